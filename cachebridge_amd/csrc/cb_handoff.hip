// CacheBridge online handoff path for MI355X (gfx950): fused source gather,
// RoPE un-rotation, split-bf16 MFMA affine map, bias, RoPE rotation, cast and
// paged scatter into the target KV pool; plus row copy (gather / install) and
// the plan that pre-packs the fitted maps.
//
// Reference algorithm (cb/ = src/cachebridge/ of the reference repository):
//   cb/mapper.py:117-239 (map_page), cb/rope.py:9-89 (RoPE),
//   cb/online/blocks.py:47-111 (pack_source_block, map_write_block).
//
// Precision: W is split at plan time into bf16 terms w = w0 + w1 (+ w2 for
// fp32 I/O); the un-rotated fp32 key is split the same way in registers.
// Products whose term indices sum below the term count are accumulated in
// fp32 by MFMA (Henry, Tang, Heinecke, "Leveraging the bfloat16 AI datatype
// for higher-precision computations", ARITH 2019): bf16 keys 3 products, bf16
// values 2 (values are bf16-exact), fp32 I/O 6.
//
// Un-rotation uses plan tables cos/m and sin/m with m = max(cos^2+sin^2, tiny)
// (cb/rope.py:86-89), so the per-element IEEE divide of the reference becomes
// a multiply; the result differs from the reference's composite rounding by at
// most a few fp32 ulp, far below the split-bf16 contraction error.

#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <numeric>
#include <string>
#include <type_traits>
#include <vector>

#include "../../include/cachebridge_hip.h"

namespace {

thread_local std::string g_last_error;

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

#define CB_HIP(expr)                                                                       \
  do {                                                                                     \
    hipError_t e_ = (expr);                                                                \
    if (e_ != hipSuccess) return fail(CB_EHIP, "%s: %s", #expr, hipGetErrorString(e_)); \
  } while (0)

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// Global-address-space pointers. Generic (flat) loads and stores also count
// against the LDS wait counter, which would make every LDS wait drain all
// outstanding HBM traffic, so every pool/table access goes through these.
#if defined(__HIP_DEVICE_COMPILE__)
#define CB_GLOBAL __attribute__((address_space(1)))
#define CB_CONST __attribute__((address_space(4)))
#define CB_LDS __attribute__((address_space(3)))
#else
#define CB_GLOBAL
#define CB_CONST
#define CB_LDS
#endif
typedef const CB_GLOBAL char* gcptr;
typedef CB_GLOBAL char* gptr;
template <typename V>
__device__ inline V gload(gcptr p) {
  return *reinterpret_cast<const CB_GLOBAL V*>(p);
}
template <typename V>
__device__ inline void gstore(gptr p, const V& v) {
  *reinterpret_cast<CB_GLOBAL V*>(p) = v;
}
// Plan metadata (job, unit and pair tables, layer pointer arrays) is read-only
// for a launch: loading it through the constant address space lets the
// compiler use scalar loads for wave-uniform indices instead of vector loads
// whose results would have to wait for every older vector load.
template <typename V>
__device__ inline V cload(const V* p) {
  return *(const CB_CONST V*)(p);
}
__device__ inline gcptr as_global(const void* p) { return (gcptr)p; }
__device__ inline gptr as_global(void* p) { return (gptr)p; }
__device__ inline const CB_GLOBAL float* gtab(const float* p) { return (const CB_GLOBAL float*)p; }

// Cache-policy operand of the LDS-DMA builtin: the non-temporal bit.
constexpr int kCachePolicyNT = 2;

constexpr int kWave = 64;
constexpr int kWaves = 4;
constexpr int kThreads = kWave * kWaves;
constexpr int kMaxClasses = CB_MAX_WINDOW_CLASSES;
constexpr int kMaxStreamBlocks = 256;  // streaming-kernel workgroups (one per CU)

// ---------------------------------------------------------------------------
// Element helpers
// ---------------------------------------------------------------------------

__device__ inline float bf2f(uint16_t h) { return __uint_as_float(static_cast<uint32_t>(h) << 16); }
__device__ inline float lo_bf(uint32_t w) { return __uint_as_float(w << 16); }
__device__ inline float hi_bf(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// Two fp32 -> packed bf16 pair, round to nearest even (v_cvt_pk_bf16_f32).
__device__ inline uint32_t pack_bf16(float a, float b) {
  const f32x2 f = {a, b};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f, bf16x2));
}

// Round-to-nearest-even fp32 -> bf16 bits (plan-time packing).
__device__ inline uint16_t f2bf(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0;
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}

template <typename IO>
struct IOTraits;
template <>
struct IOTraits<uint16_t> {  // bf16 storage
  static constexpr int NTW = 2;
  static constexpr int XT_K = 2;
  static constexpr int XT_V = 1;
  static constexpr int BYTES = 2;
};
template <>
struct IOTraits<float> {
  static constexpr int NTW = 3;
  static constexpr int XT_K = 3;
  static constexpr int XT_V = 3;
  static constexpr int BYTES = 4;
};

// Split fp32 values into XT bf16 terms (x = t0 + t1 (+ t2) + residual); N even.
// Term t of elements 2p, 2p+1 lands in dst[t][p] (packed bf16 pair).
template <int XT, int N>
__device__ inline void split_terms(const float* x, uint32_t (*dst)[N / 2]) {
#pragma unroll
  for (int p = 0; p < N / 2; ++p) {
    float a = x[2 * p], b = x[2 * p + 1];
#pragma unroll
    for (int t = 0; t < XT; ++t) {
      const uint32_t w = pack_bf16(a, b);
      dst[t][p] = w;
      a = a - lo_bf(w);
      b = b - hi_bf(w);
    }
  }
}

template <int N>
__device__ inline void load_f32(const CB_GLOBAL float* p, float* out) {
  const CB_GLOBAL float4* q = reinterpret_cast<const CB_GLOBAL float4*>(p);
#pragma unroll
  for (int u = 0; u < N / 4; ++u) {
    const float4 v = q[u];
    out[4 * u] = v.x;
    out[4 * u + 1] = v.y;
    out[4 * u + 2] = v.z;
    out[4 * u + 3] = v.w;
  }
}

// Plan RoPE tables are stored in blocks of 16 positions. Lane group g (of
// four, G = D/8 values each) holds half-row values j = g*G + 4u + e; within a
// block, the four values (u, g) of the 16 positions are consecutive float4s:
// value j of position pos sits at (pos/16)*(16*D/2) + (4u + g)*64 + (pos%16)*4
// + e. One table load of a 16-token sub-tile (16 consecutive positions x 4
// lane groups) then reads 1 KB of contiguous memory.
constexpr int kTabBlock = 16;  // positions per table block
__host__ __device__ inline int64_t tab_offset(int half, int64_t pos, int j) {
  const int G = half / 4;
  const int g = j / G, r = j % G;
  return (pos / kTabBlock) * (static_cast<int64_t>(half) * kTabBlock) + ((r / 4) * 4 + g) * 64 +
         (pos % kTabBlock) * 4 + (r % 4);
}

// Float offset of value group (u, g) of position pos (see tab_offset).
template <int G>
__device__ inline int64_t tab_chunk(int64_t pos, int u, int g) {
  return (pos / kTabBlock) * (G * 64) + (4 * u + g) * 64 + (pos % kTabBlock) * 4;
}

// Load the G table values of lane group g at position pos.
template <int G>
__device__ inline void load_tab(const CB_GLOBAL float* tab, int64_t pos, int g, float* out) {
#pragma unroll
  for (int u = 0; u < G / 4; ++u) {
    const float4 v = *reinterpret_cast<const CB_GLOBAL float4*>(tab + tab_chunk<G>(pos, u, g));
    out[4 * u] = v.x;
    out[4 * u + 1] = v.y;
    out[4 * u + 2] = v.z;
    out[4 * u + 3] = v.w;
  }
}

// Unpack 16 raw bytes of IO elements to fp32 (8 bf16 or 4 fp32).
template <typename IO>
__device__ inline void unpack16(const uint4& v, float* out) {
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
  if constexpr (IOTraits<IO>::BYTES == 2) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      out[2 * i] = lo_bf(w[i]);
      out[2 * i + 1] = hi_bf(w[i]);
    }
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) out[i] = __uint_as_float(w[i]);
  }
}

// Store N fp32 values as IO elements (N * BYTES a multiple of 8).
template <typename IO, int N>
__device__ inline void store_elems(gptr p, const float* v) {
  if constexpr (IOTraits<IO>::BYTES == 2) {
    uint32_t w[N / 2];
#pragma unroll
    for (int i = 0; i < N / 2; ++i) w[i] = pack_bf16(v[2 * i], v[2 * i + 1]);
    if constexpr (N % 8 == 0) {
#pragma unroll
      for (int u = 0; u < N / 8; ++u)
        gstore<uint4>(p + 16 * u, make_uint4(w[4 * u], w[4 * u + 1], w[4 * u + 2], w[4 * u + 3]));
    } else {
      static_assert(N == 4, "bf16 store width");
      gstore<uint2>(p, make_uint2(w[0], w[1]));
    }
  } else {
    static_assert(N % 4 == 0, "fp32 store width");
#pragma unroll
    for (int u = 0; u < N / 4; ++u)
      gstore<float4>(p + 16 * u, make_float4(v[4 * u], v[4 * u + 1], v[4 * u + 2], v[4 * u + 3]));
  }
}

// ---------------------------------------------------------------------------
// Addressing
// ---------------------------------------------------------------------------

struct DevRows {
  const void* const* k_layers;
  const void* const* v_layers;
  const char* k_base;
  const char* v_base;
  int64_t layer_stride_b;
  int64_t row_stride_b;
  int64_t rows;
  const void* index;
  int64_t index_offset;
  int32_t index_kind;
  int32_t page_size;
  int32_t head_offset;
  int32_t pad;
};

__device__ inline int64_t row_of(const DevRows& R, int t) {
  const int64_t u = t + R.index_offset;
  switch (R.index_kind) {
    case CB_INDEX_IDENTITY: return u;
    case CB_INDEX_I32: return reinterpret_cast<const CB_GLOBAL int32_t*>(as_global(R.index))[u];
    case CB_INDEX_I64: return reinterpret_cast<const CB_GLOBAL int64_t*>(as_global(R.index))[u];
    default: {
      const uint32_t ps = static_cast<uint32_t>(R.page_size);
      const uint32_t uu = static_cast<uint32_t>(u);
      const int64_t page = reinterpret_cast<const CB_GLOBAL int32_t*>(as_global(R.index))[uu / ps];
      return page * ps + uu % ps;
    }
  }
}

// row_of in two steps, so the loaded index is not consumed in the iteration
// that loads it. row_fetch issues exactly two 4-byte loads for every index
// kind (addresses chosen by uniform selects; words an index kind does not
// need read `spare`, any valid device word), so the loop's memory-operation
// count is static and nothing waits on the loads; row_finish (one iteration
// later) assembles the row: identity u, int32 slot, int64 slot, or block
// table entry * page_size + u % page_size.
__device__ inline uint2 row_fetch(const DevRows& R, int t, const CB_GLOBAL uint32_t* spare) {
  const int64_t u = t + R.index_offset;
  const uint32_t ps = static_cast<uint32_t>(R.page_size > 0 ? R.page_size : 1);
  const CB_GLOBAL uint32_t* idx =
      R.index ? reinterpret_cast<const CB_GLOBAL uint32_t*>(as_global(R.index)) : spare;
  const int k = R.index_kind;
  const int64_t w0 = k == CB_INDEX_I64 ? 2 * u : k == CB_INDEX_I32 ? u : static_cast<uint32_t>(u) / ps;
  const CB_GLOBAL uint32_t* p0 = k == CB_INDEX_IDENTITY ? spare : idx + w0;
  const CB_GLOBAL uint32_t* p1 = k == CB_INDEX_I64 ? idx + w0 + 1 : spare;
  return make_uint2(*p0, *p1);
}

__device__ inline int64_t row_finish(const DevRows& R, int t, uint2 f) {
  const int64_t u = t + R.index_offset;
  switch (R.index_kind) {
    case CB_INDEX_IDENTITY: return u;
    case CB_INDEX_I32: return static_cast<int32_t>(f.x);
    case CB_INDEX_I64: return static_cast<int64_t>((static_cast<uint64_t>(f.y) << 32) | f.x);
    default: {
      const uint32_t ps = static_cast<uint32_t>(R.page_size);
      return static_cast<int64_t>(static_cast<int32_t>(f.x)) * ps + static_cast<uint32_t>(u) % ps;
    }
  }
}

__device__ inline gcptr layer_base(const DevRows& R, int kind, int layer) {
  const void* const* arr = kind ? R.v_layers : R.k_layers;
  if (arr) return as_global(cload(arr + layer));
  return as_global(kind ? R.v_base : R.k_base) + layer * R.layer_stride_b;
}

// ---------------------------------------------------------------------------
// Launch arguments and work decode
// ---------------------------------------------------------------------------

struct MapArgs {
  const uint4* w;
  const float* bias;
  const int4* jobs;
  const int32_t* pairs;
  const int32_t* unit_job;      // first job of each unit (jobs of a unit are consecutive)
  const int32_t* unit_njobs;    // jobs in each unit
  const int32_t* unit_group;    // source group of each unit
  const int32_t* group_unit_start;
  const int32_t* group_unit_count;
  const float* cos_tab;   // rotation tables [theta][pos][D/2]
  const float* sin_tab;
  const float* ucos_tab;  // un-rotation tables cos/m, sin/m
  const float* usin_tab;
  int64_t theta_stride;   // elements per theta table
  DevRows src;
  DevRows tgt;
  int32_t n_tokens;
  int32_t position_start;
  int32_t support;
  int32_t chunk;
  int32_t ncls;
  int32_t cls_unit_begin[kMaxClasses];
  int32_t cls_tok_first[kMaxClasses];
  int32_t cls_tok_count[kMaxClasses];
  int32_t cls_nchunks[kMaxClasses];
  int32_t cls_item_begin[kMaxClasses + 1];
  int32_t total_items;
  int32_t padded_items;
  // Streaming kernel: cost-balanced ranges (one workgroup per CU).
  int32_t cls_unit_end[kMaxClasses];
  int32_t cls_subtiles[kMaxClasses];     // 16-token sub-tiles of each class's tokens
  int32_t num_units;
  int32_t num_blocks;
  // Range r of the cost line covers (unit, sub-tile) from blk_unit/sub[r] to
  // blk_unit/sub[r + 1] (cut on the host, split_cost_line).
  int32_t blk_unit[kMaxStreamBlocks + 1];
  int32_t blk_sub[kMaxStreamBlocks + 1];
  int32_t* err;
  void* sink;  // scratch destination of stores without a target row
  const void* zero;  // one all-zero head row: the gather source of tokens without a source row
  // Batched launches: position of every token (tokens then index resolved
  // rows: src/tgt are int32 row vectors over the same token space). Null for
  // one request, whose token t sits at position_start + t.
  const int32_t* pos;
  // Streaming kernel work pool: after its own range, each workgroup claims
  // chunks of the cost line's tail [(pool_u0, pool_s0), end) until pool_n are
  // taken (pool_n 0: no pool). Chunks hold pool_gs sub-tiles (fewer at a
  // unit's end) and never span two units.
  uint32_t* pool_ctr;  // this launch's (claims, finished workgroups)
  int32_t pool_n;
  int32_t pool_u0;
  int32_t pool_s0;
  int32_t pool_gs;
};

// Job flag (meta.z): un-rotation uses the rotation table (same theta, unit norm).
constexpr int kJobSharedTables = 1;

struct Work {
  int job, njobs, tok_lo, tok_hi;
};

// Logical item L (in XCD-aware order) -> (unit, token range). Items are
// ordered window class, source group, chunk, unit-in-group, so units that
// read the same source rows run back to back on one XCD and share its L2.
__device__ inline bool decode_work(const MapArgs& a, Work* w) {
  const int per = a.padded_items >> 3;
  const int L = (blockIdx.x & 7) * per + (blockIdx.x >> 3);
  if (L >= a.total_items) return false;
  int c = 0;
  while (c + 1 < a.ncls && L >= a.cls_item_begin[c + 1]) ++c;
  const int lc = L - a.cls_item_begin[c];
  const int nch = a.cls_nchunks[c];
  const int ub = a.cls_unit_begin[c];
  const int grp = a.unit_group[ub + lc / nch];
  const int us = a.group_unit_start[grp];
  const int un = a.group_unit_count[grp];
  const int r = lc - (us - ub) * nch;
  const int chunk_id = r / un;
  const int unit = us + r % un;
  w->job = cload(a.unit_job + unit);
  w->njobs = cload(a.unit_njobs + unit);
  w->tok_lo = a.cls_tok_first[c] + chunk_id * a.chunk;
  w->tok_hi = min(w->tok_lo + a.chunk, a.cls_tok_first[c] + a.cls_tok_count[c]);
  return true;
}

// Streaming kernel work split: workgroup b takes range (b & 7) *
// (num_blocks / 8) + (b >> 3) of the cost line, so each XCD owns one
// contiguous eighth of it and units that read the same source rows (adjacent
// in the unit order) share that XCD's L2.
struct Pos {
  int unit, sub;
};
static_assert(sizeof(MapArgs) <= 4096, "kernel arguments must fit 4 KB");

// Position of token t of the launch (see MapArgs::pos).
__device__ inline int position_of(const MapArgs& a, int t) {
  return a.pos ? reinterpret_cast<const CB_GLOBAL int32_t*>(as_global(a.pos))[t] : a.position_start + t;
}

__host__ __device__ inline int class_of_unit(const MapArgs& a, int u) {
  int c = 0;
  while (c + 1 < a.ncls && u >= a.cls_unit_end[c]) ++c;
  return c;
}

// Work-pool chunk idx -> (unit, first sub-tile), or false past the pool. The
// tail from (pool_u0, pool_s0) is cut unit by unit into chunks of pool_gs
// sub-tiles (the first unit's from pool_s0); every unit of a window class has
// the same sub-tiles, so a class's chunks are counted in closed form from the
// kernel arguments alone (no memory loads).
__host__ __device__ inline bool pool_chunk(const MapArgs& a, int64_t idx, int* unit, int* sub) {
  const int gs = a.pool_gs;
  int u = a.pool_u0;
  int c = class_of_unit(a, u);
  {
    const int ns = a.cls_subtiles[c];
    const int64_t first = ns > a.pool_s0 ? (ns - a.pool_s0 + gs - 1) / gs : 0;
    if (idx < first) {
      *unit = u;
      *sub = a.pool_s0 + static_cast<int>(idx) * gs;
      return true;
    }
    idx -= first;
    ++u;
  }
  for (; c < a.ncls && u < a.num_units; ++c) {
    const int cend = c + 1 < a.ncls ? a.cls_unit_end[c] : a.num_units;
    if (u >= cend) continue;
    const int64_t per = (a.cls_subtiles[c] + gs - 1) / gs;
    const int64_t n = static_cast<int64_t>(cend - u) * per;
    if (idx < n) {
      *unit = u + static_cast<int>(idx / per);
      *sub = static_cast<int>(idx % per) * gs;
      return true;
    }
    idx -= n;
    u = cend;
  }
  return false;
}

// MFMA product schedule: term pairs (i of x, j of w) with i + j < NTW, small first.
template <int XT, int NTW, typename F>
__device__ inline void for_products(F&& f) {
#pragma unroll
  for (int lvl = NTW - 1; lvl >= 0; --lvl) {
#pragma unroll
    for (int i = 0; i < XT; ++i) {
      const int j = lvl - i;
      if (j >= 0 && j < NTW) f(i, j);
    }
  }
}

__device__ inline f32x4 mfma(const bf16x8& a, const bf16x8& b, const f32x4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// Input dim of (k-step ks, lane group g, element e): lane group g holds dims
// [g*D/8, (g+1)*D/8) of both halves, k-steps walk the first half then the second.
__host__ __device__ inline int in_dim(int D, int ks, int g, int e) {
  const int per_half = D / 64;
  return (ks / per_half) * (D / 2) + g * (D / 8) + (ks % per_half) * 8 + e;
}

// ---------------------------------------------------------------------------
// Streaming kernel (support s == 1)
//
// Workgroup = 8 waves; it owns one unit -- up to two jobs of the same kind
// that read the same source (layer, head) -- and a contiguous token range.
// The split-term W blocks and biases of the unit's jobs are staged in LDS once
// (64 KB per job for D=128 bf16); then each wave independently streams
// 16-token sub-tiles (sub-tile w, w+8, ...) with no further barriers, so the
// waves of a CU drift apart and one wave's MFMAs overlap another's gather,
// un-rotation and stores. Per sub-tile the source rows, RoPE table rows,
// target slots and the un-rotated split fragments are produced once and used
// by every job of the unit.
//
// Lane (col, g) holds token col of the sub-tile and input dims
// [g*D/8, (g+1)*D/8) of both halves; output dims are permuted at pack time so
// the lane holds the same dims of the result: RoPE partners j and j+D/2 sit
// in one lane, and un-rotation and rotation read the same table rows.
// ---------------------------------------------------------------------------

constexpr int kUnitJobs = 2;                     // jobs per streaming unit
constexpr int kStreamWaves = 8;
constexpr int kStreamThreads = kWave * kStreamWaves;
constexpr int kSubTokens = 16;                   // tokens per wave sub-tile
constexpr int kSinkBytes = kWave * 128 * 4;       // one head row (D <= 128, fp32) per lane
constexpr int kZeroBytes = 128 * 4;               // one zero head row, after the sink

__host__ __device__ inline int gen_out_dim(int D, int rt, int r) {
  const int per_half = D / 32;
  return (rt / per_half) * (D / 2) + (r / 4) * (D / 8) + 4 * (rt % per_half) + (r % 4);
}

// Stage NU4 uint4 into LDS with NT threads (NU4 a multiple of NT).
template <int NU4, int NT, int MAXB = 8>
__device__ inline void copy_to_lds(uint4* lds, const uint4* __restrict__ src) {
  constexpr int PER = NU4 / NT;
  constexpr int B = PER < MAXB ? PER : MAXB;
  static_assert(NU4 % NT == 0 && PER % B == 0, "block size");
  for (int base = 0; base < NU4; base += NT * B) {
    uint4 v[B];
#pragma unroll
    for (int i = 0; i < B; ++i) v[i] = src[base + i * NT + threadIdx.x];
#pragma unroll
    for (int i = 0; i < B; ++i) lds[base + i * NT + threadIdx.x] = v[i];
  }
}

template <int D, typename IO>
struct Gm {
  using T = IOTraits<IO>;
  static constexpr int NTW = T::NTW;
  static constexpr int BYTES = T::BYTES;
  static constexpr int HALF = D / 2;
  static constexpr int KS = D / 32;
  static constexpr int RT = D / 16;
  static constexpr int G = D / 8;                 // dims per lane group per half
  static constexpr int E16 = 16 / BYTES;          // elements per 16-byte load
  static constexpr int RUN_U4 = G / E16;          // 16-byte loads per half-run
  static constexpr int W_U4 = RT * KS * NTW * kWave;
};

template <int D, typename IO, bool IS_K, bool SHARED, int NJ, int CT, bool POS>
__device__ void stream_run(const MapArgs& a, uint4* lds_w, float* lds_bias, int* lds_next, const Work& wk) {
  // No implicit contraction: every fused multiply-add is written out, so every
  // instantiation rounds identically and a job's rows are bit-identical
  // whichever unit shape or plan computes them. (The rotations use explicit
  // FMAs; the reference's separately rounded fp32 ops differ from them by at
  // most one fp32 rounding, far below the bf16 result's.)
#pragma clang fp contract(off)
  using C = Gm<D, IO>;
  using T = IOTraits<IO>;
  constexpr int NTW = C::NTW;
  constexpr int XT = IS_K ? T::XT_K : T::XT_V;
  constexpr int KS = C::KS, RT = C::RT, G = C::G, HALF = C::HALF;
  constexpr int kind = IS_K ? CB_KIND_K : CB_KIND_V;
  constexpr int TG = IS_K ? G : 1;   // un-rotation table values per lane (keys only)
  constexpr int NGRP = RT / 4;       // row-tile groups: tiles {2h, 2h+1} and partners {2h, 2h+1} + RT/2
  constexpr int NSTEP = 4 * KS;      // (row tile, k-step) steps of one group
  constexpr int SUBT = 16 * CT;      // tokens per wave sub-tile (CT column tiles share each W fragment)
  // Keys of a batched launch read each token's position from a.pos (issued
  // with the index words); otherwise token t sits at position_start + t.
  constexpr bool PV = POS && IS_K;

  const int lane = threadIdx.x & (kWave - 1);
  // Wave-uniform (scalar), so sub-tile indices and the loop stay uniform.
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int g = lane >> 4;
  const int col = lane & 15;

  // Job metadata: scalar loads at a wave-uniform index.
  const int job = __builtin_amdgcn_readfirstlane(wk.job);
  const int* jm = reinterpret_cast<const int*>(a.jobs + job);  // int4 per job: x, y, z, w
  const int meta_y = cload(jm + 1);
  const int sth = (meta_y >> 16) & 0xff;
  const int tth = (meta_y >> 24) & 0xff;
  const int pr = cload(a.pairs + job);
  const int sl = pr & 0xffff;
  const int sh = pr >> 16;

  gptr tbase[NJ];
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const int mx = cload(jm + 4 * j);
    tbase[j] = const_cast<gptr>(layer_base(a.tgt, kind, mx & 0xffff)) +
               static_cast<int64_t>((mx >> 16) - a.tgt.head_offset) * D * C::BYTES;
  }
  // Stores of tokens without a target row go to a scratch sink, so every
  // iteration issues a fixed number of memory operations (the compiler can
  // then wait for the prefetched loads without also waiting for the stores).
  gptr sink = as_global(a.sink) + lane * (D * C::BYTES);

  gcptr sbase = layer_base(a.src, kind, sl) + static_cast<int64_t>(sh - a.src.head_offset) * D * C::BYTES;
  const CB_GLOBAL float* ucos = gtab(SHARED ? a.cos_tab : a.ucos_tab) + sth * a.theta_stride;
  const CB_GLOBAL float* usin = gtab(SHARED ? a.sin_tab : a.usin_tab) + sth * a.theta_stride;
  const CB_GLOBAL float* rcos = gtab(a.cos_tab) + tth * a.theta_stride;
  const CB_GLOBAL float* rsin = gtab(a.sin_tab) + tth * a.theta_stride;

  const int n = wk.tok_hi - wk.tok_lo;
  const int nsub = (n + SUBT - 1) / SUBT;
  int errbits = 0;
  // Source and target rows of this lane's tokens in sub-tile `sub` (-1: skip).
  // Index loads are issued four sub-tiles (of this wave) ahead and resolved
  // two ahead, when that sub-tile's source dims are requested; tokens past
  // the range re-read the range's last token and are masked.
  const CB_GLOBAL uint32_t* spare = reinterpret_cast<const CB_GLOBAL uint32_t*>(as_global(a.sink));
  auto index_of = [&](int sub, int ct) { return sub * SUBT + ct * 16 + col; };
  auto token_of = [&](int sub, int ct) { return wk.tok_lo + min(index_of(sub, ct), n - 1); };
  auto fetch_rows = [&](int sub, uint2 (&fs)[CT], uint2 (&fd)[CT], int32_t (&fp)[CT]) {
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) {
      fs[ct] = row_fetch(a.src, token_of(sub, ct), spare);
      fd[ct] = row_fetch(a.tgt, token_of(sub, ct), spare);
      if constexpr (PV) fp[ct] = reinterpret_cast<const CB_GLOBAL int32_t*>(as_global(a.pos))[token_of(sub, ct)];
    }
  };
  auto finish_rows = [&](int sub, const uint2 (&fs)[CT], const uint2 (&fd)[CT], const int32_t (&fp)[CT],
                         int32_t (&sr)[CT], int32_t (&tr)[CT], int32_t (&pr)[CT]) {
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) {
      const int t = token_of(sub, ct);
      pr[ct] = PV ? fp[ct] : a.position_start + t;
      const int64_t s = row_finish(a.src, t, fs[ct]);
      const int64_t d = row_finish(a.tgt, t, fd[ct]);
      const bool live = index_of(sub, ct) < n;
      const bool sok = s >= 0 && s < a.src.rows;
      const bool dok = d >= 0 && d < a.tgt.rows;
      errbits |= live ? (sok ? 0 : 1) | (dok ? 0 : 2) : 0;
      // A token whose source row is out of range writes nothing: its store
      // goes to the sink, so its target row keeps its old contents.
      sr[ct] = live && sok ? static_cast<int32_t>(s) : -1;
      tr[ct] = live && dok && sok ? static_cast<int32_t>(d) : -1;
    }
  };

  // Source dims of this wave's sub-tiles are requested two sub-tiles ahead
  // (slot = k & 1 for its k-th sub-tile; first-touch source rows come from
  // HBM), un-rotation tables one ahead (they are shared by every key unit and
  // stay cached).
  uint4 xr[2][CT][2][C::RUN_U4];
  float uc[CT][TG], us[CT][TG];
  gcptr zrow = as_global(a.zero);
  auto prefetch_x = [&](auto slot, const int32_t (&srow)[CT]) {
    constexpr int st = decltype(slot)::value;
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) {
      // Tokens without a source row gather the plan's zero row.
      gcptr p = (srow[ct] >= 0 ? sbase + static_cast<int64_t>(srow[ct]) * a.src.row_stride_b : zrow) +
                g * G * C::BYTES;
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int u = 0; u < C::RUN_U4; ++u)
          xr[st][ct][h][u] = gload<uint4>(p + (h * HALF + u * C::E16) * C::BYTES);
    }
  };
  auto prefetch_tab = [&](int sub, const int32_t (&prow)[CT]) {
    if constexpr (IS_K) {
#pragma unroll
      for (int ct = 0; ct < CT; ++ct) {
        const int64_t pos = PV ? prow[ct] : a.position_start + token_of(sub, ct);
        load_tab<G>(ucos, pos, g, uc[ct]);
        load_tab<G>(usin, pos, g, us[ct]);
      }
    }
  };

  // Sub-tiles are claimed in order by each wave: its first three statically
  // (wave + 8k), the rest from a workgroup counter in LDS as the wave moves
  // along, so faster waves take more of the segment and all waves finish
  // within about one sub-tile of each other. A claim is made when its index
  // loads are issued, three sub-tiles ahead of its multiply.
  constexpr int SW = kStreamWaves;
  constexpr int kStatic = 3 * SW;
  int c0 = wave, c1 = wave + SW, c2 = wave + 2 * SW;  // current, next, after-next
  auto claim = [&]() {  // one claim per wave, broadcast to all lanes
    int v = 0;
    if (lane == 0) v = atomicAdd(lds_next, 1);
    return __builtin_amdgcn_readfirstlane(v);
  };

  // Segment start: the first three sub-tiles' rows and the first two's source
  // dims are requested before waiting for the workgroup's previous segment
  // to release LDS, so their latency overlaps that segment's tail.
  int32_t tr_a[CT], pr_a[CT], tr_b[CT], pr_b[CT];  // rows / positions of the current and next sub-tile
  uint2 fs_c[CT], fd_c[CT];                        // index words of the sub-tile after next
  int32_t fp_c[CT];                                // its position words (batched keys)
  {
    uint2 fs_a[CT], fd_a[CT], fs_b[CT], fd_b[CT];
    int32_t fp_a[CT], fp_b[CT], sr0[CT], sr1[CT];
    fetch_rows(c0, fs_a, fd_a, fp_a);
    fetch_rows(c1, fs_b, fd_b, fp_b);
    fetch_rows(c2, fs_c, fd_c, fp_c);
    finish_rows(c0, fs_a, fd_a, fp_a, sr0, tr_a, pr_a);
    finish_rows(c1, fs_b, fd_b, fp_b, sr1, tr_b, pr_b);
    prefetch_x(std::integral_constant<int, 0>{}, sr0);
    prefetch_x(std::integral_constant<int, 1>{}, sr1);
    prefetch_tab(c0, pr_a);
  }
  constexpr int WPER = NJ * C::W_U4 / kStreamThreads;
  static_assert(NJ * C::W_U4 % kStreamThreads == 0 && NJ * D <= kStreamThreads, "staging split");
  const float breg = threadIdx.x < NJ * D ? a.bias[static_cast<size_t>(job) * D + threadIdx.x] : 0.f;
  __syncthreads();  // the previous segment no longer reads LDS (nor claims)
  // The unit's W goes straight from memory into LDS (16 bytes per lane, each
  // wave filling 1 KB runs), with no register staging. Waiting for every
  // older load here costs little: W is the last thing requested, and the
  // loop then starts with nothing outstanding. The loads are non-temporal
  // (W is read once per segment), which leaves L2 to the source rows and
  // RoPE tables.
  {
    gcptr wsrc = as_global(a.w + static_cast<size_t>(job) * C::W_U4);
    const int wv = __builtin_amdgcn_readfirstlane(wave);
#pragma unroll
    for (int i = 0; i < WPER; ++i)
      __builtin_amdgcn_global_load_lds(wsrc + (i * kStreamThreads + threadIdx.x) * 16,
                                       (CB_LDS void*)(lds_w + i * kStreamThreads + wv * kWave), 16, 0,
                                       kCachePolicyNT);
    __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0) expcnt(7) lgkmcnt(15)
  }
  if (threadIdx.x < NJ * D) lds_bias[threadIdx.x] = breg;
  if (threadIdx.x == 0) *lds_next = kStatic;
  __syncthreads();  // W, bias and claim counter ready

  // One sub-tile of this wave; the source slot is a compile-time constant
  // (register arrays indexed at run time would be placed in scratch memory).
  auto body = [&](auto slot) {
    constexpr int st = decltype(slot)::value;
    const int sub = c0;
    // W fragments are re-read from LDS every sub-tile: keep the compiler from
    // hoisting them into registers.
    asm volatile("" ::: "memory");
    int32_t trow[CT], prow[CT];
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) {
      trow[ct] = tr_a[ct];
      prow[ct] = pr_a[ct];
    }
    // Keys with separate rotation tables: this sub-tile's rotation values are
    // requested first, before this iteration's prefetches, so the epilogue's
    // wait for them leaves those prefetches in flight (loads and stores share
    // one in-order counter).
    constexpr bool RSEP = IS_K && !SHARED;
    float rcb[RSEP ? CT : 1][RSEP ? NGRP : 1][8], rsb[RSEP ? CT : 1][RSEP ? NGRP : 1][8];
    if constexpr (RSEP) {
#pragma unroll
      for (int ct = 0; ct < CT; ++ct) {
        const int64_t pos = PV ? prow[ct] : a.position_start + token_of(sub, ct);
#pragma unroll
        for (int hg = 0; hg < NGRP; ++hg)
#pragma unroll
          for (int u = 0; u < 2; ++u) {
            const int64_t off = tab_chunk<G>(pos, 2 * hg + u, g);
            const float4 cv = *reinterpret_cast<const CB_GLOBAL float4*>(rcos + off);
            const float4 sv = *reinterpret_cast<const CB_GLOBAL float4*>(rsin + off);
            float* c = rcb[ct][hg] + 4 * u;
            float* sn = rsb[ct][hg] + 4 * u;
            c[0] = cv.x; c[1] = cv.y; c[2] = cv.z; c[3] = cv.w;
            sn[0] = sv.x; sn[1] = sv.y; sn[2] = sv.z; sn[3] = sv.w;
          }
      }
    }

    // Un-rotate (keys) and split the current sub-tile into B fragments.
    // Values stored as bf16 are their own single term: the loaded 16 bytes
    // (8 consecutive dims of one half) are the fragment of k-step ks.
    bf16x8 bx[CT][KS][XT];
    float tc[CT][SHARED ? G : 1], ts[CT][SHARED ? G : 1];
    constexpr bool RAW = !IS_K && XT == 1 && C::BYTES == 2;
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) {
      if constexpr (RAW) {
#pragma unroll
        for (int ks = 0; ks < KS; ++ks)
          bx[ct][ks][0] = __builtin_bit_cast(bf16x8, xr[st][ct][ks / (KS / 2)][ks % (KS / 2)]);
        continue;
      }
      float x1[G], x2[G];
#pragma unroll
      for (int u = 0; u < C::RUN_U4; ++u) {
        unpack16<IO>(xr[st][ct][0][u], x1 + u * C::E16);
        unpack16<IO>(xr[st][ct][1][u], x2 + u * C::E16);
      }
      if constexpr (IS_K) {
#pragma unroll
        for (int e = 0; e < G; ++e) {
          const float k1 = __builtin_fmaf(x1[e], uc[ct][e], x2[e] * us[ct][e]);
          const float k2 = __builtin_fmaf(x2[e], uc[ct][e], -(x1[e] * us[ct][e]));
          x1[e] = k1;
          x2[e] = k2;
        }
        if constexpr (SHARED) {
#pragma unroll
          for (int e = 0; e < G; ++e) {
            tc[ct][e] = uc[ct][e];
            ts[ct][e] = us[ct][e];
          }
        }
      }
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const float* src = (ks / (KS / 2) ? x2 : x1) + (ks % (KS / 2)) * 8;
        uint32_t tw[XT][4];
        split_terms<XT, 8>(src, tw);
#pragma unroll
        for (int x = 0; x < XT; ++x)
          bx[ct][ks][x] = __builtin_bit_cast(bf16x8, make_uint4(tw[x][0], tw[x][1], tw[x][2], tw[x][3]));
      }
    }
    // Next sub-tile's tables; the one after: resolve its rows and request its
    // source dims into the slot just consumed; claim the next and issue its
    // index loads.
    prefetch_tab(c1, pr_b);
    int c3;
    {
      int32_t sr2[CT], tr2[CT], pr2[CT];
      finish_rows(c2, fs_c, fd_c, fp_c, sr2, tr2, pr2);
      prefetch_x(slot, sr2);
      c3 = claim();
      fetch_rows(c3, fs_c, fd_c, fp_c);
#pragma unroll
      for (int ct = 0; ct < CT; ++ct) {
        tr_a[ct] = tr_b[ct];
        pr_a[ct] = pr_b[ct];
        tr_b[ct] = tr2[ct];
        pr_b[ct] = pr2[ct];
      }
    }

    // Store rows of this sub-tile, once per job and column tile (the sink for
    // tokens without a target row), chosen without branches.
    gptr dst[NJ][CT];
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) {
      const int64_t roff = static_cast<int64_t>(max(trow[ct], 0)) * a.tgt.row_stride_b;
#pragma unroll
      for (int j = 0; j < NJ; ++j) dst[j][ct] = trow[ct] >= 0 ? tbase[j] + roff : sink;
    }

#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const uint4* wj = lds_w + j * C::W_U4;
#pragma unroll
      for (int hg = 0; hg < NGRP; ++hg) {
        // Row tiles of this group: 2hg, 2hg+1 and their partners.
        auto tile = [&](int q) { return 2 * hg + (q & 1) + (q >> 1) * (RT / 2); };
        // The bias of each row tile is the accumulator input of its first
        // product (no register copies per column tile).
        f32x4 acc[4][CT], bq[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const float* b = lds_bias + j * D + gen_out_dim(D, tile(q), 4 * g);
          bq[q] = f32x4{b[0], b[1], b[2], b[3]};
        }
        // W fragments flow through a three-slot ring, read two steps ahead;
        // each fragment feeds the CT column tiles.
        bf16x8 ring[3][NTW];
        auto read_w = [&](int t, bf16x8 (&dst)[NTW]) {
          const int rt = tile(t / KS), ks = t % KS;
#pragma unroll
          for (int w = 0; w < NTW; ++w)
            dst[w] = __builtin_bit_cast(bf16x8, wj[((rt * KS + ks) * NTW + w) * kWave + lane]);
        };
        {
          read_w(0, ring[0]);
          read_w(1, ring[1]);
#pragma unroll
          for (int t = 0; t < NSTEP; ++t) {
            if (t + 2 < NSTEP) read_w(t + 2, ring[(t + 2) % 3]);
            const int ks = t % KS, q = t / KS;
#pragma unroll
            for (int ct = 0; ct < CT; ++ct) {
              int pi = 0;
              for_products<XT, NTW>([&](int ii, int jj) {
                const f32x4 c = ks == 0 && pi == 0 ? bq[q] : acc[q][ct];
                acc[q][ct] = mfma(ring[t % 3][jj], bx[ct][ks][ii], c);
                ++pi;
              });
            }
            __builtin_amdgcn_sched_barrier(0);
          }
        }
        // Epilogue of the group: 8 output dims of each half, target RoPE
        // (keys), cast, 16-byte stores.
#pragma unroll
        for (int ct = 0; ct < CT; ++ct) {
          float o1[8], o2[8];
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            o1[q] = acc[0][ct][q];
            o1[4 + q] = acc[1][ct][q];
            o2[q] = acc[2][ct][q];
            o2[4 + q] = acc[3][ct][q];
          }
          if constexpr (IS_K) {
            float cbuf[8], sbuf[8];
            if constexpr (SHARED) {
#pragma unroll
              for (int e = 0; e < 8; ++e) {
                cbuf[e] = tc[ct][8 * hg + e];
                sbuf[e] = ts[ct][8 * hg + e];
              }
            } else {
#pragma unroll
              for (int e = 0; e < 8; ++e) {
                cbuf[e] = rcb[RSEP ? ct : 0][RSEP ? hg : 0][e];
                sbuf[e] = rsb[RSEP ? ct : 0][RSEP ? hg : 0][e];
              }
            }
#pragma unroll
            for (int e = 0; e < 8; ++e) {
              const float y1 = o1[e], y2 = o2[e];
              o1[e] = __builtin_fmaf(y1, cbuf[e], -(y2 * sbuf[e]));
              o2[e] = __builtin_fmaf(y2, cbuf[e], y1 * sbuf[e]);
            }
          }
          gptr p = dst[j][ct];
          store_elems<IO, 8>(p + (g * G + 8 * hg) * C::BYTES, o1);
          store_elems<IO, 8>(p + (HALF + g * G + 8 * hg) * C::BYTES, o2);
        }
      }
    }
    c0 = c1;
    c1 = c2;
    c2 = c3;
  };
  while (c0 < nsub) {
    body(std::integral_constant<int, 0>{});
    if (c0 >= nsub) break;
    body(std::integral_constant<int, 1>{});
  }
  if (errbits) atomicOr(a.err, errbits);
}

template <int D, typename IO, bool POS>
__global__ __launch_bounds__(kStreamThreads) void map_install_stream_kernel(MapArgs a) {
  __shared__ uint4 lds_w[kUnitJobs * Gm<D, IO>::W_U4];
  __shared__ float lds_bias[kUnitJobs * D];
  __shared__ int lds_next;  // next sub-tile to claim in the current segment
  __shared__ int lds_chunk;  // work-pool chunk claimed by the workgroup
  const int per = a.num_blocks >> 3;
  const int r = (blockIdx.x & 7) * per + (blockIdx.x >> 3);
  Pos cur{a.blk_unit[r], a.blk_sub[r]};
  const Pos end{a.blk_unit[r + 1], a.blk_sub[r + 1]};
  // One segment: sub-tiles [sub0, stop) of unit u_in (stop > sub0).
  auto seg = [&](int u_in, int sub0, int stop) __attribute__((always_inline)) {
    const int c = class_of_unit(a, u_in);
    {
      Work wk;
      const int unit = __builtin_amdgcn_readfirstlane(u_in);  // wave-uniform: scalar loads
      wk.job = __builtin_amdgcn_readfirstlane(cload(a.unit_job + unit));
      wk.njobs = cload(a.unit_njobs + unit);
      wk.tok_lo = a.cls_tok_first[c] + sub0 * kSubTokens;
      wk.tok_hi = min(a.cls_tok_first[c] + stop * kSubTokens, a.cls_tok_first[c] + a.cls_tok_count[c]);
      const int* mp = reinterpret_cast<const int*>(a.jobs + wk.job);
      const int meta_y = cload(mp + 1), meta_z = cload(mp + 2);
      const bool two = wk.njobs == 2;
      if ((meta_y & 0xff) == CB_KIND_K) {
        if (meta_z & kJobSharedTables) {
          if (two) stream_run<D, IO, true, true, 2, 1, POS>(a, lds_w, lds_bias, &lds_next, wk);
          else stream_run<D, IO, true, true, 1, 1, POS>(a, lds_w, lds_bias, &lds_next, wk);
        } else {
          if (two) stream_run<D, IO, true, false, 2, 1, POS>(a, lds_w, lds_bias, &lds_next, wk);
          else stream_run<D, IO, true, false, 1, 1, POS>(a, lds_w, lds_bias, &lds_next, wk);
        }
      } else {
        if (two) stream_run<D, IO, false, false, 2, 2, POS>(a, lds_w, lds_bias, &lds_next, wk);
        else stream_run<D, IO, false, false, 1, 2, POS>(a, lds_w, lds_bias, &lds_next, wk);
      }
    }
  };
  while (cur.unit < end.unit || (cur.unit == end.unit && cur.sub < end.sub)) {
    const int c = class_of_unit(a, cur.unit);
    const int stop = cur.unit == end.unit ? end.sub : a.cls_subtiles[c];
    if (stop > cur.sub) seg(cur.unit, cur.sub, stop);
    cur = Pos{cur.unit + 1, 0};
  }
  if (a.pool_n <= 0) return;
  // Work pool: a workgroup done with its own range claims chunks of the
  // line's tail in order until all pool_n are taken. (The segment body is
  // instantiated twice: one loop for both kinds of segments made the compiler
  // reserve a private segment.)
  for (;;) {
    __syncthreads();  // every wave has read the previous claim
    if (threadIdx.x == 0) lds_chunk = static_cast<int>(atomicAdd(a.pool_ctr, 1u));
    __syncthreads();
    const int idx = __builtin_amdgcn_readfirstlane(lds_chunk);
    if (idx >= a.pool_n) break;
    int pu = 0, ps = 0;
    if (!pool_chunk(a, idx, &pu, &ps)) {  // pool_n exceeds the tail's chunks: a host-side bug
      if (threadIdx.x == 0) atomicOr(a.err, 4);
      break;
    }
    seg(pu, ps, min(a.cls_subtiles[class_of_unit(a, pu)], ps + a.pool_gs));
  }
  // The last workgroup to finish clears the launch's counter pair (every
  // claim of the launch has been made by then), so the next launch on this
  // pair starts from zero without a host-side clear. A launch that had the
  // pair to itself made exactly pool_n successful claims plus one failed
  // claim per workgroup; any other count means another launch shared the
  // pair (chunks may have gone to it and rows may be missing), which is
  // reported in bit 3 of the error word instead of passing silently.
  if (threadIdx.x == 0) {
    const uint32_t done = atomicAdd(a.pool_ctr + 1, 1u);
    if (done == gridDim.x - 1) {
      const uint32_t claims = atomicExch(a.pool_ctr, 0u);
      atomicExch(a.pool_ctr + 1, 0u);
      if (claims != static_cast<uint32_t>(a.pool_n) + gridDim.x) atomicOr(a.err, 8);
    } else if (done >= gridDim.x) {
      atomicOr(a.err, 8);
    }
  }
}

// ---------------------------------------------------------------------------
// Support kernel (support s > 1, head_dim 128, bf16 K/V).
//
// A target job's feature row is the concatenation of its s source rows, so a
// job is a [T x s*128] . [s*128 x 128] contraction. An item is one 256-token
// block of one job; the 8 waves of the (persistent, one per CU) workgroup
// work on the same item, wave w on its tokens 32w .. 32w + 31, and each wave
// computes all 128 outputs of its tokens with v_mfma_f32_32x32x16_bf16 into
// 64 accumulator VGPRs (four 32-row tiles).
//
// Stages: the item's input dims stream in 32-dim k-steps ks of each support
// member k, in pairs (k-step q, then its RoPE partners q + 2), q = 0 for every
// member, then q = 1: 4 s stages per item. Members are visited in ascending
// (source layer, head) order.
//
// Memory traffic of the stage loop is LDS DMA only (global_load_lds_dwordx4,
// nothing staged in registers), waited for with explicit counts:
//   - each stage's split W (four row tiles x two 16-dim MFMA k-steps x two
//     bf16 terms, 16 KB) goes into a four-slot LDS ring three stages ahead,
//     one workgroup barrier per stage publishing the stage after next and
//     freeing the slot just used;
//   - each wave's source rows of a k-step pair (its 32 tokens x 64 bytes,
//     and their RoPE partners) go into its own two-buffer LDS area two
//     stages ahead, 16 tokens x one 64-byte sector per instruction.
// Without these two distances the gathers' latency, not the MFMAs, set the
// kernel's pace: the token rows are scattered 64-byte sectors, many of them
// from beyond L2.
//
// Every wave produces its own input: the split bf16 terms of the next k-step
// pair are built (keys un-rotated, split) from its LDS rows while the current
// pair's MFMAs run, half of them in each of the pair's two stages. On gfx950
// an MFMA leaves its own wave free to issue other instructions while it
// executes, but a second wave's VALU work on the same SIMD does not overlap
// another wave's MFMAs; keeping the conversion inside the MFMA wave's
// instruction stream is what lets it hide.
//
// Items go to XCDs in runs of adjacent jobs (SupItems below), so that the
// items running on one XCD at a time share source rows in its L2.
//
// Lane layout (lane l: token n = l % 32 of the wave, half h = l / 32):
//   input: MFMA k-step kk of 32-dim k-step ks covers member dims
//          32 ks + 16 h + 8 kk + e (e = 0..7) in lane half h, so a lane
//          reads 32 contiguous bytes of its token's row per k-step and its
//          RoPE partners (ks + 2) sit in the same lane;
//   output: row r = 8v + 4h' + u of row tile t is output dim
//          64 (t >> 1) + 32 (t & 1) + 16 (v >> 1) + 8 h' + 4 (v & 1) + u; the
//          accumulator register 4v + u of lane (n, h) holds row 8v + 4h + u,
//          so tiles t and t + 2 hold RoPE partners in the same register and a
//          lane's outputs are runs of 8 dims (16-byte stores).
// W is packed [job][stage][kk][row tile][term][lane][8 bf16] in the order the
// stages are consumed: stage i covers pair p = i / 2 (k-step half q = p / S,
// member p % S) at 32-dim k-step q + 2 (i & 1).
// ---------------------------------------------------------------------------

// s_waitcnt immediates (vmcnt in bits 3:0, expcnt 6:4, lgkmcnt 11:8; the
// other counters left at their maximum, i.e. not waited for).
constexpr int kVmcnt0 = 0x0f70;
constexpr int kVmcnt2 = 0x0f72;
constexpr int kVmcnt6 = 0x0f76;

constexpr int kSupTile = 256;                  // tokens per item
constexpr int kSupWaves = 8;
constexpr int kSupThreads = kSupWaves * kWave;
constexpr int kSupStageU4 = 4 * 2 * 2 * kWave;  // uint4 per stage (16 KB)

__host__ __device__ inline int sup_out_dim(int t, int r) {
  const int v = r >> 3, h = (r >> 2) & 1, u = r & 3;
  return 64 * (t >> 1) + 32 * (t & 1) + 16 * (v >> 1) + 8 * h + 4 * (v & 1) + u;
}
__host__ __device__ inline int sup_in_dim(int ks, int kk, int h, int e) { return 32 * ks + 16 * h + 8 * kk + e; }

typedef float f32x16 __attribute__((ext_vector_type(16)));

__device__ inline f32x16 mfma32(const bf16x8& a, const bf16x8& b, const f32x16& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

__global__ void pack_support_kernel(const float* __restrict__ w, const float* __restrict__ bias,
                                     const int32_t* __restrict__ order, const int32_t* __restrict__ mperm,
                                     int njobs, int S, uint16_t* __restrict__ wp, float* __restrict__ bp) {
  constexpr int D = 128;
  const int64_t per_member = static_cast<int64_t>(kSupStageU4) * 4 * 8;  // bf16 values: 4 ks x 16 KB
  const int64_t total = per_member * S * njobs;
  for (int64_t idx = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; idx < total;
       idx += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    int64_t rem = idx;
    const int e = rem % 8; rem /= 8;
    const int lane = rem % kWave; rem /= kWave;
    const int term = rem % 2; rem /= 2;
    const int t = rem % 4; rem /= 4;
    const int kk = rem % 2; rem /= 2;
    const int i = rem % (4 * S); rem /= 4 * S;  // stage of the item
    const int pr = i >> 1, q = pr >= S ? 1 : 0, k = pr - q * S, ks = q + 2 * (i & 1);
    const int j = static_cast<int>(rem);
    const int fo = sup_out_dim(t, lane & 31);
    const int fi = mperm[static_cast<int64_t>(order[j]) * S + k] * D + sup_in_dim(ks, kk, lane >> 5, e);
    float r = w[(static_cast<int64_t>(order[j]) * S * D + fi) * D + fo];
    uint16_t hb = 0;
    for (int tt = 0; tt <= term; ++tt) {
      hb = f2bf(r);
      r = r - bf2f(hb);
    }
    wp[idx] = hb;
  }
  const int64_t nb = static_cast<int64_t>(njobs) * D;
  for (int64_t idx = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; idx < nb;
       idx += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int j = static_cast<int>(idx / D);
    bp[idx] = bias[static_cast<int64_t>(order[j]) * D + idx % D];
  }
}

// Items of the support kernel: XCD x takes units x, x + 8, ... of each class
// (the plan orders the units so that these are a run of adjacent keys jobs
// and a run of adjacent values jobs in the sorted job order, whose support
// lists share source layers) and runs them in groups of kSupJobGroup jobs,
// the group's jobs interleaved per token chunk, so that the items an XCD
// runs at one time read overlapping source rows and share its L2.
constexpr int kSupJobGroup = 16;
struct SupItems {
  int x, nwg;
  int64_t next;  // position in XCD x's item list

  struct Item {
    int job, lo, hi;
  };

  __device__ __attribute__((always_inline)) bool get(const MapArgs& a, SupItems::Item& it) const {
    int64_t p = next;
    for (int c = 0; c < a.ncls; ++c) {
      const int nj = a.cls_unit_end[c] - a.cls_unit_begin[c];
      const int mine = nj > x ? (nj - x + 7) / 8 : 0;
      const int nch = a.cls_nchunks[c];
      const int64_t count = static_cast<int64_t>(mine) * nch;
      if (p < count) {
        const int64_t gsz = static_cast<int64_t>(kSupJobGroup) * nch;
        const int g = static_cast<int>(p / gsz);
        const int r = static_cast<int>(p - g * gsz);
        const int gj = min(kSupJobGroup, mine - g * kSupJobGroup);
        const int ch = r / gj, jl = g * kSupJobGroup + (r - ch * gj);
        it.job = cload(a.unit_job + a.cls_unit_begin[c] + x + 8 * jl);
        it.lo = a.cls_tok_first[c] + ch * kSupTile;
        it.hi = min(it.lo + kSupTile, a.cls_tok_first[c] + a.cls_tok_count[c]);
        return true;
      }
      p -= count;
    }
    return false;
  }
};

// One wave's view of an item: its token's rows and position, the job's maps
// and tables.
struct SupLane {
  int job, kind, lo, hi;
  bool live;          // this lane's token is inside the item
  int64_t soff;       // source row byte offset (-1: the zero row)
  int32_t trow;       // target row (-1: write nothing)
  int pos;            // position of this lane's token
  const CB_GLOBAL float* ucos;
  const CB_GLOBAL float* usin;
};

template <bool IS_K>
__device__ __attribute__((always_inline)) void support_item(const MapArgs& a, uint4* lds, uint4* xa, uint4* xb,
                                                         const SupLane& I, int wave, uint32_t& slot) {
#pragma clang fp contract(off)
  constexpr int D = 128;
  constexpr int XT = IS_K ? 2 : 1;          // input terms
  const int lane = threadIdx.x & (kWave - 1);
  const int h = lane >> 5;
  const int S = a.support;
  const int npair = 2 * S;                   // (q, member) pairs; two stages each
  const int* jm = reinterpret_cast<const int*>(a.jobs + I.job);
  const int mx = cload(jm), meta_y = cload(jm + 1);
  const int tth = (meta_y >> 24) & 0xff;

  // W stages of the job, 16 KB each, packed in the order they are consumed.
  gcptr wjob = as_global(a.w + static_cast<size_t>(I.job) * S * 4 * kSupStageU4);
  const int nst = 4 * S;
  // Lane j < 2S holds the address of pair j's source head (its layer's base,
  // the head and the k-step half q = j / S) for the row requests, which read
  // it with readlane: no scalar loads (and their waits) in the stage loop.
  // A token without a source row (outside the item, or a row out of range)
  // reads row 0 instead (pools have at least one row): it writes only to the
  // sink, and a token's products touch only its own outputs.
  uint64_t pbase;
  {
    const int j = min(lane, npair - 1);
    const int q = j >= S ? 1 : 0, k = j - q * S;
    const int pr = *(reinterpret_cast<const CB_GLOBAL int*>(as_global(a.pairs)) + static_cast<size_t>(I.job) * S + k);
    const int layer = pr & 0xffff;
    const void* const* arr = I.kind ? a.src.v_layers : a.src.k_layers;
    gcptr lb = arr ? *(reinterpret_cast<const gcptr CB_GLOBAL*>(as_global(arr)) + layer)
                   : as_global(I.kind ? a.src.v_base : a.src.k_base) + layer * a.src.layer_stride_b;
    pbase = reinterpret_cast<uint64_t>(lb + static_cast<int64_t>((pr >> 16) - a.src.head_offset) * D * 2 + 64 * q);
  }
  const uint32_t pb_lo = static_cast<uint32_t>(pbase), pb_hi = static_cast<uint32_t>(pbase >> 32);
  // Accumulators start at the bias: register 4v + u of tile t holds output
  // dim sup_out_dim(t, 8v + 4h + u).
  f32x16 acc[4];
  {
    const CB_GLOBAL float* bj = reinterpret_cast<const CB_GLOBAL float*>(as_global(a.bias)) + static_cast<size_t>(I.job) * D;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const int base = 64 * (t >> 1) + 32 * (t & 1) + 8 * h;
      const float4 b0 = *reinterpret_cast<const CB_GLOBAL float4*>(bj + base);
      const float4 b1 = *reinterpret_cast<const CB_GLOBAL float4*>(bj + base + 4);
      const float4 b2 = *reinterpret_cast<const CB_GLOBAL float4*>(bj + base + 16);
      const float4 b3 = *reinterpret_cast<const CB_GLOBAL float4*>(bj + base + 20);
      acc[t] = f32x16{b0.x, b0.y, b0.z, b0.w, b1.x, b1.y, b1.z, b1.w,
                      b2.x, b2.y, b2.z, b2.w, b3.x, b3.y, b3.z, b3.w};
    }
  }

  // Un-rotation values (keys) of k-step q for this lane's 16 dims
  // 32q + 16h + 8kk + e: table group g = 2q + h, value groups 2kk, 2kk + 1.
  float tc[2][8], ts[2][8];
  auto load_tab_q = [&](int q) __attribute__((always_inline)) {
    if constexpr (IS_K) {
#pragma unroll
      for (int kk = 0; kk < 2; ++kk)
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          const int64_t off = tab_chunk<16>(I.pos, 2 * kk + u, 2 * q + h);
          const float4 c4 = *reinterpret_cast<const CB_GLOBAL float4*>(I.ucos + off);
          const float4 s4 = *reinterpret_cast<const CB_GLOBAL float4*>(I.usin + off);
          float* c = tc[kk] + 4 * u;
          float* sn = ts[kk] + 4 * u;
          c[0] = c4.x; c[1] = c4.y; c[2] = c4.z; c[3] = c4.w;
          sn[0] = s4.x; sn[1] = s4.y; sn[2] = s4.z; sn[3] = s4.w;
        }
    }
  };

  // Fragments of a k-step pair: [stage of the pair][kk][term][element pair]
  // (dword c of a fragment holds dims 2c, 2c + 1 of its 8). The current
  // pair's are read by the MFMAs while the next pair's are built, in two
  // buffers that swap roles every pair (the pair loop is unrolled by two,
  // so the roles are compile-time).
  typedef uint32_t Frags[2][2][XT][4];
  Frags fa, fb;

  // Memory traffic of the stage loop is LDS DMA only, issued from inline
  // assembly and waited for with explicit counts (the compiler, unaware of
  // it, adds no waits of its own). In issue order, stage i of the item
  // requests W stage i + 3 (2 instructions), then in the first stage of a
  // pair the source rows of the pair after next (4 instructions); both
  // complete in issue order.
  //
  // W ring: four 16 KB slots, stage j in slot (s0 + j) % 4. W stage i + 3
  // goes into the slot stage i - 1 used (free after the barrier that opens
  // stage i) and must have landed before the barrier that opens stage i + 2
  // (its first reads, a step ahead, are in stage i + 2's last step):
  // before opening stage i + 1 a wave waits until at most 6 of its DMA
  // instructions are outstanding, which leaves only those issued after
  // W stage i + 2.
  //
  // Source rows: pair k's go to buffer k & 1 of the wave (4 KB), two stages
  // before its fragments are built (in pair k - 1); the buffer was last read
  // in pair k - 2. DMA instruction r = 2 part + tg covers 16 tokens x 64
  // bytes (part 0: dims 32q..32q+31, part 1: their partners; tg: tokens
  // 16 tg..16 tg+15): DMA lane L loads 16-byte chunk (L & 3) ^ ((L >> 4) & 3)
  // of token L >> 2, so each 4-lane quad reads one 64-byte sector and the
  // readers' 16-lane groups hit distinct banks. Before the first read of
  // pair k's rows (start of pair k - 1) at most 2 DMA instructions (the W
  // stage requested since) may be outstanding.
  auto dma16 = [&](gcptr src, const uint4* dst) __attribute__((always_inline)) {
    const uint32_t la = __builtin_amdgcn_readfirstlane(
        static_cast<uint32_t>(reinterpret_cast<uintptr_t>((CB_LDS const uint4*)dst)));
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off"
                 :: "v"(reinterpret_cast<uint64_t>(src)), "s"(la) : "memory", "m0");
  };
  auto w_dma = [&](int j, uint32_t sl) __attribute__((always_inline)) {
    gcptr src = wjob + static_cast<int64_t>(min(j, nst - 1)) * (kSupStageU4 * 16) + (wave * 128 + lane) * 16;
    const uint4* dst = lds + sl * kSupStageU4 + wave * 128;
    dma16(src, dst);
    dma16(src + kWave * 16, dst + kWave);
  };
  uint64_t doff[2];
  {
    const int c = (lane & 3) ^ ((lane >> 4) & 3);
    const uint64_t mine = static_cast<uint64_t>(I.soff < 0 ? 0 : I.soff);
#pragma unroll
    for (int tg = 0; tg < 2; ++tg) {
      const int from = (16 * tg + (lane >> 2)) * 4;
      const uint32_t lo = __builtin_amdgcn_ds_bpermute(from, static_cast<int>(static_cast<uint32_t>(mine)));
      const uint32_t hi = __builtin_amdgcn_ds_bpermute(from, static_cast<int>(static_cast<uint32_t>(mine >> 32)));
      doff[tg] = ((static_cast<uint64_t>(hi) << 32) | lo) + 16 * c;
    }
  }
  auto src_dma = [&](int p, uint4* X) __attribute__((always_inline)) {
    const int pp = min(p, npair - 1);
    const uint64_t b = (static_cast<uint64_t>(static_cast<uint32_t>(__builtin_amdgcn_readlane(pb_hi, pp))) << 32) |
                       static_cast<uint32_t>(__builtin_amdgcn_readlane(pb_lo, pp));
#pragma unroll
    for (int r = 0; r < 4; ++r)
      dma16(reinterpret_cast<gcptr>(b + doff[r & 1] + 128 * (r >> 1)), X + wave * 256 + r * 64);
  };
  uint4 raw[2];  // first-half dims and partners of one kk half, this lane's 8 each
  const int xn16 = lane & 15, xtg = (lane >> 4) & 1;
  auto read_raw = [&](int kk, const uint4* X) __attribute__((always_inline)) {
    const int cc = (2 * h + kk) ^ (xn16 >> 2);
    raw[0] = X[wave * 256 + xtg * 64 + 4 * xn16 + cc];
    raw[1] = X[wave * 256 + (2 + xtg) * 64 + 4 * xn16 + cc];
  };
  // Element pair c (dims 2c, 2c + 1 of the 8) of the kk half held in raw:
  // keys un-rotated and split into two bf16 terms, values copied.
  auto produce = [&](Frags& nx, int kk, int c) __attribute__((always_inline)) {
    const uint32_t w1 = c == 0 ? raw[0].x : c == 1 ? raw[0].y : c == 2 ? raw[0].z : raw[0].w;
    const uint32_t w2 = c == 0 ? raw[1].x : c == 1 ? raw[1].y : c == 2 ? raw[1].z : raw[1].w;
    if constexpr (IS_K) {
      const float a1 = lo_bf(w1), b1 = hi_bf(w1), a2 = lo_bf(w2), b2 = hi_bf(w2);
      const float c0 = tc[kk][2 * c], c1 = tc[kk][2 * c + 1], s0 = ts[kk][2 * c], s1 = ts[kk][2 * c + 1];
      const float k1a = __builtin_fmaf(a1, c0, a2 * s0), k1b = __builtin_fmaf(b1, c1, b2 * s1);
      const float k2a = __builtin_fmaf(a2, c0, -(a1 * s0)), k2b = __builtin_fmaf(b2, c1, -(b1 * s1));
      const uint32_t h1 = pack_bf16(k1a, k1b), h2 = pack_bf16(k2a, k2b);
      nx[0][kk][0][c] = h1;
      nx[0][kk][1][c] = pack_bf16(k1a - lo_bf(h1), k1b - hi_bf(h1));
      nx[1][kk][0][c] = h2;
      nx[1][kk][1][c] = pack_bf16(k2a - lo_bf(h2), k2b - hi_bf(h2));
      // Keep the work in this step (next to this step's products) rather
      // than sunk toward the pair's end, where its results are first read.
      asm volatile("" :: "v"(nx[0][kk][0][c]), "v"(nx[0][kk][1][c]), "v"(nx[1][kk][0][c]), "v"(nx[1][kk][1][c]));
    } else {
      nx[0][kk][0][c] = w1;
      nx[1][kk][0][c] = w2;
    }
  };
  auto frag = [&](const uint32_t (&f)[4]) __attribute__((always_inline)) {
    return __builtin_bit_cast(bf16x8, make_uint4(f[0], f[1], f[2], f[3]));
  };
  auto ring = [](uint32_t sl, int d) __attribute__((always_inline)) { return (sl + d) & 3u; };

  // Prologue: W stages 0-2 into the three slots after the previous item's
  // last one (that slot may still be read by other waves; the other three
  // were last read before the barrier that opened the previous item's last
  // stage) and the first two pairs' rows; everything this wave has in
  // flight (including the previous item's stores) is waited for, then the
  // barrier publishes W, and the first pair's fragments are built.
  const uint32_t s0 = ring(slot, 1);
  load_tab_q(0);
  w_dma(0, s0);
  w_dma(1, ring(s0, 1));
  w_dma(2, ring(s0, 2));
  src_dma(0, xa);
  src_dma(1, xb);
  __builtin_amdgcn_s_waitcnt(kVmcnt0);
  asm volatile("s_barrier" ::: "memory");
#pragma unroll
  for (int kk = 0; kk < 2; ++kk) {
    read_raw(kk, xa);
#pragma unroll
    for (int c = 0; c < 4; ++c) produce(fa, kk, c);
  }
  if (IS_K && S == 1) {
    load_tab_q(1);
    __builtin_amdgcn_s_waitcnt(kVmcnt0);
  }
  slot = s0;  // slot of the current stage

  // W fragments [ring][tile 0/1 of the step's pair][term], read a step ahead.
  bf16x8 wf[2][4];
  auto read_w = [&](uint32_t sl, int step, bf16x8 (&dst)[4]) __attribute__((always_inline)) {
    const uint4* ws = lds + sl * kSupStageU4;
    const int kk = step >> 1, tp = step & 1;
#pragma unroll
    for (int f = 0; f < 4; ++f)
      dst[f] = __builtin_bit_cast(bf16x8, ws[((kk * 4 + 2 * tp + (f >> 1)) * 2 + (f & 1)) * kWave + lane]);
  };
  read_w(slot, 0, wf[0]);

  // One k-step pair: stages 2p (k-step q) and 2p + 1 (q + 2) with the
  // fragments in cur, building the next pair's (rows in buffer xr) into
  // nxt; the pair after next's rows go to buffer xw. Steps (kk, tile pair
  // tp) of a stage run that step's products of tiles 2tp and 2tp + 1
  // alternately, with element pair `step` of the next pair's kk = half
  // half produced beside them.
  auto pair = [&](int p, Frags& cur, Frags& nxt, const uint4* xr, uint4* xw) __attribute__((always_inline)) {
    if (IS_K && p + 1 == S && S > 1) {  // the next pair starts q = 1
      // Waited for here, once per item, so that no later wait (which would
      // also drain the DMA in flight) is needed for them.
      load_tab_q(1);
      __builtin_amdgcn_s_waitcnt(kVmcnt0);
    }
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      const int i = 2 * p + half;  // stage of the item
      if (half == 0) {
        __builtin_amdgcn_s_waitcnt(kVmcnt2);  // pair p + 1's rows
        asm volatile("" ::: "memory");
      }
      read_raw(half, xr);
      w_dma(i + 3, ring(slot, 3));
      if (half == 0) src_dma(p + 2, xw);
      const uint32_t nsl = ring(slot, 1);
#pragma unroll
      for (int step = 0; step < 4; ++step) {
        if (step < 3) read_w(slot, step + 1, wf[(step + 1) & 1]);
        else read_w(nsl, 0, wf[0]);
        const int kk = step >> 1, t0 = 2 * (step & 1);
        const bf16x8* w = wf[step & 1];  // {t0 term0, t0 term1, t1 term0, t1 term1}
        const bf16x8 x0 = frag(cur[half][kk][0]);
        if constexpr (IS_K) {
          const bf16x8 x1 = frag(cur[half][kk][XT - 1]);
          acc[t0] = mfma32(w[1], x0, acc[t0]);
          acc[t0 + 1] = mfma32(w[3], x0, acc[t0 + 1]);
          acc[t0] = mfma32(w[0], x1, acc[t0]);
          acc[t0 + 1] = mfma32(w[2], x1, acc[t0 + 1]);
          acc[t0] = mfma32(w[0], x0, acc[t0]);
          acc[t0 + 1] = mfma32(w[2], x0, acc[t0 + 1]);
        } else {
          acc[t0] = mfma32(w[1], x0, acc[t0]);
          acc[t0 + 1] = mfma32(w[3], x0, acc[t0 + 1]);
          acc[t0] = mfma32(w[0], x0, acc[t0]);
          acc[t0 + 1] = mfma32(w[2], x0, acc[t0 + 1]);
        }
        produce(nxt, half, step);
        __builtin_amdgcn_sched_barrier(0);
      }
      // Close stage i: W stage i + 2 must have landed (at most 6 younger
      // DMA instructions outstanding), then the barrier publishes it and
      // frees stage i's slot.
      __builtin_amdgcn_s_waitcnt(kVmcnt6);
      asm volatile("s_barrier" ::: "memory");
      slot = nsl;
    }
  };
  for (int p = 0; p < npair; p += 2) {  // npair = 2 S is even
    pair(p, fa, fb, xb, xa);
    pair(p + 1, fb, fa, xa, xb);
  }
  // slot is now one past the item's last stage: step back to it.
  slot = ring(slot, 3);

  // Epilogue: target RoPE (keys), cast, store. Tile tt (0, 1) and its
  // partner tt + 2; register 4v + u is first-half dim
  // 32 tt + 16 (v >> 1) + 8h + 4 (v & 1) + u.
  gptr tbase = const_cast<gptr>(layer_base(a.tgt, I.kind, mx & 0xffff)) +
               static_cast<int64_t>((mx >> 16) - a.tgt.head_offset) * D * 2;
  gptr dst = I.trow >= 0 ? tbase + static_cast<int64_t>(I.trow) * a.tgt.row_stride_b
                         : as_global(a.sink) + lane * 512;
  const CB_GLOBAL float* rcos = gtab(a.cos_tab) + tth * a.theta_stride;
  const CB_GLOBAL float* rsin = gtab(a.sin_tab) + tth * a.theta_stride;
#pragma unroll
  for (int tt = 0; tt < 2; ++tt) {
    float y1[16], y2[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      y1[r] = acc[tt][r];
      y2[r] = acc[tt + 2][r];
    }
    if constexpr (IS_K) {
      float cv[16], sv[16];
#pragma unroll
      for (int vh = 0; vh < 2; ++vh)      // v >> 1: table group 2tt + vh
#pragma unroll
        for (int vl = 0; vl < 2; ++vl) {  // v & 1: value group 2h + vl
          const int64_t off = tab_chunk<16>(I.pos, 2 * h + vl, 2 * tt + vh);
          const float4 c4 = *reinterpret_cast<const CB_GLOBAL float4*>(rcos + off);
          const float4 s4 = *reinterpret_cast<const CB_GLOBAL float4*>(rsin + off);
          const int r0 = 4 * (2 * vh + vl);
          cv[r0] = c4.x; cv[r0 + 1] = c4.y; cv[r0 + 2] = c4.z; cv[r0 + 3] = c4.w;
          sv[r0] = s4.x; sv[r0 + 1] = s4.y; sv[r0 + 2] = s4.z; sv[r0 + 3] = s4.w;
        }
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float a1 = y1[r], a2 = y2[r];
        y1[r] = __builtin_fmaf(a1, cv[r], -(a2 * sv[r]));
        y2[r] = __builtin_fmaf(a2, cv[r], a1 * sv[r]);
      }
    }
#pragma unroll
    for (int vh = 0; vh < 2; ++vh) {
      // Run v = 2vh, 2vh + 1: dims 32tt + 16vh + 8h + 0..7 (16 bytes).
      uint32_t o1[4], o2[4];
#pragma unroll
      for (int i2 = 0; i2 < 4; ++i2) {
        o1[i2] = pack_bf16(y1[8 * vh + 2 * i2], y1[8 * vh + 2 * i2 + 1]);
        o2[i2] = pack_bf16(y2[8 * vh + 2 * i2], y2[8 * vh + 2 * i2 + 1]);
      }
      const int off = (32 * tt + 16 * vh + 8 * h) * 2;
      gstore<uint4>(dst + off, make_uint4(o1[0], o1[1], o1[2], o1[3]));
      gstore<uint4>(dst + off + 128, make_uint4(o2[0], o2[1], o2[2], o2[3]));
    }
  }
}

__global__ __launch_bounds__(kSupThreads, 1) void map_install_support_kernel(MapArgs a) {
  __shared__ uint4 lds[4 * kSupStageU4];  // W ring: four 16 KB stage slots
  __shared__ uint4 lds_xa[kSupWaves * 256];  // source rows of even pairs, 4 KB per wave
  __shared__ uint4 lds_xb[kSupWaves * 256];  // and of odd pairs
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  SupItems items;
  items.x = blockIdx.x & 7;
  items.nwg = gridDim.x >> 3;
  items.next = blockIdx.x >> 3;
  uint32_t slot = 0;  // ring slot of the last stage run
  int errbits = 0;
  SupItems::Item it;
  for (; items.get(a, it); items.next += items.nwg) {
    SupLane I;
    I.job = __builtin_amdgcn_readfirstlane(it.job);
    const int* jm = reinterpret_cast<const int*>(a.jobs + I.job);
    const int meta_y = cload(jm + 1), meta_z = cload(jm + 2);
    I.kind = meta_y & 0xff;
    I.lo = it.lo;
    I.hi = it.hi;
    const int sth = (meta_y >> 16) & 0xff;
    const bool shared = (meta_z & kJobSharedTables) != 0;
    I.ucos = gtab(shared ? a.cos_tab : a.ucos_tab) + sth * a.theta_stride;
    I.usin = gtab(shared ? a.sin_tab : a.usin_tab) + sth * a.theta_stride;
    const int n = it.hi - it.lo;
    const int pt = 32 * wave + (lane & 31);
    const int tk = it.lo + min(pt, n - 1);
    I.live = pt < n;
    const int64_t srow = row_of(a.src, tk);
    const int64_t drow = row_of(a.tgt, tk);
    const bool sok = srow >= 0 && srow < a.src.rows;
    const bool dok = drow >= 0 && drow < a.tgt.rows;
    if (I.live && lane < 32) errbits |= (sok ? 0 : 1) | (dok ? 0 : 2);
    I.soff = I.live && sok ? srow * a.src.row_stride_b : -1;
    // A token whose source row is out of range writes nothing.
    I.trow = I.live && sok && dok ? static_cast<int32_t>(drow) : -1;
    I.pos = position_of(a, tk);
    if (I.kind == CB_KIND_K) support_item<true>(a, lds, lds_xa, lds_xb, I, wave, slot);
    else support_item<false>(a, lds, lds_xa, lds_xb, I, wave, slot);
  }
  // The last item's trailing W and row requests (repeats of its last stage)
  // write LDS: they land before the workgroup ends.
  __builtin_amdgcn_s_waitcnt(kVmcnt0);
  if (errbits) atomicOr(a.err, errbits);
}

// ---------------------------------------------------------------------------
// General kernel (any support s): W block of the current support staged in
// LDS, source fragments in registers; each wave covers all output dims of 32
// tokens. Output dims permuted so lane group g holds dims [g*D/8, (g+1)*D/8)
// of both halves.
// ---------------------------------------------------------------------------

constexpr int kGenColTiles = 2;
constexpr int kGenWaveTokens = 16 * kGenColTiles;
constexpr int kGenSubTokens = kWaves * kGenWaveTokens;

template <int D, typename IO, bool IS_K>
__device__ void gen_run(const MapArgs& a, uint4* lds_w, const Work& wk, int4 meta) {
  using T = IOTraits<IO>;
  using C = Gm<D, IO>;
  constexpr int NTW = T::NTW;
  constexpr int XT = IS_K ? T::XT_K : T::XT_V;
  constexpr int KS = C::KS, RT = C::RT, G = C::G, HALF = C::HALF;
  constexpr int kind = IS_K ? CB_KIND_K : CB_KIND_V;

  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int g = lane >> 4;
  const int col = lane & 15;

  const int tl = meta.x & 0xffff;
  const int th = meta.x >> 16;
  const int sth = (meta.y >> 16) & 0xff;
  const int tth = (meta.y >> 24) & 0xff;
  const int S = a.support;
  const uint4* wj = a.w + static_cast<size_t>(wk.job) * S * C::W_U4;
  const int32_t* pj = a.pairs + static_cast<size_t>(wk.job) * S;

  float bias1[G], bias2[G];
  load_f32<G>(gtab(a.bias) + static_cast<size_t>(wk.job) * D + g * G, bias1);
  load_f32<G>(gtab(a.bias) + static_cast<size_t>(wk.job) * D + HALF + g * G, bias2);

  gptr tbase = const_cast<gptr>(layer_base(a.tgt, kind, tl)) +
                static_cast<int64_t>(th - a.tgt.head_offset) * D * T::BYTES;
  const CB_GLOBAL float* ucos = gtab(a.ucos_tab) + sth * a.theta_stride;
  const CB_GLOBAL float* usin = gtab(a.usin_tab) + sth * a.theta_stride;
  const CB_GLOBAL float* rcos = gtab(a.cos_tab) + tth * a.theta_stride;
  const CB_GLOBAL float* rsin = gtab(a.sin_tab) + tth * a.theta_stride;

  if (S == 1) {
    copy_to_lds<C::W_U4, kThreads>(lds_w, wj);
    __syncthreads();
  }

  for (int sub = wk.tok_lo; sub < wk.tok_hi; sub += kGenSubTokens) {
    int tok[kGenColTiles];
    bool valid[kGenColTiles];
#pragma unroll
    for (int ct = 0; ct < kGenColTiles; ++ct) {
      tok[ct] = sub + wave * kGenWaveTokens + ct * 16 + col;
      valid[ct] = tok[ct] < wk.tok_hi;
    }
    bool src_bad[kGenColTiles] = {};  // a support row out of range: the token writes nothing
    f32x4 acc[RT][kGenColTiles];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
      for (int ct = 0; ct < kGenColTiles; ++ct) acc[rt][ct] = f32x4{0.f, 0.f, 0.f, 0.f};

    for (int k = 0; k < S; ++k) {
      if (S > 1) {
        __syncthreads();
        copy_to_lds<C::W_U4, kThreads>(lds_w, wj + static_cast<size_t>(k) * C::W_U4);
        __syncthreads();
      }
      const int pr = pj[k];
      const int sl = pr & 0xffff;
      const int sh = pr >> 16;
      gcptr sbase = layer_base(a.src, kind, sl) + static_cast<int64_t>(sh - a.src.head_offset) * D * T::BYTES;

      bf16x8 bx[KS][kGenColTiles][XT];
#pragma unroll
      for (int ct = 0; ct < kGenColTiles; ++ct) {
        float x1[G], x2[G];
        bool ok = valid[ct];
        int64_t row = 0;
        if (ok) {
          row = row_of(a.src, tok[ct]);
          if (row < 0 || row >= a.src.rows) {
            atomicOr(a.err, 1);
            ok = false;
            src_bad[ct] = true;
          }
        }
        if (ok) {
          gcptr p = sbase + row * a.src.row_stride_b;
#pragma unroll
          for (int u = 0; u < G / C::E16; ++u) {
            unpack16<IO>(gload<uint4>(p + (g * G + u * C::E16) * T::BYTES), x1 + u * C::E16);
            unpack16<IO>(gload<uint4>(p + (HALF + g * G + u * C::E16) * T::BYTES), x2 + u * C::E16);
          }
          if constexpr (IS_K) {
            const int64_t pos = position_of(a, tok[ct]);
            float c[G], s[G];
            load_tab<G>(ucos, pos, g, c);
            load_tab<G>(usin, pos, g, s);
#pragma unroll
            for (int e = 0; e < G; ++e) {
              const float k1 = __builtin_fmaf(x1[e], c[e], x2[e] * s[e]);
              const float k2 = __builtin_fmaf(x2[e], c[e], -(x1[e] * s[e]));
              x1[e] = k1;
              x2[e] = k2;
            }
          }
        } else {
#pragma unroll
          for (int e = 0; e < G; ++e) x1[e] = x2[e] = 0.f;
        }
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
          const float* src = (ks / (KS / 2) ? x2 : x1) + (ks % (KS / 2)) * 8;
          uint32_t tw[XT][4];
          split_terms<XT, 8>(src, tw);
#pragma unroll
          for (int x = 0; x < XT; ++x)
            bx[ks][ct][x] = __builtin_bit_cast(bf16x8, make_uint4(tw[x][0], tw[x][1], tw[x][2], tw[x][3]));
        }
      }

#pragma unroll
      for (int rt = 0; rt < RT; ++rt) {
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
          bf16x8 aw[NTW];
#pragma unroll
          for (int t = 0; t < NTW; ++t)
            aw[t] = __builtin_bit_cast(bf16x8, lds_w[((rt * KS + ks) * NTW + t) * kWave + lane]);
#pragma unroll
          for (int ct = 0; ct < kGenColTiles; ++ct)
            for_products<XT, NTW>([&](int i, int j) { acc[rt][ct] = mfma(aw[j], bx[ks][ct][i], acc[rt][ct]); });
        }
      }
    }

#pragma unroll
    for (int ct = 0; ct < kGenColTiles; ++ct) {
      if (!valid[ct] || src_bad[ct]) continue;
      const int64_t row = row_of(a.tgt, tok[ct]);
      if (row < 0 || row >= a.tgt.rows) {
        atomicOr(a.err, 2);
        continue;
      }
      float o1[G], o2[G];
      float c[G], s[G];
      if constexpr (IS_K) {
        const int64_t pos = position_of(a, tok[ct]);
        load_tab<G>(rcos, pos, g, c);
        load_tab<G>(rsin, pos, g, s);
      }
#pragma unroll
      for (int rt = 0; rt < RT / 2; ++rt) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int e = 4 * rt + i;
          const float y1 = acc[rt][ct][i] + bias1[e];
          const float y2 = acc[rt + RT / 2][ct][i] + bias2[e];
          if constexpr (IS_K) {
            o1[e] = __builtin_fmaf(y1, c[e], -(y2 * s[e]));
            o2[e] = __builtin_fmaf(y2, c[e], y1 * s[e]);
          } else {
            o1[e] = y1;
            o2[e] = y2;
          }
        }
      }
      gptr p = tbase + row * a.tgt.row_stride_b;
      store_elems<IO, G>(p + (g * G) * T::BYTES, o1);
      store_elems<IO, G>(p + (HALF + g * G) * T::BYTES, o2);
    }
  }
}

template <int D, typename IO>
__global__ __launch_bounds__(kThreads) void map_install_gen_kernel(MapArgs a) {
  __shared__ uint4 lds_w[Gm<D, IO>::W_U4];
  Work wk;
  if (!decode_work(a, &wk)) return;
  const int4 meta = a.jobs[wk.job];
  if ((meta.y & 0xff) == CB_KIND_K)
    gen_run<D, IO, true>(a, lds_w, wk, meta);
  else
    gen_run<D, IO, false>(a, lds_w, wk, meta);
}

// ---------------------------------------------------------------------------
// Plan-time kernels
// ---------------------------------------------------------------------------

// Pack fp32 W[orig][s*D][D] into bf16 split terms in MFMA A-fragment order,
// and permute the bias to sorted job order.
template <int D, int NTW>
__global__ void pack_weights_kernel(const float* __restrict__ w, const float* __restrict__ bias,
                                    const int32_t* __restrict__ order, int njobs, int S,
                                    uint16_t* __restrict__ wp, float* __restrict__ bp) {
  constexpr int KS = D / 32, RT = D / 16;
  const int64_t per_block = static_cast<int64_t>(RT) * KS * NTW * kWave * 8;
  const int64_t total = per_block * S * njobs;
  for (int64_t idx = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; idx < total;
       idx += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    int64_t rem = idx;
    const int e = rem % 8; rem /= 8;
    const int lane = rem % kWave; rem /= kWave;
    const int t = rem % NTW; rem /= NTW;
    const int ks = rem % KS; rem /= KS;
    const int rt = rem % RT; rem /= RT;
    const int fo = gen_out_dim(D, rt, lane & 15);
    const int k = rem % S; rem /= S;
    const int j = static_cast<int>(rem);
    const int src_job = order[j];
    const int fi = k * D + in_dim(D, ks, lane >> 4, e);
    float r = w[(static_cast<int64_t>(src_job) * S * D + fi) * D + fo];
    uint16_t h = 0;
    for (int tt = 0; tt <= t; ++tt) {
      h = f2bf(r);
      r = r - bf2f(h);
    }
    wp[idx] = h;
  }
  const int64_t nb = static_cast<int64_t>(njobs) * D;
  for (int64_t idx = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; idx < nb;
       idx += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int j = static_cast<int>(idx / D);
    bp[idx] = bias[static_cast<int64_t>(order[j]) * D + idx % D];
  }
}

// ---------------------------------------------------------------------------
// Generic kernel: any even head_dim up to 512, any support, bf16 / fp16 /
// fp32 K/V, computed in fp32 with FMAs (no split terms, no MFMA). It serves
// the shapes and dtypes the MFMA kernels do not take; the configured
// workloads never reach it.
//
// One workgroup of 256 threads per item (one job, a token range), 32-token
// tiles. Per tile and support member k, the tile's source rows are gathered,
// keys un-rotated (dims p and p + D/2 of a thread's pairs together), and the
// fp32 values staged in LDS; each thread owns one output dim pair p, p + D/2
// (threads_per_pair = 256 / (D/2) threads share a pair and split the
// tokens) and accumulates sum_i x[t][i] * W[k*D + i][p] over the member's D
// input dims. After the last member: + bias (the reference adds it after
// the product), target RoPE on the pair, cast (round to nearest even),
// store. Plan data for this kernel: W as fp32 [job][s*D][D] and the RoPE
// tables in natural [theta][position][D/2] order.
// ---------------------------------------------------------------------------

constexpr int kAnyThreads = 256;
constexpr int kAnyTile = 32;        // tokens per tile
constexpr int kAnyMaxDim = 512;
constexpr int kAnyMaxTok = kAnyTile;  // tokens per thread at most (one thread per pair)

template <typename IO>
struct AnyIO;
template <>
struct AnyIO<uint16_t> {  // bf16
  static __device__ float get(const CB_GLOBAL uint16_t* p) { return bf2f(*p); }
  static __device__ void put(CB_GLOBAL uint16_t* p, float v) { *p = f2bf(v); }
};
template <>
struct AnyIO<_Float16> {
  static __device__ float get(const CB_GLOBAL _Float16* p) { return static_cast<float>(*p); }
  static __device__ void put(CB_GLOBAL _Float16* p, float v) { *p = static_cast<_Float16>(v); }
};
template <>
struct AnyIO<float> {
  static __device__ float get(const CB_GLOBAL float* p) { return *p; }
  static __device__ void put(CB_GLOBAL float* p, float v) { *p = v; }
};

template <typename IO>
__global__ __launch_bounds__(kAnyThreads) void map_install_any_kernel(MapArgs a, int D) {
#pragma clang fp contract(off)
  __shared__ float xs[kAnyTile][kAnyMaxDim];
  __shared__ int64_t trow[kAnyTile];
  __shared__ int64_t srow[kAnyTile];  // source row, -1: zero source values
  __shared__ int32_t tpos[kAnyTile];
  Work wk;
  if (!decode_work(a, &wk)) return;
  const int S = a.support;
  const int half = D / 2;
  const int job = wk.job;
  const int* jm = reinterpret_cast<const int*>(a.jobs + job);
  const int mx = cload(jm), meta_y = cload(jm + 1);
  const int kind = meta_y & 0xff;
  const bool is_k = kind == CB_KIND_K;
  const int sth = (meta_y >> 16) & 0xff, tth = (meta_y >> 24) & 0xff;
  const int64_t eb = sizeof(IO);
  // Un-rotation tables cos/m, sin/m and rotation tables, natural order.
  const CB_GLOBAL float* ucos = gtab(a.ucos_tab) + sth * a.theta_stride;
  const CB_GLOBAL float* usin = gtab(a.usin_tab) + sth * a.theta_stride;
  const CB_GLOBAL float* rcos = gtab(a.cos_tab) + tth * a.theta_stride;
  const CB_GLOBAL float* rsin = gtab(a.sin_tab) + tth * a.theta_stride;
  gptr tbase = const_cast<gptr>(layer_base(a.tgt, kind, mx & 0xffff)) +
               static_cast<int64_t>((mx >> 16) - a.tgt.head_offset) * D * eb;
  const CB_GLOBAL float* W = gtab(reinterpret_cast<const float*>(a.w)) + static_cast<int64_t>(job) * S * D * D;
  const CB_GLOBAL float* bias = gtab(a.bias) + static_cast<int64_t>(job) * D;
  // This thread's dim pair and tokens.
  const int tpp = max(1, kAnyThreads / half);       // threads per pair
  const int p = threadIdx.x / tpp, sub = threadIdx.x % tpp;
  const bool active = p < half;
  const int toks = (kAnyTile + tpp - 1) / tpp;      // tokens per thread
  int errbits = 0;

  for (int lo = wk.tok_lo; lo < wk.tok_hi; lo += kAnyTile) {
    const int n = min(kAnyTile, wk.tok_hi - lo);
    __syncthreads();  // the previous tile's LDS reads are done
    if (threadIdx.x < kAnyTile) {
      const int t = threadIdx.x;
      const int tk = lo + min(t, n - 1);
      const int64_t s = row_of(a.src, tk), d = row_of(a.tgt, tk);
      const bool live = t < n;
      const bool sok = s >= 0 && s < a.src.rows, dok = d >= 0 && d < a.tgt.rows;
      if (live) errbits |= (sok ? 0 : 1) | (dok ? 0 : 2);
      // A token whose source row is out of range writes nothing.
      trow[t] = live && sok && dok ? d : -1;
      srow[t] = live && sok ? s : -1;
      tpos[t] = position_of(a, tk);
    }
    float acc[kAnyMaxTok][2];
#pragma unroll
    for (int m = 0; m < kAnyMaxTok; ++m) acc[m][0] = acc[m][1] = 0.f;
    for (int k = 0; k < S; ++k) {
      __syncthreads();  // rows ready / previous member's reads done
      const int pr = cload(a.pairs + static_cast<size_t>(job) * S + k);
      gcptr sbase = layer_base(a.src, kind, pr & 0xffff) + static_cast<int64_t>((pr >> 16) - a.src.head_offset) * D * eb;
      for (int e = threadIdx.x; e < kAnyTile * half; e += kAnyThreads) {
        const int t = e / half, j = e % half;
        const int pos = tpos[t];
        const int64_t s = srow[t];
        float x1 = 0.f, x2 = 0.f;
        if (s >= 0) {
          const CB_GLOBAL IO* row = reinterpret_cast<const CB_GLOBAL IO*>(sbase + s * a.src.row_stride_b);
          x1 = AnyIO<IO>::get(row + j);
          x2 = AnyIO<IO>::get(row + j + half);
        }
        if (is_k) {
          const float c = ucos[static_cast<int64_t>(pos) * half + j];
          const float sn = usin[static_cast<int64_t>(pos) * half + j];
          const float k1 = __builtin_fmaf(x1, c, x2 * sn);
          const float k2 = __builtin_fmaf(x2, c, -(x1 * sn));
          x1 = k1;
          x2 = k2;
        }
        xs[t][j] = x1;
        xs[t][j + half] = x2;
      }
      __syncthreads();
      if (active) {
        const CB_GLOBAL float* wk_ = W + static_cast<int64_t>(k) * D * D;
        for (int i = 0; i < D; ++i) {
          const float w1 = wk_[static_cast<int64_t>(i) * D + p];
          const float w2 = wk_[static_cast<int64_t>(i) * D + p + half];
#pragma unroll
          for (int m = 0; m < kAnyMaxTok; ++m) {
            if (m < toks) {
              const int t = sub + m * tpp;
              if (t < kAnyTile) {
                const float x = xs[t][i];
                acc[m][0] = __builtin_fmaf(x, w1, acc[m][0]);
                acc[m][1] = __builtin_fmaf(x, w2, acc[m][1]);
              }
            }
          }
        }
      }
    }
    if (active) {
      const float b1 = bias[p], b2 = bias[p + half];
#pragma unroll
      for (int m = 0; m < kAnyMaxTok; ++m) {
        if (m >= toks) continue;
        const int t = sub + m * tpp;
        if (t >= n) continue;
        const int64_t row = trow[t];
        if (row < 0) continue;
        float y1 = acc[m][0] + b1, y2 = acc[m][1] + b2;
        if (is_k) {
          const int pos = tpos[t];
          const float c = rcos[static_cast<int64_t>(pos) * half + p];
          const float sn = rsin[static_cast<int64_t>(pos) * half + p];
          const float r1 = __builtin_fmaf(y1, c, -(y2 * sn));
          const float r2 = __builtin_fmaf(y2, c, y1 * sn);
          y1 = r1;
          y2 = r2;
        }
        CB_GLOBAL IO* out = reinterpret_cast<CB_GLOBAL IO*>(tbase + row * a.tgt.row_stride_b);
        AnyIO<IO>::put(out + p, y1);
        AnyIO<IO>::put(out + p + half, y2);
      }
    }
  }
  if (errbits) atomicOr(a.err, errbits);
}

// Plan data of the generic kernel: W [job][s*D][D] and bias [job][D] copied
// in sorted job order.
__global__ void copy_weights_kernel(const float* __restrict__ w, const float* __restrict__ bias,
                                    const int32_t* __restrict__ order, int njobs, int per_job_w, int D,
                                    float* __restrict__ wp, float* __restrict__ bp) {
  const int64_t total = static_cast<int64_t>(njobs) * per_job_w;
  for (int64_t idx = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; idx < total;
       idx += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t j = idx / per_job_w;
    wp[idx] = w[static_cast<int64_t>(order[j]) * per_job_w + idx % per_job_w];
  }
  const int64_t nb = static_cast<int64_t>(njobs) * D;
  for (int64_t idx = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; idx < nb;
       idx += static_cast<int64_t>(gridDim.x) * blockDim.x)
    bp[idx] = bias[static_cast<int64_t>(order[idx / D]) * D + idx % D];
}

// Plan tables from standard [theta][pos][D/2] cos/sin: rotation tables and
// un-rotation tables cos/m, sin/m (m = max(cos^2 + sin^2, FLT_MIN)), both in
// the permuted half-row layout; also max |m - 1| per theta set (as float bits).
// Grid: (blocks per theta set, theta sets); each block reduces its maximum in
// LDS and issues one atomic.
__global__ __launch_bounds__(256) void prepare_tables_kernel(
    const float* __restrict__ c, const float* __restrict__ s, float* __restrict__ rc,
    float* __restrict__ rs, float* __restrict__ uc, float* __restrict__ us, int half,
    int64_t per_theta, int64_t out_per_theta, unsigned* __restrict__ norm_dev, int natural) {
#pragma clang fp contract(off)
  __shared__ unsigned red[256];
  const int64_t base = static_cast<int64_t>(blockIdx.y) * per_theta;
  unsigned dev = 0u;
  for (int64_t k = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; k < per_theta;
       k += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t i = base + k;
    const float cc = c[i], ss = s[i];
    const float m = fmaxf(cc * cc + ss * ss, 1.17549435e-38f);
    const int64_t o = blockIdx.y * out_per_theta +
                      (natural ? k : tab_offset(half, k / half, static_cast<int>(k % half)));
    rc[o] = cc;
    rs[o] = ss;
    uc[o] = cc / m;
    us[o] = ss / m;
    dev = max(dev, __float_as_uint(fabsf(m - 1.0f)));
  }
  red[threadIdx.x] = dev;
  __syncthreads();
  for (int w = 128; w > 0; w >>= 1) {
    if (threadIdx.x < w) red[threadIdx.x] = max(red[threadIdx.x], red[threadIdx.x + w]);
    __syncthreads();
  }
  if (threadIdx.x == 0) atomicMax(norm_dev + blockIdx.y, red[0]);
}

// ---------------------------------------------------------------------------
// Row copy: dst layer l row(t) <- src layer l row(t), 16-byte chunks.
// ---------------------------------------------------------------------------

struct CopyArgs {
  DevRows src, dst;
  int32_t num_tokens;
  int32_t chunks_per_row;
  int32_t tokens_per_block;
  int32_t blocks_per_layer;
  int32_t* err;
};

// Each thread moves kCopyUnroll 16-byte pieces: first every piece's rows are
// resolved (index loads), then every source piece is loaded, then stored, so
// a thread keeps kCopyUnroll loads in flight instead of one dependent
// index-load / load / store chain at a time. A workgroup covers 256 *
// kCopyUnroll pieces (one pass), so many small workgroups fill the chip.
constexpr int kCopyUnroll = 4;

__global__ __launch_bounds__(256) void copy_rows_kernel(CopyArgs a) {
  const int lk = blockIdx.x / a.blocks_per_layer;  // layer * 2 + kind
  const int tb = blockIdx.x % a.blocks_per_layer;
  const int layer = lk >> 1, kind = lk & 1;
  gcptr sbase = layer_base(a.src, kind, layer);
  gptr dbase = const_cast<gptr>(layer_base(a.dst, kind, layer));
  const int t0 = tb * a.tokens_per_block;
  const int n = min(a.tokens_per_block, a.num_tokens - t0);
  const int cpr = a.chunks_per_row;
  const int total = n * cpr;
  for (int base = threadIdx.x; base < total; base += blockDim.x * kCopyUnroll) {
    int64_t so[kCopyUnroll], dof[kCopyUnroll];  // byte offsets; -1: piece not copied
#pragma unroll
    for (int u = 0; u < kCopyUnroll; ++u) {
      const int idx = base + u * blockDim.x;
      so[u] = -1;
      dof[u] = -1;
      if (idx < total) {
        const int t = t0 + idx / cpr;
        const int ch = idx % cpr;
        const int64_t sr = row_of(a.src, t);
        const int64_t dr = row_of(a.dst, t);
        const bool sok = sr >= 0 && sr < a.src.rows;
        const bool dok = dr >= 0 && dr < a.dst.rows;
        if (a.err && ch == 0 && !(sok && dok)) atomicOr(a.err, sok ? 2 : 1);
        if (sok && dok) {
          so[u] = sr * a.src.row_stride_b + 16 * ch;
          dof[u] = dr * a.dst.row_stride_b + 16 * ch;
        }
      }
    }
    uint4 v[kCopyUnroll];
#pragma unroll
    for (int u = 0; u < kCopyUnroll; ++u)
      if (so[u] >= 0) v[u] = gload<uint4>(sbase + so[u]);
#pragma unroll
    for (int u = 0; u < kCopyUnroll; ++u)
      if (dof[u] >= 0) gstore<uint4>(dbase + dof[u], v[u]);
  }
}

// ---------------------------------------------------------------------------
// Recurrent (DeltaNet) state transform: out[b] = A[b]^T . U[b] . B[b]
// (cb/architectures/qwen35.py:52-61) with U [k, v], A [k, kp], B [v, vp],
// out [kp, vp], row-major fp32 or fp64. One workgroup per (batch entry,
// 16-row block of out): stage 1 forms the block's 16 rows of T = A^T U in LDS,
// stage 2 multiplies them by B. Both stages are 16x16x4 MFMAs (lane l holds
// A[l % 16][l / 16] and B[l / 16][l % 16]; the result rows 4(l / 16) + j of
// column l % 16), with operands outside the matrices read as zero.
// ---------------------------------------------------------------------------

constexpr int kDeltaMaxV = 512;  // LDS holds 16 rows of T (16 x v, fp64)

typedef double f64x4 __attribute__((ext_vector_type(4)));

template <typename T>
struct DeltaMfma;
template <>
struct DeltaMfma<float> {
  using V = f32x4;
  static __device__ inline V op(float a, float b, V c) { return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0); }
};
template <>
struct DeltaMfma<double> {
  using V = f64x4;
  static __device__ inline V op(double a, double b, V c) { return __builtin_amdgcn_mfma_f64_16x16x4f64(a, b, c, 0, 0, 0); }
};

struct DeltaArgs {
  const void* u;
  const void* a;
  const void* b;
  void* out;
  int64_t su, sa, sb, so;  // batch strides in elements (0: one matrix for every entry)
  int32_t k, v, kp, vp;
};

template <typename T>
__global__ __launch_bounds__(256) void delta_state_kernel(DeltaArgs p) {
  __shared__ double tblk_raw[16 * kDeltaMaxV];
  T* tblk = reinterpret_cast<T*>(tblk_raw);
  using M = DeltaMfma<T>;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = lane & 15, q = lane >> 4;
  const int64_t bi = blockIdx.x;
  const int i0 = blockIdx.y * 16;
  const T* U = static_cast<const T*>(p.u) + bi * p.su;
  const T* A = static_cast<const T*>(p.a) + bi * p.sa;
  const T* B = static_cast<const T*>(p.b) + bi * p.sb;
  T* out = static_cast<T*>(p.out) + bi * p.so;
  // Stage 1: T[i0 + row][c] = sum_k A[k][i0 + row] * U[k][c] for the block's 16 rows.
  for (int c0 = wave * 16; c0 < p.v; c0 += 64) {
    typename M::V acc = {0, 0, 0, 0};
    const int ia = i0 + r, cu = c0 + r;
#pragma unroll 4
    for (int kk = 0; kk < p.k; kk += 4) {
      const int kr = kk + q;
      const T av = kr < p.k && ia < p.kp ? A[static_cast<int64_t>(kr) * p.kp + ia] : T(0);
      const T bv = kr < p.k && cu < p.v ? U[static_cast<int64_t>(kr) * p.v + cu] : T(0);
      acc = M::op(av, bv, acc);
    }
    if (cu < p.v) {
#pragma unroll
      for (int j = 0; j < 4; ++j) tblk[(4 * q + j) * p.v + cu] = acc[j];
    }
  }
  __syncthreads();
  // Stage 2: out[i0 + row][c] = sum_v T[row][v] * B[v][c].
  for (int c0 = wave * 16; c0 < p.vp; c0 += 64) {
    typename M::V acc = {0, 0, 0, 0};
    const int cb = c0 + r;
#pragma unroll 4
    for (int vv = 0; vv < p.v; vv += 4) {
      const int vr = vv + q;
      const T av = vr < p.v ? tblk[r * p.v + vr] : T(0);
      const T bv = vr < p.v && cb < p.vp ? B[static_cast<int64_t>(vr) * p.vp + cb] : T(0);
      acc = M::op(av, bv, acc);
    }
    if (cb < p.vp) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int row = i0 + 4 * q + j;
        if (row < p.kp) out[static_cast<int64_t>(row) * p.vp + cb] = acc[j];
      }
    }
  }
}

// fp32 states with every dimension 128 (the DeltaNet head size): one
// workgroup of 8 waves per batch entry, two workgroups per CU. Wave w owns
// the 16 rows [16w, 16w + 16) of T and of out.
//   Stage 1 forms T^T = U^T A as eight 16x16 tiles (v-block vb, row block w):
//   A operand U[k][16vb + r], B operand A[k][16w + r], over four 32-row
//   chunks of A and U staged through LDS (double-buffered; the next chunk's
//   loads are in flight during the current chunk's MFMAs).
//   Stage 2 uses those accumulators directly as the A operand of out = T B:
//   lane (q, r) of tile vb holds T[16w + r][16vb + 4q + e], so k-step (vb, e)
//   pairs lane q with row 16vb + 4q + e of B (a permuted k order; the sum over
//   v is the same). B streams through the same LDS buffers.
// Chunk rows are padded to 144 floats, so every operand read of a k-step hits
// 64 distinct banks.
constexpr int kDs = 128;        // matrix size of the fast path
constexpr int kDsChunk = 32;    // rows per staged chunk
constexpr int kDsPadC = 144;    // chunk row stride (floats)
constexpr int kDsChunkFloats = kDsChunk * kDsPadC;

__global__ __launch_bounds__(512, 2) void delta_state128_kernel(DeltaArgs p) {
  __shared__ float lds[4 * kDsChunkFloats];  // stage 1: A0 U0 A1 U1; stage 2: B0 B1
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r = lane & 15, q = lane >> 4;
  const int64_t bi = blockIdx.x;
  const float* U = static_cast<const float*>(p.u) + bi * p.su;
  const float* A = static_cast<const float*>(p.a) + bi * p.sa;
  const float* B = static_cast<const float*>(p.b) + bi * p.sb;
  float* out = static_cast<float*>(p.out) + bi * p.so;
  // Chunk staging: thread t moves 16 bytes of rows t / 32 and t / 32 + 16.
  const int srow = threadIdx.x >> 5, scol = (threadIdx.x & 31) * 4;
  auto load_chunk = [&](const float* m, int c, float4& v0, float4& v1) {
    v0 = *reinterpret_cast<const float4*>(m + (c * kDsChunk + srow) * kDs + scol);
    v1 = *reinterpret_cast<const float4*>(m + (c * kDsChunk + srow + 16) * kDs + scol);
  };
  auto store_chunk = [&](float* dst, const float4& v0, const float4& v1) {
    *reinterpret_cast<float4*>(dst + srow * kDsPadC + scol) = v0;
    *reinterpret_cast<float4*>(dst + (srow + 16) * kDsPadC + scol) = v1;
  };
  constexpr int NC = kDs / kDsChunk;
  constexpr int NB = kDs / 16;

  // Stage 1: tt[vb] = (U^T A) tile (vb, w), i.e. T[16w + r][16vb + 4q + e].
  f32x4 tt[NB];
#pragma unroll
  for (int vb = 0; vb < NB; ++vb) tt[vb] = f32x4{0.f, 0.f, 0.f, 0.f};
  float4 a0, a1, u0, u1, b0, b1;
  load_chunk(A, 0, a0, a1);
  load_chunk(U, 0, u0, u1);
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    float* bufA = lds + (c & 1) * 2 * kDsChunkFloats;
    float* bufU = bufA + kDsChunkFloats;
    store_chunk(bufA, a0, a1);
    store_chunk(bufU, u0, u1);
    __syncthreads();
    if (c + 1 < NC) {
      load_chunk(A, c + 1, a0, a1);
      load_chunk(U, c + 1, u0, u1);
    } else {
      load_chunk(B, 0, b0, b1);
    }
#pragma unroll
    for (int kk = 0; kk < kDsChunk; kk += 4) {
      const float bv = bufA[(kk + q) * kDsPadC + 16 * w + r];
#pragma unroll
      for (int vb = 0; vb < NB; ++vb)
        tt[vb] = __builtin_amdgcn_mfma_f32_16x16x4f32(bufU[(kk + q) * kDsPadC + 16 * vb + r], bv, tt[vb], 0, 0, 0);
    }
  }

  // Stage 2: oo[jb] = out tile (w, jb) = sum over v of T[16w + .][v] B[v][16jb + .].
  f32x4 oo[NB];
#pragma unroll
  for (int jb = 0; jb < NB; ++jb) oo[jb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    float* bufB = lds + (c & 1) * kDsChunkFloats;
    __syncthreads();  // the buffer's previous readers (stage 1, or chunk c - 2) are done
    store_chunk(bufB, b0, b1);
    __syncthreads();
    if (c + 1 < NC) load_chunk(B, c + 1, b0, b1);
#pragma unroll
    for (int h = 0; h < 2; ++h) {        // v-blocks 2c, 2c + 1 of this chunk
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int vrow = 16 * h + 4 * q + e;
        const float av = tt[2 * c + h][e];  // c and h are unrolled constants
#pragma unroll
        for (int jb = 0; jb < NB; ++jb)
          oo[jb] = __builtin_amdgcn_mfma_f32_16x16x4f32(av, bufB[vrow * kDsPadC + 16 * jb + r], oo[jb], 0, 0, 0);
      }
    }
  }
#pragma unroll
  for (int jb = 0; jb < NB; ++jb)
#pragma unroll
    for (int e = 0; e < 4; ++e) out[(16 * w + 4 * q + e) * kDs + 16 * jb + r] = oo[jb][e];
}

// ---------------------------------------------------------------------------
// Batched launches: every kept token of every request gets a slot in one
// token space, class by class (class c's kept tokens of request r occupy
// [vbase, vbase + count)). This kernel resolves each slot's source row,
// target row and position once; the map kernel then reads them as int32 row
// vectors, so a batch runs as one map launch.
// ---------------------------------------------------------------------------

constexpr int kBatchSpans = 32;  // requests per resolve launch (kernel arguments)

struct BatchArgs {
  DevRows src, tgt;
  int32_t* src_row;
  int32_t* tgt_row;
  int32_t* pos;
  int32_t nspans;
  int32_t ncls;
  int64_t src_off[kBatchSpans];
  int64_t tgt_off[kBatchSpans];
  int32_t pos0[kBatchSpans];
  int32_t first[kMaxClasses][kBatchSpans];  // first kept token of the request in the class
  int32_t count[kMaxClasses][kBatchSpans];
  int32_t vbase[kMaxClasses][kBatchSpans];
};
static_assert(sizeof(BatchArgs) <= 4096, "kernel arguments must fit 4 KB");

// Row of u = t + index_offset under R's index rule; -1 outside [0, rows).
__device__ inline int32_t resolve_row(const DevRows& R, int64_t t) {
  const int64_t u = t + R.index_offset;
  int64_t row;
  switch (R.index_kind) {
    case CB_INDEX_IDENTITY: row = u; break;
    case CB_INDEX_I32: row = reinterpret_cast<const CB_GLOBAL int32_t*>(as_global(R.index))[u]; break;
    case CB_INDEX_I64: row = reinterpret_cast<const CB_GLOBAL int64_t*>(as_global(R.index))[u]; break;
    default: {
      const int64_t ps = R.page_size;
      row = static_cast<int64_t>(reinterpret_cast<const CB_GLOBAL int32_t*>(as_global(R.index))[u / ps]) * ps + u % ps;
    }
  }
  return row >= 0 && row < R.rows ? static_cast<int32_t>(row) : -1;
}

__global__ __launch_bounds__(256) void resolve_batch_kernel(BatchArgs b) {
  const int c = blockIdx.y / b.nspans, r = blockIdx.y % b.nspans;
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i >= b.count[c][r]) return;
  const int t = b.first[c][r] + i;
  const int v = b.vbase[c][r] + i;
  b.pos[v] = b.pos0[r] + t;
  b.src_row[v] = resolve_row(b.src, b.src_off[r] + t);
  b.tgt_row[v] = resolve_row(b.tgt, b.tgt_off[r] + t);
}

}  // namespace

// Workspace of cb_map_install_batch_noalloc: a file-scope device array, one
// copy per GPU, held until the process ends. Host code never uses this name
// as an address (it is a host-side stand-in there); it uses the per-device
// pointer that hipGetSymbolAddress returns (scratch_setup).
static __device__ __align__(256) char scratch[CB_NOALLOC_WORKSPACE_BYTES];
static_assert(3 * ((int64_t{CB_NOALLOC_MAX_TOKENS} * 4 + 255) / 256 * 256) <= CB_NOALLOC_WORKSPACE_BYTES,
              "the no-allocation workspace holds CB_NOALLOC_MAX_TOKENS tokens");

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------

constexpr int kPoolSlots = 64;     // work-pool counter pairs that direct launches rotate over
constexpr int kCapturePairs = 64;  // further pairs, each given to one launch recorded into a HIP graph

struct cb_plan {
  int device = 0;
  cb_plan_info info{};
  int ntw = 2;
  int elem_bytes = 2;
  bool support_gemm = false;  // support > 1, head_dim 128, bf16: map_install_support_kernel
  bool generic = false;       // map_install_any_kernel: shapes / dtypes the MFMA kernels do not take
  int num_windows = 1;
  int window_size[kMaxClasses] = {0, 0, 0, 0};
  int cls_unit_begin[kMaxClasses] = {0, 0, 0, 0};
  int cls_unit_end[kMaxClasses] = {0, 0, 0, 0};
  int max_src_layer = 0, min_src_head = 0, max_src_head = 0;
  int max_tgt_layer = 0, min_tgt_head = 0, max_tgt_head = 0;
  void* d_w = nullptr;
  float* d_bias = nullptr;
  int4* d_jobs = nullptr;
  int32_t* d_pairs = nullptr;
  int32_t* d_unit_job = nullptr;
  int32_t* d_unit_njobs = nullptr;
  int32_t* d_unit_group = nullptr;
  int32_t* d_group_unit_start = nullptr;
  int32_t* d_group_unit_count = nullptr;
  int num_units = 0;
  int num_cus = 256;
  std::vector<int32_t> unit_weight;  // cost of one 16-token sub-tile of each unit
  // Last cost-line split (it depends only on the blocks and the sub-tiles of
  // each window class), reused by launches with the same shape.
  mutable std::mutex split_mu;
  mutable std::vector<int32_t> split_key, split_unit, split_sub;
  mutable int32_t split_pool[4] = {0, 0, 0, 0};  // pool_n, pool_u0, pool_s0, pool_gs
  // Work-pool counters of the streaming kernel: kPoolSlots + kCapturePairs
  // pairs (claims, finished workgroups), zero between launches. Direct
  // launch k uses pair k % kPoolSlots. A launch recorded into a HIP graph
  // keeps its pair for every replay, so each one gets a pair of its own from
  // the capture range, which direct launches never use; once that range is
  // spent, captured launches run without the pool (static ranges only).
  uint32_t* d_pool = nullptr;
  mutable std::atomic<uint32_t> pool_seq{0};
  mutable std::atomic<uint32_t> capture_seq{0};
  // Completion event and stream of the last pooled direct launch on each
  // pair (created with the plan; guarded by split_mu). A pooled launch whose
  // pair's previous pooled launch may still run on another stream makes its
  // own stream wait for it, so launches in flight never share a pair: two
  // that did would take chunk indices from one counter, and each would then
  // write some of the other's chunks with its own request's rows.
  hipEvent_t pair_done[kPoolSlots] = {};
  mutable hipStream_t pair_stream[kPoolSlots] = {};
  // The last launch's split, for callers and tests (cb_plan_last_split).
  mutable std::atomic<int32_t> last_pool_chunks{0};
  mutable std::atomic<int32_t> last_workgroups{0};
  float* d_cos = nullptr;
  float* d_sin = nullptr;
  float* d_ucos = nullptr;
  float* d_usin = nullptr;
  int32_t* d_err = nullptr;
  void* d_sink = nullptr;
};

namespace {

void plan_free(cb_plan* p) {
  if (!p) return;
  void* ptrs[] = {p->d_w,         p->d_bias,         p->d_jobs,           p->d_pairs,
                  p->d_unit_job,  p->d_unit_njobs,   p->d_unit_group,     p->d_group_unit_start,
                  p->d_group_unit_count, p->d_cos,   p->d_sin,            p->d_ucos,
                  p->d_usin,      p->d_err,          p->d_sink,
                  p->d_pool};
  for (void* q : ptrs)
    if (q) (void)hipFree(q);
  for (hipEvent_t e : p->pair_done)
    if (e) (void)hipEventDestroy(e);
  delete p;
}

template <typename Tp>
int upload(Tp** dst, const void* src, size_t bytes, int64_t* total) {
  CB_HIP(hipMalloc(reinterpret_cast<void**>(dst), bytes));
  *total += static_cast<int64_t>(bytes);
  if (src) CB_HIP(hipMemcpy(*dst, src, bytes, hipMemcpyHostToDevice));
  return CB_OK;
}

// align: the byte alignment the launch needs of strides and bases (16 for the
// vector kernels, one element for the generic kernel).
int to_dev_rows(const cb_rows& r, int elem_bytes, DevRows* out, int align = 16) {
  out->k_layers = r.k_layers;
  out->v_layers = r.v_layers;
  out->k_base = static_cast<const char*>(r.k_base);
  out->v_base = static_cast<const char*>(r.v_base);
  out->layer_stride_b = r.layer_stride * elem_bytes;
  out->row_stride_b = r.row_stride * elem_bytes;
  out->rows = r.rows;
  out->index = r.index;
  out->index_offset = r.index_offset;
  out->index_kind = r.index_kind;
  out->page_size = r.page_size;
  out->head_offset = r.head_offset;
  out->pad = 0;
  if (r.index_kind < CB_INDEX_IDENTITY || r.index_kind > CB_INDEX_BLOCK_TABLE)
    return fail(CB_EINVAL, "unknown index_kind %d", r.index_kind);
  if (r.index_kind != CB_INDEX_IDENTITY && !r.index)
    return fail(CB_EINVAL, "index pointer required for index_kind %d", r.index_kind);
  if (r.index_kind == CB_INDEX_BLOCK_TABLE && r.page_size <= 0)
    return fail(CB_EINVAL, "block table needs page_size > 0");
  if (r.index_offset < 0 || r.index_offset > (int64_t{1} << 30))
    return fail(CB_EINVAL, "index_offset out of range");
  if (r.rows <= 0) return fail(CB_EINVAL, "rows must be > 0");
  if (!r.k_layers && (!r.k_base || !r.v_base))
    return fail(CB_EINVAL, "either per-layer pointer arrays or k_base/v_base are required");
  if (r.k_layers && !r.v_layers) return fail(CB_EINVAL, "v_layers required with k_layers");
  if ((out->row_stride_b % align) || (out->layer_stride_b % align))
    return fail(CB_EINVAL, "row and layer strides must be multiples of %d bytes", align);
  if ((reinterpret_cast<uintptr_t>(r.k_base) | reinterpret_cast<uintptr_t>(r.v_base)) % align)
    return fail(CB_EINVAL, "k_base/v_base must be %d-byte aligned", align);
  return CB_OK;
}

template <int D, int NTW>
void launch_pack(const cb_plan_desc* d, const int32_t* d_order, uint16_t* wp, float* bp) {
  hipLaunchKernelGGL((pack_weights_kernel<D, NTW>), dim3(1024), dim3(256), 0, 0, d->d_weight,
                     d->d_bias, d_order, d->num_jobs, d->support, wp, bp);
}

template <typename SameGroup>
int plan_build(const cb_plan_desc* d, const std::vector<int>& order, const std::vector<int>& mperm,
               SameGroup same_group, cb_plan* p) {
  const int D = d->head_dim, S = d->support, nj = d->num_jobs;
  int64_t bytes = 0;
  CB_HIP(hipGetDevice(&p->device));
  p->ntw = d->io_dtype == CB_DTYPE_BF16 ? 2 : 3;
  p->elem_bytes = d->io_dtype == CB_DTYPE_F32 ? 4 : 2;
  p->generic = !((d->io_dtype == CB_DTYPE_BF16 && (D == 64 || D == 128)) ||
                 (d->io_dtype == CB_DTYPE_F32 && D == 64));
  p->support_gemm = !p->generic && S > 1 && D == 128 && p->ntw == 2;
  p->num_windows = d->num_windows;
  for (int c = 0; c < kMaxClasses; ++c) {
    p->window_size[c] = c < d->num_windows ? d->window_size[c] : 0;
    p->cls_unit_begin[c] = p->cls_unit_end[c] = c < d->num_windows ? -1 : 0;
  }
  std::vector<int4> jobs(nj);
  std::vector<int32_t> pairs(static_cast<size_t>(nj) * S);
  std::vector<int32_t> unit_job, unit_njobs, unit_group, group_unit_start, group_unit_count;
  p->max_src_layer = 0;
  p->min_src_head = 1 << 30;
  p->max_src_head = 0;
  p->max_tgt_layer = 0;
  p->min_tgt_head = 1 << 30;
  p->max_tgt_head = 0;
  // Units: runs of up to kUnitJobs consecutive jobs of one group for the
  // streaming kernel (s == 1); single jobs for the general kernel.
  const int unit_cap = S == 1 && !p->generic ? kUnitJobs : 1;
  for (int i = 0; i < nj; ++i) {
    const int j = order[i];
    jobs[i] = make_int4(d->job_target_layer[j] | (d->job_target_head[j] << 16),
                        d->job_kind[j] | (d->job_window[j] << 8) | (d->job_source_theta[j] << 16) |
                            (d->job_target_theta[j] << 24),
                        0, j);
    for (int k = 0; k < S; ++k) {
      const int m = mperm[static_cast<size_t>(j) * S + k];
      const int sl = d->job_source_layer[j * S + m], sh = d->job_source_head[j * S + m];
      pairs[static_cast<size_t>(i) * S + k] = sl | (sh << 16);
      p->max_src_layer = std::max(p->max_src_layer, sl);
      p->min_src_head = std::min(p->min_src_head, sh);
      p->max_src_head = std::max(p->max_src_head, sh);
    }
    p->max_tgt_layer = std::max(p->max_tgt_layer, d->job_target_layer[j]);
    p->min_tgt_head = std::min(p->min_tgt_head, d->job_target_head[j]);
    p->max_tgt_head = std::max(p->max_tgt_head, d->job_target_head[j]);
    const bool new_group = i == 0 || !same_group(order[i - 1], j);
    if (new_group) {
      group_unit_start.push_back(static_cast<int32_t>(unit_job.size()));
      group_unit_count.push_back(0);
    }
    if (new_group || unit_njobs.back() == unit_cap) {
      unit_job.push_back(i);
      unit_njobs.push_back(0);
      unit_group.push_back(static_cast<int32_t>(group_unit_start.size() - 1));
      group_unit_count.back() += 1;
      const int c = d->job_window[j];
      const int u = static_cast<int>(unit_job.size() - 1);
      if (p->cls_unit_begin[c] < 0) p->cls_unit_begin[c] = u;
      p->cls_unit_end[c] = u + 1;
    }
    unit_njobs.back() += 1;
  }
  for (int c = 0; c < d->num_windows; ++c)
    if (p->cls_unit_begin[c] < 0) p->cls_unit_begin[c] = p->cls_unit_end[c] = 0;
  p->num_units = static_cast<int>(unit_job.size());
  if (p->support_gemm) {
    // The support kernel gives XCD x units x, x + 8, ... of each class. Place
    // the units so that these are a contiguous run of the sorted keys jobs
    // followed by one of the sorted values jobs (each XCD gets its share of
    // both kinds, whose costs differ), so that jobs an XCD runs together
    // share source layers. Units are single jobs here.
    for (int c = 0; c < d->num_windows; ++c) {
      const int cb = p->cls_unit_begin[c], n = p->cls_unit_end[c] - cb;
      std::vector<int32_t> kj, vj;
      for (int u = cb; u < cb + n; ++u) ((jobs[unit_job[u]].y & 0xff) == CB_KIND_K ? kj : vj).push_back(u);
      std::vector<int32_t> perm(n);
      bool ok = true;
      int kpos = 0, vpos = 0;
      for (int x = 0; x < 8 && ok; ++x) {
        const int mine = n > x ? (n - x + 7) / 8 : 0;
        const int nk = static_cast<int>(kj.size()) * (x + 1) / 8 - static_cast<int>(kj.size()) * x / 8;
        const int nv = mine - nk;
        if (nv < 0 || vpos + nv > static_cast<int>(vj.size())) ok = false;
        for (int jl = 0; ok && jl < mine; ++jl) perm[x + 8 * jl] = jl < nk ? kj[kpos + jl] : vj[vpos + jl - nk];
        kpos += nk;
        vpos += std::max(nv, 0);
      }
      if (!ok) continue;  // leave the sorted order
      std::vector<int32_t> uj(n), un(n), ug(n);
      for (int i = 0; i < n; ++i) {
        uj[i] = unit_job[perm[i]];
        un[i] = unit_njobs[perm[i]];
        ug[i] = unit_group[perm[i]];
      }
      std::copy(uj.begin(), uj.end(), unit_job.begin() + cb);
      std::copy(un.begin(), un.end(), unit_njobs.begin() + cb);
      std::copy(ug.begin(), ug.end(), unit_group.begin() + cb);
    }
  }
  {
    int cus = 0;
    CB_HIP(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, p->device));
    p->num_cus = std::max(8, std::min(cus, kMaxStreamBlocks) / 8 * 8);
  }

  const size_t w_bytes = p->generic ? static_cast<size_t>(nj) * S * D * D * 4
                                    : static_cast<size_t>(nj) * S * (D / 16) * (D / 32) * p->ntw * kWave * 8 * 2;
  const int64_t padded_positions = (static_cast<int64_t>(d->table_positions) + kTabBlock - 1) / kTabBlock * kTabBlock;
  const size_t table = static_cast<size_t>(d->num_thetas) * padded_positions * (D / 2);
  int rc;
  if ((rc = upload(&p->d_pairs, pairs.data(), pairs.size() * 4, &bytes))) return rc;
  if ((rc = upload(&p->d_unit_job, unit_job.data(), unit_job.size() * 4, &bytes))) return rc;
  if ((rc = upload(&p->d_unit_njobs, unit_njobs.data(), unit_njobs.size() * 4, &bytes))) return rc;
  if ((rc = upload(&p->d_unit_group, unit_group.data(), unit_group.size() * 4, &bytes))) return rc;
  if ((rc = upload(&p->d_group_unit_start, group_unit_start.data(), group_unit_start.size() * 4, &bytes))) return rc;
  if ((rc = upload(&p->d_group_unit_count, group_unit_count.data(), group_unit_count.size() * 4, &bytes))) return rc;
  if ((rc = upload(&p->d_w, nullptr, w_bytes, &bytes))) return rc;
  if ((rc = upload(&p->d_bias, nullptr, static_cast<size_t>(nj) * D * 4, &bytes))) return rc;
  if ((rc = upload(&p->d_cos, nullptr, table * 4, &bytes))) return rc;
  if ((rc = upload(&p->d_sin, nullptr, table * 4, &bytes))) return rc;
  if ((rc = upload(&p->d_ucos, nullptr, table * 4, &bytes))) return rc;
  if ((rc = upload(&p->d_usin, nullptr, table * 4, &bytes))) return rc;
  if ((rc = upload(&p->d_err, nullptr, 4, &bytes))) return rc;
  if ((rc = upload(&p->d_sink, nullptr, kSinkBytes + kZeroBytes, &bytes))) return rc;
  CB_HIP(hipMemset(p->d_err, 0, 4));
  CB_HIP(hipMemset(static_cast<char*>(p->d_sink) + kSinkBytes, 0, kZeroBytes));
  // Rotation / un-rotation tables in the permuted layout, and which theta sets
  // have unit norm (|cos^2 + sin^2 - 1| <= 2 ulp) so keys can share one table.
  {
    unsigned* d_norm = nullptr;
    CB_HIP(hipMalloc(reinterpret_cast<void**>(&d_norm), d->num_thetas * sizeof(unsigned)));
    std::vector<unsigned> norm(d->num_thetas, 0u);
    hipError_t e = hipMemset(d_norm, 0, d->num_thetas * sizeof(unsigned));
    if (e == hipSuccess) {
      hipLaunchKernelGGL(prepare_tables_kernel, dim3(256, d->num_thetas), dim3(256), 0, 0,
                         d->d_cos, d->d_sin, p->d_cos, p->d_sin, p->d_ucos, p->d_usin, D / 2,
                         static_cast<int64_t>(d->table_positions) * (D / 2), padded_positions * (D / 2), d_norm,
                         p->generic ? 1 : 0);
      e = hipGetLastError();
    }
    if (e == hipSuccess) e = hipMemcpy(norm.data(), d_norm, norm.size() * sizeof(unsigned), hipMemcpyDeviceToHost);
    (void)hipFree(d_norm);
    if (e != hipSuccess) return fail(CB_EHIP, "plan table preparation failed: %s", hipGetErrorString(e));
    for (int i = 0; i < nj; ++i) {
      const int sth = (jobs[i].y >> 16) & 0xff, tth = (jobs[i].y >> 24) & 0xff;
      float dev;
      std::memcpy(&dev, &norm[sth], sizeof(dev));
      if (sth == tth && dev <= 2.4e-7f) jobs[i].z |= kJobSharedTables;
    }
    if ((rc = upload(&p->d_jobs, jobs.data(), jobs.size() * sizeof(int4), &bytes))) return rc;
  }
  // Relative cost of one 16-token sub-tile of each unit (streaming kernel),
  // from per-segment timestamps on MI355X: a two-job key unit 28, a one-job
  // key unit 21, a two-job value unit 20, a one-job value unit 14 (one job
  // still pays the whole gather, and keys the un-rotation and tables); keys
  // with separate rotation tables load them too (+4). A unit that is the only
  // one reading its source rows fetches all of them from HBM (otherwise
  // another unit of the group has usually brought them into the MALL first)
  // and runs ~30% slower per token.
  p->unit_weight.assign(unit_job.size(), 0);
  for (size_t u = 0; u < unit_job.size(); ++u) {
    const int4 m = jobs[unit_job[u]];
    const bool key = (m.y & 0xff) == CB_KIND_K;
    const bool two = unit_njobs[u] == 2;
    int w = key ? (two ? 28 : 21) : (two ? 20 : 14);
    if (key && !(m.z & kJobSharedTables)) w += 4;
    if (group_unit_count[unit_group[u]] == 1) w = (w * 13 + 5) / 10;
    p->unit_weight[u] = w;
  }
  const size_t pool_bytes = 2 * (kPoolSlots + kCapturePairs) * sizeof(uint32_t);
  if ((rc = upload(&p->d_pool, nullptr, pool_bytes, &bytes))) return rc;
  CB_HIP(hipMemset(p->d_pool, 0, pool_bytes));
  for (hipEvent_t& e : p->pair_done) CB_HIP(hipEventCreateWithFlags(&e, hipEventDisableTiming));
  int32_t* d_order = nullptr;
  int32_t* d_mperm = nullptr;
  CB_HIP(hipMalloc(reinterpret_cast<void**>(&d_order), (order.size() + mperm.size()) * 4));
  d_mperm = d_order + order.size();
  hipError_t e = hipMemcpy(d_order, order.data(), order.size() * 4, hipMemcpyHostToDevice);
  if (e == hipSuccess) e = hipMemcpy(d_mperm, mperm.data(), mperm.size() * 4, hipMemcpyHostToDevice);
  if (e == hipSuccess) {
    uint16_t* wp = static_cast<uint16_t*>(p->d_w);
    if (p->generic)
      hipLaunchKernelGGL(copy_weights_kernel, dim3(1024), dim3(256), 0, 0, d->d_weight, d->d_bias, d_order,
                         nj, S * D * D, D, static_cast<float*>(p->d_w), p->d_bias);
    else if (D == 64 && p->ntw == 2)
      launch_pack<64, 2>(d, d_order, wp, p->d_bias);
    else if (D == 64)
      launch_pack<64, 3>(d, d_order, wp, p->d_bias);
    else if (p->support_gemm)
      hipLaunchKernelGGL(pack_support_kernel, dim3(1024), dim3(256), 0, 0, d->d_weight, d->d_bias, d_order,
                         d_mperm, d->num_jobs, d->support, wp, p->d_bias);
    else
      launch_pack<128, 2>(d, d_order, wp, p->d_bias);
    e = hipGetLastError();
  }
  if (e == hipSuccess) e = hipDeviceSynchronize();
  (void)hipFree(d_order);
  if (e != hipSuccess) return fail(CB_EHIP, "plan weight pack failed: %s", hipGetErrorString(e));
  p->info.head_dim = D;
  p->info.support = S;
  p->info.io_dtype = d->io_dtype;
  p->info.num_jobs = nj;
  p->info.target_layers = d->target_layers;
  p->info.target_heads = d->target_heads;
  p->info.num_groups = static_cast<int32_t>(group_unit_start.size());
  p->info.num_thetas = d->num_thetas;
  p->info.table_positions = d->table_positions;
  p->info.weight_terms = p->generic ? 1 : p->ntw;
  p->info.device_bytes = bytes;
  return CB_OK;
}

// Default tokens per workgroup: about three workgroups per CU over the launch
// (one resident per CU for the streaming kernel), at least 512 tokens.
int default_chunk(const cb_plan* p, int n) {
  if (p->generic) return 8 * kAnyTile;
  if (p->info.support != 1) return kGenSubTokens;
  int64_t units = 0;
  for (int c = 0; c < p->num_windows; ++c) units += p->cls_unit_end[c] - p->cls_unit_begin[c];
  const int64_t target_items = 768;
  int64_t chunk = (units * n + target_items - 1) / target_items;
  chunk = std::max<int64_t>(512, (chunk + kSubTokens - 1) / kSubTokens * kSubTokens);
  return static_cast<int>(std::min<int64_t>(chunk, 1 << 20));
}

// Geometry checks shared by single and batched launches (before anything is
// enqueued).
int check_sides(const cb_plan* p, const cb_rows& sr, const cb_rows& tr) {
  const int D = p->info.head_dim;
  if (sr.num_layers <= p->max_src_layer)
    return fail(CB_EINVAL, "source has %d layers; the plan reads layer %d", sr.num_layers,
                p->max_src_layer);
  if (p->min_src_head < sr.head_offset || p->max_src_head >= sr.head_offset + sr.heads)
    return fail(CB_EINVAL, "source rows hold heads [%d, %d); the plan reads heads %d..%d",
                sr.head_offset, sr.head_offset + sr.heads, p->min_src_head, p->max_src_head);
  if (tr.num_layers <= p->max_tgt_layer)
    return fail(CB_EINVAL, "target has %d layers; the plan writes layer %d", tr.num_layers,
                p->max_tgt_layer);
  if (p->min_tgt_head < tr.head_offset || p->max_tgt_head >= tr.head_offset + tr.heads)
    return fail(CB_EINVAL, "target rows hold heads [%d, %d); the plan writes heads %d..%d",
                tr.head_offset, tr.head_offset + tr.heads, p->min_tgt_head, p->max_tgt_head);
  if (static_cast<int64_t>(sr.heads) * D > sr.row_stride ||
      static_cast<int64_t>(tr.heads) * D > tr.row_stride)
    return fail(CB_EINVAL, "row_stride is smaller than heads * head_dim");
  if (tr.index_kind == CB_INDEX_IDENTITY && sr.index_kind == CB_INDEX_IDENTITY &&
      tr.k_base == sr.k_base && tr.k_base)
    return fail(CB_EINVAL, "target aliases the source");
  // The streaming and support kernels keep row indices in 32 bits; the
  // generic kernels take 64-bit rows.
  const bool rows32 = !p->generic && (p->info.support == 1 || p->support_gemm);
  if (rows32 && (sr.rows > INT32_MAX || tr.rows > INT32_MAX))
    return fail(CB_EINVAL, "pools with more than 2^31 rows are not supported");
  return CB_OK;
}

// Kept tokens of each window class for a request of n tokens at positions
// position_start.. of a prefix of `prefix` tokens: [first[c], first[c] +
// count[c]). A sliding class keeps the last min(prefix, window - 1) tokens of
// the prefix (cb/architectures/gemma3.py:52); a full class keeps all.
void class_ranges(const cb_plan* p, int64_t n, int64_t position_start, int64_t prefix,
                  int64_t* first, int64_t* count) {
  for (int c = 0; c < p->num_windows; ++c) {
    int64_t first_pos = 0;
    if (p->window_size[c] > 0) first_pos = prefix - std::min<int64_t>(prefix, p->window_size[c] - 1);
    const int64_t f = std::max<int64_t>(0, first_pos - position_start);
    count[c] = std::max<int64_t>(0, n - f);
    first[c] = std::min<int64_t>(f, n);
  }
}

// Fixed cost of one segment (a workgroup's pass over part of one unit), in
// sub-tile weight units: staging the unit's W into LDS, the pipeline ramp and
// the wait for the slowest wave (tuned on MI355X with the TP4-share and
// whole-model handoffs).
constexpr int64_t kSegmentCost = 256;

// Work pool of the streaming kernel. Workgroups drift apart over a long
// launch (memory contention differs between XCDs and over time), so when a
// workgroup's share of the cost line is long the line's tail is not cut into
// static ranges but handed out in chunks to whichever workgroup is free.
// Every chunk pays a segment start, so short launches keep static ranges
// only. Per-workgroup budgets are in sub-tile weight units (the TP4-share
// 4096-token handoff: about 3.2K; the whole 64x8 model: 13K; the 32K-token
// history and the 64-request batch: about 100K). Measured on MI355X.
#ifndef CB_POOL_MID_BUDGET
#define CB_POOL_MID_BUDGET 8192   // below: no pool
#endif
#ifndef CB_POOL_LONG_BUDGET
#define CB_POOL_LONG_BUDGET 32768
#endif
#ifndef CB_POOL_MID_PCT           // share of the line in the pool, chunk cost (% of a budget)
#define CB_POOL_MID_PCT 15
#endif
#ifndef CB_POOL_MID_CHUNK_PCT
#define CB_POOL_MID_CHUNK_PCT 8
#endif
#ifndef CB_POOL_LONG_PCT
#define CB_POOL_LONG_PCT 25
#endif
#ifndef CB_POOL_LONG_CHUNK_PCT
#define CB_POOL_LONG_CHUNK_PCT 5
#endif

// Cut the units' sub-tiles, in order, into a.num_blocks contiguous ranges and
// store the cut points in a.blk_unit / a.blk_sub. A range costs kSegmentCost
// per unit it touches plus its sub-tiles' weights; the cuts minimise the
// largest range cost (greedy fill for a given budget, bisection on the
// budget), so ranges that cross a unit boundary get fewer sub-tiles. With a
// work pool, the ranges are filled to a smaller budget and the rest of the
// line becomes the pool (a->pool_*).
void split_cost_line(const cb_plan* p, MapArgs* a, bool allow_pool) {
  const int nu = p->num_units, nb = a->num_blocks;
  std::vector<int32_t> ns(nu, 0);
  int64_t total = 0;
  int c = 0;
  for (int u = 0; u < nu; ++u) {
    while (c + 1 < p->num_windows && u >= a->cls_unit_end[c]) ++c;
    ns[u] = a->cls_subtiles[c];
    if (ns[u] > 0) total += kSegmentCost + static_cast<int64_t>(p->unit_weight[u]) * ns[u];
  }
  // Greedy fill with budget T per range; returns the ranges used (cuts into
  // blk_* when `out`). With `out`, at most nb ranges are cut and the rest of
  // the line, from (u, sub), is left to the pool; cuts past the last range
  // all sit at that point.
  int u = 0, sub = 0;
  auto fill = [&](int64_t T, bool out) {
    u = 0;
    sub = 0;
    int r = 0;
    while (u < nu && ns[u] == 0) ++u;
    while (u < nu && !(out && r == nb)) {
      if (out) {
        a->blk_unit[r] = u;
        a->blk_sub[r] = sub;
      }
      int64_t budget = T - kSegmentCost;
      bool first = true;
      while (u < nu) {
        const int64_t w = p->unit_weight[u];
        int64_t k = std::min<int64_t>(ns[u] - sub, std::max<int64_t>(budget, 0) / w);
        if (first && k == 0) k = 1;  // every range makes progress
        first = false;
        sub += static_cast<int>(k);
        budget -= k * w;
        if (sub < ns[u]) break;
        int nxt = u + 1;
        while (nxt < nu && ns[nxt] == 0) ++nxt;
        u = nxt;
        sub = 0;
        if (u >= nu || budget < kSegmentCost + p->unit_weight[u]) break;
        budget -= kSegmentCost;
      }
      ++r;
      if (r > nb && !out) return r;
    }
    if (out) {
      for (int q = r; q <= nb; ++q) {
        a->blk_unit[q] = u;
        a->blk_sub[q] = sub;
      }
    }
    return r;
  };
  int64_t lo = 1, hi = total + kSegmentCost;
  while (lo < hi) {
    const int64_t mid = lo + (hi - lo) / 2;
    if (fill(mid, false) <= nb) hi = mid;
    else lo = mid + 1;
  }
  int64_t pool_pct = 0, chunk_pct = 0;
  if (!allow_pool) {
  } else if (lo >= CB_POOL_LONG_BUDGET) {
    pool_pct = CB_POOL_LONG_PCT;
    chunk_pct = CB_POOL_LONG_CHUNK_PCT;
  } else if (lo >= CB_POOL_MID_BUDGET) {
    pool_pct = CB_POOL_MID_PCT;
    chunk_pct = CB_POOL_MID_CHUNK_PCT;
  }
  a->pool_n = 0;
  a->pool_u0 = nu;
  a->pool_s0 = 0;
  a->pool_gs = 1;
  if (pool_pct <= 0) {
    fill(lo, true);
    return;
  }
  fill(lo * (100 - pool_pct) / 100, true);  // leaves (u, sub) at the pool's start
  // Chunks of about chunk_pct% of a budget: sub-tiles at the pool's mean
  // sub-tile weight, at least 4.
  int64_t pool_w = 0, pool_subs = 0;
  for (int v = u; v < nu; ++v) {
    const int s0 = v == u ? sub : 0;
    if (ns[v] > s0) {
      pool_w += static_cast<int64_t>(p->unit_weight[v]) * (ns[v] - s0);
      pool_subs += ns[v] - s0;
    }
  }
  if (pool_subs == 0) return;  // the ranges reach the line's end
  const int64_t gs = std::max<int64_t>(4, lo * chunk_pct / 100 * pool_subs / pool_w);
  int64_t chunks = 0;
  for (int v = u; v < nu; ++v) {
    const int s0 = v == u ? sub : 0;
    if (ns[v] > s0) chunks += (ns[v] - s0 + gs - 1) / gs;
  }
  if (chunks > (int64_t{1} << 24) || gs > INT32_MAX) {  // not a useful pool: static ranges only
    fill(lo, true);
    return;
  }
  a->pool_n = static_cast<int32_t>(chunks);
  a->pool_u0 = u;
  a->pool_s0 = sub;
  a->pool_gs = static_cast<int32_t>(gs);
}

// Enqueue the map kernel over class token ranges [first[c], first[c] +
// count[c]) of the launch's token space. `a` carries the two sides (and, for
// batches, the position vector); the plan fields are filled in here.
// tokens_per_workgroup > 0 caps the unit-tokens per workgroup.
int launch_map(const cb_plan* p, MapArgs& a, const int64_t* first, const int64_t* count,
               int tokens_per_workgroup, int default_tokens, hipStream_t s) {
  const int D = p->info.head_dim;
  const bool ws = p->info.support == 1 && !p->generic;
  const int unit = p->generic ? kAnyTile : ws ? kSubTokens : kGenSubTokens;
  int chunk = tokens_per_workgroup > 0 ? tokens_per_workgroup : default_tokens;
  if (tokens_per_workgroup < 0 || chunk < unit || chunk % unit)
    return fail(CB_EINVAL, "tokens_per_workgroup must be a positive multiple of %d", unit);
  // The support kernel's items are fixed 256-token blocks; the knob does not apply.
  if (p->support_gemm) chunk = kSupTile;
  a.w = static_cast<const uint4*>(p->d_w);
  a.bias = p->d_bias;
  a.jobs = p->d_jobs;
  a.pairs = p->d_pairs;
  a.unit_job = p->d_unit_job;
  a.unit_njobs = p->d_unit_njobs;
  a.unit_group = p->d_unit_group;
  a.group_unit_start = p->d_group_unit_start;
  a.group_unit_count = p->d_group_unit_count;
  a.cos_tab = p->d_cos;
  a.sin_tab = p->d_sin;
  a.ucos_tab = p->d_ucos;
  a.usin_tab = p->d_usin;
  a.theta_stride = (static_cast<int64_t>(p->info.table_positions) + kTabBlock - 1) / kTabBlock * kTabBlock * (D / 2);
  a.support = p->info.support;
  a.chunk = chunk;
  a.err = p->d_err;
  a.sink = p->d_sink;
  a.zero = static_cast<const char*>(p->d_sink) + kSinkBytes;
  int64_t items = 0, n_total = 0;
  a.ncls = p->num_windows;
  for (int c = 0; c < p->num_windows; ++c) {
    if (first[c] + count[c] > INT32_MAX) return fail(CB_EINVAL, "launch too large");
    const int64_t nch = (count[c] + chunk - 1) / chunk;
    a.cls_unit_begin[c] = p->cls_unit_begin[c];
    a.cls_unit_end[c] = p->cls_unit_end[c];
    a.cls_tok_first[c] = static_cast<int32_t>(first[c]);
    a.cls_tok_count[c] = static_cast<int32_t>(count[c]);
    a.cls_nchunks[c] = static_cast<int32_t>(std::max<int64_t>(nch, 1));
    a.cls_item_begin[c] = static_cast<int32_t>(items);
    items += static_cast<int64_t>(p->cls_unit_end[c] - p->cls_unit_begin[c]) * nch;
    n_total = std::max(n_total, first[c] + count[c]);
  }
  a.n_tokens = static_cast<int32_t>(n_total);
  a.cls_item_begin[p->num_windows] = static_cast<int32_t>(items);
  if (items == 0) return CB_OK;
  if (items > (int64_t{1} << 30)) return fail(CB_EINVAL, "request too large for one launch");
  a.total_items = static_cast<int32_t>(items);
  a.padded_items = static_cast<int32_t>((items + 7) / 8 * 8);
  int64_t grid_blocks = a.padded_items;
  // Held from the cost-line split through the launch and its pair event.
  std::unique_lock<std::mutex> held;
  int tracked_pair = -1;
  if (ws) {
    int64_t unit_tokens = 0, subtiles = 0;
    for (int c = 0; c < p->num_windows; ++c) {
      const int64_t sub = (static_cast<int64_t>(a.cls_tok_count[c]) + kSubTokens - 1) / kSubTokens;
      a.cls_unit_end[c] = p->cls_unit_end[c];
      a.cls_subtiles[c] = static_cast<int32_t>(sub);
      unit_tokens += static_cast<int64_t>(p->cls_unit_end[c] - p->cls_unit_begin[c]) * a.cls_tok_count[c];
      subtiles += sub;
    }
    if (subtiles == 0) return CB_OK;
    a.num_units = p->num_units;
    int64_t nb = p->num_cus;
    if (tokens_per_workgroup > 0)  // cap on unit-tokens per workgroup
      nb = std::min<int64_t>(nb, std::max<int64_t>(8, (unit_tokens + chunk - 1) / chunk));
    a.num_blocks = static_cast<int32_t>(std::max<int64_t>(8, nb / 8 * 8));
    grid_blocks = a.num_blocks;
    // A launch recorded into a HIP graph keeps its counter pair for every
    // replay: it takes a pair of its own from the capture range, or runs
    // without the pool once that range is spent.
    bool allow_pool = true, captured = false;
    uint32_t capture_pair = 0;
    {
      hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
      CB_HIP(hipStreamIsCapturing(s, &cs));
      if (cs != hipStreamCaptureStatusNone) {
        captured = true;
        capture_pair = p->capture_seq.fetch_add(1, std::memory_order_relaxed);
        allow_pool = capture_pair < static_cast<uint32_t>(kCapturePairs);
      }
    }
    std::vector<int32_t> key{a.num_blocks, p->num_windows, allow_pool ? 1 : 0};
    for (int c = 0; c < p->num_windows; ++c) key.push_back(a.cls_subtiles[c]);
    const size_t nbk = static_cast<size_t>(a.num_blocks) + 1;
    held = std::unique_lock<std::mutex>(p->split_mu);
    if (key == p->split_key) {
      std::copy(p->split_unit.begin(), p->split_unit.end(), a.blk_unit);
      std::copy(p->split_sub.begin(), p->split_sub.end(), a.blk_sub);
      a.pool_n = p->split_pool[0];
      a.pool_u0 = p->split_pool[1];
      a.pool_s0 = p->split_pool[2];
      a.pool_gs = p->split_pool[3];
    } else {
      split_cost_line(p, &a, allow_pool);
      p->split_key = key;
      p->split_unit.assign(a.blk_unit, a.blk_unit + nbk);
      p->split_sub.assign(a.blk_sub, a.blk_sub + nbk);
      p->split_pool[0] = a.pool_n;
      p->split_pool[1] = a.pool_u0;
      p->split_pool[2] = a.pool_s0;
      p->split_pool[3] = a.pool_gs;
    }
    // (Without the pool the kernel never touches its pair.)
    const uint32_t pair = captured ? (allow_pool ? static_cast<uint32_t>(kPoolSlots) + capture_pair : 0u)
                                   : p->pool_seq.fetch_add(1, std::memory_order_relaxed) % kPoolSlots;
    a.pool_ctr = p->d_pool + 2 * static_cast<size_t>(pair);
    if (!captured && a.pool_n > 0) {
      // The pair's previous pooled launch ran on this stream (finished
      // before this one starts) or is waited for unless it has finished.
      if (p->pair_stream[pair] != s) {
        const hipError_t q = hipEventQuery(p->pair_done[pair]);
        if (q == hipErrorNotReady) CB_HIP(hipStreamWaitEvent(s, p->pair_done[pair], 0));
        else if (q != hipSuccess) return fail(CB_EHIP, "hipEventQuery: %s", hipGetErrorString(q));
      }
      tracked_pair = static_cast<int>(pair);
    }
  }
  p->last_pool_chunks.store(ws ? a.pool_n : 0, std::memory_order_relaxed);
  p->last_workgroups.store(static_cast<int32_t>(grid_blocks), std::memory_order_relaxed);
  const dim3 grid(static_cast<unsigned>(grid_blocks)), block(ws ? kStreamThreads : kThreads);
  if (ws) {
    const bool pv = a.pos != nullptr;
    if (D == 128 && p->ntw == 2) {
      if (pv) hipLaunchKernelGGL((map_install_stream_kernel<128, uint16_t, true>), grid, block, 0, s, a);
      else hipLaunchKernelGGL((map_install_stream_kernel<128, uint16_t, false>), grid, block, 0, s, a);
    } else if (D == 64 && p->ntw == 2) {
      if (pv) hipLaunchKernelGGL((map_install_stream_kernel<64, uint16_t, true>), grid, block, 0, s, a);
      else hipLaunchKernelGGL((map_install_stream_kernel<64, uint16_t, false>), grid, block, 0, s, a);
    } else {
      if (pv) hipLaunchKernelGGL((map_install_stream_kernel<64, float, true>), grid, block, 0, s, a);
      else hipLaunchKernelGGL((map_install_stream_kernel<64, float, false>), grid, block, 0, s, a);
    }
    if (tracked_pair >= 0) {
      CB_HIP(hipGetLastError());
      CB_HIP(hipEventRecord(p->pair_done[tracked_pair], s));
      p->pair_stream[tracked_pair] = s;
    }
  } else if (p->generic) {
    const dim3 g(static_cast<unsigned>(grid_blocks)), b(kAnyThreads);
    if (p->info.io_dtype == CB_DTYPE_BF16) hipLaunchKernelGGL(map_install_any_kernel<uint16_t>, g, b, 0, s, a, D);
    else if (p->info.io_dtype == CB_DTYPE_F16) hipLaunchKernelGGL(map_install_any_kernel<_Float16>, g, b, 0, s, a, D);
    else hipLaunchKernelGGL(map_install_any_kernel<float>, g, b, 0, s, a, D);
  } else if (p->support_gemm) {
    // One persistent workgroup per CU; 8 per XCD at least.
    const unsigned per_xcd = static_cast<unsigned>(std::max(1, p->num_cus / 8));
    hipLaunchKernelGGL(map_install_support_kernel, dim3(8 * per_xcd), dim3(kSupThreads), 0, s, a);
  } else {
    if (D == 128 && p->ntw == 2)
      hipLaunchKernelGGL((map_install_gen_kernel<128, uint16_t>), grid, block, 0, s, a);
    else if (D == 64 && p->ntw == 2)
      hipLaunchKernelGGL((map_install_gen_kernel<64, uint16_t>), grid, block, 0, s, a);
    else
      hipLaunchKernelGGL((map_install_gen_kernel<64, float>), grid, block, 0, s, a);
  }
  CB_HIP(hipGetLastError());
  return CB_OK;
}

// Token space of a batched launch: class by class, request by request, the
// kept tokens of request r in class c occupy [vbase, vbase + count) (arrays
// indexed c * num_spans + r).
struct BatchLayout {
  std::vector<int64_t> first, count, vbase;
  int64_t cls_base[kMaxClasses] = {0, 0, 0, 0};
  int64_t cls_count[kMaxClasses] = {0, 0, 0, 0};
  int64_t total = 0;
};

int batch_layout(const cb_plan* p, const cb_span* spans, int32_t num_spans, BatchLayout* L) {
  if (num_spans < 0 || (num_spans > 0 && !spans)) return fail(CB_EINVAL, "bad request array");
  const size_t cells = static_cast<size_t>(p->num_windows) * num_spans;
  L->first.assign(cells, 0);
  L->count.assign(cells, 0);
  L->vbase.assign(cells, 0);
  for (int r = 0; r < num_spans; ++r) {
    const cb_span& sp = spans[r];
    const int64_t n = sp.num_tokens;
    if (n < 0) return fail(CB_EINVAL, "request %d: num_tokens must be >= 0", r);
    if (sp.position_start < 0 || sp.position_start + n > p->info.table_positions)
      return fail(CB_EINVAL, "request %d: positions [%d, %lld) exceed the RoPE table (%d positions)",
                  r, sp.position_start, static_cast<long long>(sp.position_start + n),
                  p->info.table_positions);
    if (sp.source_offset < 0 || sp.target_offset < 0 || sp.source_offset > (int64_t{1} << 40) ||
        sp.target_offset > (int64_t{1} << 40))
      return fail(CB_EINVAL, "request %d: index offsets out of range", r);
    if (sp.reserved != 0) return fail(CB_EINVAL, "request %d: reserved must be 0", r);
    const int64_t prefix = sp.prefix_length > 0 ? sp.prefix_length : sp.position_start + n;
    if (prefix < sp.position_start + n)
      return fail(CB_EINVAL, "request %d: prefix_length is shorter than the block end", r);
    int64_t first[kMaxClasses], count[kMaxClasses];
    class_ranges(p, n, sp.position_start, prefix, first, count);
    for (int c = 0; c < p->num_windows; ++c) {
      L->first[static_cast<size_t>(c) * num_spans + r] = first[c];
      L->count[static_cast<size_t>(c) * num_spans + r] = count[c];
    }
  }
  for (int c = 0; c < p->num_windows; ++c) {
    L->cls_base[c] = L->total;
    for (int r = 0; r < num_spans; ++r) {
      const size_t k = static_cast<size_t>(c) * num_spans + r;
      L->vbase[k] = L->total;
      L->total += L->count[k];
    }
    L->cls_count[c] = L->total - L->cls_base[c];
  }
  if (L->total > INT32_MAX) return fail(CB_EINVAL, "batch too large for one launch");
  return CB_OK;
}

// Workspace of a batch: int32 source rows, target rows and positions of every
// token of the batch's token space, each section 256-byte aligned.
int64_t batch_workspace(int64_t tokens) { return 3 * ((tokens * 4 + 255) / 256 * 256); }

// Device address of `scratch` on each GPU, looked up once per device with
// that device current (at plan creation on it).
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

int scratch_setup(int device) {
  if (device < 0 || device >= kMaxDevices)
    return fail(CB_EINVAL, "device %d is beyond the %d devices the no-allocation workspace covers",
                device, kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[device]) return CB_OK;
  void* ptr = nullptr;
  CB_HIP(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)));
  if (!ptr) return fail(CB_EHIP, "hipGetSymbolAddress returned a null workspace address");
  g_scratch_ptr[device] = ptr;
  return CB_OK;
}

void* scratch_on(int device) {
  if (device < 0 || device >= kMaxDevices) return nullptr;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  return g_scratch_ptr[device];
}

}  // namespace

extern "C" {

const char* cb_last_error(void) { return g_last_error.c_str(); }

int cb_abi_version(void) { return CB_ABI_VERSION; }

int cb_plan_create(const cb_plan_desc* d, cb_plan** out) {
  g_last_error.clear();
  if (!d || !out) return fail(CB_EINVAL, "null descriptor or output");
  *out = nullptr;
  const int D = d->head_dim, S = d->support, nj = d->num_jobs;
  if (D < 2 || D > kAnyMaxDim || (D & 1))
    return fail(CB_EINVAL, "head_dim must be even and in [2, %d] (got %d)", kAnyMaxDim, D);
  if (S < 1 || S > CB_MAX_SUPPORT) return fail(CB_EINVAL, "support must be in [1, %d]", CB_MAX_SUPPORT);
  if (d->io_dtype != CB_DTYPE_BF16 && d->io_dtype != CB_DTYPE_F32 && d->io_dtype != CB_DTYPE_F16)
    return fail(CB_EINVAL, "io_dtype must be CB_DTYPE_BF16, CB_DTYPE_F16 or CB_DTYPE_F32");
  if (nj < 1 || d->target_layers < 1 || d->target_heads < 1)
    return fail(CB_EINVAL, "num_jobs, target_layers and target_heads must be positive");
  if (nj > (1 << 20)) return fail(CB_EINVAL, "too many jobs");
  if (!d->job_target_layer || !d->job_target_head || !d->job_kind || !d->job_window ||
      !d->job_source_theta || !d->job_target_theta || !d->job_source_layer || !d->job_source_head)
    return fail(CB_EINVAL, "job arrays must not be NULL");
  if (!d->d_weight || !d->d_bias || !d->d_cos || !d->d_sin)
    return fail(CB_EINVAL, "device weight, bias and RoPE tables must not be NULL");
  if (d->num_thetas < 1 || d->num_thetas > 255 || d->table_positions < 1)
    return fail(CB_EINVAL, "num_thetas must be in [1,255] and table_positions positive");
  if (d->num_windows < 1 || d->num_windows > kMaxClasses)
    return fail(CB_EINVAL, "num_windows must be in [1, %d]", kMaxClasses);
  for (int c = 0; c < d->num_windows; ++c)
    if (d->window_size[c] < 0 || d->window_size[c] == 1)
      return fail(CB_EINVAL, "window_size must be 0 (full) or >= 2");
  if (d->target_layers > 0xffff || d->target_heads > 0x7fff)
    return fail(CB_EINVAL, "target layers/heads out of range");

  std::vector<int> seen(static_cast<size_t>(d->target_layers) * d->target_heads * 2, 0);
  for (int j = 0; j < nj; ++j) {
    const int tl = d->job_target_layer[j], th = d->job_target_head[j], kd = d->job_kind[j];
    if (tl < 0 || tl >= d->target_layers || th < 0 || th >= d->target_heads)
      return fail(CB_EINVAL, "job %d: target (layer %d, head %d) out of range", j, tl, th);
    if (kd != CB_KIND_K && kd != CB_KIND_V) return fail(CB_EINVAL, "job %d: bad kind %d", j, kd);
    if (d->job_window[j] < 0 || d->job_window[j] >= d->num_windows)
      return fail(CB_EINVAL, "job %d: window class out of range", j);
    if (d->job_source_theta[j] < 0 || d->job_source_theta[j] >= d->num_thetas ||
        d->job_target_theta[j] < 0 || d->job_target_theta[j] >= d->num_thetas)
      return fail(CB_EINVAL, "job %d: theta index out of range", j);
    int& s = seen[(static_cast<size_t>(tl) * d->target_heads + th) * 2 + kd];
    if (s) return fail(CB_EINVAL, "duplicate job for target (layer %d, head %d, kind %d)", tl, th, kd);
    s = 1;
    for (int k = 0; k < S; ++k) {
      const int sl = d->job_source_layer[j * S + k], sh = d->job_source_head[j * S + k];
      if (sl < 0 || sl > 0xffff || sh < 0 || sh > 0x7fff)
        return fail(CB_EINVAL, "job %d: source pair (%d, %d) out of range", j, sl, sh);
    }
  }

  // Member order within a job: as given, except for the support kernel
  // (bf16, head_dim 128, support > 1), which visits a job's source pairs in
  // ascending (layer, head) order so that jobs sharing source layers visit
  // them at about the same time (the sum over members is then taken in that
  // order; its W rows are packed to match).
  std::vector<int> mperm(static_cast<size_t>(nj) * S);
  for (int j = 0; j < nj; ++j) {
    int* m = mperm.data() + static_cast<size_t>(j) * S;
    std::iota(m, m + S, 0);
    if (S > 1 && D == 128 && d->io_dtype == CB_DTYPE_BF16)
      std::stable_sort(m, m + S, [&](int u, int v) {
        const int lu = d->job_source_layer[j * S + u], lv = d->job_source_layer[j * S + v];
        if (lu != lv) return lu < lv;
        return d->job_source_head[j * S + u] < d->job_source_head[j * S + v];
      });
  }
  auto src_layer = [&](int j, int k) { return d->job_source_layer[j * S + mperm[static_cast<size_t>(j) * S + k]]; };
  auto src_head = [&](int j, int k) { return d->job_source_head[j * S + mperm[static_cast<size_t>(j) * S + k]]; };

  // Sort jobs: window class, kind, RoPE theta sets, source pairs, then target
  // position. A group (same class, kind, thetas and source pairs) reads the
  // same source rows and tables.
  std::vector<int> order(nj);
  std::iota(order.begin(), order.end(), 0);
  auto key_less = [&](int x, int y) {
    if (d->job_window[x] != d->job_window[y]) return d->job_window[x] < d->job_window[y];
    if (d->job_kind[x] != d->job_kind[y]) return d->job_kind[x] < d->job_kind[y];
    if (d->job_source_theta[x] != d->job_source_theta[y])
      return d->job_source_theta[x] < d->job_source_theta[y];
    if (d->job_target_theta[x] != d->job_target_theta[y])
      return d->job_target_theta[x] < d->job_target_theta[y];
    // Support lists usually keep to one source head: jobs of a head sort
    // together, in the order of their source layers (depth).
    if (S > 1 && src_head(x, 0) != src_head(y, 0)) return src_head(x, 0) < src_head(y, 0);
    for (int k = 0; k < S; ++k) {
      const int a0 = src_layer(x, k), b0 = src_layer(y, k);
      if (a0 != b0) return a0 < b0;
      const int a1 = src_head(x, k), b1 = src_head(y, k);
      if (a1 != b1) return a1 < b1;
    }
    if (d->job_target_layer[x] != d->job_target_layer[y])
      return d->job_target_layer[x] < d->job_target_layer[y];
    return d->job_target_head[x] < d->job_target_head[y];
  };
  std::stable_sort(order.begin(), order.end(), key_less);
  auto same_group = [&](int x, int y) {
    if (d->job_window[x] != d->job_window[y] || d->job_kind[x] != d->job_kind[y] ||
        d->job_source_theta[x] != d->job_source_theta[y] ||
        d->job_target_theta[x] != d->job_target_theta[y])
      return false;
    for (int k = 0; k < S; ++k)
      if (src_layer(x, k) != src_layer(y, k) || src_head(x, k) != src_head(y, k)) return false;
    return true;
  };

  cb_plan* p = new cb_plan();
  int rc = plan_build(d, order, mperm, same_group, p);
  // The plan's device is current here: look up its no-allocation workspace.
  if (rc == CB_OK) rc = scratch_setup(p->device);
  if (rc != CB_OK) {
    plan_free(p);
    return rc;
  }
  *out = p;
  return CB_OK;
}

void cb_plan_destroy(cb_plan* plan) { plan_free(plan); }

int cb_plan_get_info(const cb_plan* plan, cb_plan_info* info) {
  if (!plan || !info) return fail(CB_EINVAL, "null plan or info");
  *info = plan->info;
  return CB_OK;
}

int cb_plan_last_split(const cb_plan* plan, int32_t* pool_chunks, int32_t* workgroups) {
  if (!plan || !pool_chunks || !workgroups) return fail(CB_EINVAL, "null plan or output");
  *pool_chunks = plan->last_pool_chunks.load(std::memory_order_relaxed);
  *workgroups = plan->last_workgroups.load(std::memory_order_relaxed);
  return CB_OK;
}

int cb_map_install(const cb_plan* p, const cb_request* rq, void* stream) {
  if (!p || !rq) return fail(CB_EINVAL, "null plan or request");
  const int n = rq->num_tokens;
  if (n < 1) return fail(CB_EINVAL, "num_tokens must be positive");
  if (rq->position_start < 0 ||
      static_cast<int64_t>(rq->position_start) + n > p->info.table_positions)
    return fail(CB_EINVAL, "positions [%d, %lld) exceed the RoPE table (%d positions)",
                rq->position_start, static_cast<long long>(rq->position_start) + n,
                p->info.table_positions);
  const cb_rows& sr = rq->source;
  const cb_rows& tr = rq->target;
  int rc;
  if ((rc = check_sides(p, sr, tr))) return rc;
  MapArgs a{};
  const int align = p->generic ? p->elem_bytes : 16;
  if ((rc = to_dev_rows(sr, p->elem_bytes, &a.src, align))) return rc;
  if ((rc = to_dev_rows(tr, p->elem_bytes, &a.tgt, align))) return rc;
  const int64_t prefix = rq->prefix_length > 0 ? rq->prefix_length
                                               : static_cast<int64_t>(rq->position_start) + n;
  if (prefix < static_cast<int64_t>(rq->position_start) + n)
    return fail(CB_EINVAL, "prefix_length is shorter than the block end");
  int64_t first[kMaxClasses], count[kMaxClasses];
  class_ranges(p, n, rq->position_start, prefix, first, count);
  a.position_start = rq->position_start;
  return launch_map(p, a, first, count, rq->tokens_per_workgroup, default_chunk(p, n),
                    static_cast<hipStream_t>(stream));
}

int cb_batch_workspace_bytes(const cb_plan* p, const cb_span* spans, int32_t num_spans, int64_t* bytes) {
  if (!p || !bytes) return fail(CB_EINVAL, "null plan or output");
  BatchLayout L;
  int rc;
  if ((rc = batch_layout(p, spans, num_spans, &L))) return rc;
  *bytes = batch_workspace(L.total);
  return CB_OK;
}

int cb_map_install_batch(const cb_plan* p, const cb_rows* source, const cb_rows* target,
                         const cb_span* spans, int32_t num_spans, void* d_workspace,
                         int64_t workspace_bytes, void* stream) {
  if (!p || !source || !target) return fail(CB_EINVAL, "null plan, source or target");
  int rc;
  if ((rc = check_sides(p, *source, *target))) return rc;
  if (source->rows > INT32_MAX || target->rows > INT32_MAX)
    return fail(CB_EINVAL, "batched launches address at most 2^31 rows per side");
  BatchArgs b{};
  const int align = p->generic ? p->elem_bytes : 16;
  if ((rc = to_dev_rows(*source, p->elem_bytes, &b.src, align))) return rc;
  if ((rc = to_dev_rows(*target, p->elem_bytes, &b.tgt, align))) return rc;
  BatchLayout L;
  if ((rc = batch_layout(p, spans, num_spans, &L))) return rc;
  for (int r = 0; r < num_spans; ++r) {
    const int64_t n = spans[r].num_tokens;
    const cb_rows* sides[2] = {source, target};
    const int64_t offs[2] = {spans[r].source_offset, spans[r].target_offset};
    for (int k = 0; k < 2; ++k)
      if (sides[k]->index_kind == CB_INDEX_BLOCK_TABLE &&
          sides[k]->index_offset + offs[k] + n > INT32_MAX)
        return fail(CB_EINVAL, "request %d: block-table token offset beyond 2^31", r);
  }
  if (L.total == 0) return CB_OK;
  const int64_t need = batch_workspace(L.total);
  if (!d_workspace || workspace_bytes < need)
    return fail(CB_EINVAL, "batch workspace of %lld bytes is smaller than the %lld needed",
                static_cast<long long>(workspace_bytes), static_cast<long long>(need));
  if (reinterpret_cast<uintptr_t>(d_workspace) % 256)
    return fail(CB_EINVAL, "batch workspace must be 256-byte aligned");
  const int64_t section = need / 3;
  char* ws = static_cast<char*>(d_workspace);
  b.src_row = reinterpret_cast<int32_t*>(ws);
  b.tgt_row = reinterpret_cast<int32_t*>(ws + section);
  b.pos = reinterpret_cast<int32_t*>(ws + 2 * section);
  b.ncls = p->num_windows;
  hipStream_t s = static_cast<hipStream_t>(stream);
  for (int r0 = 0; r0 < num_spans; r0 += kBatchSpans) {
    b.nspans = std::min(kBatchSpans, num_spans - r0);
    int64_t widest = 0;
    for (int i = 0; i < b.nspans; ++i) {
      const cb_span& sp = spans[r0 + i];
      b.src_off[i] = sp.source_offset;
      b.tgt_off[i] = sp.target_offset;
      b.pos0[i] = sp.position_start;
      for (int c = 0; c < p->num_windows; ++c) {
        const size_t k = static_cast<size_t>(c) * num_spans + r0 + i;
        b.first[c][i] = static_cast<int32_t>(L.first[k]);
        b.count[c][i] = static_cast<int32_t>(L.count[k]);
        b.vbase[c][i] = static_cast<int32_t>(L.vbase[k]);
        widest = std::max(widest, L.count[k]);
      }
    }
    if (widest == 0) continue;
    const dim3 grid(static_cast<unsigned>((widest + 255) / 256), static_cast<unsigned>(b.nspans * b.ncls));
    hipLaunchKernelGGL(resolve_batch_kernel, grid, dim3(256), 0, s, b);
    CB_HIP(hipGetLastError());
  }
  // The map launch reads the resolved rows as int32 row vectors over the
  // batch's token space, and each key token's position from the third section.
  MapArgs a{};
  a.src = b.src;
  a.tgt = b.tgt;
  for (DevRows* side : {&a.src, &a.tgt}) {
    side->index_kind = CB_INDEX_I32;
    side->index_offset = 0;
    side->page_size = 0;
  }
  a.src.index = b.src_row;
  a.tgt.index = b.tgt_row;
  a.pos = b.pos;
  a.position_start = 0;
  return launch_map(p, a, L.cls_base, L.cls_count, 0,
                    default_chunk(p, static_cast<int>(std::min<int64_t>(L.total, INT32_MAX))), s);
}

int cb_map_install_batch_noalloc(const cb_plan* p, const cb_rows* source, const cb_rows* target,
                                 const cb_span* spans, int32_t num_spans, void* stream) {
  if (!p) return fail(CB_EINVAL, "null plan");
  BatchLayout L;
  int rc;
  if ((rc = batch_layout(p, spans, num_spans, &L))) return rc;
  const int64_t need = batch_workspace(L.total);
  if (need > CB_NOALLOC_WORKSPACE_BYTES)
    return fail(CB_EINVAL,
                "batch of %lld kept tokens needs %lld workspace bytes; the no-allocation entry point "
                "holds %lld (%lld tokens)",
                static_cast<long long>(L.total), static_cast<long long>(need),
                static_cast<long long>(CB_NOALLOC_WORKSPACE_BYTES),
                static_cast<long long>(CB_NOALLOC_MAX_TOKENS));
  void* ws = scratch_on(p->device);
  if (!ws) return fail(CB_EINVAL, "no-allocation workspace is not set up on device %d", p->device);
  return cb_map_install_batch(p, source, target, spans, num_spans, ws, CB_NOALLOC_WORKSPACE_BYTES,
                              stream);
}

int cb_copy_rows(const cb_rows* src, const cb_rows* dst, int32_t num_layers, int32_t num_tokens,
                 int32_t row_elements, int32_t dtype, int32_t* d_error_flag, void* stream) {
  if (!src || !dst) return fail(CB_EINVAL, "null rows");
  if (dtype != CB_DTYPE_BF16 && dtype != CB_DTYPE_F32 && dtype != CB_DTYPE_F16)
    return fail(CB_EINVAL, "bad dtype");
  const int eb = dtype == CB_DTYPE_F32 ? 4 : 2;
  if (num_layers < 1 || num_tokens < 0 || row_elements < 1)
    return fail(CB_EINVAL, "num_layers and row_elements must be positive");
  if ((static_cast<int64_t>(row_elements) * eb) % 16)
    return fail(CB_EINVAL, "row bytes must be a multiple of 16");
  if (src->num_layers < num_layers || dst->num_layers < num_layers)
    return fail(CB_EINVAL, "fewer layers than num_layers");
  if (row_elements > src->row_stride || row_elements > dst->row_stride)
    return fail(CB_EINVAL, "row_elements exceeds a row stride");
  if (num_tokens == 0) return CB_OK;
  CopyArgs a{};
  int rc;
  if ((rc = to_dev_rows(*src, eb, &a.src))) return rc;
  if ((rc = to_dev_rows(*dst, eb, &a.dst))) return rc;
  a.num_tokens = num_tokens;
  a.chunks_per_row = row_elements * eb / 16;
  a.tokens_per_block = std::max(1, 256 * kCopyUnroll / a.chunks_per_row);
  a.blocks_per_layer = (num_tokens + a.tokens_per_block - 1) / a.tokens_per_block;
  a.err = d_error_flag;
  const int64_t grid = static_cast<int64_t>(num_layers) * 2 * a.blocks_per_layer;
  if (grid > 0x7fffffff) return fail(CB_EINVAL, "copy too large");
  hipLaunchKernelGGL(copy_rows_kernel, dim3(static_cast<unsigned>(grid)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), a);
  CB_HIP(hipGetLastError());
  return CB_OK;
}

int cb_plan_read_errors(cb_plan* p, int32_t* flags, void* stream) {
  if (!p || !flags) return fail(CB_EINVAL, "null plan or flags");
  hipStream_t s = static_cast<hipStream_t>(stream);
  CB_HIP(hipMemcpyAsync(flags, p->d_err, 4, hipMemcpyDeviceToHost, s));
  CB_HIP(hipStreamSynchronize(s));
  CB_HIP(hipMemsetAsync(p->d_err, 0, 4, s));
  CB_HIP(hipStreamSynchronize(s));
  return CB_OK;
}

int cb_delta_state_transform(int32_t dtype, int64_t batch, int32_t k, int32_t v, int32_t kp, int32_t vp,
                             const void* d_state, int64_t state_stride, const void* d_key_basis,
                             int64_t key_stride, const void* d_value_basis, int64_t value_stride,
                             void* d_out, int64_t out_stride, void* stream) {
  if (dtype != CB_DTYPE_F32 && dtype != CB_DTYPE_F64) return fail(CB_EINVAL, "delta state dtype must be fp32 or fp64");
  if (batch < 0) return fail(CB_EINVAL, "negative batch");
  if (k < 1 || v < 1 || kp < 1 || vp < 1) return fail(CB_EINVAL, "matrix dimensions must be positive");
  if (v > kDeltaMaxV) return fail(CB_EINVAL, "value dimension above %d", kDeltaMaxV);
  if (state_stride < 0 || key_stride < 0 || value_stride < 0 || out_stride < 0)
    return fail(CB_EINVAL, "negative batch stride");
  if (batch == 0) return CB_OK;
  if (!d_state || !d_key_basis || !d_value_basis || !d_out) return fail(CB_EINVAL, "null matrix pointer");
  if (out_stride < static_cast<int64_t>(kp) * vp && batch > 1)
    return fail(CB_EINVAL, "output batch stride overlaps entries");
  if (batch > 0x7fffffff) return fail(CB_EINVAL, "batch too large");
  DeltaArgs a{d_state, d_key_basis, d_value_basis, d_out, state_stride, key_stride, value_stride, out_stride,
              k, v, kp, vp};
  const dim3 grid(static_cast<unsigned>(batch), static_cast<unsigned>((kp + 15) / 16));
  const bool square128 = k == kDs && v == kDs && kp == kDs && vp == kDs;
  if (dtype == CB_DTYPE_F32 && square128)
    hipLaunchKernelGGL(delta_state128_kernel, dim3(static_cast<unsigned>(batch)), dim3(512), 0,
                       static_cast<hipStream_t>(stream), a);
  else if (dtype == CB_DTYPE_F32)
    hipLaunchKernelGGL(delta_state_kernel<float>, grid, dim3(256), 0, static_cast<hipStream_t>(stream), a);
  else
    hipLaunchKernelGGL(delta_state_kernel<double>, grid, dim3(256), 0, static_cast<hipStream_t>(stream), a);
  CB_HIP(hipGetLastError());
  return CB_OK;
}

}  // extern "C"
