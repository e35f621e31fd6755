// CacheBridge online handoff path for MI355X (gfx950): fused source gather,
// RoPE un-rotation, split-bf16 MFMA affine map, bias, RoPE rotation, cast and
// paged scatter into the target KV pool; plus row copy (gather / install) and
// the plan that pre-packs the fitted maps.
//
// Reference algorithm (cb/ = src/cachebridge/ of the reference repository):
//   cb/mapper.py:117-239 (map_page), cb/rope.py:9-89 (RoPE),
//   cb/online/blocks.py:47-111 (pack_source_block, map_write_block).
//
// Precision: W is split on the host side of the launch (pack kernel) into
// bf16 terms w = w0 + w1 (+ w2 for fp32 I/O); the un-rotated fp32 key is split
// the same way in registers. Products with term-index sum below the term
// count are accumulated in fp32 by MFMA (Henry, Tang, Heinecke, "Leveraging
// the bfloat16 AI datatype for higher-precision computations", ARITH 2019):
// bf16 keys 3 products, bf16 values 2 (values are bf16-exact), fp32 I/O 6.

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <numeric>
#include <string>
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

#define CB_HIP(expr)                                                              \
  do {                                                                            \
    hipError_t e_ = (expr);                                                       \
    if (e_ != hipSuccess) return fail(CB_EHIP, "%s: %s", #expr, hipGetErrorString(e_)); \
  } while (0)

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kWave = 64;
constexpr int kWaves = 4;
constexpr int kThreads = kWave * kWaves;
constexpr int kColTiles = 2;                         // 16-token MFMA column tiles per wave
constexpr int kWaveTokens = 16 * kColTiles;          // tokens per wave per sub-tile
constexpr int kSubTokens = kWaves * kWaveTokens;     // tokens per workgroup sub-tile
constexpr int kMaxClasses = CB_MAX_WINDOW_CLASSES;

// Geometry of one (job, support) weight block for head_dim D with NTW terms.
//   in-dim  of (k-step ks, lane group g, element e):
//     half(ks)*D/2 + g*D/8 + (ks % (D/64))*8 + e,  half(ks) = ks / (D/64)
//   out-dim of (row tile rt, tile row r):
//     half(rt)*D/2 + (r/4)*D/8 + 4*(rt % (D/32)) + r%4, half(rt) = rt / (D/32)
// so every lane group g owns dims [g*D/8, (g+1)*D/8) of both halves, which
// puts RoPE partners j and j+D/2 in the same lane on input and output.
template <int D, int NTW>
struct Geo {
  static constexpr int HALF = D / 2;
  static constexpr int KS = D / 32;   // k-steps (MFMA K = 32)
  static constexpr int RT = D / 16;   // output row tiles (MFMA M = 16)
  static constexpr int G = D / 8;     // dims per lane group per half
  static constexpr int W_U4 = RT * KS * NTW * kWave;  // uint4 per (job, support)
};

__host__ __device__ inline int in_dim(int D, int ks, int g, int e) {
  const int per_half = D / 64;
  return (ks / per_half) * (D / 2) + g * (D / 8) + (ks % per_half) * 8 + e;
}
__host__ __device__ inline int out_dim(int D, int rt, int r) {
  const int per_half = D / 32;
  return (rt / per_half) * (D / 2) + (r / 4) * (D / 8) + 4 * (rt % per_half) + (r % 4);
}

__device__ inline float bf2f(uint16_t h) { return __uint_as_float(static_cast<uint32_t>(h) << 16); }

// Round-to-nearest-even fp32 -> bf16 bits; NaN -> canonical quiet NaN.
__device__ inline uint16_t f2bf(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0;
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}

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
    case CB_INDEX_I32: return static_cast<const int32_t*>(R.index)[u];
    case CB_INDEX_I64: return static_cast<const int64_t*>(R.index)[u];
    default: {
      const int32_t ps = R.page_size;
      const int64_t page = static_cast<const int32_t*>(R.index)[u / ps];
      return page * ps + u % ps;
    }
  }
}

__device__ inline const char* layer_base(const DevRows& R, int kind, int layer) {
  const void* const* arr = kind ? R.v_layers : R.k_layers;
  if (arr) return static_cast<const char*>(arr[layer]);
  return (kind ? R.v_base : R.k_base) + layer * R.layer_stride_b;
}

struct MapArgs {
  const uint4* w;
  const float* bias;
  const int4* jobs;
  const int32_t* pairs;
  const int32_t* group_of;
  const int32_t* group_start;
  const int32_t* group_size;
  const float* cos_tab;
  const float* sin_tab;
  int64_t theta_stride;  // elements per theta table
  DevRows src;
  DevRows tgt;
  int32_t n_tokens;
  int32_t position_start;
  int32_t support;
  int32_t chunk;
  int32_t ncls;
  int32_t cls_job_begin[kMaxClasses];
  int32_t cls_tok_first[kMaxClasses];
  int32_t cls_tok_count[kMaxClasses];
  int32_t cls_nchunks[kMaxClasses];
  int32_t cls_item_begin[kMaxClasses + 1];
  int32_t total_items;
  int32_t padded_items;
  int32_t* err;
};

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

// Load n contiguous elements (n*BYTES a multiple of 16) as fp32.
template <typename IO, int N>
__device__ inline void load_run(const char* p, float* out) {
  constexpr int U4 = N * IOTraits<IO>::BYTES / 16;
  const uint4* q = reinterpret_cast<const uint4*>(p);
#pragma unroll
  for (int u = 0; u < U4; ++u) {
    const uint4 v = q[u];
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
    if constexpr (IOTraits<IO>::BYTES == 2) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        out[u * 8 + 2 * i] = __uint_as_float(w[i] << 16);
        out[u * 8 + 2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
      }
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) out[u * 4 + i] = __uint_as_float(w[i]);
    }
  }
}

template <typename IO, int N>
__device__ inline void store_run(char* p, const float* in) {
  constexpr int U4 = N * IOTraits<IO>::BYTES / 16;
  uint4* q = reinterpret_cast<uint4*>(p);
#pragma unroll
  for (int u = 0; u < U4; ++u) {
    uint32_t w[4];
    if constexpr (IOTraits<IO>::BYTES == 2) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        w[i] = static_cast<uint32_t>(f2bf(in[u * 8 + 2 * i])) |
               (static_cast<uint32_t>(f2bf(in[u * 8 + 2 * i + 1])) << 16);
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) w[i] = __float_as_uint(in[u * 4 + i]);
    }
    q[u] = make_uint4(w[0], w[1], w[2], w[3]);
  }
}

template <int N>
__device__ inline void load_f32(const float* p, float* out) {
  const float4* q = reinterpret_cast<const float4*>(p);
#pragma unroll
  for (int u = 0; u < N / 4; ++u) {
    const float4 v = q[u];
    out[4 * u] = v.x;
    out[4 * u + 1] = v.y;
    out[4 * u + 2] = v.z;
    out[4 * u + 3] = v.w;
  }
}

// Split 8 fp32 values into XT bf16 terms: x = t0 + t1 (+ t2) + residual.
template <int XT>
__device__ inline void split8(const float* x, bf16x8* terms) {
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    float r = x[e];
#pragma unroll
    for (int t = 0; t < XT; ++t) {
      const uint16_t h = f2bf(r);
      terms[t][e] = __builtin_bit_cast(__bf16, h);
      r = r - bf2f(h);
    }
  }
}

// Stage one (job, support) weight block into LDS; NU4 is a multiple of kThreads.
template <int NU4>
__device__ inline void copy_w_to_lds(uint4* lds, const uint4* __restrict__ src) {
  constexpr int PER = NU4 / kThreads;
  constexpr int B = PER < 8 ? PER : 8;
  static_assert(NU4 % kThreads == 0 && PER % B == 0, "weight block size");
  for (int base = 0; base < NU4; base += kThreads * B) {
    uint4 v[B];
#pragma unroll
    for (int i = 0; i < B; ++i) v[i] = src[base + i * kThreads + threadIdx.x];
#pragma unroll
    for (int i = 0; i < B; ++i) lds[base + i * kThreads + threadIdx.x] = v[i];
  }
}

template <int D, typename IO, bool IS_K>
__device__ void run_job(const MapArgs& a, uint4* lds_w, int job, int tok_lo, int tok_hi,
                        int4 meta) {
#pragma clang fp contract(off)
  using T = IOTraits<IO>;
  using Gm = Geo<D, T::NTW>;
  constexpr int NTW = T::NTW;
  constexpr int XT = IS_K ? T::XT_K : T::XT_V;
  constexpr int KS = Gm::KS, RT = Gm::RT, G = Gm::G, HALF = Gm::HALF;
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
  const uint4* wj = a.w + static_cast<size_t>(job) * S * Gm::W_U4;
  const int32_t* pj = a.pairs + static_cast<size_t>(job) * S;

  float bias1[G], bias2[G];
  load_f32<G>(a.bias + static_cast<size_t>(job) * D + g * G, bias1);
  load_f32<G>(a.bias + static_cast<size_t>(job) * D + HALF + g * G, bias2);

  char* tbase = const_cast<char*>(layer_base(a.tgt, kind, tl)) +
                static_cast<int64_t>(th - a.tgt.head_offset) * D * T::BYTES;
  const float* cos_s = a.cos_tab + sth * a.theta_stride;
  const float* sin_s = a.sin_tab + sth * a.theta_stride;
  const float* cos_t = a.cos_tab + tth * a.theta_stride;
  const float* sin_t = a.sin_tab + tth * a.theta_stride;

  if (S == 1) {
    copy_w_to_lds<Gm::W_U4>(lds_w, wj);
    __syncthreads();
  }

  for (int sub = tok_lo; sub < tok_hi; sub += kSubTokens) {
    int tok[kColTiles];
    bool valid[kColTiles];
#pragma unroll
    for (int ct = 0; ct < kColTiles; ++ct) {
      tok[ct] = sub + wave * kWaveTokens + ct * 16 + col;
      valid[ct] = tok[ct] < tok_hi;
    }
    f32x4 acc[RT][kColTiles];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
      for (int ct = 0; ct < kColTiles; ++ct) acc[rt][ct] = f32x4{0.f, 0.f, 0.f, 0.f};

    for (int k = 0; k < S; ++k) {
      if (S > 1) {
        __syncthreads();
        copy_w_to_lds<Gm::W_U4>(lds_w, wj + static_cast<size_t>(k) * Gm::W_U4);
        __syncthreads();
      }
      const int pr = pj[k];
      const int sl = pr & 0xffff;
      const int sh = pr >> 16;
      const char* sbase = layer_base(a.src, kind, sl) +
                          static_cast<int64_t>(sh - a.src.head_offset) * D * T::BYTES;

      bf16x8 bx[KS][kColTiles][XT];
#pragma unroll
      for (int ct = 0; ct < kColTiles; ++ct) {
        float x1[G], x2[G];
        bool ok = valid[ct];
        int64_t row = 0;
        if (ok) {
          row = row_of(a.src, tok[ct]);
          if (row < 0 || row >= a.src.rows) {
            atomicOr(a.err, 1);
            ok = false;
          }
        }
        if (ok) {
          const char* p = sbase + row * a.src.row_stride_b;
          load_run<IO, G>(p + (g * G) * T::BYTES, x1);
          load_run<IO, G>(p + (HALF + g * G) * T::BYTES, x2);
          if constexpr (IS_K) {
            // remove_rope: (x*cos - rotate_half(x)*sin) / max(cos^2 + sin^2, tiny)
            const int pos = a.position_start + tok[ct];
            float c[G], s[G];
            load_f32<G>(cos_s + static_cast<int64_t>(pos) * HALF + g * G, c);
            load_f32<G>(sin_s + static_cast<int64_t>(pos) * HALF + g * G, s);
#pragma unroll
            for (int e = 0; e < G; ++e) {
              const float m = fmaxf(c[e] * c[e] + s[e] * s[e], 1.17549435e-38f);
              const float a1 = (x1[e] * c[e] + x2[e] * s[e]) / m;
              const float a2 = (x2[e] * c[e] - x1[e] * s[e]) / m;
              x1[e] = a1;
              x2[e] = a2;
            }
          }
        } else {
#pragma unroll
          for (int e = 0; e < G; ++e) x1[e] = x2[e] = 0.f;
        }
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
          const int half_idx = ks / (KS / 2);
          const int sub8 = ks % (KS / 2);
          split8<XT>((half_idx ? x2 : x1) + sub8 * 8, bx[ks][ct]);
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
          for (int ct = 0; ct < kColTiles; ++ct) {
            // small terms first: sum of term indices from NTW-1 down to 0
#pragma unroll
            for (int lvl = NTW - 1; lvl >= 0; --lvl) {
#pragma unroll
              for (int i = 0; i < XT; ++i) {
                const int j = lvl - i;
                if (j < 0 || j >= NTW) continue;
                acc[rt][ct] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(aw[j], bx[ks][ct][i],
                                                                      acc[rt][ct], 0, 0, 0);
              }
            }
          }
        }
      }
    }

    // Epilogue: bias, target RoPE (keys), cast, scatter through the target index.
#pragma unroll
    for (int ct = 0; ct < kColTiles; ++ct) {
      if (!valid[ct]) continue;
      const int64_t row = row_of(a.tgt, tok[ct]);
      if (row < 0 || row >= a.tgt.rows) {
        atomicOr(a.err, 2);
        continue;
      }
      float o1[G], o2[G];
      float c[G], s[G];
      if constexpr (IS_K) {
        const int pos = a.position_start + tok[ct];
        load_f32<G>(cos_t + static_cast<int64_t>(pos) * HALF + g * G, c);
        load_f32<G>(sin_t + static_cast<int64_t>(pos) * HALF + g * G, s);
      }
#pragma unroll
      for (int rt = 0; rt < RT / 2; ++rt) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int e = 4 * rt + i;
          const float y1 = acc[rt][ct][i] + bias1[e];
          const float y2 = acc[rt + RT / 2][ct][i] + bias2[e];
          if constexpr (IS_K) {
            // apply_rope: x*cos + rotate_half(x)*sin
            o1[e] = y1 * c[e] - y2 * s[e];
            o2[e] = y2 * c[e] + y1 * s[e];
          } else {
            o1[e] = y1;
            o2[e] = y2;
          }
        }
      }
      char* p = tbase + row * a.tgt.row_stride_b;
      store_run<IO, G>(p + (g * G) * T::BYTES, o1);
      store_run<IO, G>(p + (HALF + g * G) * T::BYTES, o2);
    }
  }
}

template <int D, typename IO>
__global__ __launch_bounds__(kThreads) void map_install_kernel(MapArgs a) {
  __shared__ uint4 lds_w[Geo<D, IOTraits<IO>::NTW>::W_U4];
  // XCD-aware order: consecutive logical items land on the same XCD, so jobs
  // that share source rows (adjacent after plan sorting) share that L2.
  const int per = a.padded_items >> 3;
  const int L = (blockIdx.x & 7) * per + (blockIdx.x >> 3);
  if (L >= a.total_items) return;
  int c = 0;
  while (c + 1 < a.ncls && L >= a.cls_item_begin[c + 1]) ++c;
  const int lc = L - a.cls_item_begin[c];
  const int nch = a.cls_nchunks[c];
  const int jb = a.cls_job_begin[c];
  const int grp = a.group_of[jb + lc / nch];
  const int gs = a.group_start[grp];
  const int gn = a.group_size[grp];
  const int r = lc - (gs - jb) * nch;
  const int chunk_id = r / gn;
  const int job = gs + r % gn;
  const int tok_lo = a.cls_tok_first[c] + chunk_id * a.chunk;
  const int tok_hi = min(tok_lo + a.chunk, a.cls_tok_first[c] + a.cls_tok_count[c]);
  const int4 meta = a.jobs[job];
  if ((meta.y & 0xff) == CB_KIND_K)
    run_job<D, IO, true>(a, lds_w, job, tok_lo, tok_hi, meta);
  else
    run_job<D, IO, false>(a, lds_w, job, tok_lo, tok_hi, meta);
}

// Pack fp32 W[orig][s*D][D] into bf16 split terms in MFMA A-fragment order,
// and permute the bias to sorted job order.
template <int D, int NTW>
__global__ void pack_weights_kernel(const float* __restrict__ w, const float* __restrict__ bias,
                                    const int32_t* __restrict__ order, int njobs, int S,
                                    uint16_t* __restrict__ wp, float* __restrict__ bp) {
  using Gm = Geo<D, NTW>;
  const int64_t per_block = static_cast<int64_t>(Gm::W_U4) * 8;  // bf16 per (job, support)
  const int64_t total = per_block * S * njobs;
  for (int64_t idx = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; idx < total;
       idx += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    int64_t rem = idx;
    const int e = rem % 8; rem /= 8;
    const int lane = rem % kWave; rem /= kWave;
    const int t = rem % NTW; rem /= NTW;
    const int ks = rem % Gm::KS; rem /= Gm::KS;
    const int rt = rem % Gm::RT; rem /= Gm::RT;
    const int k = rem % S; rem /= S;
    const int j = static_cast<int>(rem);
    const int src_job = order[j];
    const int fi = k * D + in_dim(D, ks, lane >> 4, e);
    const int fo = out_dim(D, rt, lane & 15);
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

// Row copy: dst layer l row(t) <- src layer l row(t), 16-byte chunks.
struct CopyArgs {
  DevRows src, dst;
  int32_t num_tokens;
  int32_t chunks_per_row;
  int32_t tokens_per_block;
  int32_t blocks_per_layer;
  int32_t* err;
};

__global__ __launch_bounds__(256) void copy_rows_kernel(CopyArgs a) {
  const int lk = blockIdx.x / a.blocks_per_layer;  // layer * 2 + kind
  const int tb = blockIdx.x % a.blocks_per_layer;
  const int layer = lk >> 1, kind = lk & 1;
  const char* sbase = layer_base(a.src, kind, layer);
  char* dbase = const_cast<char*>(layer_base(a.dst, kind, layer));
  const int t0 = tb * a.tokens_per_block;
  const int n = min(a.tokens_per_block, a.num_tokens - t0);
  const int cpr = a.chunks_per_row;
  for (int idx = threadIdx.x; idx < n * cpr; idx += blockDim.x) {
    const int t = t0 + idx / cpr;
    const int ch = idx % cpr;
    const int64_t sr = row_of(a.src, t);
    const int64_t dr = row_of(a.dst, t);
    if (sr < 0 || sr >= a.src.rows) {
      if (a.err && ch == 0) atomicOr(a.err, 1);
      continue;
    }
    if (dr < 0 || dr >= a.dst.rows) {
      if (a.err && ch == 0) atomicOr(a.err, 2);
      continue;
    }
    const uint4 v = reinterpret_cast<const uint4*>(sbase + sr * a.src.row_stride_b)[ch];
    reinterpret_cast<uint4*>(dbase + dr * a.dst.row_stride_b)[ch] = v;
  }
}

}  // namespace

struct cb_plan {
  int device = 0;
  cb_plan_info info{};
  int ntw = 2;
  int elem_bytes = 2;
  int num_windows = 1;
  int window_size[kMaxClasses] = {0, 0, 0, 0};
  int cls_job_begin[kMaxClasses] = {0, 0, 0, 0};
  int cls_job_end[kMaxClasses] = {0, 0, 0, 0};
  int max_src_layer = 0, min_src_head = 0, max_src_head = 0;
  int max_tgt_layer = 0, min_tgt_head = 0, max_tgt_head = 0;
  void* d_w = nullptr;
  float* d_bias = nullptr;
  int4* d_jobs = nullptr;
  int32_t* d_pairs = nullptr;
  int32_t* d_group_of = nullptr;
  int32_t* d_group_start = nullptr;
  int32_t* d_group_size = nullptr;
  float* d_cos = nullptr;
  float* d_sin = nullptr;
  int32_t* d_err = nullptr;
};

namespace {

void plan_free(cb_plan* p) {
  if (!p) return;
  void* ptrs[] = {p->d_w, p->d_bias, p->d_jobs, p->d_pairs, p->d_group_of, p->d_group_start,
                  p->d_group_size, p->d_cos, p->d_sin, p->d_err};
  for (void* q : ptrs)
    if (q) (void)hipFree(q);
  delete p;
}

template <typename Tp>
int upload(Tp** dst, const void* src, size_t bytes, int64_t* total) {
  CB_HIP(hipMalloc(reinterpret_cast<void**>(dst), bytes));
  *total += static_cast<int64_t>(bytes);
  if (src) CB_HIP(hipMemcpy(*dst, src, bytes, hipMemcpyHostToDevice));
  return CB_OK;
}

int to_dev_rows(const cb_rows& r, int elem_bytes, DevRows* out) {
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
  if (r.index_offset < 0) return fail(CB_EINVAL, "index_offset must be >= 0");
  if (r.rows <= 0) return fail(CB_EINVAL, "rows must be > 0");
  if (!r.k_layers && (!r.k_base || !r.v_base))
    return fail(CB_EINVAL, "either per-layer pointer arrays or k_base/v_base are required");
  if (r.k_layers && !r.v_layers) return fail(CB_EINVAL, "v_layers required with k_layers");
  if ((out->row_stride_b % 16) || (out->layer_stride_b % 16))
    return fail(CB_EINVAL, "row and layer strides must be multiples of 16 bytes");
  if ((reinterpret_cast<uintptr_t>(r.k_base) | reinterpret_cast<uintptr_t>(r.v_base)) % 16)
    return fail(CB_EINVAL, "k_base/v_base must be 16-byte aligned");
  return CB_OK;
}


template <typename SameGroup>
int plan_build(const cb_plan_desc* d, const std::vector<int>& order, SameGroup same_group,
               cb_plan* p) {
  const int D = d->head_dim, S = d->support, nj = d->num_jobs;
  int64_t bytes = 0;
  CB_HIP(hipGetDevice(&p->device));
  p->ntw = d->io_dtype == CB_DTYPE_BF16 ? 2 : 3;
  p->elem_bytes = d->io_dtype == CB_DTYPE_BF16 ? 2 : 4;
  p->num_windows = d->num_windows;
  for (int c = 0; c < kMaxClasses; ++c) {
    p->window_size[c] = c < d->num_windows ? d->window_size[c] : 0;
    p->cls_job_begin[c] = p->cls_job_end[c] = c < d->num_windows ? -1 : 0;
  }
  std::vector<int4> jobs(nj);
  std::vector<int32_t> pairs(static_cast<size_t>(nj) * S), group_of(nj);
  std::vector<int32_t> gstart, gsize;
  p->max_src_layer = 0;
  p->min_src_head = 1 << 30;
  p->max_src_head = 0;
  p->max_tgt_layer = 0;
  p->min_tgt_head = 1 << 30;
  p->max_tgt_head = 0;
  for (int i = 0; i < nj; ++i) {
    const int j = order[i];
    jobs[i] = make_int4(d->job_target_layer[j] | (d->job_target_head[j] << 16),
                        d->job_kind[j] | (d->job_window[j] << 8) |
                            (d->job_source_theta[j] << 16) | (d->job_target_theta[j] << 24),
                        0, j);
    for (int k = 0; k < S; ++k) {
      const int sl = d->job_source_layer[j * S + k], sh = d->job_source_head[j * S + k];
      pairs[static_cast<size_t>(i) * S + k] = sl | (sh << 16);
      p->max_src_layer = std::max(p->max_src_layer, sl);
      p->min_src_head = std::min(p->min_src_head, sh);
      p->max_src_head = std::max(p->max_src_head, sh);
    }
    p->max_tgt_layer = std::max(p->max_tgt_layer, d->job_target_layer[j]);
    p->min_tgt_head = std::min(p->min_tgt_head, d->job_target_head[j]);
    p->max_tgt_head = std::max(p->max_tgt_head, d->job_target_head[j]);
    if (i == 0 || !same_group(order[i - 1], j)) {
      gstart.push_back(i);
      gsize.push_back(0);
    }
    gsize.back() += 1;
    group_of[i] = static_cast<int32_t>(gstart.size() - 1);
    const int c = d->job_window[j];
    if (p->cls_job_begin[c] < 0) p->cls_job_begin[c] = i;
    p->cls_job_end[c] = i + 1;
  }
  for (int c = 0; c < d->num_windows; ++c)
    if (p->cls_job_begin[c] < 0) p->cls_job_begin[c] = p->cls_job_end[c] = 0;

  const size_t w_elems = static_cast<size_t>(nj) * S * (D / 16) * (D / 32) * p->ntw * kWave * 8;
  const size_t table = static_cast<size_t>(d->num_thetas) * d->table_positions * (D / 2);
  int rc;
  if ((rc = upload(&p->d_jobs, jobs.data(), jobs.size() * sizeof(int4), &bytes))) return rc;
  if ((rc = upload(&p->d_pairs, pairs.data(), pairs.size() * 4, &bytes))) return rc;
  if ((rc = upload(&p->d_group_of, group_of.data(), group_of.size() * 4, &bytes))) return rc;
  if ((rc = upload(&p->d_group_start, gstart.data(), gstart.size() * 4, &bytes))) return rc;
  if ((rc = upload(&p->d_group_size, gsize.data(), gsize.size() * 4, &bytes))) return rc;
  if ((rc = upload(&p->d_w, nullptr, w_elems * 2, &bytes))) return rc;
  if ((rc = upload(&p->d_bias, nullptr, static_cast<size_t>(nj) * D * 4, &bytes))) return rc;
  if ((rc = upload(&p->d_cos, nullptr, table * 4, &bytes))) return rc;
  if ((rc = upload(&p->d_sin, nullptr, table * 4, &bytes))) return rc;
  if ((rc = upload(&p->d_err, nullptr, 4, &bytes))) return rc;
  CB_HIP(hipMemcpy(p->d_cos, d->d_cos, table * 4, hipMemcpyDeviceToDevice));
  CB_HIP(hipMemcpy(p->d_sin, d->d_sin, table * 4, hipMemcpyDeviceToDevice));
  CB_HIP(hipMemset(p->d_err, 0, 4));
  int32_t* d_order = nullptr;
  CB_HIP(hipMalloc(reinterpret_cast<void**>(&d_order), order.size() * 4));
  hipError_t e = hipMemcpy(d_order, order.data(), order.size() * 4, hipMemcpyHostToDevice);
  if (e == hipSuccess) {
    const dim3 grid(1024), block(256);
    uint16_t* wp = static_cast<uint16_t*>(p->d_w);
    if (D == 64 && p->ntw == 2)
      hipLaunchKernelGGL((pack_weights_kernel<64, 2>), grid, block, 0, 0, d->d_weight, d->d_bias,
                         d_order, nj, S, wp, p->d_bias);
    else if (D == 64)
      hipLaunchKernelGGL((pack_weights_kernel<64, 3>), grid, block, 0, 0, d->d_weight, d->d_bias,
                         d_order, nj, S, wp, p->d_bias);
    else
      hipLaunchKernelGGL((pack_weights_kernel<128, 2>), grid, block, 0, 0, d->d_weight, d->d_bias,
                         d_order, nj, S, wp, p->d_bias);
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
  p->info.num_groups = static_cast<int32_t>(gstart.size());
  p->info.num_thetas = d->num_thetas;
  p->info.table_positions = d->table_positions;
  p->info.weight_terms = p->ntw;
  p->info.device_bytes = bytes;
  return CB_OK;
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
  if (D != 64 && D != 128) return fail(CB_EINVAL, "head_dim must be 64 or 128 (got %d)", D);
  if (S < 1 || S > CB_MAX_SUPPORT) return fail(CB_EINVAL, "support must be in [1, %d]", CB_MAX_SUPPORT);
  if (d->io_dtype != CB_DTYPE_BF16 && d->io_dtype != CB_DTYPE_F32)
    return fail(CB_EINVAL, "io_dtype must be CB_DTYPE_BF16 or CB_DTYPE_F32");
  if (d->io_dtype == CB_DTYPE_F32 && D != 64)
    return fail(CB_EINVAL, "fp32 I/O is supported for head_dim 64 only");
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

  // Sort jobs: window class, kind, source pairs, then target position.
  std::vector<int> order(nj);
  std::iota(order.begin(), order.end(), 0);
  auto key_less = [&](int x, int y) {
    if (d->job_window[x] != d->job_window[y]) return d->job_window[x] < d->job_window[y];
    if (d->job_kind[x] != d->job_kind[y]) return d->job_kind[x] < d->job_kind[y];
    for (int k = 0; k < S; ++k) {
      const int a0 = d->job_source_layer[x * S + k], b0 = d->job_source_layer[y * S + k];
      if (a0 != b0) return a0 < b0;
      const int a1 = d->job_source_head[x * S + k], b1 = d->job_source_head[y * S + k];
      if (a1 != b1) return a1 < b1;
    }
    if (d->job_target_layer[x] != d->job_target_layer[y])
      return d->job_target_layer[x] < d->job_target_layer[y];
    return d->job_target_head[x] < d->job_target_head[y];
  };
  std::stable_sort(order.begin(), order.end(), key_less);
  auto same_group = [&](int x, int y) {
    if (d->job_window[x] != d->job_window[y] || d->job_kind[x] != d->job_kind[y]) return false;
    for (int k = 0; k < S; ++k)
      if (d->job_source_layer[x * S + k] != d->job_source_layer[y * S + k] ||
          d->job_source_head[x * S + k] != d->job_source_head[y * S + k])
        return false;
    return true;
  };

  cb_plan* p = new cb_plan();
  const int rc = plan_build(d, order, same_group, p);
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

int cb_map_install(const cb_plan* p, const cb_request* rq, void* stream) {
  if (!p || !rq) return fail(CB_EINVAL, "null plan or request");
  const int D = p->info.head_dim;
  const int n = rq->num_tokens;
  if (n < 1) return fail(CB_EINVAL, "num_tokens must be positive");
  if (rq->position_start < 0 ||
      static_cast<int64_t>(rq->position_start) + n > p->info.table_positions)
    return fail(CB_EINVAL, "positions [%d, %lld) exceed the RoPE table (%d positions)",
                rq->position_start, static_cast<long long>(rq->position_start) + n,
                p->info.table_positions);
  const cb_rows& sr = rq->source;
  const cb_rows& tr = rq->target;
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
  if (static_cast<int64_t>(sr.heads) * D > sr.row_stride || static_cast<int64_t>(tr.heads) * D > tr.row_stride)
    return fail(CB_EINVAL, "row_stride is smaller than heads * head_dim");
  if (tr.index_kind == CB_INDEX_IDENTITY && sr.index_kind == CB_INDEX_IDENTITY &&
      tr.k_base == sr.k_base && tr.k_base)
    return fail(CB_EINVAL, "target aliases the source");
  MapArgs a{};
  int rc;
  if ((rc = to_dev_rows(sr, p->elem_bytes, &a.src))) return rc;
  if ((rc = to_dev_rows(tr, p->elem_bytes, &a.tgt))) return rc;
  int chunk = rq->tokens_per_workgroup;
  if (chunk == 0) chunk = p->info.support == 1 ? 512 : kSubTokens;
  if (chunk < kSubTokens || chunk % kSubTokens)
    return fail(CB_EINVAL, "tokens_per_workgroup must be a positive multiple of %d", kSubTokens);
  a.w = static_cast<const uint4*>(p->d_w);
  a.bias = p->d_bias;
  a.jobs = p->d_jobs;
  a.pairs = p->d_pairs;
  a.group_of = p->d_group_of;
  a.group_start = p->d_group_start;
  a.group_size = p->d_group_size;
  a.cos_tab = p->d_cos;
  a.sin_tab = p->d_sin;
  a.theta_stride = static_cast<int64_t>(p->info.table_positions) * (D / 2);
  a.n_tokens = n;
  a.position_start = rq->position_start;
  a.support = p->info.support;
  a.chunk = chunk;
  a.err = p->d_err;
  const int64_t prefix = rq->prefix_length > 0 ? rq->prefix_length
                                               : static_cast<int64_t>(rq->position_start) + n;
  if (prefix < static_cast<int64_t>(rq->position_start) + n)
    return fail(CB_EINVAL, "prefix_length is shorter than the block end");
  int64_t items = 0;
  a.ncls = p->num_windows;
  for (int c = 0; c < p->num_windows; ++c) {
    int64_t first_pos = 0;
    if (p->window_size[c] > 0) first_pos = prefix - std::min<int64_t>(prefix, p->window_size[c] - 1);
    const int64_t first = std::max<int64_t>(0, first_pos - rq->position_start);
    const int64_t count = std::max<int64_t>(0, n - first);
    const int64_t nch = (count + chunk - 1) / chunk;
    a.cls_job_begin[c] = p->cls_job_begin[c];
    a.cls_tok_first[c] = static_cast<int32_t>(std::min<int64_t>(first, n));
    a.cls_tok_count[c] = static_cast<int32_t>(count);
    a.cls_nchunks[c] = static_cast<int32_t>(std::max<int64_t>(nch, 1));
    a.cls_item_begin[c] = static_cast<int32_t>(items);
    items += static_cast<int64_t>(p->cls_job_end[c] - p->cls_job_begin[c]) * nch;
  }
  a.cls_item_begin[p->num_windows] = static_cast<int32_t>(items);
  if (items == 0) return CB_OK;
  if (items > (int64_t{1} << 30)) return fail(CB_EINVAL, "request too large for one launch");
  a.total_items = static_cast<int32_t>(items);
  a.padded_items = static_cast<int32_t>((items + 7) / 8 * 8);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (D == 128 && p->ntw == 2)
    hipLaunchKernelGGL((map_install_kernel<128, uint16_t>), dim3(a.padded_items), dim3(kThreads), 0, s, a);
  else if (D == 64 && p->ntw == 2)
    hipLaunchKernelGGL((map_install_kernel<64, uint16_t>), dim3(a.padded_items), dim3(kThreads), 0, s, a);
  else
    hipLaunchKernelGGL((map_install_kernel<64, float>), dim3(a.padded_items), dim3(kThreads), 0, s, a);
  CB_HIP(hipGetLastError());
  return CB_OK;
}

int cb_copy_rows(const cb_rows* src, const cb_rows* dst, int32_t num_layers, int32_t num_tokens,
                 int32_t row_elements, int32_t dtype, int32_t* d_error_flag, void* stream) {
  if (!src || !dst) return fail(CB_EINVAL, "null rows");
  if (dtype != CB_DTYPE_BF16 && dtype != CB_DTYPE_F32) return fail(CB_EINVAL, "bad dtype");
  const int eb = dtype == CB_DTYPE_BF16 ? 2 : 4;
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
  a.tokens_per_block = std::max(1, 4096 / a.chunks_per_row);
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

}  // extern "C"
