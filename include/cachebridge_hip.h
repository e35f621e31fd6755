/*
 * cachebridge_hip.h -- C ABI of the MI355X (gfx950) CacheBridge handoff path.
 *
 * The library maps source-model KV pages to target-model KV with per
 * (target layer, target KV head) affine maps and installs the result into the
 * target's paged KV pool:
 *
 *   for each target (layer l, head h) and kind in {K, V}:
 *     X  = concat_k source[(layer, head) pair k of (l, h)]   rows of the block
 *     K: X <- remove_rope(X, source theta)                    (fp32)
 *     Y  = X . W[l,h] + b[l,h]                                 (W is [s*D, D] fp32)
 *     K: Y <- apply_rope(Y, target theta)
 *     target_pool[l][row(t)][h] = cast(Y)                      (bf16 RNE or fp32)
 *
 * All entry points return 0 on success or a negative errno-style code
 * (CB_EINVAL, CB_ENOMEM, CB_EHIP) with a message from cb_last_error().
 * Every pointer named d_* or described as "device" is a HIP device pointer;
 * buffers are owned by the caller and must stay alive until the stream work
 * that uses them completes. Launches are asynchronous on the given stream and
 * never synchronize the device, except plan creation and cb_plan_read_errors.
 *
 * Reference interfaces replaced (paths relative to the reference repository,
 * cb/ = src/cachebridge/, rt/ = src/cachebridge/backends/sglang/runtime/):
 *   cb_plan_create     <- PageMapper.__init__ (cb/mapper.py:35-110): weight
 *                         load + TP head slice, here plus MFMA pre-packing and
 *                         resident RoPE tables (cb/rope.py:16-72).
 *   cb_map_install     <- PageMapper.map_page (cb/mapper.py:117-239) fused with
 *                         map_write_block / set_kv_buffer
 *                         (cb/online/blocks.py:86-111,
 *                         rt/r010_core.py:16-43) and the
 *                         run-segmented install of _DirectMappedPoolCodec
 *                         (rt/source_mapper_adapter.py:366-428).
 *                         With an identity target index it is map_page's
 *                         dense [2, Lt, n, Ht, D] output (cb/mapper.py:216-239).
 *   cb_delta_state_transform <- qwen35.transform_delta_state
 *                         (cb/architectures/qwen35.py:52-61).
 *   cb_copy_rows       <- pack_source_block (cb/online/blocks.py:47-82) and the
 *                         per-run install copies of _DirectMappedPoolCodec.copy
 *                         (rt/source_mapper_adapter.py:400-420).
 */
#ifndef CACHEBRIDGE_HIP_H
#define CACHEBRIDGE_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define CB_ABI_VERSION 1

#define CB_OK 0
#define CB_EINVAL (-22)
#define CB_ENOMEM (-12)
#define CB_EHIP (-5)

/* Element type of pages, pools and outputs. */
#define CB_DTYPE_BF16 0
#define CB_DTYPE_F32 1
#define CB_DTYPE_F64 2 /* cb_delta_state_transform only */
#define CB_DTYPE_F16 3 /* map / install / row copy I/O */

/* Job kinds. */
#define CB_KIND_K 0
#define CB_KIND_V 1

/* How a token index t of a request maps to a row of a K/V buffer. */
#define CB_INDEX_IDENTITY 0    /* row = t + index_offset                          */
#define CB_INDEX_I32 1         /* row = index[t + index_offset]  (int32)          */
#define CB_INDEX_I64 2         /* row = index[t + index_offset]  (int64)          */
#define CB_INDEX_BLOCK_TABLE 3 /* u = t + index_offset; row = bt[u / page_size] * page_size + u % page_size (int32 bt) */

/* Maximum number of window classes (e.g. sliding vs full attention layers). */
#define CB_MAX_WINDOW_CLASSES 4
/* Maximum support size s (source pairs per target head). */
#define CB_MAX_SUPPORT 16

/*
 * Description of one side's K/V buffers (the source pool or page, the target
 * pool or output). Layer l's K buffer is k_layers[l] when k_layers is not
 * NULL (a device array of device pointers, e.g. one tensor per layer as in
 * SGLang's MHATokenToKVPool), else k_base + l * layer_stride elements.
 * Row r of a layer starts row_stride elements after the layer base and holds
 * `heads` consecutive heads of head_dim elements, the first of which is head
 * index head_offset (global source head index for sources; local target head
 * index for targets).
 */
typedef struct cb_rows {
  const void* const* k_layers;
  const void* const* v_layers;
  const void* k_base;
  const void* v_base;
  int64_t layer_stride; /* elements */
  int64_t row_stride;   /* elements */
  int64_t rows;         /* rows per layer; a token whose source or target row is outside
                           [0, rows) writes nothing and is flagged (cb_plan_read_errors) */
  int32_t num_layers;   /* layers addressable through this description */
  int32_t head_offset;
  int32_t heads;
  int32_t index_kind; /* CB_INDEX_* */
  const void* index;  /* device; slot vector or block table */
  int64_t index_offset;
  int32_t page_size; /* CB_INDEX_BLOCK_TABLE only */
  int32_t reserved;
} cb_rows;

/*
 * Mapper plan description. Jobs are (target layer, target head, kind); each
 * job has `support` source (layer, head) pairs and a [support*head_dim,
 * head_dim] fp32 weight with y = x . W (x is the concatenation of the
 * support rows in pair order) plus a [head_dim] fp32 bias.
 */
typedef struct cb_plan_desc {
  int32_t head_dim;  /* even, 2..512. bf16 at 64 and 128 and fp32 at 64 take the
                        MFMA kernels; every other head_dim or dtype takes the
                        generic fp32 kernel (same results within the parity bar) */
  int32_t support;   /* 1..CB_MAX_SUPPORT */
  int32_t io_dtype;  /* CB_DTYPE_* */
  int32_t num_jobs;
  int32_t target_layers; /* local target layers of the plan */
  int32_t target_heads;  /* local target heads of the plan */
  /* host arrays, one entry per job */
  const int32_t* job_target_layer; /* [num_jobs] in [0, target_layers) */
  const int32_t* job_target_head;  /* [num_jobs] in [0, target_heads) */
  const int32_t* job_kind;         /* [num_jobs] CB_KIND_* */
  const int32_t* job_window;       /* [num_jobs] window class in [0, num_windows) */
  const int32_t* job_source_theta; /* [num_jobs] table index for un-rotation (K only) */
  const int32_t* job_target_theta; /* [num_jobs] table index for rotation (K only) */
  const int32_t* job_source_layer; /* [num_jobs * support] */
  const int32_t* job_source_head;  /* [num_jobs * support] global source head */
  /* device fp32 arrays in job order */
  const float* d_weight; /* [num_jobs][support*head_dim][head_dim] */
  const float* d_bias;   /* [num_jobs][head_dim] */
  /* RoPE tables: [num_thetas][table_positions][head_dim/2] fp32 (device).
     Entry [i][p][j] is qwen_rope(p)[j] of theta set i (the halves of the
     reference's [tokens, head_dim] table are equal, so only one is kept). */
  int32_t num_thetas;
  int32_t table_positions;
  const float* d_cos;
  const float* d_sin;
  /* Window classes: window_size[c] == 0 keeps every token; otherwise the
     class keeps the last min(prefix_length, window_size[c] - 1) tokens of
     the prefix (Gemma 3 sliding layers, cb/architectures/gemma3.py:52). */
  int32_t num_windows;
  int32_t window_size[CB_MAX_WINDOW_CLASSES];
} cb_plan_desc;

/* One handoff block: tokens [0, num_tokens) at positions position_start + t. */
typedef struct cb_request {
  cb_rows source;
  cb_rows target;
  int32_t num_tokens;
  int32_t position_start;
  int32_t prefix_length; /* whole prefix length for windows; 0 means position_start + num_tokens */
  /* 0 = library default. Otherwise a cap on the tokens each workgroup maps
     per unit of work: a positive multiple of 16 for the streaming kernel
     (bf16 / fp32 maps with support 1 at head_dim 64 or 128) and of 32 for the
     generic kernels; the support kernel (support > 1 at head_dim 128, bf16)
     ignores it. For the streaming kernel a cap below the default shrinks the
     grid to about (tokens x units) / cap workgroups, which can make each
     workgroup's share long enough for the work pool. */
  int32_t tokens_per_workgroup;
} cb_request;

typedef struct cb_plan cb_plan;

typedef struct cb_plan_info {
  int32_t head_dim, support, io_dtype, num_jobs, target_layers, target_heads;
  int32_t num_groups, num_thetas, table_positions, weight_terms;
  int64_t device_bytes;
} cb_plan_info;

/* Message of the last failed call on this thread ("" if none). */
const char* cb_last_error(void);
int cb_abi_version(void);

/* Validate, sort jobs by (window class, kind, source pairs) so that jobs
   reading the same source rows are adjacent, pre-pack W into bf16 split
   terms in MFMA fragment order and copy the RoPE tables. Synchronous. */
int cb_plan_create(const cb_plan_desc* desc, cb_plan** out);
void cb_plan_destroy(cb_plan* plan);
int cb_plan_get_info(const cb_plan* plan, cb_plan_info* info);
/* Work split of the plan's last map launch (host-side values, no device
   access): the work-pool chunks its workgroups claimed dynamically (0: static
   ranges only) and its workgroups. No counterpart in the reference; it lets
   a caller or test see which scheduling a launch used. */
int cb_plan_last_split(const cb_plan* plan, int32_t* pool_chunks, int32_t* workgroups);

/* Fused gather -> un-rotate -> MFMA affine map -> bias -> rotate -> cast ->
   scatter for every job of the plan over one request block. Asynchronous. */
int cb_map_install(const cb_plan* plan, const cb_request* request, void* stream);

/*
 * One request of a batched launch: tokens [0, num_tokens) of its history at
 * positions position_start + t. Its source row of token t is the shared
 * source description's row of u = source_offset + t (the cb_rows index
 * rules, including that description's index_offset), and likewise for the
 * target. With SGLang's req_to_token table, for example, the offsets are the
 * request's row times the table's row length.
 */
typedef struct cb_span {
  int64_t source_offset;
  int64_t target_offset;
  int32_t num_tokens;     /* >= 0; a request with 0 tokens is skipped */
  int32_t position_start; /* >= 0 */
  int32_t prefix_length;  /* whole prefix for windows; 0 means position_start + num_tokens */
  int32_t reserved;       /* 0 */
} cb_span;

/* Device workspace bytes cb_map_install_batch needs for these spans (host
   array). */
int cb_batch_workspace_bytes(const cb_plan* plan, const cb_span* spans, int32_t num_spans,
                             int64_t* bytes);

/* Every job of the plan over every request of a ragged batch, as one map
   launch (after one small launch per 32 requests that resolves each kept
   token's source row, target row and position into the workspace). Same
   results, row for row, as one cb_map_install per request. `spans` is a host
   array (read before the call returns); `d_workspace` is caller-owned device
   memory of at least cb_batch_workspace_bytes bytes, 256-byte aligned, that
   no other launch may use until this one completes. Asynchronous.
   Replaces the reference's one-request-at-a-time mapper transactions over an
   admitted cohort (begin_next_mapper / publish_active_mapper,
   cb/online/admission.py:466-499), each a map_page + install
   (cb/online/blocks.py:86-111). */
int cb_map_install_batch(const cb_plan* plan, const cb_rows* source, const cb_rows* target,
                         const cb_span* spans, int32_t num_spans, void* d_workspace,
                         int64_t workspace_bytes, void* stream);

/* Workspace limit of cb_map_install_batch_noalloc: 16 MiB per GPU, which
   holds the resolved rows and positions (12 bytes per kept token, three
   256-byte-aligned sections) of CB_NOALLOC_MAX_TOKENS tokens. */
#define CB_NOALLOC_WORKSPACE_BYTES 16777216
#define CB_NOALLOC_MAX_TOKENS 1398080

/* cb_map_install_batch without a caller workspace and without any device
   allocation: the resolve workspace is a fixed device array of
   CB_NOALLOC_WORKSPACE_BYTES per GPU, looked up once per device at
   cb_plan_create and held until the process ends. No counterpart in the
   reference: this is for callers that cannot allocate device memory (code
   under HIP graph capture, serving loops that forbid hipMalloc). Same rows,
   row for row, as cb_map_install_batch. A batch needing more workspace is
   rejected (CB_EINVAL) before anything is enqueued. Every call on one GPU
   shares that GPU's array: calls that overlap on one GPU (two streams, or
   a second call before the first completes on another stream) race; calls
   on one stream are ordered. Asynchronous. */
int cb_map_install_batch_noalloc(const cb_plan* plan, const cb_rows* source,
                                 const cb_rows* target, const cb_span* spans,
                                 int32_t num_spans, void* stream);

/* Copy the first row_elements elements of rows of layers [0, num_layers)
   from src to dst, K and V: dst layer l row dst_row(t) <- src layer l row
   src_row(t) for t in [0, num_tokens). row_elements * element size must be a
   multiple of 16 bytes. Rows outside [0, rows) are skipped and flagged in
   *d_error_flag (bit 0 source, bit 1 target) when it is not NULL.
   Asynchronous. */
int cb_copy_rows(const cb_rows* src, const cb_rows* dst, int32_t num_layers,
                 int32_t num_tokens, int32_t row_elements, int32_t dtype,
                 int32_t* d_error_flag, void* stream);

/* Recurrent-state transform of a linear-attention (DeltaNet) layer:
   out[b] = A[b]^T . U[b] . B[b] for b in [0, batch), with U the source state
   [k, v], A the key basis [k, kp], B the value basis [v, vp] and out [kp, vp],
   all row-major device matrices of dtype CB_DTYPE_F32 or CB_DTYPE_F64. Entry
   b of each operand starts b * stride elements after its pointer (stride 0
   uses one matrix for every entry). v <= 512. Asynchronous.
   Replaces qwen35.transform_delta_state (cb/architectures/qwen35.py:52-61),
   key_basis^T @ source_state @ value_basis over the batch dimensions. */
int cb_delta_state_transform(int32_t dtype, int64_t batch, int32_t k, int32_t v, int32_t kp, int32_t vp,
                             const void* d_state, int64_t state_stride, const void* d_key_basis,
                             int64_t key_stride, const void* d_value_basis, int64_t value_stride,
                             void* d_out, int64_t out_stride, void* stream);

/* Read and clear the plan's device error word (bit 0: source row out of
   range, bit 1: target row out of range, bit 2: a work-pool claim of the
   streaming kernel fell past its pool, a host-side inconsistency; bit 3: a
   streaming launch found its work-pool counter pair shared with another
   launch of the plan in flight, so rows may be missing). The word is one per
   plan: bits from launches that overlap are merged. Synchronizes `stream`.

   Work-pool counters: direct launches of one plan rotate over 64 counter
   pairs. A launch that uses the pool and whose pair's previous such launch
   ran on another stream makes its stream wait for that launch (an event
   recorded with it) unless it has finished, so any number of direct launches
   may be queued on any streams and none shares its pair. A launch recorded
   into a HIP graph takes a pair of its own (64 per plan; later captured
   launches run without the pool), so graph replays never share a pair with
   direct launches. Two replays of one graph that overlap in time do share
   their pair: they set bit 3. */
int cb_plan_read_errors(cb_plan* plan, int32_t* flags, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* CACHEBRIDGE_HIP_H */
