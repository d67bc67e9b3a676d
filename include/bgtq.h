/* bgtq.h — C ABI of the MI355X (gfx950) Block-GTQ hot path.
 *
 * Replaces the WebGPU substrate under the reference's TypeScript runtime
 * (src/webgpu) with HIP kernels. Every entry point takes plain pointers and
 * sizes, returns a bgtq_status (0 = success) and leaves a thread-local
 * message in bgtq_last_error(). On failure no object state changes: lengths
 * advance only after the device work of an append has completed
 * (src/runtime/packed-keys.ts:47), and validation happens before any launch.
 *
 * Two layers:
 *  1. Objects that mirror the reference's classes one to one (context =
 *     GPUDevice + queue, tables = tables(p), keys/values stores, attention
 *     sessions). Host buffers in, device-resident state, reads for tests.
 *  2. Stream-ordered batched entry points over caller-owned device memory for
 *     model geometry (the src/model dispatch names encode_k / compressed_dot /
 *     softmax / weighted / append), used for layers x sequences x heads.
 */
#ifndef BGTQ_H
#define BGTQ_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef int32_t bgtq_status;
#define BGTQ_OK 0
#define BGTQ_ERR_RANGE 1       /* invalid argument; the reference throws RangeError */
#define BGTQ_ERR_STATE 2       /* invalid object state; the reference throws Error */
#define BGTQ_ERR_DEVICE 3      /* HIP runtime failure */
#define BGTQ_ERR_UNSUPPORTED 4 /* valid input this build does not handle */
#define BGTQ_ERR_NOMEM 5

#define BGTQ_DTYPE_F32 0
#define BGTQ_DTYPE_F16 1

/* Roles of src/webgpu/buffers.ts:1 (Allocation.role). */
#define BGTQ_ROLE_PERSISTENT_K 0
#define BGTQ_ROLE_PERSISTENT_V 1
#define BGTQ_ROLE_SHARED 2
#define BGTQ_ROLE_SCRATCH 3

typedef struct {
  char name[48];
  int32_t role;
  uint64_t bytes;
} bgtq_allocation;

/* Thread-local message of the last failing call on this thread. */
const char *bgtq_last_error(void);
/* 2: bgtq_tables_info gained device_bytes. 3: bgtq_model_submit, bgtq_buffer_*, bgtq_allocate_bits,
 * bgtq_layout_groups, bgtq_layout_build. 4: bgtq_decode_noalloc; q_rotated closes the decode and
 * prefill descriptors; bgtq_bake_qproj; bgtq_timestamps_*; the prefill workspace is always needed
 * (at least BGTQ_PREFILL_COUNTER_BYTES, 16-byte aligned, its counter prefix zeroed before the first
 * call). 5: bgtq_attention_record_timed; attention over FP32 V runs on the fused kernel. 6:
 * bgtq_prefill_append; the decode workspace holds one more partial per query head and the prefill
 * workspace the appended rows' partials (allocate what the *_workspace_size calls return). */
int32_t bgtq_abi_version(void);

/* ---- context: replaces GPUDevice + GPUQueue ------------------------------ */
typedef struct bgtq_context bgtq_context;
bgtq_status bgtq_context_create(int32_t device, bgtq_context **out);
void bgtq_context_destroy(bgtq_context *ctx);
/* Queue-ordered completion, replaces device.queue.onSubmittedWorkDone(). */
bgtq_status bgtq_context_synchronize(bgtq_context *ctx);
/* The hipStream_t all work of this context is ordered on. A caller may set a
 * stream it owns (for example PyTorch's current stream); NULL restores the
 * context's own stream. Calls reuse context-owned device state (the encode
 * job table, the staging area), so setting a different stream makes it wait
 * for the work queued on the previous one (an event; not while either stream
 * is capturing a graph, where the caller orders the two). */
void *bgtq_context_stream(bgtq_context *ctx);
bgtq_status bgtq_context_set_stream(bgtq_context *ctx, void *hip_stream);

/* ---- GPU timestamps: replace a GPUQuerySet of type "timestamp" ----------- *
 * device.createQuerySet({type:"timestamp",count}), the timestampWrites of a
 * compute pass (src/attention/attention.ts:44-58, benchmarks/timing.ts:13-16)
 * and encoder.resolveQuerySet (benchmarks/timing.ts:20). write() records
 * index on the context's stream: the time all work queued before it on the
 * stream completed. resolve() waits for the writes and gives nanoseconds on
 * one time base per call (differences are durations); indices never written
 * resolve to 0. */
typedef struct bgtq_timestamps bgtq_timestamps;
bgtq_status bgtq_timestamps_create(bgtq_context *ctx, uint32_t count, bgtq_timestamps **out);
bgtq_status bgtq_timestamps_write(bgtq_timestamps *t, uint32_t index);
bgtq_status bgtq_timestamps_resolve(bgtq_timestamps *t, uint32_t first, uint32_t count, uint64_t *ns);
void bgtq_timestamps_destroy(bgtq_timestamps *t);

/* ---- calibration tables: replaces tables(p)/validateLayout --------------- *
 * src/webgpu/layout.ts:8-31. integer = [dim, groups, rowBytes, normStride,
 * nibbleDims, maxCentroids, o_perm, o_groupOf, o_posToCb, o_lut] ++ perm ++
 * groupOf ++ positionToCodebook ++ codeLut (one u32 per LUT byte); floating =
 * rotation[d*d] (y_j = sum_i x_i R[j*d+i]) ++ centroids[d*maxC] ++
 * offsets[d] ++ inverseScales[d]. The per-head model calibration blob
 * (src/model/calibration.ts:15-20) has the same format. Validation also
 * applies the PackedKeys constructor checks (src/runtime/packed-keys.ts:16-23):
 * contiguous groups, zero off-group rotation. */
typedef struct bgtq_tables bgtq_tables;
typedef struct {
  int32_t dim, groups, row_bytes, norm_stride, nibble_dims, max_centroids;
  int32_t n_codebooks, n_books; /* LUT rows; distinct centroid rows */
  uint64_t device_bytes;        /* device memory the tables hold */
} bgtq_tables_info;
bgtq_status bgtq_tables_create(bgtq_context *ctx, const uint32_t *integer, size_t n_integer,
                               const float *floating, size_t n_floating, bgtq_tables **out);
bgtq_status bgtq_tables_info_get(const bgtq_tables *t, bgtq_tables_info *out);
void bgtq_tables_destroy(bgtq_tables *t);

/* ---- key stores: replace KeyStore implementations ------------------------ *
 * FP16Keys (src/runtime/keys.ts:16-27), PackedKeys (src/runtime/packed-keys.ts:7-52),
 * CompressedKeys (src/runtime/compressed-keys.ts:5-59; packed storage plus a
 * materialised FP32 K for phase-3 attention). append() takes FP16 bit patterns
 * of whole rows and validates like appendCount (src/runtime/keys.ts:11-15). */
typedef struct bgtq_keys bgtq_keys;
#define BGTQ_KEYS_FP16 0
#define BGTQ_KEYS_PACKED 1
#define BGTQ_KEYS_COMPRESSED 2
bgtq_status bgtq_fp16_keys_create(bgtq_context *ctx, uint32_t dim, uint32_t capacity, bgtq_keys **out);
bgtq_status bgtq_packed_keys_create(bgtq_tables *t, uint32_t capacity, bgtq_keys **out);
bgtq_status bgtq_compressed_keys_create(bgtq_tables *t, uint32_t capacity, bgtq_keys **out);
bgtq_status bgtq_keys_append(bgtq_keys *k, const uint16_t *fp16_bits, size_t n_values);
/* PackedKeys.ready(): Error "K storage not ready" while empty. */
bgtq_status bgtq_keys_ready(const bgtq_keys *k);
int32_t bgtq_keys_kind(const bgtq_keys *k);
uint32_t bgtq_keys_length(const bgtq_keys *k);
uint32_t bgtq_keys_capacity(const bgtq_keys *k);
uint32_t bgtq_keys_dim(const bgtq_keys *k);
/* readBuffer(packed) / readBuffer(norms): capacity*rowBytes bytes and
 * capacity*normStride FP16 bit patterns, row major (packed/compressed kinds). */
bgtq_status bgtq_keys_read_packed(const bgtq_keys *k, uint8_t *packed, size_t packed_bytes,
                                  uint16_t *norms, size_t norm_count);
/* FP16 kind: the raw FP16 K rows [capacity*dim]. */
bgtq_status bgtq_keys_read_fp16(const bgtq_keys *k, uint16_t *out, size_t count);
/* CompressedKeys.prepare(): materialise FP32 K [length*dim] (head order) on
 * the device; with out != NULL also copy it to the host. */
bgtq_status bgtq_keys_prepare(bgtq_keys *k, float *out, size_t count);
bgtq_status bgtq_keys_allocations(const bgtq_keys *k, bgtq_allocation *out, size_t cap, size_t *n);
void bgtq_keys_destroy(bgtq_keys *k);

/* ---- Values (src/runtime/values.ts:3-16) --------------------------------- *
 * dtype BGTQ_DTYPE_F32 stores FP32 V exactly (the synthetic path); F16 stores
 * RNE-rounded FP16 V (src/model/append.wgsl:6-10). append() is synchronous.
 * Attention over F32 V runs on the fused kernel, which splits each value into
 * three FP16 parts that add back to it exactly, while every appended
 * |v| < 65504; a larger value sends the store to the general kernels. */
typedef struct bgtq_values bgtq_values;
bgtq_status bgtq_values_create(bgtq_context *ctx, uint32_t dim, uint32_t capacity, int32_t dtype,
                               bgtq_values **out);
bgtq_status bgtq_values_append(bgtq_values *v, const float *values, size_t n_values);
uint32_t bgtq_values_length(const bgtq_values *v);
bgtq_status bgtq_values_allocations(const bgtq_values *v, bgtq_allocation *out, size_t cap, size_t *n);
void bgtq_values_destroy(bgtq_values *v);

/* ---- attention sessions -------------------------------------------------- *
 * OptimizedAttention (src/attention/optimized.ts:5-45) over PACKED keys, and
 * AttentionSession (src/attention/attention.ts:19-70) over FP16 or
 * COMPRESSED keys. set_queries validates like setQueries; record enqueues the
 * work; attend = set_queries + record + wait. read() returns the inspect()
 * buffers: which = 0 logits [n*T], 1 probabilities [n*T], 2 output [n*dim].
 * Logits and probabilities are materialised only when the session was made
 * with materialize != 0 (the fused path otherwise never writes them). */
typedef struct bgtq_attention bgtq_attention;
bgtq_status bgtq_attention_create(bgtq_keys *k, bgtq_values *v, uint32_t max_queries,
                                  int32_t materialize, bgtq_attention **out);
bgtq_status bgtq_attention_set_queries(bgtq_attention *a, const float *q, size_t n_q_values,
                                       const uint32_t *positions, size_t n_positions, int32_t causal);
bgtq_status bgtq_attention_record(bgtq_attention *a);
/* record() with timestamps: index begin_index written on the stream after the
 * queries' upload, right before the attention passes, end_index right after
 * them (record(encoder, {querySet, beginningOfPassWriteIndex,
 * endOfPassWriteIndex}), src/attention/attention.ts:44-58). */
bgtq_status bgtq_attention_record_timed(bgtq_attention *a, bgtq_timestamps *ts, uint32_t begin_index,
                                        uint32_t end_index);
bgtq_status bgtq_attention_attend(bgtq_attention *a, const float *q, size_t n_q_values,
                                  const uint32_t *positions, size_t n_positions, int32_t causal);
bgtq_status bgtq_attention_read(const bgtq_attention *a, int32_t which, float *out, size_t count);
uint32_t bgtq_attention_queries(const bgtq_attention *a);
bgtq_status bgtq_attention_allocations(const bgtq_attention *a, bgtq_allocation *out, size_t cap, size_t *n);
void bgtq_attention_destroy(bgtq_attention *a);

/* ---- batched, caller-owned device memory --------------------------------- */

/* K encode of strided rows into packed rows (src/model/codec.wgsl:11-33 and
 * src/webgpu/mixed.wgsl:14-41, arithmetic of src/reference/production_math.py:4-24).
 * src holds FP16 bits (BGTQ_DTYPE_F16) or FP32 values that are first rounded
 * to FP16 (BGTQ_DTYPE_F32, src/model/codec.wgsl:14). Row r of a job reads
 * src + r*src_row_stride elements and writes packed row dst_row0 + r
 * (tables->row_bytes bytes, every byte written) and norms row dst_row0 + r. */
typedef struct {
  const bgtq_tables *tables;
  const void *src;
  int64_t src_row_stride; /* elements */
  int64_t rows;
  uint8_t *packed;
  uint16_t *norms;
  int64_t dst_row0;
} bgtq_encode_job;
bgtq_status bgtq_encode_batched(bgtq_context *ctx, int32_t src_dtype, const bgtq_encode_job *jobs,
                                size_t n_jobs);

/* Decode attention for one layer: B sequences x Hkv KV heads, G = Hq/Hkv
 * query heads per KV head (src/model/compressed-dot.wgsl:14-31 +
 * src/model/attention.wgsl:24-39 fused). Query head h uses KV head h / G.
 * key_format: BGTQ_KEYS_PACKED (packed rows + FP16 scales, tables[kv]) or
 * BGTQ_KEYS_FP16 (k_f16 rows). Layouts (element strides for norms/V/K):
 *   packed[b*packed_seq_stride + kv*packed_head_stride + t*row_bytes]
 *   norms [b*norms_seq_stride  + kv*norms_head_stride  + t*norm_stride]
 *   v/k   [b*seq_stride        + kv*head_stride        + t*dim]
 *   batch: 1..65535 sequences.
 *   q, out: [B, Hq, dim] FP32 contiguous; lengths: device uint32 [B] (tokens
 *   attended per sequence, 1..max_length). workspace: device memory of at
 *   least bgtq_decode_workspace_size() bytes, zero-filled by the caller
 *   before its first use (it holds per-(sequence, KV head) split counters
 *   that every call leaves at zero again); calls sharing a workspace must be
 *   ordered on one stream. The counters occupy a prefix of 64 bytes per
 *   (sequence, KV head) pair, at least BGTQ_DECODE_COUNTER_UNITS pairs long,
 *   which calls of up to that many pairs never write otherwise: such calls
 *   share a workspace whatever their geometries. A call with more pairs uses
 *   a longer prefix, which calls of other geometries may have written: zero
 *   it again before such a call when geometries mix. */
#define BGTQ_DECODE_COUNTER_UNITS 1024
typedef struct {
  int32_t batch, q_heads, kv_heads, dim;
  int32_t key_format;
  const bgtq_tables *tables[16];
  const uint8_t *packed;
  int64_t packed_seq_stride, packed_head_stride; /* bytes */
  const uint16_t *norms;
  int64_t norms_seq_stride, norms_head_stride;   /* elements */
  const uint16_t *k_f16;
  int64_t k_seq_stride, k_head_stride;           /* elements */
  const void *v;
  int32_t v_dtype;
  int64_t v_seq_stride, v_head_stride;           /* elements */
  const float *q;
  float *out;
  const uint32_t *lengths;
  uint32_t max_length;
  int32_t splits; /* token splits per (sequence, KV head); 0 = choose */
  void *workspace;
  size_t workspace_bytes;
  /* 0: q as the model produces it. 1 (packed K only): q is already in the
   * code domain of its KV head's tables, qr[j] = sum_i R[j][i] q[perm[i]]
   * (the query of vendor/blockgtq/quantizer.py:1160-1188,
   * rotate_q_for_packed_kernel, e.g. from a projection baked with
   * bgtq_bake_qproj), and the kernels skip their own rotation. */
  int32_t q_rotated;
} bgtq_decode_desc;
bgtq_status bgtq_decode_workspace_size(const bgtq_decode_desc *d, size_t *bytes);
bgtq_status bgtq_decode(bgtq_context *ctx, const bgtq_decode_desc *d);

/* One decode step of a layer with its new token, in one launch: the model
 * step's encode_k (packed K) or append (FP16 K), the V append and the
 * attention of src/model/decoder.ts:46-56 at rows = 1 (src/model/codec.wgsl,
 * src/model/append.wgsl, then src/model/compressed-dot.wgsl:14-31 and
 * src/model/attention.wgsl:24-39). The new token of sequence b is row
 * lengths[b] - 1 of the caches: its post-RoPE K (k_new[b][kv][dim], FP32 is
 * rounded to FP16 first) is encoded with tables[kv] into packed/norms (or
 * converted into k_f16), its V (v_new) converted into the FP16 V rows, and
 * the attention covers lengths[b] tokens including it. Same results as
 * bgtq_encode_batched of those rows, the V rows written, then bgtq_decode.
 * Needs the fused kernel: FP16 V, d 64 or 128, 16-byte aligned caches and
 * strides, and a packed layout within its limits (at most four groups in any
 * 32 head-perm positions, 8 books whose code tables fit its LDS, norm_stride
 * up to 8; the reference's layouts and SmolLM2 calibration heads qualify);
 * others return BGTQ_ERR_UNSUPPORTED and write nothing (use the two calls).
 * k_new and v_new are 4-byte aligned, FP16 ones with even strides
 * (BGTQ_ERR_RANGE otherwise). The workspace is the decode's. */
typedef struct {
  const void *k_new;
  int32_t k_new_dtype; /* BGTQ_DTYPE_F32 or BGTQ_DTYPE_F16 */
  int64_t k_new_seq_stride, k_new_head_stride; /* elements */
  const void *v_new;
  int32_t v_new_dtype;
  int64_t v_new_seq_stride, v_new_head_stride;
} bgtq_append_desc;
bgtq_status bgtq_decode_append(bgtq_context *ctx, const bgtq_decode_desc *d, const bgtq_append_desc *a);

/* bgtq_decode without a caller workspace and without any allocation. No
 * counterpart in the reference: it is for callers that cannot allocate
 * device memory (code under HIP graph capture, serving loops or harnesses
 * that forbid hipMalloc). d->workspace and d->workspace_bytes are ignored;
 * the decode's workspace is a library-owned device array of
 * BGTQ_DECODE_SCRATCH_BYTES per device, held until the process ends and
 * resolved and cleared by bgtq_context_create (once per device). A launch
 * whose bgtq_decode_workspace_size exceeds it, or with more than
 * BGTQ_DECODE_COUNTER_UNITS (sequence, KV head) pairs, fails with
 * BGTQ_ERR_RANGE and queues nothing. Same kernels and results as
 * bgtq_decode. Every call on one
 * device shares that device's array: calls that may overlap on one device
 * (several streams or contexts) race and must be ordered by the caller. */
#define BGTQ_DECODE_SCRATCH_BYTES (4u << 20)
bgtq_status bgtq_decode_noalloc(bgtq_context *ctx, const bgtq_decode_desc *d);

/* Chunked-prefill attention for one layer: the model forward over a chunk of
 * prompt rows (src/model/decoder.ts:46-56 with rows > 1, called per chunk by
 * src/model/decoder.ts:82; the reference caps chunks at 32 rows,
 * src/model/decoder.ts:15, this entry point takes any number). Sequence b's
 * chunk holds `rows` query rows at positions starts[b] .. starts[b]+rows-1;
 * row r's queries attend to tokens 0 .. starts[b]+r
 * (src/model/compressed-dot.wgsl:28, src/model/attention.wgsl:19). The K/V
 * buffers already hold the chunk's own tokens (encode them first).
 *   q, out: [B, rows, Hq, dim] FP32 contiguous; query head h uses KV head h / G.
 *   starts: device uint32 [B], starts[b] + rows <= max_length (kernels clamp).
 *   v: FP16. Key formats and strides are those of bgtq_decode.
 *   workspace: 16-byte aligned device memory of at least
 *   bgtq_prefill_workspace_size() bytes for the partial results of query
 *   rows or tiles whose history several workgroups share. Its first
 *   BGTQ_PREFILL_COUNTER_BYTES bytes (split arrival counters) must be zero
 *   before the first call on it, and every call leaves them zero, whatever
 *   its geometry; the rest needs no initial contents. Calls sharing a
 *   workspace must be ordered on one stream.
 *   Chunks of at most BGTQ_PREFILL_ROWWISE_ROWS rows run every query row as
 *   a decode step over its causal history (the fused decode kernel and its
 *   split merge); longer chunks tile their queries.
 *   split_tokens: the history is divided into ranges of this many tokens, one
 *   workgroup each (tiled: every sequence, KV head and query tile's causal
 *   history, rounded up to 32; row-wise: each row's, as max_length /
 *   split_tokens splits); 0 = about two workgroups per compute unit (tiled:
 *   sized on the device for the actual starts).
 * q, V and the K scales must be finite: the tiled kernels are built without
 * NaN/Inf semantics, so a non-finite input inside a history gives an
 * unspecified output (packed K codes are always finite).
 * Layouts: FP16 K, or packed layouts the fused decode takes (see
 * bgtq_decode_append) whose centroid books (n_books * max_centroids floats)
 * fit 4 KB at d=64, 8 KB at d=128; others return BGTQ_ERR_UNSUPPORTED. */
#define BGTQ_PREFILL_COUNTER_BYTES (4u * 65536u)
#define BGTQ_PREFILL_ROWWISE_ROWS 32
typedef struct {
  int32_t batch, rows, q_heads, kv_heads, dim;
  int32_t key_format;
  const bgtq_tables *tables[16];
  const uint8_t *packed;
  int64_t packed_seq_stride, packed_head_stride; /* bytes */
  const uint16_t *norms;
  int64_t norms_seq_stride, norms_head_stride;   /* elements */
  const uint16_t *k_f16;
  int64_t k_seq_stride, k_head_stride;           /* elements */
  const uint16_t *v;
  int64_t v_seq_stride, v_head_stride;           /* elements */
  const float *q;
  float *out;
  const uint32_t *starts;
  uint32_t max_length;
  int32_t split_tokens; /* history tokens per workgroup range, rounded up to 32; 0 = choose */
  void *workspace;
  size_t workspace_bytes;
  int32_t q_rotated; /* as in bgtq_decode_desc */
} bgtq_prefill_desc;
bgtq_status bgtq_prefill_workspace_size(const bgtq_prefill_desc *d, size_t *bytes);
bgtq_status bgtq_prefill(bgtq_context *ctx, const bgtq_prefill_desc *d);

/* One chunk of a layer's prefill with the chunk's own rows, in one launch:
 * the model step's encode_k, V append and attention passes of
 * src/model/decoder.ts:46-56 for rows > 1 (called per chunk by
 * src/model/decoder.ts:82, chunks of up to 32 rows: src/model/decoder.ts:15).
 * Row r of sequence b (post-RoPE K at k_new + b k_new_seq_stride + r
 * k_new_row_stride + kv k_new_head_stride, FP32 rounded to FP16 first; V
 * likewise) is encoded with tables[kv] into packed/norms and its V converted
 * into the FP16 V rows at cache row min(starts[b], max_length - rows) + r,
 * and the chunk's queries attend causally to the history and to the chunk's
 * rows. Same caches as bgtq_encode_batched of those rows plus the V rows
 * written, same outputs (within the attention tolerance) as bgtq_prefill
 * after them. Packed K, rows up to BGTQ_PREFILL_ROWWISE_ROWS, the layouts
 * bgtq_decode_append takes (others: BGTQ_ERR_UNSUPPORTED, nothing written);
 * the workspace is bgtq_prefill_workspace_size()'s. New rows 4-byte aligned,
 * FP16 ones with even strides. */
typedef struct {
  const void *k_new;
  int32_t k_new_dtype; /* BGTQ_DTYPE_F32 or BGTQ_DTYPE_F16 */
  int64_t k_new_seq_stride, k_new_row_stride, k_new_head_stride; /* elements */
  const void *v_new;
  int32_t v_new_dtype;
  int64_t v_new_seq_stride, v_new_row_stride, v_new_head_stride;
} bgtq_prefill_append_desc;
bgtq_status bgtq_prefill_append(bgtq_context *ctx, const bgtq_prefill_desc *d, const bgtq_prefill_append_desc *a);

/* ---- calibration-table pipeline (host only, no device needed) ------------
 * The setup that produces the tables(p) blobs bgtq_tables_create takes:
 * bgtq_allocate_bits is the greedy per-pair allocation
 * (src/reference/allocator.py:4-17: one more bit to the first argmax of
 * s * 4^-w, FP32 scores, FP64 powers, until the budget is spent or every
 * pair is at max_bits or no priority is positive). bgtq_layout_groups gives
 * the groups of a width allocation (src/reference/mixed_layout.py:5-18:
 * pairs stably sorted by width, one group per distinct width, ascending):
 * their widths and dimensions, so that the caller can supply each group's
 * codebook and rotation. bgtq_layout_build then forms the full table set:
 * head_perm, group_of, the per-position code LUTs (one per distinct
 * codebook), bin offsets and inverse widths
 * (vendor/blockgtq/quant_kernels.py:276-364), the block-diagonal rotation and
 * the centroid table, serialised as src/webgpu/layout.ts:24-31. groups[k]
 * holds group k's 2^bits ascending centroids and its m x m rotation
 * (row-major, y_j = sum_i x_i R[j*m+i]; NULL = identity, which the reference
 * uses below 2 bits). row_bytes / norm_stride 0 take the natural values.
 * Called with integer or floating NULL it only returns the element counts. */
bgtq_status bgtq_allocate_bits(const float *scores, size_t n_pairs, int64_t budget, int32_t min_bits,
                               int32_t max_bits, int64_t *widths);
bgtq_status bgtq_layout_groups(const int64_t *widths, size_t n_pairs, int32_t *n_groups, int32_t *bits /*[8]*/,
                               int32_t *group_dims /*[8]*/);
typedef struct {
  const float *centroids;
  const float *rotation;
} bgtq_group_tables;
bgtq_status bgtq_layout_build(const int64_t *widths, size_t n_pairs, const bgtq_group_tables *groups, size_t n_groups,
                              int32_t row_bytes, int32_t norm_stride, uint32_t *integer, size_t *n_integer,
                              float *floating, size_t *n_floating);

/* Bakes a KV head's head permutation and rotation into the query projection
 * of its query heads, so the queries it produces are already in the code
 * domain and the attention kernels skip their rotation (the optimisation of
 * vendor/blockgtq/quantizer.py:1190-1244, bake_permutation_into_qproj; the
 * packing permutation is the identity in the reference,
 * tests/oracles/calibrate_model.py:34). integer/floating: the KV head's
 * tables(p) blobs (src/webgpu/layout.ts:24-31), checked as bgtq_tables_create
 * checks them. weight: the projection rows of `heads` query heads,
 * [heads * dim][in_features] row-major FP32; bias: [heads * dim] or NULL.
 * Per head h: out[h*dim + j][c] = sum_i R[j][i] w[h*dim + perm[i]][c], and
 * the same for the bias, accumulated in FP64 and rounded once. Queries from
 * the baked projection go to bgtq_decode / bgtq_prefill with q_rotated = 1.
 * Host only; no device is used. */
bgtq_status bgtq_bake_qproj(const uint32_t *integer, size_t n_integer, const float *floating, size_t n_floating,
                            int32_t heads, int64_t in_features, const float *weight, const float *bias,
                            float *weight_out, float *bias_out);

/* ---- device buffers: storage / upload / readBuffer (src/webgpu/buffers.ts:3-25)
 * For callers without their own device allocator (the Node mirror). A buffer
 * holds `bytes` rounded up to a multiple of 4, zero-filled (WebGPU buffers
 * start zeroed). Writes are ordered on the context stream and complete
 * before returning; reads wait for the stream. */
typedef struct bgtq_buffer bgtq_buffer;
bgtq_status bgtq_buffer_create(bgtq_context *ctx, size_t bytes, bgtq_buffer **out);
void *bgtq_buffer_device_ptr(const bgtq_buffer *b);
size_t bgtq_buffer_size(const bgtq_buffer *b);
bgtq_status bgtq_buffer_write(bgtq_buffer *b, size_t offset, const void *src, size_t bytes);
bgtq_status bgtq_buffer_read(const bgtq_buffer *b, size_t offset, void *dst, size_t bytes);
void bgtq_buffer_destroy(bgtq_buffer *b);

/* ---- the model step's kernel protocol --------------------------------------
 * Commands.dispatch(name, parameters, buffers, x, y) then submit()
 * (src/model/ops.ts:24-30) for the attention-path names of ModelOps
 * (src/model/ops.ts:6-12), as src/model/decoder.ts:46-56 dispatches them.
 * One bgtq_model_dispatch per dispatch, with the reference's parameters
 * (unused slots zero) and bindings in its binding order, the uniform slot
 * left out. A binding is device memory (ptr, bytes); the config and table
 * slots of encode_k and compressed_dot instead name the head's calibration
 * tables (tables; both slots may carry the same handle). Layouts are the
 * reference's: q and post-RoPE K/V rows [rows][heads][head_dim] FP32, caches
 * [kv_heads][capacity][head_dim] FP16, packed K and scales per head
 * [token][row_bytes] / [token][norm_stride], scores and probabilities
 * [rows*q_heads][tokens], attention output [rows*q_heads][head_dim] FP32.
 *   append         [rows,start,capacity,heads]   bindings input, cache
 *                  (src/model/append.wgsl:6-10; 64 dims, FP32 -> FP16 RNE)
 *   encode_k       [rows,start,head,kv_heads]    config, table, kr, codes, norms
 *                  (src/model/codec.wgsl:11-33; = bgtq_encode_batched of the
 *                  FP32 rows, which writes every byte of each row where the
 *                  reference ORs codes into zeroed rows)
 *   compressed_dot [rows,start,head,tokens,q_heads,gqa,head_dim]
 *                  config, table, q, codes, norms, ranges (unused), scores
 *                  (src/model/compressed-dot.wgsl:14-31)
 *   dot, softmax, weighted [rows,tokens,capacity,start,q_heads,kv_heads,gqa,head_dim]
 *                  q, k, v, scores, probabilities, attention
 *                  (src/model/attention.wgsl:13-39)
 * x and y are the dispatch's workgroup counts: each pass covers the work
 * items those workgroups cover in the reference, clamped to the parameters'
 * extents. head_dim is 64 or 128 (the reference's kernels fix 64), gqa at
 * most 16, q_heads = kv_heads * gqa. Every dispatch is checked, bindings
 * against the extents its pass reads and writes, before any work is queued;
 * a failed check returns BGTQ_ERR_RANGE (BGTQ_ERR_UNSUPPORTED for the
 * model's other kernels: embedding, matmul, norm, element, rope) and queues
 * nothing. The work is queued on the context stream in order (consecutive
 * encode_k dispatches share one launch); bgtq_context_synchronize waits for
 * it, as the reference's submit() awaits the queue. */
typedef struct {
  void *ptr;
  size_t bytes;
  const bgtq_tables *tables;
} bgtq_binding;
typedef struct {
  const char *name;
  uint32_t params[8];
  const bgtq_binding *bindings;
  size_t n_bindings;
  uint32_t x, y;
} bgtq_model_dispatch;
bgtq_status bgtq_model_submit(bgtq_context *ctx, const bgtq_model_dispatch *dispatches, size_t n);

#ifdef __cplusplus
}
#endif
#endif
