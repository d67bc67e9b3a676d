// Internal structures shared by the host library and the gfx950 kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "bgtq.h"

namespace bgtq {

constexpr int kMaxDim = 128;
constexpr int kMaxGroups = 8;
constexpr int kMaxKvHeads = 16;
constexpr int kEncodeJobsPerLaunch = 60;  // 64-byte jobs: the launch stays under 4 KB of kernel arguments
constexpr int kEncodeJobTable = 4096;     // jobs in a context's device job table (thread-per-row encoders)

// Device-resident calibration tables, built once on the host from the
// reference's serialized tables (src/webgpu/layout.ts:24-31). Fixed header,
// then variable sections at byte offsets from the start of the struct.
struct DevTables {
  int32_t dim, groups, row_bytes, norm_stride, nibble_dims, max_centroids, n_books, n_codebooks;
  int32_t gstart[kMaxGroups], gend[kMaxGroups], gsize[kMaxGroups];  // group ranges (head-perm order)
  uint32_t off_lut, off_books, off_rot, off_rot_t, off_mfma, off_rot_q, off_gdesc, off_glane, total_bytes;
  int32_t cent_exp;  // 2^cent_exp * max|centroid| <= 2^14: fp16 hi/lo split range for MFMA operands
  // The fused decode of any packed layout: its leading pair K-steps (see
  // off_glane) and the books whose pair tables it keeps in LDS for them
  // (byte i = book of pair slot i, 0xff = unused).
  int32_t pair_lead;
  uint32_t pair_books;
  uint8_t perm[kMaxDim];      // head_perm
  uint8_t group_of[kMaxDim];
  uint8_t pos_cb[kMaxDim];    // position -> code LUT row
  uint8_t pos_book[kMaxDim];  // position -> distinct centroid row
  float lut_off[kMaxDim];
  float lut_inv[kMaxDim];
  // [off_lut]   uint8 code_lut[n_codebooks*256]
  // [off_books] float books[n_books*max_centroids]
  // [off_rot]   float rotation[dim*dim], y_j = sum_i x_i R[j*dim+i]
  // [off_rot_t] float rotation transposed, Rt[i*dim+j] = R[j*dim+i]
  // [off_mfma]  per book, kMfmaTableBytes: the fp16 (hi, lo) split of
  //             centroid * 2^cent_exp as MFMA lookup tables,
  //             uint32 pair[256][2]: hi pair, lo pair (entry = packed
  //                    nibble byte, low nibble in the low half of each pair)
  //             uint32 code[256]: hi | lo << 16 (entry = byte code)
  // [off_rot_q] the rotation with the head permutation folded in,
  //             Rq[j][c] = R[j][i] for c = perm[i] (qr = Rq q), as fp16
  //             (hi, lo) MFMA A operands: for 16-row tile n, 32-column step
  //             s and lane l, 8 hi then 8 lo halves of
  //             Rq[16 n + l % 16][32 s + 8 (l / 16) + 0..7] (kRotQBytes).
  // [off_gdesc] per head-perm position j, for the fused decode of any packed
  //             layout: uint32 byte offset in the packed row | nibble shift << 8
  //             | nibble flag << 11 | book << 12 | group << 16.
  // [off_glane]  (d % 32 == 0) the fused decode's per-lane code-lookup
  //             records, [K-step s][lane group gq][kLaneRecordWords] uint32
  //             for positions j = 32 s + 8 gq + k: koff (row byte of code 0),
  //             hib (byte where the word of codes 4..7 starts), glo (group of
  //             position 32 s), nsl (groups in the K-step), ext[8] (bit offset
  //             of each code in its word), tbo[8] (LDS offset of its book's
  //             code table plus its field width), gmask[4][4] (per slot i, the
  //             fp16 halves of the 8 positions in group glo + i), then for a
  //             pair K-step phi[4] and plo[4]: the LDS offsets, among the pair
  //             slots (kPairSlots of 2 KB, 8-byte (hi pair, lo pair) entries),
  //             of the pair tables of positions 2 k2, 2 k2 + 1 (plo = phi + 1024,
  //             unused by the kernel, which reads both halves at phi). A pair K-step
  //             (all 32 positions nibble codes, each even position in the book
  //             of the next; only leading K-steps, pair_lead of them) reads
  //             two codes per packed byte.
};
constexpr int kMfmaTableBytes = 3072;
constexpr int kPairSlots = 4;         // pair tables (2 KB each) the fused decode keeps in LDS
constexpr int kLaneRecordWords = 44;
constexpr int kCounterStride = 16;   // words between the decode's split counters (one per 64-byte line)  // words of one per-lane code-lookup record
__host__ __device__ constexpr int rot_q_bytes(int dim) { return dim * dim * 4; }

__host__ __device__ inline const uint8_t *tables_lut(const DevTables *t) {
  return reinterpret_cast<const uint8_t *>(t) + t->off_lut;
}
__host__ __device__ inline const float *tables_books(const DevTables *t) {
  return reinterpret_cast<const float *>(reinterpret_cast<const uint8_t *>(t) + t->off_books);
}
__host__ __device__ inline const float *tables_rot(const DevTables *t) {
  return reinterpret_cast<const float *>(reinterpret_cast<const uint8_t *>(t) + t->off_rot);
}
__host__ __device__ inline const float *tables_rot_t(const DevTables *t) {
  return reinterpret_cast<const float *>(reinterpret_cast<const uint8_t *>(t) + t->off_rot_t);
}
__host__ __device__ inline const uint8_t *tables_mfma(const DevTables *t) {
  return reinterpret_cast<const uint8_t *>(t) + t->off_mfma;
}
__host__ __device__ inline const uint8_t *tables_rot_q(const DevTables *t) {
  return reinterpret_cast<const uint8_t *>(t) + t->off_rot_q;
}

struct EncodeJobDev {
  const DevTables *t;
  const void *src;
  uint8_t *packed;
  uint16_t *norms;
  int64_t rows;
  int64_t dst_row0;
  int32_t src_stride;  // elements
  int32_t dst_step;    // destination row step per source row (>= 1)
  int32_t enc_bytes;   // bytes of the table set's header, code LUT and books (off_rot)
  int32_t off_rot_t;   // byte offset of the transposed rotation
};
static_assert(sizeof(EncodeJobDev) == 64, "encode job layout");

struct EncodeLaunch {
  EncodeJobDev jobs[kEncodeJobsPerLaunch];
  int32_t n_jobs;
};

// Pointers into global memory typed as such. The compiler knows the address
// space of pointers it loads from kernel arguments, not of pointers it loads
// from device memory (the encoders' job table): typed generic, wave-uniform
// table reads become per-lane flat loads instead of scalar loads. (The host
// pass of a HIP source parses kernels too; there the qualifier is empty.)
#if defined(__HIP_DEVICE_COMPILE__)
#define BGTQ_GLOBAL __attribute__((address_space(1)))
#else
#define BGTQ_GLOBAL
#endif
template <typename X>
__host__ __device__ __forceinline__ BGTQ_GLOBAL X *to_global(X *p) {
  return (BGTQ_GLOBAL X *)p;
}
#if defined(__HIP_DEVICE_COMPILE__)
__device__ inline const BGTQ_GLOBAL uint8_t *tables_lut(const BGTQ_GLOBAL DevTables *t) {
  return reinterpret_cast<const BGTQ_GLOBAL uint8_t *>(t) + t->off_lut;
}
__device__ inline const BGTQ_GLOBAL float *tables_books(const BGTQ_GLOBAL DevTables *t) {
  return reinterpret_cast<const BGTQ_GLOBAL float *>(reinterpret_cast<const BGTQ_GLOBAL uint8_t *>(t) + t->off_books);
}
__device__ inline const BGTQ_GLOBAL float *tables_rot(const BGTQ_GLOBAL DevTables *t) {
  return reinterpret_cast<const BGTQ_GLOBAL float *>(reinterpret_cast<const BGTQ_GLOBAL uint8_t *>(t) + t->off_rot);
}
__device__ inline const BGTQ_GLOBAL float *tables_rot_t(const BGTQ_GLOBAL DevTables *t) {
  return reinterpret_cast<const BGTQ_GLOBAL float *>(reinterpret_cast<const BGTQ_GLOBAL uint8_t *>(t) + t->off_rot_t);
}
#endif

// Decode attention of one layer. Units are (sequence, KV head); each unit
// serves G query heads (GQA). Work per unit is split over token ranges.
struct DecodeParams {
  const DevTables *tables[kMaxKvHeads];
  int32_t batch, q_heads, kv_heads, dim, G;
  int32_t key_format;  // 0 = FP16 K rows, 1 = packed, 2 = FP32 K rows
  const uint8_t *packed;
  int64_t packed_seq_stride, packed_head_stride;  // bytes
  const uint16_t *norms;
  int64_t norms_seq_stride, norms_head_stride;  // elements
  const void *k;
  int64_t k_seq_stride, k_head_stride;  // elements
  const void *v;
  int32_t v_dtype;  // 0 = FP32, 1 = FP16
  int32_t waves;          // decode workgroup waves of the fused kernel: 8 (d=64, few units), else 4
  int32_t splits_forced;  // the caller fixed the split count
  int32_t v_f32_split;  // FP32 V with every |v| < 65504: the fused kernel may split it into FP16 parts
  int64_t v_seq_stride, v_head_stride;  // elements
  const float *q;         // [B*Hq*dim] queries
  int32_t q_rotated;      // 1: q is already R q[perm] (code domain); the kernels do not rotate it
  const float *qr;        // [B*Hq*dim] rotated, permuted, scaled by 1/sqrt(dim)
  const uint32_t *lengths;  // [B]; kernels clamp them to max_length
  // Chunked prefill through the fused decode kernel (small chunks): row r of
  // sequence b attends to the first min(starts[b], max_length - rows) + r + 1
  // tokens; q and out are indexed by query row b * rows + r instead of b. A
  // unit is unit_cols (8 or 16) query columns of one (sequence, KV head): the
  // chunk's rows x G heads flattened row-major, qgroups = ceil(rows * G /
  // unit_cols) units per (sequence, KV head), partials at row unit *
  // unit_cols + column. A unit runs min(splits, ceil(history / split_floor))
  // of its splits. Plain decode: rows = 1, starts = null.
  int32_t rows;
  const uint32_t *starts;
  int32_t qgroups, split_floor, unit_cols;
  int32_t max_length;       // tokens every K/V buffer holds per (sequence, KV head)
  const int32_t *ends;      // optional [B*Hq] exclusive causal ends
  int32_t splits, split_tokens;
  float inv_sqrt_d;
  uint32_t *counters;  // split arrival counters, one per unit: zero between launches
  // Words from one unit's counter to the next (0 counts as 1): counters on
  // lines of their own keep the arrivals of different units from queueing
  // behind each other at the memory's atomic unit.
  int32_t counter_stride;
  float *part;    // [B*Hq*splits*(dim+2)] (m, l, o[dim])
  float *stats;   // [B*Hq*2] final (m, l)
  float *out;     // [B*Hq*dim]
  float *logits;  // optional [B*Hq*logit_stride]
  float *probs;   // optional [B*Hq*logit_stride]
  int64_t logit_stride;
  int32_t lds_bytes;  // dynamic LDS of the split kernel
  // Decode-step append (fused kernel only), null otherwise: the newest token
  // of sequence b sits at row lengths[b] - 1 of the caches; its post-RoPE K
  // [b][kv][dim] is encoded into packed/norms (or converted into the FP16 K
  // rows) and its V converted into the FP16 V rows within the launch.
  // Row-wise prefill with the chunk's rows appended (packed K): row r of
  // sequence b at k_new + b seq_stride + r row_stride + kv head_stride goes to
  // cache row min(starts[b], max_length - rows) + r.
  const void *k_new, *v_new;
  int32_t k_new_f32, v_new_f32;
  int64_t k_new_seq_stride, k_new_head_stride, v_new_seq_stride, v_new_head_stride;  // elements
  int64_t k_new_row_stride, v_new_row_stride;                                        // elements
  // Workgroups per (sequence, KV head) or row-wise unit that take the
  // appended rows (packed K: decode 1; row-wise prefill one row per wave),
  // after the splits in the split dimension; each leaves one partial.
  int32_t app_parts;
};

// Chunked-prefill attention of one layer (prefill.hip). Units are (sequence,
// KV head); a unit's queries are its chunk's rows x G heads (qi = row*G + h),
// tiled by tile_queries and split over token ranges.
struct PrefillParams {
  const DevTables *tables[kMaxKvHeads];
  int32_t batch, rows, q_heads, kv_heads, dim, G;
  int32_t key_format;  // 0 = FP16 K rows, 1 = packed
  const uint8_t *packed;
  int64_t packed_seq_stride, packed_head_stride;  // bytes
  const uint16_t *norms;
  int64_t norms_seq_stride, norms_head_stride;  // elements
  const void *k;
  int64_t k_seq_stride, k_head_stride;  // elements
  const void *v;                        // FP16
  int64_t v_seq_stride, v_head_stride;  // elements
  const float *q;           // [B*rows*Hq*dim] queries
  int32_t q_rotated;        // 1: q is already R q[perm] (code domain); the kernel does not rotate it
  float inv_sqrt_d;
  const uint32_t *starts;   // [B] position of each chunk's first row
  int32_t max_length;       // tokens every K/V buffer holds; kernels clamp starts to max_length - rows
  int32_t tiles;            // query tiles per (sequence, KV head)
  int32_t tile_queries;     // 64 or 64 * prefill_column_blocks(dim)
  int32_t ranges;           // workgroups: each takes an equal range of the flattened work
  int32_t range_blocks;     // cost units per range; 0 = ceil(work / ranges), at least kPrefillMinRange
  int32_t first_round;      // > 0: the first first_round ranges are 1.5 times the others
  float *part;              // two records per workgroup: (m, l, o[dim]) per query of a tile
  int32_t *tile_info;       // per (KV head, sequence, tile): first and last workgroup, first one's record
  float *out;               // [B*rows*Hq*dim]
};
// Most 16-query MFMA column blocks per wave of the prefill kernel (four waves per tile).
__host__ __device__ constexpr int prefill_column_blocks(int dim) { return dim == 64 ? 4 : 2; }
constexpr int kPrefillMinRange = 2;       // cost units per workgroup range the kernel picks at least
constexpr int kPrefillSegmentCost = 4;    // cost units of a tile's set-up (a 32-token block is one)
constexpr int kPrefillMaxRanges = 2048;   // workgroups of one launch at most (bounds the records)
// Chunks of at most this many rows run row-wise through the fused decode
// kernel (a unit per query row and KV head, its split merge); longer chunks
// tile their queries in the prefill kernel.
constexpr int kPrefillRowwiseRows = BGTQ_PREFILL_ROWWISE_ROWS;
// Row-wise prefill: waves per workgroup (d=64: 8, so a split covers twice
// the tokens and a unit merges half the partials; d=128 keeps 4, whose ring
// would not fit twice), tokens per split at least (two 32-token chunks per
// wave), splits per unit at most.
constexpr int decode_fast_prefill_waves(int dim) { return dim == 64 ? 8 : 4; }
constexpr int prefill_split_floor(int dim) { return 64 * decode_fast_prefill_waves(dim); }
constexpr int kPrefillMaxSplits = 16;
// Rows each wave of a row-wise prefill append workgroup encodes (side by
// side). One: two or four rows per wave took as long per row as one (their
// encode chains did not overlap), so fewer, longer append workgroups ended
// later (4096-token prompt in 32-row chunks, one launch per chunk and layer:
// 42.7 ms with one row per wave, 48.3 ms with two, 57.4 ms with four).
constexpr int kPrefillAppendRowsPerWave = 1;
// Row-wise prefill: query columns per unit (8 or 16).
constexpr int kPrefillUnitCols = 16;
// The prefill workspace starts with the row-wise path's split counters (a
// word per unit, up to 65535 units): zero before a workspace's first call,
// left zero by every call, never written by the tiled path.
constexpr size_t kPrefillCounterBytes = BGTQ_PREFILL_COUNTER_BYTES;

// The model step's separate attention passes (model_ops.hip), in the
// reference's buffer layouts: q [rows][q_heads][dim] FP32, K/V caches
// [kv_heads][capacity][dim] FP16, scores/probabilities [rows*q_heads][tokens].
struct ModelAppendParams {
  const float *input;  // [rows][heads][64]
  uint32_t *cache;     // FP16 pairs, [heads][capacity][32]
  int64_t pairs;       // pairs converted (rows*heads*32 or fewer)
  int32_t start, capacity, heads;
};
struct ModelScoresParams {
  const DevTables *tables;  // packed K (one KV head per dispatch), else null
  const float *q;
  const uint8_t *packed;    // [tokens][row_bytes] of the dispatch's head
  const uint16_t *norms;    // [tokens][norm_stride]
  const uint16_t *k;        // FP16 K cache
  float *scores;
  int32_t rows, start, q_heads, gqa, dim, capacity;
  int32_t tokens;  // score row length
  int32_t n_tok;   // tokens scored: min(tokens, the dispatch's x)
  int32_t head0;   // first KV head of the launch (grid z adds to it)
  int32_t y_limit; // the dispatch's y: workgroup rows of 128 query items
  float scale;     // 1/sqrt(dim)
};
struct ModelAttnParams {
  const float *scores;
  float *probs;
  const uint16_t *v;
  float *out;
  int32_t tokens, start, q_heads, gqa, dim, capacity;
  int64_t x_limit;  // outputs written (weighted): min(x, rows*q_heads*dim)
};

// Structure of a layout the fused matrix-core decode handles: every 32-dim
// K-step of the head-perm order lies in one group and one centroid book and is
// either all nibble codes or all byte codes (nibble steps first); at most two
// groups (norm_stride 2), group 0 first; rows 8-byte aligned.
struct FastLayout {
  int32_t book[4];  // centroid book of each K-step
  // Per KV head, resolved on the host so the kernel's first loads need no
  // dependent read of the tables' header: the MFMA lookup tables, the
  // permuted rotation's MFMA operands and cent_exp.
  const uint8_t *mfma[kMaxKvHeads];
  const uint8_t *rot_q[kMaxKvHeads];
  int32_t cent_exp[kMaxKvHeads];
  // The decode-step append's encoder: transposed rotation, and the bytes of
  // the table set's header, code LUT and books (contiguous from its start).
  const float *rot_t[kMaxKvHeads];
  int32_t enc_bytes[kMaxKvHeads];
  // Where that copy starts in the table set: 0 (header, LUT, books), or
  // off_lut (LUT and books only; the encoder reads the header in device
  // memory). enc_bytes 0: no copy, the encoder reads the tables in place.
  int32_t enc_from[kMaxKvHeads];
  // Packed layouts of any structure (the kernel's per-position code
  // lookup): position descriptors, row bytes, norm stride, book count, bytes
  // of each book's code table in LDS (whole 256-byte pieces), books of
  // nibble codes (bit mask), and whether every lane's row bytes start on a
  // word (row bytes a multiple of 4 and nibble positions a multiple of 8).
  const uint32_t *gdesc[kMaxKvHeads];
  const uint32_t *glane[kMaxKvHeads];
  int16_t grb[kMaxKvHeads], gns[kMaxKvHeads], gnb[kMaxKvHeads], gbstride[kMaxKvHeads];
  uint8_t gbnib[kMaxKvHeads], galign[kMaxKvHeads];
  uint32_t gpair[kMaxKvHeads];  // DevTables::pair_books
  int32_t gpair_lead;           // leading pair K-steps of every head of the launch
};

// Sets the calling thread's bgtq_last_error() message; returns code.
int32_t set_error(int32_t code, const char *msg);

// Launchers (kernels live in encode.hip / decode.hip / decode_fast_kernel.h / reconstruct.hip).
// The thread-per-row encoders read their jobs from a device job table
// (jobs[0 .. n_jobs), one grid row per job); launch_encode_upload writes up to
// kEncodeJobsPerLaunch jobs of a chunk (kernel arguments) to table[base ..]
// on the stream, so the table's contents are stream-ordered and a captured
// graph re-writes them on every replay.
hipError_t launch_encode_upload(const EncodeLaunch &chunk, EncodeJobDev *table, int base, hipStream_t stream);
hipError_t launch_encode(const EncodeJobDev *jobs, int n_jobs, int dim, int src_f32, int64_t max_rows,
                         hipStream_t stream);
// Wave-per-row encode (encode_wave.hip): dynamic LDS for a job whose table
// set's header, LUT and books take enc_bytes, and its launcher (wgs_per_job
// workgroups of four waves per job, each wave striding over the job's rows).
int encode_wave_lds_bytes(int dim, int enc_bytes);
hipError_t launch_encode_wave(const EncodeLaunch &launch, int dim, int src_f32, int wgs_per_job, int lds_bytes,
                              hipStream_t stream);
// Bulk thread-per-row encode (encode_bulk.hip) for layouts of two equal
// contiguous groups with nibble codes in the first (layout B at d 64 / 128):
// kind 1 (d=64) or 2 (d=128), 0 when the layout does not qualify. wg rows per
// workgroup: 256 (d=64) or 128 (d=128). The launch needs
// encode_bulk_lds_bytes of dynamic LDS for the largest LUT (bytes) and book
// set (floats) among its jobs.
int encode_bulk_kind(const DevTables *T);
int encode_bulk_lds_bytes(int kind, int wg, int lut_bytes, int book_floats);
hipError_t launch_encode_bulk(const EncodeJobDev *jobs, int n_jobs, int kind, int wg, int src_f32, int64_t max_rows,
                              int lut_bytes, int book_floats, hipStream_t stream);
hipError_t launch_rotate_q(const DecodeParams &p, const float *q, float *qr, hipStream_t stream);
// Device address of this device's bgtq_decode_noalloc scratch (decode_scratch.hip).
hipError_t decode_scratch_setup(int device, hipStream_t stream, uint8_t **out);
int decode_lds_bytes(int G, int dim, int key_format, int books_bytes, int row_bytes, int norm_stride);
hipError_t launch_decode(const DecodeParams &p, int lds_bytes, hipStream_t stream);
// LSE merge of split partials and the optional probabilities pass.
hipError_t launch_decode_tail(const DecodeParams &p, hipStream_t stream);
// Materialised probabilities exp(logit - m)/l from the final statistics.
hipError_t launch_decode_probs(const DecodeParams &p, hipStream_t stream);
// Fused decode (decode_fast_kernel.h): nn leading nibble K-steps, sg K-steps in group 0;
// nn = -1: a packed layout of any structure (per-position code lookup).
bool decode_fast_supported(int dim, int key_format, int nn, int sg);
// LDS bytes the per-position path holds for the books' code tables
// (n_books * (table bytes + 32) must fit) at head dim `dim`, its largest norm
// stride there (6 at d=64, 8 at d=128) and its groups per 32 positions.
int decode_general_table_bytes(int dim);
int decode_general_max_norm_stride(int dim);
constexpr int kDecodeGeneralMaxGroupsPerStep = 4;
// LDS bytes of centroid books (n_books * max_centroids floats) the prefill
// kernel's per-position build holds at head dim `dim`.
int prefill_general_book_bytes(int dim);
// LDS bytes the fused kernel gives the append's copy of a table set's
// header, code LUT and books.
int decode_fast_enc_capacity(int dim, int nn);
// Row bytes of the packed layout with nn leading nibble K-steps (no padding).
int decode_fast_row_bytes(int dim, int nn);
hipError_t launch_decode_fast(const DecodeParams &p, const FastLayout &fl, int nn, int sg, hipStream_t stream);
// Chunked prefill (prefill.hip, the kernel and, with several splits, the
// merge), same layout requirements as the fused decode.
hipError_t launch_prefill(const PrefillParams &p, const FastLayout &fl, int nn, int sg, hipStream_t stream);
hipError_t launch_reconstruct(const DevTables *t, const uint8_t *packed, const uint16_t *norms,
                              int64_t rows, float *out, hipStream_t stream);
int model_scores_lds_bytes(int dim, int book_floats);
hipError_t launch_model_append(const ModelAppendParams &p, hipStream_t stream);
hipError_t launch_model_scores(const ModelScoresParams &p, int kv_count, int lds_bytes, hipStream_t stream);
hipError_t launch_model_softmax(const ModelAttnParams &p, int64_t score_rows, hipStream_t stream);
hipError_t launch_model_weighted(const ModelAttnParams &p, int64_t score_rows, hipStream_t stream);
hipError_t launch_half_convert(const float *src, uint16_t *dst, int64_t n, hipStream_t stream);

}  // namespace bgtq
