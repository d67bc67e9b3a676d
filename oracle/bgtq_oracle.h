/* Block-GTQ CPU oracle: TEST INFRASTRUCTURE ONLY.
 *
 * A plain-C restatement of the reference's Python path (encode, pack, unpack,
 * reconstruct, attention, allocator). Only tests/, the smoke check
 * and bench.py's CPU-baseline leg may load it, and only as the checker. The
 * product library (libbgtq.so) never links or calls anything declared here.
 */
#ifndef BGTQ_ORACLE_H
#define BGTQ_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Tables in the reference's calibration format (src/webgpu/layout.ts:2-6). */
typedef struct {
  int32_t dim, groups, row_bytes, norm_stride, nibble_dims, max_centroids;
  int32_t n_codebooks;              /* code_lut rows */
  const uint32_t *perm;             /* head_perm [dim] */
  const uint32_t *group_of;         /* [dim] */
  const uint32_t *pos_to_cb;        /* [dim] */
  const uint8_t *code_lut;          /* [n_codebooks*256] */
  const float *rotation;            /* [dim*dim], y_j = sum_i x_i R[j*dim+i] */
  const float *centroids;           /* [dim*max_centroids] */
  const float *offsets;             /* [dim] */
  const float *inv_scales;          /* [dim] */
} bgtq_oracle_layout;

/* Which CPU reduction tree the reference's torch ran with.
 * sum_lanes: ATen Vectorized<float>::size() (8 = AVX2, 16 = AVX-512).
 * gemm_mode: summation order of the K loop in the CPU sgemm (see .c). */
typedef struct { int32_t sum_lanes; int32_t gemm_mode; } bgtq_oracle_profile;

uint16_t bgtq_oracle_f32_to_f16(float x);
float bgtq_oracle_f16_to_f32(uint16_t h);
float bgtq_oracle_aten_sum(const float *x, int32_t n, int32_t lanes);

/* out[n x m] = a[n x k] @ b[m x k]^T with the sgemm K-loop order of gemm_mode. */
void bgtq_oracle_gemm_abt(const float *a, const float *b, int64_t n, int32_t k, int32_t m, int32_t mode,
                          float *out);

/* encode (src/reference/production_math.py:4-24). x holds FP16-valued floats
 * [rows*dim]. Outputs: codes [rows*dim] (head_perm order, pack_perm = identity),
 * raw/corrected [rows*groups], y [rows*dim] (may be NULL). */
int32_t bgtq_oracle_encode(const bgtq_oracle_layout *L, const bgtq_oracle_profile *P,
                           const float *x, int64_t rows, uint8_t *codes, float *raw,
                           float *corrected, float *y);

/* Same as encode, then pack + FP16 scales: the persistent cache row format. */
int32_t bgtq_oracle_encode_pack(const bgtq_oracle_layout *L, const bgtq_oracle_profile *P,
                                const uint16_t *k_half, int64_t rows, uint8_t *packed,
                                uint16_t *norms);

void bgtq_oracle_pack(const uint8_t *codes, int64_t rows, int32_t dim, int32_t nibble_dims,
                      int32_t row_bytes, uint8_t *out);
void bgtq_oracle_unpack(const uint8_t *packed, int64_t rows, int32_t dim, int32_t nibble_dims,
                        int32_t row_bytes, uint8_t *codes);

/* reconstruct (production_math.py:27-31): k = ((c*s) @ R)[inv_head_perm]. */
void bgtq_oracle_reconstruct(const bgtq_oracle_layout *L, const uint8_t *codes,
                             const float *scales, int32_t scale_stride, int64_t rows,
                             float *k_out);

/* attention (src/reference/attention.py:5-22), accumulated in double.
 * k/v: [T*dim] float; out logits/probs [nq*T] (may be NULL), out [nq*dim]. */
int32_t bgtq_oracle_attention(const float *q, int32_t nq, const float *k, const float *v,
                              int64_t T, int32_t dim, const uint32_t *positions, int32_t causal,
                              float *logits, float *probs, float *out);
/* The same in FP32 (the reference's arithmetic type), for the CPU baseline. */
int32_t bgtq_oracle_attention_f32(const float *q, int32_t nq, const float *k, const float *v,
                                  int64_t T, int32_t dim, const uint32_t *positions, int32_t causal,
                                  float *logits, float *probs, float *out);

/* allocate_bits (src/reference/allocator.py:4-17). */
void bgtq_oracle_allocate_bits(const float *scores, int32_t n, int64_t budget, int32_t min_bits,
                               int32_t max_bits, int64_t *widths);

#ifdef __cplusplus
}
#endif
#endif
