/* Block-GTQ CPU oracle: TEST INFRASTRUCTURE ONLY (see bgtq_oracle.h).
 *
 * Bit-exact restatement of the reference encoder as its Python/torch code
 * evaluates on the CPU, including the order of every FP32 reduction:
 *   - src/reference/production_math.py:12  ((xp*xp)*mask).sum(1)  -> aten_sum
 *   - src/reference/production_math.py:14  (n*mask).sum(1)/m       -> aten_sum
 *   - src/reference/production_math.py:16  normalized @ R.T        -> gemm_dot
 *   - src/reference/production_math.py:23  ((c*c)*mask).sum(1)     -> aten_sum
 * Built with -ffp-contract=off so that every a*b+c written here rounds twice
 * unless fmaf() is called explicitly.
 */
#include "bgtq_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* IEEE binary32 -> binary16, round to nearest even, subnormals, overflow to
 * inf (torch .half(); src/webgpu/half.wgsl:2-12 states the same rule). */
uint16_t bgtq_oracle_f32_to_f16(float x) {
  uint32_t b;
  memcpy(&b, &x, 4);
  uint32_t sign = (b >> 16) & 0x8000u;
  uint32_t e = (b >> 23) & 0xffu;
  uint32_t m = b & 0x7fffffu;
  if (e == 0xffu) return (uint16_t)(sign | 0x7c00u | (m ? 0x200u : 0u));
  int32_t he = (int32_t)e - 127 + 15;
  if (he >= 31) return (uint16_t)(sign | 0x7c00u);
  uint32_t mant, shift;
  if (he <= 0) {
    if (he < -10) return (uint16_t)sign;
    mant = m | 0x800000u;
    shift = (uint32_t)(14 - he);
  } else {
    mant = m;
    shift = 13;
  }
  uint32_t base = mant >> shift;
  uint32_t rem = mant & ((1u << shift) - 1u);
  uint32_t half = 1u << (shift - 1u);
  uint32_t inc = (rem > half || (rem == half && (base & 1u))) ? 1u : 0u;
  uint32_t exp_bits = he > 0 ? ((uint32_t)he << 10) : 0u;
  return (uint16_t)(sign | (exp_bits + base + inc));
}

float bgtq_oracle_f16_to_f32(uint16_t h) {
  uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
  uint32_t e = (h >> 10) & 31u, m = h & 1023u, b;
  if (e == 0) {
    float v = (float)m * 5.9604644775390625e-8f; /* 2^-24, exact */
    return (h & 0x8000u) ? -v : v;
  }
  if (e == 31) b = sign | 0x7f800000u | (m << 13);
  else b = sign | ((e + 112u) << 23) | (m << 13);
  float f;
  memcpy(&f, &b, 4);
  return f;
}

/* ATen's contiguous inner-dimension float sum (cascade_sum ->
 * vectorized_inner_sum -> row_sum -> multi_row_sum, 1 thread): lanes-wide
 * vectors, 4 interleaved vector accumulators, the cascade levels (which only
 * engage at >= 64 vectors), a scalar tail, then a sequential horizontal sum. */
float bgtq_oracle_aten_sum(const float *x, int32_t n, int32_t lanes) {
  /* Rows shorter than one vector take scalar_inner_sum: the same row_sum
   * structure over single floats and no horizontal step. */
  const int32_t W = n < lanes ? 1 : lanes;
  int32_t nvec = n / W;
  int32_t size_ilp = nvec / 4;
  float acc[4][4][16];
  memset(acc, 0, sizeof(acc));
  int32_t ceil_log2 = 0;
  while ((1 << ceil_log2) < size_ilp) ++ceil_log2;
  int32_t level_power = ceil_log2 / 4 > 4 ? ceil_log2 / 4 : 4;
  int32_t level_step = 1 << level_power, level_mask = level_step - 1;
  int32_t i = 0;
  for (; i + level_step <= size_ilp;) {
    for (int32_t j = 0; j < level_step; ++j, ++i)
      for (int32_t k = 0; k < 4; ++k)
        for (int32_t l = 0; l < W; ++l) acc[0][k][l] += x[(i * 4 + k) * W + l];
    for (int32_t j = 1; j < 4; ++j) {
      for (int32_t k = 0; k < 4; ++k)
        for (int32_t l = 0; l < W; ++l) {
          acc[j][k][l] += acc[j - 1][k][l];
          acc[j - 1][k][l] = 0.0f;
        }
      if ((i & (level_mask << (j * level_power))) != 0) break;
    }
  }
  for (; i < size_ilp; ++i)
    for (int32_t k = 0; k < 4; ++k)
      for (int32_t l = 0; l < W; ++l) acc[0][k][l] += x[(i * 4 + k) * W + l];
  for (int32_t j = 1; j < 4; ++j)
    for (int32_t k = 0; k < 4; ++k)
      for (int32_t l = 0; l < W; ++l) acc[0][k][l] += acc[j][k][l];
  for (int32_t v = size_ilp * 4; v < nvec; ++v)
    for (int32_t l = 0; l < W; ++l) acc[0][0][l] += x[v * W + l];
  for (int32_t k = 1; k < 4; ++k)
    for (int32_t l = 0; l < W; ++l) acc[0][0][l] += acc[0][k][l];
  if (W == 1) return acc[0][0][0];
  float final_acc = 0.0f;
  for (int32_t t = nvec * W; t < n; ++t) final_acc += x[t];
  for (int32_t l = 0; l < W; ++l) final_acc += acc[0][0][l];
  return final_acc;
}

/* One output of `normalized @ R.T` (production_math.py:16): the K loop of the
 * CPU sgemm. mode 0: one FMA chain, k ascending from +0. mode 1: separately
 * rounded products, k ascending. mode 2: FMA chain, k descending. */
static float gemm_dot(const float *a, const float *b, int32_t n, int32_t mode) {
  float acc = 0.0f;
  if (mode == 0) {
    for (int32_t k = 0; k < n; ++k) acc = fmaf(a[k], b[k], acc);
  } else if (mode == 1) {
    for (int32_t k = 0; k < n; ++k) acc += a[k] * b[k];
  } else if (mode >= 3) {
    /* K split into blocks of kc = 16*(mode-2): FMA chain per block, block sums added in order */
    int32_t kc = 16 * (mode - 2);
    for (int32_t k0 = 0; k0 < n; k0 += kc) {
      float part = 0.0f;
      for (int32_t k = k0; k < n && k < k0 + kc; ++k) part = fmaf(a[k], b[k], part);
      acc = k0 == 0 ? part : acc + part;
    }
  } else {
    for (int32_t k = n - 1; k >= 0; --k) acc = fmaf(a[k], b[k], acc);
  }
  return acc;
}

void bgtq_oracle_gemm_abt(const float *a, const float *b, int64_t n, int32_t k, int32_t m, int32_t mode,
                          float *out) {
  /* out[i*m+j] = sum_t a[i*k+t] b[j*k+t] with the K-loop order of gemm_dot. */
  for (int64_t i = 0; i < n; ++i)
    for (int32_t j = 0; j < m; ++j) out[i * m + j] = gemm_dot(a + i * k, b + (int64_t)j * k, k, mode);
}

int32_t bgtq_oracle_encode(const bgtq_oracle_layout *L, const bgtq_oracle_profile *P,
                           const float *x, int64_t rows, uint8_t *codes, float *raw,
                           float *corrected, float *y_out) {
  const int32_t d = L->dim, ng = L->groups, mc = L->max_centroids, W = P->sum_lanes;
  if (d < 2 || d > 128 || ng < 1 || ng > 8) return -1;
  float xp[128], tmp[128], xn[128], y[128], cents[128], rowR[128], nrm[8], rw[8];
  int32_t members[8] = {0};
  for (int32_t j = 0; j < d; ++j) members[L->group_of[j]]++;
  for (int64_t r = 0; r < rows; ++r) {
    const float *xr = x + r * d;
    for (int32_t i = 0; i < d; ++i) xp[i] = xr[L->perm[i]];
    for (int32_t g = 0; g < ng; ++g) {
      /* production_math.py:12  n = ((xp*xp)*mask).sum(1).add(1e-30).sqrt() */
      for (int32_t i = 0; i < d; ++i) {
        float sq = xp[i] * xp[i];
        tmp[i] = sq * (L->group_of[i] == (uint32_t)g ? 1.0f : 0.0f);
      }
      float n = sqrtf(bgtq_oracle_aten_sum(tmp, d, W) + 1e-30f);
      nrm[g] = n;
      /* production_math.py:14  raw = (n*mask).sum(1)/mask.sum() when ng > 1 */
      if (ng > 1) {
        for (int32_t i = 0; i < d; ++i) tmp[i] = n * (L->group_of[i] == (uint32_t)g ? 1.0f : 0.0f);
        rw[g] = bgtq_oracle_aten_sum(tmp, d, W) / (float)members[g];
      } else {
        rw[g] = n;
      }
    }
    /* production_math.py:15  normalized = xp / where(n > 1e-10, n, 1) */
    for (int32_t i = 0; i < d; ++i) {
      float n = nrm[L->group_of[i]];
      xn[i] = xp[i] / (n > 1e-10f ? n : 1.0f);
    }
    /* production_math.py:16-18 */
    for (int32_t j = 0; j < d; ++j) {
      for (int32_t i = 0; i < d; ++i) rowR[i] = L->rotation[(size_t)j * d + i];
      y[j] = gemm_dot(xn, rowR, d, P->gemm_mode);
      float t = (y[j] - L->offsets[j]) * L->inv_scales[j];
      t = t < 0.0f ? 0.0f : t;          /* clamp(0, 255) */
      t = t > 255.0f ? 255.0f : t;
      int32_t bin = (int32_t)t;         /* .long() truncates */
      uint8_t code = L->code_lut[(size_t)L->pos_to_cb[j] * 256 + bin];
      codes[r * d + j] = code;
      cents[j] = L->centroids[(size_t)j * mc + code];
    }
    /* production_math.py:21-23 */
    for (int32_t g = 0; g < ng; ++g) {
      for (int32_t j = 0; j < d; ++j) {
        float sq = cents[j] * cents[j];
        tmp[j] = sq * (L->group_of[j] == (uint32_t)g ? 1.0f : 0.0f);
      }
      float c = sqrtf(bgtq_oracle_aten_sum(tmp, d, W));
      c = c < 1e-10f ? 1e-10f : c;
      if (raw) raw[r * ng + g] = rw[g];
      if (corrected) corrected[r * ng + g] = rw[g] / c;
    }
    if (y_out) memcpy(y_out + r * d, y, sizeof(float) * d);
  }
  return 0;
}

void bgtq_oracle_pack(const uint8_t *codes, int64_t rows, int32_t dim, int32_t nibble_dims,
                      int32_t row_bytes, uint8_t *out) {
  /* src/reference/mixed_layout.py:21-27 */
  for (int64_t r = 0; r < rows; ++r) {
    const uint8_t *c = codes + r * dim;
    uint8_t *o = out + r * row_bytes;
    memset(o, 0, (size_t)row_bytes);
    for (int32_t k = 0; k < nibble_dims / 2; ++k)
      o[k] = (uint8_t)((c[2 * k] & 15) | ((c[2 * k + 1] & 15) << 4));
    for (int32_t j = nibble_dims; j < dim; ++j) o[nibble_dims / 2 + j - nibble_dims] = c[j];
  }
}

void bgtq_oracle_unpack(const uint8_t *packed, int64_t rows, int32_t dim, int32_t nibble_dims,
                        int32_t row_bytes, uint8_t *codes) {
  /* src/reference/mixed_layout.py:30-37 */
  for (int64_t r = 0; r < rows; ++r) {
    const uint8_t *p = packed + r * row_bytes;
    uint8_t *c = codes + r * dim;
    for (int32_t k = 0; k < nibble_dims / 2; ++k) {
      c[2 * k] = p[k] & 15;
      c[2 * k + 1] = p[k] >> 4;
    }
    for (int32_t j = nibble_dims; j < dim; ++j) c[j] = p[nibble_dims / 2 + j - nibble_dims];
  }
}

int32_t bgtq_oracle_encode_pack(const bgtq_oracle_layout *L, const bgtq_oracle_profile *P,
                                const uint16_t *k_half, int64_t rows, uint8_t *packed,
                                uint16_t *norms) {
  /* tests/oracles/export_attention.py:27-31: encode(k.float()), scales.half(),
   * zero-padded to norm_stride, pack(codes). Processed in blocks of rows. */
  const int32_t d = L->dim, ng = L->groups;
  enum { BLOCK = 256 };
  float *x = (float *)malloc(sizeof(float) * BLOCK * d);
  uint8_t *codes = (uint8_t *)malloc((size_t)BLOCK * d);
  float *corr = (float *)malloc(sizeof(float) * BLOCK * ng);
  if (!x || !codes || !corr) {
    free(x); free(codes); free(corr);
    return -2;
  }
  int32_t rc = 0;
  for (int64_t r0 = 0; r0 < rows && rc == 0; r0 += BLOCK) {
    int64_t n = rows - r0 < BLOCK ? rows - r0 : BLOCK;
    for (int64_t i = 0; i < n * d; ++i) x[i] = bgtq_oracle_f16_to_f32(k_half[r0 * d + i]);
    rc = bgtq_oracle_encode(L, P, x, n, codes, NULL, corr, NULL);
    bgtq_oracle_pack(codes, n, d, L->nibble_dims, L->row_bytes, packed + r0 * L->row_bytes);
    for (int64_t r = 0; r < n; ++r)
      for (int32_t g = 0; g < L->norm_stride; ++g)
        norms[(r0 + r) * L->norm_stride + g] =
            g < ng ? bgtq_oracle_f32_to_f16(corr[r * ng + g]) : (uint16_t)0;
  }
  free(x); free(codes); free(corr);
  return rc;
}

void bgtq_oracle_reconstruct(const bgtq_oracle_layout *L, const uint8_t *codes,
                             const float *scales, int32_t scale_stride, int64_t rows,
                             float *k_out) {
  const int32_t d = L->dim, mc = L->max_centroids;
  float yv[128], acc[128];
  for (int64_t r = 0; r < rows; ++r) {
    for (int32_t j = 0; j < d; ++j)
      yv[j] = L->centroids[(size_t)j * mc + codes[r * d + j]] * scales[r * scale_stride + L->group_of[j]];
    /* k[i] = fma chain over j ascending (the sgemm K-loop of y @ R); the
     * loops run j outer so the d independent chains advance together. */
    for (int32_t i = 0; i < d; ++i) acc[i] = 0.0f;
    for (int32_t j = 0; j < d; ++j) {
      const float y = yv[j];
      const float *row = L->rotation + (size_t)j * d;
      for (int32_t i = 0; i < d; ++i) acc[i] = fmaf(y, row[i], acc[i]);
    }
    for (int32_t i = 0; i < d; ++i) k_out[r * d + L->perm[i]] = acc[i];
  }
}

int32_t bgtq_oracle_attention(const float *q, int32_t nq, const float *k, const float *v,
                              int64_t T, int32_t dim, const uint32_t *positions, int32_t causal,
                              float *logits, float *probs, float *out) {
  /* src/reference/attention.py:7-16: validation, raised as negative codes. */
  if (nq < 1 || T < 1 || dim < 1) return -1;
  for (int32_t r = 0; r < nq; ++r)
    if ((int64_t)positions[r] >= T) return -2;
  for (int64_t i = 0; i < (int64_t)nq * dim; ++i) if (!isfinite(q[i])) return -3;
  for (int64_t i = 0; i < T * dim; ++i) if (!isfinite(k[i]) || !isfinite(v[i])) return -3;
  double *l = (double *)malloc(sizeof(double) * (size_t)T);
  double *acc = (double *)malloc(sizeof(double) * (size_t)dim);
  if (!l || !acc) { free(l); free(acc); return -4; }
  const double inv = 1.0 / sqrt((double)dim);
  for (int32_t r = 0; r < nq; ++r) {
    int64_t end = causal ? (int64_t)positions[r] + 1 : T;
    double mx = -INFINITY;
    for (int64_t t = 0; t < T; ++t) {
      if (t >= end) { l[t] = -INFINITY; continue; }
      double s = 0.0;
      for (int32_t i = 0; i < dim; ++i) s += (double)q[(int64_t)r * dim + i] * (double)k[t * dim + i];
      l[t] = s * inv;
      if (l[t] > mx) mx = l[t];
    }
    double den = 0.0;
    for (int64_t t = 0; t < end; ++t) den += exp(l[t] - mx);
    for (int32_t i = 0; i < dim; ++i) acc[i] = 0.0;
    for (int64_t t = 0; t < T; ++t) {
      double p = t < end ? exp(l[t] - mx) / den : 0.0;
      if (logits) logits[(int64_t)r * T + t] = (float)l[t];
      if (probs) probs[(int64_t)r * T + t] = (float)p;
      if (p != 0.0)
        for (int32_t i = 0; i < dim; ++i) acc[i] += p * (double)v[t * dim + i];
    }
    for (int32_t i = 0; i < dim; ++i) out[(int64_t)r * dim + i] = (float)acc[i];
  }
  free(l);
  free(acc);
  return 0;
}

/* src/reference/attention.py:17-21 in FP32 (q.float() @ k.float().T / sqrt(d),
 * softmax, @ v.float()), with sums in ascending order: a float restatement of
 * the reference's own arithmetic type, within the fixtures' tolerances of its
 * results, for timing the CPU path. Logits of 16 tokens accumulate together
 * (independent chains); validation as bgtq_oracle_attention. */
int32_t bgtq_oracle_attention_f32(const float *q, int32_t nq, const float *k, const float *v,
                                  int64_t T, int32_t dim, const uint32_t *positions, int32_t causal,
                                  float *logits, float *probs, float *out) {
  if (nq < 1 || T < 1 || dim < 1) return -1;
  for (int32_t r = 0; r < nq; ++r)
    if ((int64_t)positions[r] >= T) return -2;
  for (int64_t i = 0; i < (int64_t)nq * dim; ++i) if (!isfinite(q[i])) return -3;
  for (int64_t i = 0; i < T * dim; ++i) if (!isfinite(k[i]) || !isfinite(v[i])) return -3;
  float *l = (float *)malloc(sizeof(float) * (size_t)T);
  float *acc = (float *)malloc(sizeof(float) * (size_t)dim);
  if (!l || !acc) { free(l); free(acc); return -4; }
  const float scale = (float)sqrt((double)dim);
  for (int32_t r = 0; r < nq; ++r) {
    const float *qr = q + (int64_t)r * dim;
    const int64_t end = causal ? (int64_t)positions[r] + 1 : T;
    float mx = -INFINITY;
    int64_t t = 0;
    for (; t + 16 <= end; t += 16) {
      float s[16] = {0.0f};
      for (int32_t i = 0; i < dim; ++i)
        for (int b = 0; b < 16; ++b) s[b] = fmaf(qr[i], k[(t + b) * dim + i], s[b]);
      for (int b = 0; b < 16; ++b) {
        l[t + b] = s[b] / scale;
        if (l[t + b] > mx) mx = l[t + b];
      }
    }
    for (; t < end; ++t) {
      float s = 0.0f;
      for (int32_t i = 0; i < dim; ++i) s = fmaf(qr[i], k[t * dim + i], s);
      l[t] = s / scale;
      if (l[t] > mx) mx = l[t];
    }
    for (; t < T; ++t) l[t] = -INFINITY;
    float den = 0.0f;
    for (t = 0; t < end; ++t) den += expf(l[t] - mx);
    for (int32_t i = 0; i < dim; ++i) acc[i] = 0.0f;
    for (t = 0; t < T; ++t) {
      const float p = t < end ? expf(l[t] - mx) / den : 0.0f;
      if (logits) logits[(int64_t)r * T + t] = l[t];
      if (probs) probs[(int64_t)r * T + t] = p;
      if (p != 0.0f) {
        const float *vt = v + t * dim;
        for (int32_t i = 0; i < dim; ++i) acc[i] = fmaf(p, vt[i], acc[i]);
      }
    }
    for (int32_t i = 0; i < dim; ++i) out[(int64_t)r * dim + i] = acc[i];
  }
  free(l);
  free(acc);
  return 0;
}

void bgtq_oracle_allocate_bits(const float *scores, int32_t n, int64_t budget, int32_t min_bits,
                               int32_t max_bits, int64_t *widths) {
  /* src/reference/allocator.py:4-17: FP32 scores times FP64 powers of 4,
   * argmax with the first index winning ties, stop at a nonpositive best. */
  int64_t total = 0;
  for (int32_t i = 0; i < n; ++i) { widths[i] = min_bits; total += min_bits; }
  int64_t remaining = budget - total;
  while (remaining > 0 && n > 0) {
    int32_t best = -1;
    double best_p = 0.0;
    for (int32_t i = 0; i < n; ++i) {
      double p = widths[i] >= max_bits ? -1.0 : (double)scores[i] * pow(4.0, -(double)widths[i]);
      if (best < 0 || p > best_p) { best = i; best_p = p; }
    }
    if (best_p <= 0.0) break;
    widths[best] += 1;
    remaining -= 1;
  }
}
