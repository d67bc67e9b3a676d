// The model step's separate attention passes, by the reference's dispatch
// names (src/model/ops.ts:6-12): append (src/model/append.wgsl:6-10), dot,
// softmax and weighted (src/model/attention.wgsl:13-39) and compressed_dot
// (src/model/compressed-dot.wgsl:14-31). They keep the reference's buffer
// layouts, including the materialised scores and probabilities
// [rows*qHeads, tokens]; the fused decode and prefill kernels are the fast
// path for the same step. Each pass covers the work items the reference's
// dispatch of x (and y) workgroups covers, clamped to the parameters' extents.
#include <hip/hip_fp16.h>

#include "bgtq_internal.h"

namespace bgtq {
namespace {

constexpr int kMaxGqa = 16;

__device__ __forceinline__ float h2f(uint16_t h) { return __half2float(__ushort_as_half(h)); }
__device__ __forceinline__ uint16_t f2h(float v) { return __half_as_ushort(__float2half_rn(v)); }

// append.wgsl:6-10: pair i of the rows x heads x 32 pairs (64 dims) of the
// FP32 input, rounded to FP16, into cache[head][start + row][pair].
__global__ __launch_bounds__(256) void model_append_kernel(ModelAppendParams p) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= p.pairs) return;
  const int64_t per_row = (int64_t)p.heads * 32;
  const int64_t row = i / per_row;
  const int head = (int)((i / 32) % p.heads), pair = (int)(i % 32);
  const int64_t at = ((int64_t)head * p.capacity + p.start + row) * 32 + pair;
  const float2 v = reinterpret_cast<const float2 *>(p.input)[i];
  p.cache[at] = (uint32_t)f2h(v.x) | ((uint32_t)f2h(v.y) << 16);
}

// Scores of one query row against every token of one KV head, a thread per
// token for the head's gqa query heads (compressed-dot.wgsl:14-31 with packed
// K, attention.wgsl:13-23 with FP16 K rows). The packed-K dot uses the
// rotated query: q . (R^T c)[perm^-1] = sum_j c_j (R q_perm)_j, with
// c_j = centroid(code_j) * scale(group of j) as the reference forms it.
// Grid: (token blocks of 256, query rows, KV heads of the dispatch).
template <int KF>
__global__ __launch_bounds__(256) void model_scores_kernel(ModelScoresParams p) {
  extern __shared__ __align__(16) uint8_t smem[];
  const int row = blockIdx.y, kv = p.head0 + blockIdx.z, tid = threadIdx.x;
  const int d = p.dim, G = p.gqa;
  const int qbase = kv * G;
  float *qr = reinterpret_cast<float *>(smem);  // [kMaxGqa][d]
  float *books = qr + kMaxGqa * d;
  const DevTables *T = KF == 1 ? p.tables : nullptr;
  const int mc = KF == 1 ? T->max_centroids : 0;
  for (int e = tid; e < G * d; e += 256) {
    const int g = e / d, j = e - g * d;
    const float *qv = p.q + ((int64_t)row * p.q_heads + qbase + g) * d;
    float r;
    if (KF == 1) {
      const float *R = tables_rot(T);
      const int grp = T->group_of[j];
      float acc = 0.0f;
      for (int i = T->gstart[grp]; i < T->gend[grp]; ++i) acc = __builtin_fmaf(R[j * d + i], qv[T->perm[i]], acc);
      r = acc;
    } else {
      r = qv[j];
    }
    qr[g * d + j] = r;
  }
  if (KF == 1) {
    const float *bg = tables_books(T);
    for (int e = tid; e < T->n_books * mc; e += 256) books[e] = bg[e];
  }
  __syncthreads();
  const int t = blockIdx.x * 256 + tid;
  if (t >= p.n_tok) return;
  // Work item (row, g) of the reference's dispatch: item = row*gqa + g in
  // workgroup row item / 128 (offset by the KV head's blocks for dot).
  const int blocks = (p.rows * G + 127) / 128;
  const int causal_end = p.start + row;  // tokens after it are -inf
  float acc[kMaxGqa];
#pragma unroll
  for (int g = 0; g < kMaxGqa; ++g) acc[g] = 0.0f;
  if (t <= causal_end) {
    if (KF == 1) {
      const int ns = T->nibble_dims, rb = T->row_bytes, nst = T->norm_stride;
      const uint8_t *prow = p.packed + (int64_t)t * rb;
      const uint16_t *nrow = p.norms + (int64_t)t * nst;
      float scale[kMaxGroups];
#pragma unroll
      for (int g = 0; g < kMaxGroups; ++g) scale[g] = g < T->groups ? h2f(nrow[g]) : 0.0f;
      for (int j = 0; j < d; ++j) {
        const int code = j < ns ? (prow[j >> 1] >> ((j & 1) * 4)) & 15 : prow[ns / 2 + j - ns];
        float s = scale[0];
#pragma unroll
        for (int g = 1; g < kMaxGroups; ++g) s = T->group_of[j] == g ? scale[g] : s;
        const float c = books[T->pos_book[j] * mc + code] * s;
#pragma unroll
        for (int g = 0; g < kMaxGqa; ++g)
          if (g < G) acc[g] = __builtin_fmaf(c, qr[g * d + j], acc[g]);
      }
    } else {
      const uint16_t *krow = p.k + ((int64_t)kv * p.capacity + t) * d;
      for (int j = 0; j < d; ++j) {
        const float kval = h2f(krow[j]);
#pragma unroll
        for (int g = 0; g < kMaxGqa; ++g)
          if (g < G) acc[g] = __builtin_fmaf(qr[g * d + j], kval, acc[g]);
      }
    }
  }
#pragma unroll
  for (int g = 0; g < kMaxGqa; ++g) {
    if (g >= G) break;
    const int item = row * G + g;
    const int wg_row = (KF == 1 ? 0 : (kv - p.head0) * blocks) + item / 128;
    if (wg_row >= p.y_limit) continue;
    const float lg = t <= causal_end ? acc[g] * p.scale : -INFINITY;
    p.scores[((int64_t)row * p.q_heads + qbase + g) * p.tokens + t] = lg;
  }
}

// Sum of a 256-thread workgroup's values, in a fixed order.
__device__ __forceinline__ float block_reduce(float v, float *red, bool is_max) {
  const int tid = threadIdx.x;
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float w = __shfl_xor(v, o);
    v = is_max ? fmaxf(v, w) : v + w;
  }
  if ((tid & 63) == 0) red[tid >> 6] = v;
  __syncthreads();
  const float r = is_max ? fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3])) : ((red[0] + red[1]) + red[2]) + red[3];
  __syncthreads();
  return r;
}

// attention.wgsl:24-31: one workgroup per score row r (= row*qHeads + head):
// probabilities over tokens < end = min(tokens, start + row + 1), zero after.
__global__ __launch_bounds__(256) void model_softmax_kernel(ModelAttnParams p) {
  __shared__ float red[4];
  const int64_t r = blockIdx.x;
  const int tid = threadIdx.x;
  const int end = min(p.tokens, p.start + (int)(r / p.q_heads) + 1);
  const float *lg = p.scores + r * p.tokens;
  float m = -3.4e38f;
  for (int t = tid; t < end; t += 256) m = fmaxf(m, lg[t]);
  m = block_reduce(m, red, true);
  float s = 0.0f;
  for (int t = tid; t < end; t += 256) s += expf(lg[t] - m);
  s = block_reduce(s, red, false);
  float *pr = p.probs + r * p.tokens;
  for (int t = tid; t < p.tokens; t += 256) pr[t] = (t < end ? expf(lg[t] - m) : 0.0f) / s;
}

// attention.wgsl:32-39: output[r][dm] = sum_{t < end} p[r][t] v[kv][t][dm],
// kv = (r mod qHeads) / gqa. One workgroup per score row; wave w takes tokens
// w, w + 4, ..., lane dm (and dm + 64 at head_dim 128).
__global__ __launch_bounds__(256) void model_weighted_kernel(ModelAttnParams p) {
  __shared__ float part[4][kMaxDim];
  const int64_t r = blockIdx.x;
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
  const int d = p.dim;
  const int kv = (int)(r % p.q_heads) / p.gqa;
  const int end = min(p.tokens, p.start + (int)(r / p.q_heads) + 1);
  const float *pr = p.probs + r * p.tokens;
  const uint16_t *vb = p.v + (int64_t)kv * p.capacity * d;
  float s0 = 0.0f, s1 = 0.0f;
  for (int t = w; t < end; t += 4) {
    const float pt = pr[t];
    s0 = __builtin_fmaf(pt, h2f(vb[(int64_t)t * d + lane]), s0);
    if (d > 64) s1 = __builtin_fmaf(pt, h2f(vb[(int64_t)t * d + 64 + lane]), s1);
  }
  part[w][lane] = s0;
  if (d > 64) part[w][64 + lane] = s1;
  __syncthreads();
  for (int dm = tid; dm < d; dm += 256) {
    const int64_t index = r * d + dm;
    if (index < p.x_limit) p.out[index] = ((part[0][dm] + part[1][dm]) + part[2][dm]) + part[3][dm];
  }
}

}  // namespace

int model_scores_lds_bytes(int dim, int book_floats) { return (kMaxGqa * dim + book_floats) * 4; }

hipError_t launch_model_append(const ModelAppendParams &p, hipStream_t stream) {
  if (p.pairs <= 0) return hipSuccess;
  hipLaunchKernelGGL(model_append_kernel, dim3((unsigned)((p.pairs + 255) / 256)), dim3(256), 0, stream, p);
  return hipGetLastError();
}

hipError_t launch_model_scores(const ModelScoresParams &p, int kv_count, int lds_bytes, hipStream_t stream) {
  if (p.n_tok <= 0 || p.rows <= 0 || kv_count <= 0) return hipSuccess;
  const dim3 grid((unsigned)((p.n_tok + 255) / 256), (unsigned)p.rows, (unsigned)kv_count);
  if (p.tables) hipLaunchKernelGGL(model_scores_kernel<1>, grid, dim3(256), lds_bytes, stream, p);
  else hipLaunchKernelGGL(model_scores_kernel<0>, grid, dim3(256), lds_bytes, stream, p);
  return hipGetLastError();
}

hipError_t launch_model_softmax(const ModelAttnParams &p, int64_t score_rows, hipStream_t stream) {
  if (score_rows <= 0) return hipSuccess;
  hipLaunchKernelGGL(model_softmax_kernel, dim3((unsigned)score_rows), dim3(256), 0, stream, p);
  return hipGetLastError();
}

hipError_t launch_model_weighted(const ModelAttnParams &p, int64_t score_rows, hipStream_t stream) {
  if (score_rows <= 0) return hipSuccess;
  hipLaunchKernelGGL(model_weighted_kernel, dim3((unsigned)score_rows), dim3(256), 0, stream, p);
  return hipGetLastError();
}

}  // namespace bgtq
