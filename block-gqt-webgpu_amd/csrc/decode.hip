// Compressed-K decode attention for gfx950 (flash-decoding over token splits).
//
// QK runs in the rotated domain: reconstruct() (production_math.py:27-31) is
// k = ((c*s) @ R)[inv_perm], so q.k = sum_j s_g(j) c_j[code_j] qr_j with
// qr = R q[perm] (block diagonal R, computed once per query head by
// rotate_q_kernel and pre-scaled by 1/sqrt(d)). One KV head's codes are
// unpacked once and shared by its G query heads (src/model/compressed-dot.wgsl
// serves the same GQA grouping). Online softmax replaces the materialised
// softmax pass (src/model/attention.wgsl:24-32); PV streams the FP16 or FP32 V
// rows (src/model/attention.wgsl:34-39). Each (sequence, KV head, split)
// workgroup writes (m, l, o) partials; combine_kernel merges them by LSE.
#include <hip/hip_fp16.h>

#include "bgtq_internal.h"

namespace bgtq {
namespace {

constexpr int kThreads = 256;  // 4 waves
constexpr int kTile = 256;     // tokens staged per iteration (64 per wave)

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
__device__ __forceinline__ float h2f(uint16_t h) { return __half2float(__ushort_as_half(h)); }

struct Lds {
  // byte offsets into dynamic shared memory
  int qr, books, rows, norms, probs, comb, total;
};

__host__ __device__ inline int align16(int x) { return (x + 15) & ~15; }

__host__ __device__ inline Lds lds_layout(int GP, int dim, int key_format, int books_bytes, int row_bytes,
                                          int norm_stride) {
  Lds L;
  int o = 0;
  L.qr = o; o += align16(dim * GP * 4);
  L.books = o; o += key_format == 1 ? align16(books_bytes) : 0;
  L.rows = o; o += key_format == 1 ? align16(kTile * row_bytes + 16) : 0;
  L.norms = o; o += key_format == 1 ? align16(kTile * norm_stride * 2 + 16) : 0;
  L.probs = o; o += align16(4 * 64 * GP * 4);
  L.comb = o; o += align16(4 * GP * (dim + 2) * 4);
  L.total = o;
  return L;
}

// q rotation for the compressed path: qr_j = (1/sqrt d) sum_{i in group(j)} R[j,i] q[perm[i]];
// plain scaling for FP16/FP32 K rows.
__global__ void rotate_q_kernel(DecodeParams p, const float *__restrict__ q, float *__restrict__ qr,
                                float inv_sqrt_d) {
  const int idx = blockIdx.x;  // b*Hq + h
  const int j = threadIdx.x;
  const int d = p.dim;
  if (j >= d) return;
  const int h = idx % p.q_heads;
  const float *qv = q + (int64_t)idx * d;
  float r;
  if (p.key_format == 1 && !p.q_rotated) {
    const DevTables *T = p.tables[h / p.G];
    const float *R = tables_rot(T);
    const int g = T->group_of[j];
    float acc = 0.0f;
    for (int i = T->gstart[g]; i < T->gend[g]; ++i) acc = __builtin_fmaf(R[j * d + i], qv[T->perm[i]], acc);
    r = acc;
  } else {
    r = qv[j];
  }
  qr[(int64_t)idx * d + j] = r * inv_sqrt_d;
}

template <int GP, int KF, int VT>
__global__ __launch_bounds__(kThreads) void decode_split_kernel(DecodeParams p) {
  extern __shared__ __align__(16) uint8_t smem[];
  const int unit = blockIdx.y, split = blockIdx.x;
  const int b = unit / p.kv_heads, kv = unit - b * p.kv_heads;
  const int d = p.dim, G = p.G, Hq = p.q_heads;
  const int hq0 = kv * G;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int T_b = (int)min(p.lengths[b], (uint32_t)p.max_length);
  const int t_begin = split * p.split_tokens;
  const int t_end = min(T_b, t_begin + p.split_tokens);

  const DevTables *T = KF == 1 ? p.tables[kv] : nullptr;
  const int RB = KF == 1 ? T->row_bytes : 0;
  const int NS = KF == 1 ? T->norm_stride : 0;
  const int books_bytes = KF == 1 ? T->n_books * T->max_centroids * 4 : 0;
  const Lds L = lds_layout(GP, d, KF, books_bytes, RB, NS);
  float *qr_s = reinterpret_cast<float *>(smem + L.qr);
  float *books_s = reinterpret_cast<float *>(smem + L.books);
  uint8_t *rows_s = smem + L.rows;
  uint16_t *norms_s = reinterpret_cast<uint16_t *>(smem + L.norms);
  float *p_s = reinterpret_cast<float *>(smem + L.probs);
  float *comb = reinterpret_cast<float *>(smem + L.comb);

  // Query rows (rotated, scaled) as qr_s[j*GP + g]; heads >= G are zero.
  for (int e = tid; e < d * GP; e += kThreads) {
    const int j = e / GP, g = e - j * GP;
    qr_s[e] = g < G ? p.qr[((int64_t)b * Hq + hq0 + g) * d + j] : 0.0f;
  }
  if (KF == 1) {
    const float *books = tables_books(T);
    for (int e = tid; e < books_bytes / 4; e += kThreads) books_s[e] = books[e];
  }
  int end_g[GP];
#pragma unroll
  for (int g = 0; g < GP; ++g) {
    int e = 0;
    if (g < G) e = p.ends ? min(p.ends[(int64_t)b * Hq + hq0 + g], T_b) : T_b;
    end_g[g] = e;
  }
  float m_run[GP], l_run[GP], o0[GP], o1[GP];
#pragma unroll
  for (int g = 0; g < GP; ++g) {
    m_run[g] = -INFINITY;
    l_run[g] = 0.0f;
    o0[g] = 0.0f;
    o1[g] = 0.0f;
  }
  const bool dim0 = lane < d, dim1 = lane + 64 < d;
  const uint8_t *packed = KF == 1 ? p.packed + b * p.packed_seq_stride + kv * p.packed_head_stride : nullptr;
  const uint16_t *norms = KF == 1 ? p.norms + b * p.norms_seq_stride + kv * p.norms_head_stride : nullptr;
  const int64_t vbase = b * p.v_seq_stride + kv * p.v_head_stride;
  const int64_t kbase = b * p.k_seq_stride + kv * p.k_head_stride;
  __syncthreads();

  for (int tile = t_begin; tile < t_end; tile += kTile) {
    const int tile_n = min(kTile, t_end - tile);
    int row_off = 0, nrm_off = 0;
    if (KF == 1) {
      // Stage the tile's packed rows and scales with aligned dword loads. The
      // dword covering the last byte may extend up to 3 bytes past it; the
      // host requires packed/norm buffers readable to a 16-byte boundary.
      const int64_t byte0 = (int64_t)tile * RB, byte1 = (int64_t)(tile + tile_n) * RB;
      const int64_t a0 = (reinterpret_cast<uintptr_t>(packed + byte0) & 3);
      const uint32_t *src = reinterpret_cast<const uint32_t *>(packed + byte0 - a0);
      const int nw = (int)((byte1 - byte0 + a0 + 3) >> 2);
      uint32_t *dst = reinterpret_cast<uint32_t *>(rows_s);
      for (int e = tid; e < nw; e += kThreads) dst[e] = src[e];
      row_off = (int)a0;
      const int64_t h0 = (int64_t)tile * NS, h1 = (int64_t)(tile + tile_n) * NS;
      const int64_t n0 = (reinterpret_cast<uintptr_t>(norms + h0) & 3) >> 1;
      const uint32_t *nsrc = reinterpret_cast<const uint32_t *>(norms + h0 - n0);
      const int nn = (int)((h1 - h0 + n0 + 1) >> 1);
      uint32_t *ndst = reinterpret_cast<uint32_t *>(norms_s);
      for (int e = tid; e < nn; e += kThreads) ndst[e] = nsrc[e];
      nrm_off = (int)n0;
    }
    __syncthreads();

    const int li = wave * 64 + lane;  // token index within the tile
    const int tt = tile + li;
    const bool tok = li < tile_n;
    float logit[GP];
#pragma unroll
    for (int g = 0; g < GP; ++g) logit[g] = 0.0f;
    if (tok) {
      if (KF == 1) {
        const uint8_t *row = rows_s + row_off + li * RB;
        const uint16_t *nrow = norms_s + nrm_off + li * NS;
        const int ng = T->groups, nib = T->nibble_dims, mc = T->max_centroids;
        for (int g2 = 0; g2 < ng; ++g2) {
          const float s = h2f(nrow[g2]);
          float acc[GP];
#pragma unroll
          for (int g = 0; g < GP; ++g) acc[g] = 0.0f;
          for (int j = T->gstart[g2]; j < T->gend[g2]; ++j) {
            const int code = j < nib ? (row[j >> 1] >> ((j & 1) * 4)) & 15 : row[(nib >> 1) + j - nib];
            const float c = books_s[(int)T->pos_book[j] * mc + code];
#pragma unroll
            for (int g = 0; g < GP; ++g) acc[g] = __builtin_fmaf(qr_s[j * GP + g], c, acc[g]);
          }
#pragma unroll
          for (int g = 0; g < GP; ++g) logit[g] = __builtin_fmaf(s, acc[g], logit[g]);
        }
      } else {
        for (int j = 0; j < d; ++j) {
          float kval;
          if (KF == 0) kval = h2f(static_cast<const uint16_t *>(p.k)[kbase + (int64_t)tt * d + j]);
          else kval = static_cast<const float *>(p.k)[kbase + (int64_t)tt * d + j];
#pragma unroll
          for (int g = 0; g < GP; ++g) logit[g] = __builtin_fmaf(qr_s[j * GP + g], kval, logit[g]);
        }
      }
    }
    // Online softmax update per query head (wave-wide max and sum).
#pragma unroll
    for (int g = 0; g < GP; ++g) {
      const float lg = (tok && tt < end_g[g]) ? logit[g] : -INFINITY;
      if (p.logits && tok && g < G) p.logits[((int64_t)b * Hq + hq0 + g) * p.logit_stride + tt] = lg;
      const float mn = fmaxf(m_run[g], wave_max(lg));
      const float alpha = mn == -INFINITY ? 1.0f : expf(m_run[g] - mn);
      const float pr = lg == -INFINITY ? 0.0f : expf(lg - mn);
      l_run[g] = l_run[g] * alpha + wave_sum(pr);
      o0[g] *= alpha;
      o1[g] *= alpha;
      m_run[g] = mn;
      p_s[(wave * 64 + lane) * GP + g] = pr;
    }
    __syncthreads();
    // PV over this wave's tokens: lane owns dims lane and lane + 64.
    const int nt = min(64, tile_n - wave * 64);
    for (int k = 0; k < nt; ++k) {
      const int t = tile + wave * 64 + k;
      const float *pk = p_s + (wave * 64 + k) * GP;
      float v0 = 0.0f, v1 = 0.0f;
      if (VT == 1) {
        const uint16_t *vr = static_cast<const uint16_t *>(p.v) + vbase + (int64_t)t * d;
        if (dim0) v0 = h2f(vr[lane]);
        if (dim1) v1 = h2f(vr[lane + 64]);
      } else {
        const float *vr = static_cast<const float *>(p.v) + vbase + (int64_t)t * d;
        if (dim0) v0 = vr[lane];
        if (dim1) v1 = vr[lane + 64];
      }
#pragma unroll
      for (int g = 0; g < GP; ++g) {
        o0[g] = __builtin_fmaf(pk[g], v0, o0[g]);
        o1[g] = __builtin_fmaf(pk[g], v1, o1[g]);
      }
    }
    __syncthreads();
  }

  // Merge the four waves, then write the split's partial (or the output).
#pragma unroll
  for (int g = 0; g < GP; ++g) {
    float *c = comb + (wave * GP + g) * (d + 2);
    if (lane == 0) {
      c[0] = m_run[g];
      c[1] = l_run[g];
    }
    if (dim0) c[2 + lane] = o0[g];
    if (dim1) c[2 + lane + 64] = o1[g];
  }
  __syncthreads();
  for (int e = tid; e < G * d; e += kThreads) {
    const int g = e / d, dm = e - g * d;
    float M = -INFINITY;
    for (int w = 0; w < 4; ++w) M = fmaxf(M, comb[(w * GP + g) * (d + 2)]);
    float Lsum = 0.0f, O = 0.0f;
    if (M != -INFINITY) {
      for (int w = 0; w < 4; ++w) {
        const float *c = comb + (w * GP + g) * (d + 2);
        if (c[0] == -INFINITY) continue;
        const float wgt = expf(c[0] - M);
        Lsum = __builtin_fmaf(c[1], wgt, Lsum);
        O = __builtin_fmaf(c[2 + dm], wgt, O);
      }
    }
    const int64_t head = (int64_t)b * Hq + hq0 + g;
    if (p.splits == 1) {
      p.out[head * d + dm] = O / Lsum;
      if (dm == 0 && p.stats) {
        p.stats[head * 2] = M;
        p.stats[head * 2 + 1] = Lsum;
      }
    } else {
      float *pp = p.part + (head * p.splits + split) * (d + 2);
      pp[2 + dm] = O;
      if (dm == 0) {
        pp[0] = M;
        pp[1] = Lsum;
      }
    }
  }
}

// LSE merge of the split partials: one workgroup per query head, one thread per dim.
__global__ void combine_kernel(DecodeParams p) {
  const int64_t head = blockIdx.x;
  const int dm = threadIdx.x, d = p.dim, S = p.splits;
  const float *pp = p.part + head * S * (d + 2);
  float M = -INFINITY;
  for (int s = 0; s < S; ++s) M = fmaxf(M, pp[s * (d + 2)]);
  float Lsum = 0.0f, O = 0.0f;
  for (int s = 0; s < S; ++s) {
    const float m = pp[s * (d + 2)];
    if (m == -INFINITY) continue;
    const float w = expf(m - M);
    Lsum = __builtin_fmaf(pp[s * (d + 2) + 1], w, Lsum);
    if (dm < d) O = __builtin_fmaf(pp[s * (d + 2) + 2 + dm], w, O);
  }
  if (dm < d) p.out[head * d + dm] = O / Lsum;
  if (dm == 0 && p.stats) {
    p.stats[head * 2] = M;
    p.stats[head * 2 + 1] = Lsum;
  }
}

// Materialised probabilities for inspect(): exp(logit - M)/L (0 where masked).
__global__ void probs_kernel(DecodeParams p) {
  const int64_t head = blockIdx.y;
  const int b = (int)(head / p.q_heads);
  const int T_b = (int)min(p.lengths[b], (uint32_t)p.max_length);
  const float M = p.stats[head * 2], Lsum = p.stats[head * 2 + 1];
  for (int t = blockIdx.x * blockDim.x + threadIdx.x; t < T_b; t += gridDim.x * blockDim.x) {
    const float lg = p.logits[head * p.logit_stride + t];
    p.probs[head * p.logit_stride + t] = lg == -INFINITY ? 0.0f : expf(lg - M) / Lsum;
  }
}

template <int GP>
hipError_t launch_gp(const DecodeParams &p, int lds_bytes, hipStream_t stream) {
  dim3 grid((unsigned)p.splits, (unsigned)(p.batch * p.kv_heads));
  const int kf = p.key_format, vt = p.v_dtype;
  if (kf == 1 && vt == 1) hipLaunchKernelGGL((decode_split_kernel<GP, 1, 1>), grid, dim3(kThreads), lds_bytes, stream, p);
  else if (kf == 1 && vt == 0) hipLaunchKernelGGL((decode_split_kernel<GP, 1, 0>), grid, dim3(kThreads), lds_bytes, stream, p);
  else if (kf == 0 && vt == 1) hipLaunchKernelGGL((decode_split_kernel<GP, 0, 1>), grid, dim3(kThreads), lds_bytes, stream, p);
  else if (kf == 0 && vt == 0) hipLaunchKernelGGL((decode_split_kernel<GP, 0, 0>), grid, dim3(kThreads), lds_bytes, stream, p);
  else if (kf == 2 && vt == 1) hipLaunchKernelGGL((decode_split_kernel<GP, 2, 1>), grid, dim3(kThreads), lds_bytes, stream, p);
  else hipLaunchKernelGGL((decode_split_kernel<GP, 2, 0>), grid, dim3(kThreads), lds_bytes, stream, p);
  return hipGetLastError();
}

}  // namespace

int decode_lds_bytes(int G, int dim, int key_format, int books_bytes, int row_bytes, int norm_stride) {
  const int GP = G <= 1 ? 1 : G <= 2 ? 2 : G <= 4 ? 4 : G <= 8 ? 8 : 16;
  return lds_layout(GP, dim, key_format, books_bytes, row_bytes, norm_stride).total;
}

hipError_t launch_rotate_q(const DecodeParams &p, const float *q, float *qr, hipStream_t stream) {
  const float inv = (float)(1.0 / __builtin_sqrt((double)p.dim));
  hipLaunchKernelGGL(rotate_q_kernel, dim3((unsigned)(p.batch * p.q_heads)), dim3(128), 0, stream, p, q, qr, inv);
  return hipGetLastError();
}

hipError_t launch_decode_probs(const DecodeParams &p, hipStream_t stream) {
  hipLaunchKernelGGL(probs_kernel, dim3(16, (unsigned)(p.batch * p.q_heads)), dim3(256), 0, stream, p);
  return hipGetLastError();
}

hipError_t launch_decode_tail(const DecodeParams &p, hipStream_t stream) {
  hipError_t e = hipSuccess;
  if (p.splits > 1) {
    hipLaunchKernelGGL(combine_kernel, dim3((unsigned)(p.batch * p.q_heads)), dim3(128), 0, stream, p);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  if (p.probs) {
    hipLaunchKernelGGL(probs_kernel, dim3(16, (unsigned)(p.batch * p.q_heads)), dim3(256), 0, stream, p);
    e = hipGetLastError();
  }
  return e;
}

hipError_t launch_decode(const DecodeParams &p, int lds_bytes, hipStream_t stream) {
  hipError_t e;
  const int G = p.G;
  if (G <= 1) e = launch_gp<1>(p, lds_bytes, stream);
  else if (G <= 2) e = launch_gp<2>(p, lds_bytes, stream);
  else if (G <= 4) e = launch_gp<4>(p, lds_bytes, stream);
  else if (G <= 8) e = launch_gp<8>(p, lds_bytes, stream);
  else e = launch_gp<16>(p, lds_bytes, stream);
  if (e != hipSuccess) return e;
  return launch_decode_tail(p, stream);
}

}  // namespace bgtq
