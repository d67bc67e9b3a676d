// Decode attention on the matrix cores of gfx950 (v_mfma_f32_16x16x32_f16).
//
// Same contract as decode.hip (one workgroup per (sequence, KV head, token
// split), (m, l, o) partials merged by LSE), for FP16 V and either FP16 K rows
// or packed K in a layout whose 32-dim K-steps each hold one group (FastLayout).
//
// Per wave and chunk of 32 tokens:
//   QK  D[t][h] = sum_k K[t][k] Qr[k][h] as two 16-token tiles. The A operand
//       is rebuilt from the packed codes: lane (token t = lane%16, dims
//       8*(lane/16)..+7 of a K-step) unpacks its 8 codes and gathers
//       c*2^e as an exact fp16 (hi, lo) pair from an LDS table, so
//       K = hi + lo to ~2^-22. Qr is split the same way; three MFMAs
//       (hi*hi + lo*hi + hi*lo) per K-step give FP32-level logits. The group
//       scale s_g(t) and the power-of-two factors are applied to the FP32
//       accumulator: logit = sum_g s_g(t) * D_g * 2^-(eq+ec).
//   softmax: each lane holds 4 tokens x 1 head per tile; the per-head max over
//       the chunk needs two cross-lane steps (permlane16/32 swaps).
//   PV  O[h][d] += sum_t P[h][t] V[t][d]. P (scaled by 2^15, split hi/lo) is
//       already in A-operand order: lane (head, group g) owns tokens
//       {4g..4g+3} of tile 0 and {16+4g..} of tile 1, which is the K index
//       order used for both operands. V is staged row-major in a padded LDS
//       tile and read transposed (8 x 16-bit per lane per dim tile).
#include <hip/hip_fp16.h>

#include "bgtq_internal.h"

namespace bgtq {
namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kWaves = 4;
constexpr int kChunk = 32;
constexpr float kLog2e = 1.4426950408889634f;

template <int D>
struct Geo {
  static constexpr int KS = D / 32;   // K-steps of the QK contraction
  static constexpr int DT = D / 16;   // 16-dim tiles of the PV output
  static constexpr int VSTR = D + 4;  // halfs per staged V row: rows 4 apart land 8 banks apart
};

__device__ __forceinline__ float pair_max(float v) {
  auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ __forceinline__ float pair_sum(float v) {
  auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

__device__ __forceinline__ uint32_t split_pair(float x) {
  // x = hi + lo exactly to ~2^-22 relative (both fp16, packed lo16 = hi, hi16 = lo)
  const _Float16 hi = (_Float16)x;
  const _Float16 lo = (_Float16)(x - (float)hi);
  return (uint32_t)__builtin_bit_cast(uint16_t, hi) | ((uint32_t)__builtin_bit_cast(uint16_t, lo) << 16);
}

__device__ __forceinline__ half8 gather_lo(const uint32_t (&e)[8]) {
  u32x4 r;
#pragma unroll
  for (int k = 0; k < 4; ++k) r[k] = __builtin_amdgcn_perm(e[2 * k + 1], e[2 * k], 0x05040100u);
  return __builtin_bit_cast(half8, r);
}
__device__ __forceinline__ half8 gather_hi(const uint32_t (&e)[8]) {
  u32x4 r;
#pragma unroll
  for (int k = 0; k < 4; ++k) r[k] = __builtin_amdgcn_perm(e[2 * k + 1], e[2 * k], 0x07060302u);
  return __builtin_bit_cast(half8, r);
}

__device__ __forceinline__ f32x4 mfma(half8 a, half8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

template <int D, int KF>
__global__ __launch_bounds__(256) void decode_mfma_kernel(DecodeParams p, FastLayout fl) {
  using G_ = Geo<D>;
  constexpr int KS = G_::KS, DT = G_::DT, VSTR = G_::VSTR;
  extern __shared__ __align__(16) uint8_t smem[];
  const int unit = blockIdx.y, split = blockIdx.x;
  const int b = unit / p.kv_heads, kv = unit - b * p.kv_heads;
  const int G = p.G, Hq = p.q_heads, hq0 = kv * G;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int gq = lane >> 4, col = lane & 15;
  const int T_b = (int)p.lengths[b];
  const int t_begin = split * p.split_tokens;
  const int t_end = min(T_b, t_begin + p.split_tokens);

  // LDS: [V tiles of the 4 waves | centroid (hi,lo) table]; the wave merge at
  // the end reuses the V region.
  _Float16 *v_all = reinterpret_cast<_Float16 *>(smem);
  _Float16 *v_s = v_all + wave * kChunk * VSTR;
  uint32_t *book_s = reinterpret_cast<uint32_t *>(smem + kWaves * kChunk * VSTR * 2);

  const DevTables *T = KF == 1 ? p.tables[kv] : nullptr;
  int ec = 0, mc = 0;
  if (KF == 1) {
    ec = T->cent_exp;
    mc = T->max_centroids;
    const float *books = tables_books(T);
    const float sc = __builtin_ldexpf(1.0f, ec);
    for (int e = tid; e < T->n_books * mc; e += 256) book_s[e] = split_pair(books[e] * sc);
  }

  // Query operand (B of QK): lane holds Qr[head = col][32 s + 8 gq + j].
  const bool head_ok = col < G;
  const float *qrow = p.qr + ((int64_t)b * Hq + hq0 + (head_ok ? col : 0)) * D;
  float qv[KS][8];
  float qmax = 0.0f;
#pragma unroll
  for (int s = 0; s < KS; ++s)
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      qv[s][j] = head_ok ? qrow[32 * s + 8 * gq + j] : 0.0f;
      qmax = fmaxf(qmax, fabsf(qv[s][j]));
    }
  qmax = pair_max(qmax);
  const int eq = qmax > 0.0f ? 14 - (int)ceilf(__builtin_log2f(qmax)) : 0;
  const float qsc = __builtin_ldexpf(1.0f, eq);
  half8 qhi[KS], qlo[KS];
#pragma unroll
  for (int s = 0; s < KS; ++s)
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float x = qv[s][j] * qsc;
      qhi[s][j] = (_Float16)x;
      qlo[s][j] = (_Float16)(x - (float)qhi[s][j]);
    }
  const float unscale = __builtin_ldexpf(1.0f, -(eq + ec));
  const int end_h = head_ok ? (p.ends ? min(p.ends[(int64_t)b * Hq + hq0 + col], T_b) : T_b) : 0;
  const int lim = min(end_h, t_end);

  const uint8_t *packed = KF == 1 ? p.packed + b * p.packed_seq_stride + kv * p.packed_head_stride : nullptr;
  const uint16_t *norms = KF == 1 ? p.norms + b * p.norms_seq_stride + kv * p.norms_head_stride : nullptr;
  const _Float16 *kf16 = KF == 0 ? static_cast<const _Float16 *>(p.k) + b * p.k_seq_stride + kv * p.k_head_stride
                                 : nullptr;
  const _Float16 *vbase = static_cast<const _Float16 *>(p.v) + b * p.v_seq_stride + kv * p.v_head_stride;
  const int RB = KF == 1 ? T->row_bytes : 0;
  int book_base[KS];
#pragma unroll
  for (int s = 0; s < KS; ++s) book_base[s] = KF == 1 ? fl.book[s] * mc : 0;

  float m_run = -INFINITY, l_run = 0.0f;
  f32x4 O[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) O[dt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  __syncthreads();

  for (int c0 = t_begin + wave * kChunk; c0 < t_end; c0 += kWaves * kChunk) {
    const bool tail = c0 + kChunk > t_end;
    // ---- V chunk -> LDS (rows clamped to the last valid token) ----
    {
      constexpr int PIECES = kChunk * D * 2 / 16 / 64;  // 16-byte pieces per lane
#pragma unroll
      for (int k = 0; k < PIECES; ++k) {
        const int off = (k * 64 + lane) * 16;  // byte offset within the chunk
        const int tok = off / (2 * D), inrow = off - tok * 2 * D;
        const int src_tok = min(c0 + tok, t_end - 1);
        const u32x4 x = *reinterpret_cast<const u32x4 *>(
            reinterpret_cast<const uint8_t *>(vbase + (int64_t)src_tok * D) + inrow);
        uint8_t *dst = reinterpret_cast<uint8_t *>(v_s + tok * VSTR) + inrow;
        *reinterpret_cast<u32x2 *>(dst) = u32x2{x[0], x[1]};
        *reinterpret_cast<u32x2 *>(dst + 8) = u32x2{x[2], x[3]};
      }
    }
    // ---- QK: two 16-token tiles ----
    f32x4 acc[2][KS];
    float sc[2][4][KS];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int t = min(c0 + 16 * u + col, t_end - 1);  // A-operand row of this lane
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        acc[u][s] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        if (KF == 1) {
          const uint8_t *row = packed + (int64_t)t * RB + fl.byte_off[s];
          uint32_t e[8];
          if (fl.nib[s]) {
            const uint32_t w = *reinterpret_cast<const uint32_t *>(row + 4 * gq);
#pragma unroll
            for (int j = 0; j < 8; ++j) e[j] = book_s[book_base[s] + ((w >> (4 * j)) & 15u)];
          } else {
            const u32x2 w = *reinterpret_cast<const u32x2 *>(row + 8 * gq);
#pragma unroll
            for (int j = 0; j < 8; ++j) e[j] = book_s[book_base[s] + ((w[j >> 2] >> (8 * (j & 3))) & 255u)];
          }
          const half8 ahi = gather_lo(e), alo = gather_hi(e);
          acc[u][s] = mfma(ahi, qhi[s], acc[u][s]);
          acc[u][s] = mfma(alo, qhi[s], acc[u][s]);
          acc[u][s] = mfma(ahi, qlo[s], acc[u][s]);
        } else {
          const half8 a = *reinterpret_cast<const half8 *>(kf16 + (int64_t)t * D + 32 * s + 8 * gq);
          acc[u][s] = mfma(a, qhi[s], acc[u][s]);
          acc[u][s] = mfma(a, qlo[s], acc[u][s]);
        }
      }
      if (KF == 1) {
        // FP16 scales of this lane's output rows: tokens c0 + 16u + 4gq + i, groups 0/1.
        const int t0 = c0 + 16 * u + 4 * gq;
        uint32_t w4[4];
        if (!tail) {
          const u32x4 w = *reinterpret_cast<const u32x4 *>(norms + (int64_t)t0 * 2);
#pragma unroll
          for (int i = 0; i < 4; ++i) w4[i] = w[i];
        } else {
#pragma unroll
          for (int i = 0; i < 4; ++i)
            w4[i] = *reinterpret_cast<const uint32_t *>(norms + (int64_t)min(t0 + i, t_end - 1) * 2);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int s = 0; s < KS; ++s) {
            const uint16_t h = fl.group[s] == 0 ? (uint16_t)(w4[i] & 0xffffu) : (uint16_t)(w4[i] >> 16);
            sc[u][i][s] = __half2float(__ushort_as_half(h));
          }
      }
    }
    // ---- logits and online softmax (lane: head col, tokens 4gq+i of each tile) ----
    float lg[2][4];
    float mloc = -INFINITY;
#pragma unroll
    for (int u = 0; u < 2; ++u)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float x = 0.0f;
#pragma unroll
        for (int s = 0; s < KS; ++s) x = __builtin_fmaf(KF == 1 ? sc[u][i][s] : 1.0f, acc[u][s][i], x);
        x *= unscale;
        const int tok = c0 + 16 * u + 4 * gq + i;
        if (tail || lim < t_end) x = tok < lim ? x : -INFINITY;
        if (p.logits && head_ok && tok < t_end)
          p.logits[((int64_t)b * Hq + hq0 + col) * p.logit_stride + tok] = x;
        lg[u][i] = x;
        mloc = fmaxf(mloc, x);
      }
    const float m_new = fmaxf(m_run, pair_max(mloc));
    const float alpha = m_new == -INFINITY ? 1.0f : exp2f((m_run - m_new) * kLog2e);
    const float mb = m_new == -INFINITY ? 0.0f : m_new * kLog2e;
    uint32_t ph[4], pl[4];
    float psum = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; j += 2) {
      float pr[2];
#pragma unroll
      for (int k = 0; k < 2; ++k) {
        const int jj = j + k;
        const float x = jj < 4 ? lg[0][jj] : lg[1][jj - 4];
        pr[k] = x == -INFINITY ? 0.0f : exp2f(__builtin_fmaf(x, kLog2e, -mb) + 15.0f);
        psum += pr[k];
      }
      const uint32_t a0 = split_pair(pr[0]), a1 = split_pair(pr[1]);
      ph[j / 2] = __builtin_amdgcn_perm(a1, a0, 0x05040100u);
      pl[j / 2] = __builtin_amdgcn_perm(a1, a0, 0x07060302u);
    }
    l_run = __builtin_fmaf(l_run, alpha, psum);
    m_run = m_new;
    if (__builtin_amdgcn_ballot_w64(alpha != 1.0f)) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float ai = __shfl(alpha, 4 * gq + i, 64);
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) O[dt][i] *= ai;
      }
    }
    // ---- PV ----
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const half8 pha = __builtin_bit_cast(half8, u32x4{ph[0], ph[1], ph[2], ph[3]});
    const half8 pla = __builtin_bit_cast(half8, u32x4{pl[0], pl[1], pl[2], pl[3]});
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
      half8 vb;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int tok = j < 4 ? 4 * gq + j : 16 + 4 * gq + (j - 4);
        vb[j] = v_s[tok * VSTR + 16 * dt + col];
      }
      O[dt] = mfma(pha, vb, O[dt]);
      O[dt] = mfma(pla, vb, O[dt]);
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  }

  // ---- merge the four waves (reusing the V region) ----
  const float l_tot = pair_sum(l_run) * (1.0f / 32768.0f);
  __syncthreads();
  float *comb = reinterpret_cast<float *>(smem);  // [wave][16 heads][D + 2]
  if (gq == 0) {
    comb[(wave * 16 + col) * (D + 2)] = m_run;
    comb[(wave * 16 + col) * (D + 2) + 1] = l_tot;
  }
#pragma unroll
  for (int dt = 0; dt < DT; ++dt)
#pragma unroll
    for (int i = 0; i < 4; ++i) comb[(wave * 16 + 4 * gq + i) * (D + 2) + 2 + 16 * dt + col] = O[dt][i] * (1.0f / 32768.0f);
  __syncthreads();
  for (int e = tid; e < G * D; e += 256) {
    const int g = e / D, dm = e - g * D;
    float M = -INFINITY;
    for (int w = 0; w < kWaves; ++w) M = fmaxf(M, comb[(w * 16 + g) * (D + 2)]);
    float Lsum = 0.0f, Ov = 0.0f;
    if (M != -INFINITY) {
      for (int w = 0; w < kWaves; ++w) {
        const float *c = comb + (w * 16 + g) * (D + 2);
        if (c[0] == -INFINITY) continue;
        const float wgt = exp2f((c[0] - M) * kLog2e);
        Lsum = __builtin_fmaf(c[1], wgt, Lsum);
        Ov = __builtin_fmaf(c[2 + dm], wgt, Ov);
      }
    }
    const int64_t head = (int64_t)b * Hq + hq0 + g;
    if (p.splits == 1) {
      p.out[head * D + dm] = Ov / Lsum;
      if (dm == 0 && p.stats) {
        p.stats[head * 2] = M;
        p.stats[head * 2 + 1] = Lsum;
      }
    } else {
      float *pp = p.part + (head * p.splits + split) * (D + 2);
      pp[2 + dm] = Ov;
      if (dm == 0) {
        pp[0] = M;
        pp[1] = Lsum;
      }
    }
  }
}

}  // namespace

int decode_mfma_lds_bytes(int dim, int key_format, int books_bytes) {
  const int vbytes = kWaves * kChunk * (dim + 4) * 2;
  const int comb = kWaves * 16 * (dim + 2) * 4;
  return (vbytes > comb ? vbytes : comb) + (key_format == 1 ? books_bytes : 0);
}

hipError_t launch_decode_mfma(const DecodeParams &p, const FastLayout &fl, hipStream_t stream) {
  dim3 grid((unsigned)p.splits, (unsigned)(p.batch * p.kv_heads));
  if (p.dim == 64 && p.key_format == 1)
    hipLaunchKernelGGL((decode_mfma_kernel<64, 1>), grid, dim3(256), p.lds_bytes, stream, p, fl);
  else if (p.dim == 64)
    hipLaunchKernelGGL((decode_mfma_kernel<64, 0>), grid, dim3(256), p.lds_bytes, stream, p, fl);
  else if (p.key_format == 1)
    hipLaunchKernelGGL((decode_mfma_kernel<128, 1>), grid, dim3(256), p.lds_bytes, stream, p, fl);
  else
    hipLaunchKernelGGL((decode_mfma_kernel<128, 0>), grid, dim3(256), p.lds_bytes, stream, p, fl);
  return hipGetLastError();
}

}  // namespace bgtq
