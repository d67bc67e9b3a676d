// Bulk Block-GTQ K encode for gfx950: one thread per K row, for layouts whose
// NG groups are equal, contiguous runs of the head-perm order and whose codes
// are nibbles below NS and bytes from NS on (layout B: two groups of d/2,
// nibbles first). Bit-exact with the reference encoder
// (src/reference/production_math.py:4-24) under the same contract as
// encode.hip, with the layout's structure known at compile time:
//  * the FP32 sums of production_math.py:12, :14 and :23 follow ATen's 8-lane
//    inner-sum tree; a group's leaves are the only nonzero ones, and the
//    never-negative accumulators make the skipped zero leaves exact no-ops, so
//    each sum is a fixed sequence of adds over the group's positions;
//  * y_j = sum_i xn_i R[j][i] (production_math.py:16) is one FMA chain over
//    the group of j in ascending i from +0, the order of the CPU sgemm (the
//    off-group rotation entries are exact zeros); the rotation rows are
//    wave-uniform operands read through the scalar cache;
//  * division and square root are IEEE (built with -ffp-contract=off and
//    correctly rounded fp32 division/sqrt).
// The code LUT and centroid books sit in LDS; codes are packed in registers
// as they are produced (mixed_layout.py:21-27) and each thread writes its own
// packed row and FP16 scales.
#include <hip/hip_fp16.h>

#include <type_traits>

#include "bgtq_internal.h"

namespace bgtq {
namespace {

__device__ __forceinline__ float f16_bits_to_f32(uint16_t h) { return __half2float(__ushort_as_half(h)); }
__device__ __forceinline__ uint16_t f32_to_f16_bits(float v) { return __half_as_ushort(__float2half_rn(v)); }

// f(std::integral_constant<int, I>) for I = B .. E-1, in order.
template <int B, int E, typename F>
__device__ __forceinline__ void static_for(F &&f) {
  if constexpr (B < E) {
    f(std::integral_constant<int, B>{});
    static_for<B + 1, E>(f);
  }
}

template <int D, int WG>
struct Bulk {
  static constexpr int ROWS = WG;     // rows (threads) per workgroup
  static constexpr int SSTR = D + 2;  // staged halfs per row: odd dword stride
  static constexpr int STAGE = ROWS * SSTR * 2;
};

// ATen's 8-lane inner sum (vectorized_inner_sum: four interleaved
// accumulators over the 8-wide vectors, tail vectors to the first, then
// ((a0 + a1) + a2) + a3 per lane and the 8 lanes in order) of leaves that are
// zero outside the positions [P0, P1); leaf(p) is called with constant p.
template <int D, int P0, int P1, typename F>
__device__ __forceinline__ float tree_sum(F &&leaf) {
  constexpr int NV = D / 8, SI = NV / 4, V0 = P0 / 8, V1 = P1 / 8;
  static_assert(P0 % 8 == 0 && P1 % 8 == 0, "groups cover whole 8-wide vectors");
  float total = 0.0f;
#pragma unroll
  for (int l = 0; l < 8; ++l) {
    float a[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    bool set[4] = {false, false, false, false};
#pragma unroll
    for (int v = V0; v < V1; ++v) {
      const int k = v < SI * 4 ? v % 4 : 0;
      const float x = leaf(v * 8 + l);
      a[k] = set[k] ? a[k] + x : x;
      set[k] = true;
    }
    float t = 0.0f;
    bool tset = false;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      if (!set[k]) continue;
      t = tset ? t + a[k] : a[k];
      tset = true;
    }
    total = l == 0 ? t : total + t;
  }
  return total;
}

template <int D, int NG, int NS, bool SRC_F32, int WG>
__global__ __launch_bounds__(WG) void encode_bulk_kernel(EncodeLaunch launch, int lut_area) {
  constexpr int ROWS = Bulk<D, WG>::ROWS, SSTR = Bulk<D, WG>::SSTR, GW = D / NG;
  constexpr int LOGICAL = NS / 2 + D - NS;  // packed bytes before padding
  static_assert(GW % 8 == 0 && NS % 8 == 0 && NS <= D && LOGICAL % 4 == 0, "layout");
  extern __shared__ __align__(16) uint8_t smem[];
  uint16_t *stage = reinterpret_cast<uint16_t *>(smem);
  uint8_t *lut = smem + Bulk<D, WG>::STAGE;
  float *books = reinterpret_cast<float *>(lut + lut_area);

  const EncodeJobDev job = launch.jobs[blockIdx.y];
  const int64_t row0 = (int64_t)blockIdx.x * ROWS;
  if (row0 >= job.rows) return;  // uniform for the workgroup
  const int nr = (int)min((int64_t)ROWS, job.rows - row0);
  const DevTables *__restrict__ T = job.t;
  const int tid = threadIdx.x;
  const int mc = T->max_centroids;

  // Stage the rows (FP16 bits; FP32 sources rounded to FP16 first,
  // src/model/codec.wgsl:14), the code LUT and the centroid books.
  for (int e = tid; e < nr * D; e += ROWS) {
    const int r = e / D, c = e - r * D;
    const int64_t at = (row0 + r) * job.src_stride + c;
    stage[r * SSTR + c] = SRC_F32 ? f32_to_f16_bits(static_cast<const float *>(job.src)[at])
                                  : static_cast<const uint16_t *>(job.src)[at];
  }
  {
    const uint8_t *lut_g = tables_lut(T);
    const int lut_bytes = T->n_codebooks * 256;
    for (int e = tid; e < lut_bytes; e += ROWS) lut[e] = lut_g[e];
    const float *books_g = tables_books(T);
    const int nbf = T->n_books * mc;
    for (int e = tid; e < nbf; e += ROWS) books[e] = books_g[e];
  }
  __syncthreads();
  if (tid >= nr) return;  // no barrier below

  float x[D];
#pragma unroll
  for (int i = 0; i < D; ++i) x[i] = f16_bits_to_f32(stage[tid * SSTR + T->perm[i]]);

  const float *__restrict__ R = tables_rot(T);
  uint32_t packed[LOGICAL / 4];
#pragma unroll
  for (int w = 0; w < LOGICAL / 4; ++w) packed[w] = 0u;
  uint16_t scales[NG];

  static_for<0, NG>([&](auto gc) {
    constexpr int g = decltype(gc)::value, P0 = g * GW, P1 = P0 + GW;
    // production_math.py:12-15: n_g, raw_g, x / where(n > 1e-10, n, 1)
    const float n = __builtin_sqrtf(tree_sum<D, P0, P1>([&](int p) { return x[p] * x[p]; }) + 1e-30f);
    const float raw = NG > 1 ? tree_sum<D, P0, P1>([&](int) { return n; }) / (float)GW : n;
    const float den = n > 1e-10f ? n : 1.0f;
#pragma unroll
    for (int i = P0; i < P1; ++i) x[i] = x[i] / den;
    // production_math.py:16-20 per output j of the group: FMA chain, bin,
    // LUT code, centroid; codes packed as produced.
    float c2[GW];
#pragma unroll
    for (int j = P0; j < P1; ++j) {
      const float *__restrict__ Rj = R + j * D;
      float acc = 0.0f;
#pragma unroll
      for (int i = P0; i < P1; ++i) acc = __builtin_fmaf(x[i], Rj[i], acc);
      float t = (acc - T->lut_off[j]) * T->lut_inv[j];
      t = fminf(fmaxf(t, 0.0f), 255.0f);
      const uint32_t code = lut[(int)T->pos_cb[j] * 256 + (int)t];
      const float c = books[(int)T->pos_book[j] * mc + (int)code];
      c2[j - P0] = c * c;
      const int byte = j < NS ? j / 2 : NS / 2 + (j - NS);
      const int shift = 8 * (byte % 4) + (j < NS ? 4 * (j % 2) : 0);
      packed[byte / 4] |= code << shift;
    }
    // production_math.py:21-23: corrected_g = raw_g / max(sqrt(sum c^2), 1e-10)
    const float cn = fmaxf(__builtin_sqrtf(tree_sum<D, P0, P1>([&](int p) { return c2[p - P0]; })), 1e-10f);
    scales[g] = f32_to_f16_bits(raw / cn);
  });

  // mixed_layout.py:21-27: every byte of the destination row written (zero
  // padding after the codes); FP16 scales zero-padded to norm_stride.
  const int64_t out_row = job.dst_row0 + (row0 + tid) * job.dst_step;
  const int RB = T->row_bytes, NSTR = T->norm_stride;
  uint32_t *prow = reinterpret_cast<uint32_t *>(job.packed + out_row * RB);
#pragma unroll
  for (int w = 0; w < LOGICAL / 4; ++w) prow[w] = packed[w];
  for (int w = LOGICAL / 4; w < RB / 4; ++w) prow[w] = 0u;
  uint16_t *nrow = job.norms + out_row * NSTR;
#pragma unroll
  for (int g = 0; g < NG; ++g) nrow[g] = scales[g];
  for (int g = NG; g < NSTR; ++g) nrow[g] = 0;
}

template <int D, int NG, int NS, int WG>
hipError_t launch_kind(const EncodeLaunch &launch, int src_f32, int64_t max_rows, int lut_area, int book_floats,
                       hipStream_t stream) {
  const int lds = Bulk<D, WG>::STAGE + lut_area + book_floats * 4;
  dim3 grid((unsigned)((max_rows + WG - 1) / WG), (unsigned)launch.n_jobs);
  if (src_f32)
    hipLaunchKernelGGL((encode_bulk_kernel<D, NG, NS, true, WG>), grid, dim3(WG), lds, stream, launch, lut_area);
  else
    hipLaunchKernelGGL((encode_bulk_kernel<D, NG, NS, false, WG>), grid, dim3(WG), lds, stream, launch, lut_area);
  return hipGetLastError();
}

}  // namespace

int encode_bulk_kind(const DevTables *T) {
  const int d = T->dim, ng = T->groups;
  if ((d != 64 && d != 128) || ng != 2 || T->nibble_dims != d / 2) return 0;
  if (T->gstart[0] != 0 || T->gend[0] != d / 2 || T->gstart[1] != d / 2 || T->gend[1] != d) return 0;
  if (T->row_bytes % 4 || T->row_bytes < d / 4 + d / 2) return 0;
  return d == 64 ? 1 : 2;
}

int encode_bulk_lds_bytes(int kind, int wg, int lut_bytes, int book_floats) {
  const int d = kind == 1 ? 64 : 128;
  return wg * (d + 2) * 2 + ((lut_bytes + 15) & ~15) + book_floats * 4;
}

hipError_t launch_encode_bulk(const EncodeLaunch &launch, int kind, int wg, int src_f32, int64_t max_rows,
                              int lut_bytes, int book_floats, hipStream_t stream) {
  const int lut_area = (lut_bytes + 15) & ~15;
#define BGTQ_BULK(K, DD, NS, W) \
  if (kind == K && wg == W) return launch_kind<DD, 2, NS, W>(launch, src_f32, max_rows, lut_area, book_floats, stream);
  BGTQ_BULK(1, 64, 32, 256)
  BGTQ_BULK(2, 128, 64, 128)
#undef BGTQ_BULK
  return hipErrorInvalidValue;
}

}  // namespace bgtq
