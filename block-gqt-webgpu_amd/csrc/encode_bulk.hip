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
//    off-group rotation entries are exact zeros); the group's chains advance
//    together, column i of R (a row of the stored transpose) a wave-uniform
//    operand read through the scalar cache;
//  * division and square root are IEEE (built with -ffp-contract=off and
//    correctly rounded fp32 division/sqrt); a group's 32 divisions by its
//    norm use its correctly rounded reciprocal and one FMA correction each,
//    which gives the same quotients.
// The code LUT and centroid books sit in LDS; codes are packed in registers
// as they are produced (mixed_layout.py:21-27) and each thread writes its own
// packed row and FP16 scales.
#include <hip/hip_fp16.h>

#include <type_traits>

#include "bgtq_internal.h"
#include "gfx950_common.h"

namespace bgtq {
namespace {

using gfx::dma16;
using gfx::dma4;
using gfx::f32x4;
using gfx::rsrc;
using gfx::u32x4;
using gfx::wait_vm;

// The job table and the table sets are not written while the kernel runs:
// read through the constant address space, their wave-uniform fields are
// scalar loads whatever the kernel's other memory operations are.
#define BGTQ_CONST __attribute__((address_space(4)))
template <typename X>
__device__ __forceinline__ const BGTQ_CONST X *to_const(const void *p) {
  return (const BGTQ_CONST X *)reinterpret_cast<uintptr_t>(p);
}

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
  // d <= 64: the two diagonal rotation blocks in LDS (8 KB); at d=128 (32 KB)
  // the columns are read through the scalar cache instead.
  static constexpr bool ROT_LDS = D <= 64;
  static constexpr int ROT = ROT_LDS ? 2 * (D / 2) * (D / 2) * 4 : 0;
  // The LUT and book areas are whole 256-byte pieces (the LDS DMA's unit).
  static constexpr int lut_area(int lut_bytes) { return (lut_bytes + 255) & ~255; }
  static constexpr int book_area(int book_floats) { return ((book_floats + 63) & ~63) * 4; }
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
__global__ __launch_bounds__(WG) void encode_bulk_kernel(const EncodeJobDev *__restrict__ jobs, int lut_area,
                                                         int book_floats) {
  constexpr int ROWS = Bulk<D, WG>::ROWS, SSTR = Bulk<D, WG>::SSTR, GW = D / NG;
  constexpr int LOGICAL = NS / 2 + D - NS;  // packed bytes before padding
  static_assert(GW % 8 == 0 && NS % 8 == 0 && NS <= D && LOGICAL % 4 == 0, "layout");
  extern __shared__ __align__(16) uint8_t smem[];
  uint16_t *stage = reinterpret_cast<uint16_t *>(smem);
  uint8_t *lut = smem + Bulk<D, WG>::STAGE;
  float *books = reinterpret_cast<float *>(lut + lut_area);
  // The groups' diagonal rotation blocks, rot[g][i][j] = R[P0 + j][P0 + i]
  // (column i of the block contiguous): read as wave-wide broadcasts.
  float *rot = reinterpret_cast<float *>(reinterpret_cast<uint8_t *>(books) + Bulk<D, WG>::book_area(book_floats));

  struct JobWords {
    u32x4 w[4];
  };
  static_assert(sizeof(JobWords) == sizeof(EncodeJobDev), "job words");
  const BGTQ_CONST u32x4 *jw = to_const<u32x4>(jobs + blockIdx.y);
  const EncodeJobDev job = __builtin_bit_cast(EncodeJobDev, (JobWords{{jw[0], jw[1], jw[2], jw[3]}}));
  const int64_t row0 = (int64_t)blockIdx.x * ROWS;
  if (row0 >= job.rows) return;  // uniform for the workgroup
  const int nr = (int)min((int64_t)ROWS, job.rows - row0);
  const BGTQ_CONST DevTables *T = to_const<DevTables>(job.t);
  const int tid = threadIdx.x;
  const int mc = T->max_centroids;

  // Stage the rows (FP16 bits; FP32 sources rounded to FP16 first,
  // src/model/codec.wgsl:14), the code LUT, the centroid books and the
  // rotation blocks, every load of the workgroup in flight at once: the rows
  // as 16-byte pieces into registers (lane-consecutive pieces, coalesced),
  // the tables by LDS DMA; one wait, then the rows' LDS writes.
  constexpr int PR = D / 8;  // 8-element pieces per row
  const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const uintptr_t src_addr = reinterpret_cast<uintptr_t>(job.src);
  const bool vec = src_addr % 16 == 0 && job.src_stride % 8 == 0;  // uniform
  u32x4 piece[PR];
  if (vec) {
#pragma unroll
    for (int k = 0; k < PR; ++k) {
      const int e = tid + ROWS * k, r = e / PR, c = e - r * PR;
      const int64_t at = (row0 + r) * job.src_stride + 8 * c;
      if (r < nr) {
        if constexpr (SRC_F32) {
          const BGTQ_GLOBAL f32x4 *sp = reinterpret_cast<const BGTQ_GLOBAL f32x4 *>(
              to_global(static_cast<const float *>(job.src)) + at);
          const f32x4 a = sp[0], b = sp[1];
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            piece[k][h] = (uint32_t)f32_to_f16_bits(a[2 * h]) | ((uint32_t)f32_to_f16_bits(a[2 * h + 1]) << 16);
            piece[k][2 + h] = (uint32_t)f32_to_f16_bits(b[2 * h]) | ((uint32_t)f32_to_f16_bits(b[2 * h + 1]) << 16);
          }
        } else {
          piece[k] = *reinterpret_cast<const BGTQ_GLOBAL u32x4 *>(to_global(static_cast<const uint16_t *>(job.src)) + at);
        }
      } else {
        piece[k] = u32x4{0u, 0u, 0u, 0u};
      }
    }
  }
  {
    const uint8_t *tb = reinterpret_cast<const uint8_t *>(job.t);
    constexpr int NW = WG / 64;
    const int lut_bytes = T->n_codebooks * 256;
    const __amdgpu_buffer_rsrc_t rl = rsrc(tb + T->off_lut, lut_bytes);
    for (int c = wave; c * 256 < lut_bytes; c += NW) dma4(rl, lut + c * 256, c * 256 + lane * 4, 0);
    const int nbb = T->n_books * mc * 4;  // the LDS area is whole 256-byte pieces
    const __amdgpu_buffer_rsrc_t rb = rsrc(tb + T->off_books, nbb);
    for (int c = wave; c * 256 < nbb; c += NW)
      dma4(rb, reinterpret_cast<uint8_t *>(books) + c * 256, c * 256 + lane * 4, 0);
    if constexpr (Bulk<D, WG>::ROT_LDS) {
      // Eight rows i of block g (GW = 32 floats each) per instruction:
      // lane l brings Rt[(g GW + i0 + l / 8) D + g GW + 4 (l % 8) ...+3].
      static_assert(GW == 32, "eight 128-byte block rows per 16-byte DMA");
      const __amdgpu_buffer_rsrc_t rr = rsrc(tb + T->off_rot_t, D * D * 4);
      for (int c = wave; c < NG * GW / 8; c += NW) {
        const int g = c / (GW / 8), i = 8 * c - g * GW + lane / 8;
        dma16(rr, reinterpret_cast<uint8_t *>(rot) + c * 1024, ((g * GW + i) * D + g * GW + 4 * (lane % 8)) * 4, 0);
      }
    }
  }
  if (vec) {
#pragma unroll
    for (int k = 0; k < PR; ++k) {
      const int e = tid + ROWS * k, r = e / PR, c = e - r * PR;
      uint32_t *dst = reinterpret_cast<uint32_t *>(stage + r * SSTR + 8 * c);  // 4-byte aligned: SSTR even
#pragma unroll
      for (int h = 0; h < 4; ++h) dst[h] = piece[k][h];
    }
  } else {
    for (int e = tid; e < nr * D; e += ROWS) {
      const int r = e / D, c = e - r * D;
      const int64_t at = (row0 + r) * job.src_stride + c;
      stage[r * SSTR + c] = SRC_F32 ? f32_to_f16_bits(to_global(static_cast<const float *>(job.src))[at])
                                    : to_global(static_cast<const uint16_t *>(job.src))[at];
    }
  }
  wait_vm<0>();  // the DMAs
  __syncthreads();
  if (tid >= nr) return;  // no barrier below

  const BGTQ_CONST float *Rt = to_const<float>(reinterpret_cast<const uint8_t *>(job.t) + T->off_rot_t);  // Rt[i * D + j] = R[j][i]
  uint32_t packed[LOGICAL / 4];
#pragma unroll
  for (int w = 0; w < LOGICAL / 4; ++w) packed[w] = 0u;
  uint16_t scales[NG];

  static_for<0, NG>([&](auto gc) {
    constexpr int g = decltype(gc)::value, P0 = g * GW, P1 = P0 + GW;
    // This group's inputs in head-perm order (the other groups' stay in LDS).
    float x[GW];
#pragma unroll
    for (int i = 0; i < GW; ++i) x[i] = f16_bits_to_f32(stage[tid * SSTR + T->perm[P0 + i]]);
    // production_math.py:12-15: n_g, raw_g, x / where(n > 1e-10, n, 1)
    const float n = __builtin_sqrtf(tree_sum<D, P0, P1>([&](int p) { return x[p - P0] * x[p - P0]; }) + 1e-30f);
    const float raw = NG > 1 ? tree_sum<D, P0, P1>([&](int) { return n; }) / (float)GW : n;
    const float den = n > 1e-10f ? n : 1.0f;
    // The group's divisions share the divisor: with r = 1/den correctly
    // rounded, q = x r is within an ulp of x/den and one FMA correction
    // returns the correctly rounded quotient (Markstein's theorem; checked
    // against IEEE division on every FP16 numerator, tests/host_division_check.c).
    // A -0 numerator may come out +0, which the FMA chains below, starting
    // from +0, cannot tell apart.
    const float rden = 1.0f / den;
#pragma unroll
    for (int i = 0; i < GW; ++i) {
      const float q0 = x[i] * rden;
      x[i] = __builtin_fmaf(__builtin_fmaf(-q0, den, x[i]), rden, q0);
    }
    // production_math.py:16: y_j = FMA chain over i ascending from +0 for
    // every output j of the group, the chains advanced together (input i
    // outer: column i of the group's block one broadcast LDS read, or one
    // scalar read at d=128), each in its own order.
    float y[GW];
#pragma unroll
    for (int j = 0; j < GW; ++j) y[j] = 0.0f;
#pragma unroll
    for (int i = 0; i < GW; ++i) {
      if constexpr (Bulk<D, WG>::ROT_LDS) {
        const float4 *Ci = reinterpret_cast<const float4 *>(rot + (g * GW + i) * GW);
#pragma unroll
        for (int j4 = 0; j4 < GW / 4; ++j4) {
          const float4 c = Ci[j4];
          y[4 * j4 + 0] = __builtin_fmaf(x[i], c.x, y[4 * j4 + 0]);
          y[4 * j4 + 1] = __builtin_fmaf(x[i], c.y, y[4 * j4 + 1]);
          y[4 * j4 + 2] = __builtin_fmaf(x[i], c.z, y[4 * j4 + 2]);
          y[4 * j4 + 3] = __builtin_fmaf(x[i], c.w, y[4 * j4 + 3]);
        }
      } else {
        const BGTQ_CONST float *Ci = Rt + (P0 + i) * D + P0;
#pragma unroll
        for (int j = 0; j < GW; ++j) y[j] = __builtin_fmaf(x[i], Ci[j], y[j]);
      }
    }
    // production_math.py:17-23: output j's bin, LUT code and centroid are
    // taken where the sum tree of c^2 takes its leaf j (the code packed as
    // produced), so each c^2 is folded in at once; the tree visits every leaf
    // once, in its own fixed order.
    const float csum = tree_sum<D, P0, P1>([&](int j) {
      float t = (y[j - P0] - T->lut_off[j]) * T->lut_inv[j];
      t = fminf(fmaxf(t, 0.0f), 255.0f);
      const uint32_t code = lut[(int)T->pos_cb[j] * 256 + (int)t];
      const float c = books[(int)T->pos_book[j] * mc + (int)code];
      const int byte = j < NS ? j / 2 : NS / 2 + (j - NS);
      const int shift = 8 * (byte % 4) + (j < NS ? 4 * (j % 2) : 0);
      packed[byte / 4] |= code << shift;
      return c * c;
    });
    // corrected_g = raw_g / max(sqrt(sum c^2), 1e-10)
    scales[g] = f32_to_f16_bits(raw / fmaxf(__builtin_sqrtf(csum), 1e-10f));
  });

  // mixed_layout.py:21-27: every byte of the destination row written (zero
  // padding after the codes); FP16 scales zero-padded to norm_stride.
  const int64_t out_row = job.dst_row0 + (row0 + tid) * job.dst_step;
  const int RB = T->row_bytes, NSTR = T->norm_stride;
  BGTQ_GLOBAL uint32_t *prow = reinterpret_cast<BGTQ_GLOBAL uint32_t *>(to_global(job.packed) + out_row * RB);
#pragma unroll
  for (int w = 0; w < LOGICAL / 4; ++w) prow[w] = packed[w];
  for (int w = LOGICAL / 4; w < RB / 4; ++w) prow[w] = 0u;
  BGTQ_GLOBAL uint16_t *nrow = to_global(job.norms) + out_row * NSTR;
#pragma unroll
  for (int g = 0; g < NG; ++g) nrow[g] = scales[g];
  for (int g = NG; g < NSTR; ++g) nrow[g] = 0;
}

template <int D, int NG, int NS, int WG>
hipError_t launch_kind(const EncodeJobDev *jobs, int n_jobs, int src_f32, int64_t max_rows, int lut_area,
                       int book_floats, hipStream_t stream) {
  const int lds = Bulk<D, WG>::STAGE + lut_area + Bulk<D, WG>::book_area(book_floats) + Bulk<D, WG>::ROT;
  dim3 grid((unsigned)((max_rows + WG - 1) / WG), (unsigned)n_jobs);
  if (src_f32)
    hipLaunchKernelGGL((encode_bulk_kernel<D, NG, NS, true, WG>), grid, dim3(WG), lds, stream, jobs, lut_area,
                       book_floats);
  else
    hipLaunchKernelGGL((encode_bulk_kernel<D, NG, NS, false, WG>), grid, dim3(WG), lds, stream, jobs, lut_area,
                       book_floats);
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
  return wg * (d + 2) * 2 + Bulk<64, 256>::lut_area(lut_bytes) + Bulk<64, 256>::book_area(book_floats) +
         (d <= 64 ? 2 * (d / 2) * (d / 2) * 4 : 0);
}

hipError_t launch_encode_bulk(const EncodeJobDev *jobs, int n_jobs, int kind, int wg, int src_f32, int64_t max_rows,
                              int lut_bytes, int book_floats, hipStream_t stream) {
  const int lut_area = Bulk<64, 256>::lut_area(lut_bytes);
#define BGTQ_BULK(K, DD, NS, W)                                                                           \
  if (kind == K && wg == W)                                                                               \
    return launch_kind<DD, 2, NS, W>(jobs, n_jobs, src_f32, max_rows, lut_area, book_floats, stream);
  BGTQ_BULK(1, 64, 32, 256)
  BGTQ_BULK(2, 128, 64, 128)
#undef BGTQ_BULK
  return hipErrorInvalidValue;
}

}  // namespace bgtq
