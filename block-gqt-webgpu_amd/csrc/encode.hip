// Block-GTQ K encode for gfx950: one thread per K row, bit-exact with the
// reference encoder (src/reference/production_math.py:4-24) as its torch code
// evaluates on the CPU the reference goldens were written on:
//  * group sums of squares, repeated-norm sums and centroid-norm sums follow
//    ATen's 8-lane vectorised inner-sum tree (aten_sum8 below);
//  * y = normalized @ R.T is one FMA chain per output in ascending k, the
//    order of the CPU sgemm; only 8-wide blocks that touch the output's
//    group are issued, the remaining rotation entries are exact zeros
//    (validated when the tables are built), so skipping them is exact;
//  * division and square root are IEEE (this file is built with
//    -ffp-contract=off and correctly rounded fp32 division/sqrt).
// Rows are staged through LDS with coalesced loads; packed bytes and FP16
// scales leave through coalesced byte/short stores, so adjacent rows never
// read-modify-write each other (no atomics, unlike src/webgpu/mixed.wgsl:35-40).
#include <hip/hip_fp16.h>

#include "bgtq_internal.h"

namespace bgtq {
namespace {

constexpr int kRows = 128;  // rows (threads) per workgroup

__device__ __forceinline__ uint16_t f32_to_f16_bits(float v) {
  return __half_as_ushort(__float2half_rn(v));
}
__device__ __forceinline__ float f16_bits_to_f32(uint16_t h) {
  return __half2float(__ushort_as_half(h));
}

// ATen cascade_sum over a contiguous row of D floats with 8-wide vectors
// (vectorized_inner_sum -> row_sum -> multi_row_sum, no cascade levels below
// 64 vectors): lane l accumulates four interleaved partials a_k over vectors
// 4i+k, tail vectors go to a_0, then ((a0+a1)+a2)+a3, then the 8 lanes are
// added in order. leaf(i) must return element i (compile-time i).
template <int D, typename F>
__device__ __forceinline__ float aten_sum8(F leaf) {
  constexpr int NV = D / 8, SI = NV / 4;
  float total = 0.0f;
#pragma unroll
  for (int l = 0; l < 8; ++l) {
    float a0 = 0.0f, a1 = 0.0f, a2 = 0.0f, a3 = 0.0f;
#pragma unroll
    for (int i = 0; i < SI; ++i) {
      a0 += leaf((i * 4 + 0) * 8 + l);
      a1 += leaf((i * 4 + 1) * 8 + l);
      a2 += leaf((i * 4 + 2) * 8 + l);
      a3 += leaf((i * 4 + 3) * 8 + l);
    }
#pragma unroll
    for (int v = SI * 4; v < NV; ++v) a0 += leaf(v * 8 + l);
    a0 += a1;
    a0 += a2;
    a0 += a3;
    total += a0;
  }
  return total;
}

template <int D, bool SRC_F32>
__global__ __launch_bounds__(kRows) void encode_kernel(const EncodeJobDev *__restrict__ jobs) {
  constexpr int SSTR = D + 2;  // staged halfs per row: odd dword stride, no bank conflicts
  constexpr int CSTR = D + 4;  // code bytes per row
  static_assert(kRows * CSTR <= kRows * SSTR * 2, "codes alias the staging buffer");
  __shared__ uint16_t stage[kRows * SSTR];
  __shared__ uint16_t scales[kRows * kMaxGroups];

  const EncodeJobDev job = jobs[blockIdx.y];
  const int64_t row0 = (int64_t)blockIdx.x * kRows;
  if (row0 >= job.rows) return;  // uniform for the workgroup
  const int nr = (int)min((int64_t)kRows, job.rows - row0);
  const BGTQ_GLOBAL DevTables *__restrict__ T = to_global(job.t);
  const int tid = threadIdx.x;

  // Coalesced staging of the block's rows as FP16 bits. FP32 sources are
  // first rounded to FP16 (src/model/codec.wgsl:14, x.half().float()).
  for (int e = tid; e < nr * D; e += kRows) {
    const int r = e / D, c = e - r * D;
    const int64_t at = (row0 + r) * job.src_stride + c;
    uint16_t h;
    if (SRC_F32) h = f32_to_f16_bits(to_global(static_cast<const float *>(job.src))[at]);
    else h = to_global(static_cast<const uint16_t *>(job.src))[at];
    stage[r * SSTR + c] = h;
  }
  __syncthreads();

  const bool active = tid < nr;
  float x[D];
#pragma unroll
  for (int i = 0; i < D; ++i)
    x[i] = active ? f16_bits_to_f32(stage[tid * SSTR + T->perm[i]]) : 0.0f;
  __syncthreads();  // stage is reused for codes below

  const int ng = T->groups;
  // production_math.py:12-14: n_g = sqrt(sum((x*x)*mask) + 1e-30),
  // raw_g = sum(n_g*mask)/|g| when there is more than one group.
  float nrm[kMaxGroups], raw[kMaxGroups];
#pragma unroll
  for (int g = 0; g < kMaxGroups; ++g) {
    nrm[g] = 1.0f;
    raw[g] = 0.0f;
    if (g < ng) {
      const float s = aten_sum8<D>([&](int i) { return (int)T->group_of[i] == g ? x[i] * x[i] : 0.0f; });
      const float n = __builtin_sqrtf(s + 1e-30f);
      nrm[g] = n;
      if (ng > 1) {
        const float t = aten_sum8<D>([&](int i) { return (int)T->group_of[i] == g ? n : 0.0f; });
        raw[g] = t / (float)T->gsize[g];
      } else {
        raw[g] = n;
      }
    }
  }
  // production_math.py:15: x / where(n > 1e-10, n, 1)
  float den[kMaxGroups];
#pragma unroll
  for (int g = 0; g < kMaxGroups; ++g) den[g] = nrm[g] > 1e-10f ? nrm[g] : 1.0f;
#pragma unroll
  for (int i = 0; i < D; ++i) {
    const int gi = T->group_of[i];
    float dv = den[0];
#pragma unroll
    for (int g = 1; g < kMaxGroups; ++g) dv = gi == g ? den[g] : dv;
    x[i] = x[i] / dv;
  }

  // production_math.py:16-18: y_j = sum_i xn_i R[j,i] (FMA chain, ascending i),
  // bin = trunc(clamp((y - off)*inv, 0, 255)), code = LUT[posToCb[j]][bin].
  const BGTQ_GLOBAL float *__restrict__ R = tables_rot(T);
  const BGTQ_GLOBAL uint8_t *__restrict__ lut = tables_lut(T);
  uint8_t *codes = reinterpret_cast<uint8_t *>(stage);
  for (int j = 0; j < D; ++j) {
    const int g = T->group_of[j];
    const int gs = T->gstart[g], ge = T->gend[g];
    const float *__restrict__ Rj = R + j * D;
    float acc = 0.0f;
#pragma unroll
    for (int b = 0; b < D / 8; ++b) {
      if (b * 8 < ge && b * 8 + 8 > gs) {
#pragma unroll
        for (int k = 0; k < 8; ++k) acc = __builtin_fmaf(x[b * 8 + k], Rj[b * 8 + k], acc);
      }
    }
    float t = (acc - T->lut_off[j]) * T->lut_inv[j];
    t = fminf(fmaxf(t, 0.0f), 255.0f);
    const int bin = (int)t;
    codes[tid * CSTR + j] = lut[(int)T->pos_cb[j] * 256 + bin];
  }

  // production_math.py:20-23: corrected_g = raw_g / max(sqrt(sum((c*c)*mask)), 1e-10)
  const BGTQ_GLOBAL float *__restrict__ books = tables_books(T);
  const int mc = T->max_centroids;
#pragma unroll
  for (int i = 0; i < D; ++i) {
    const float c = books[(int)T->pos_book[i] * mc + codes[tid * CSTR + i]];
    x[i] = c * c;
  }
#pragma unroll
  for (int g = 0; g < kMaxGroups; ++g) {
    if (g < ng) {
      const float s = aten_sum8<D>([&](int i) { return (int)T->group_of[i] == g ? x[i] : 0.0f; });
      const float c = fmaxf(__builtin_sqrtf(s), 1e-10f);
      scales[tid * kMaxGroups + g] = f32_to_f16_bits(raw[g] / c);
    }
  }
  __syncthreads();

  // mixed_layout.py:21-27: [nibble bytes][byte codes][zero pad], every byte of
  // each destination row written; FP16 scales zero-padded to norm_stride.
  const int RB = T->row_bytes, ns = T->nibble_dims, NS = T->norm_stride;
  const int logical = ns / 2 + D - ns;
  const int64_t step = job.dst_step;
  for (int o = tid; o < nr * RB; o += kRows) {
    const int r = o / RB, b = o - r * RB;
    const uint8_t *cr = codes + r * CSTR;
    uint8_t val = 0;
    if (b < ns / 2) val = (uint8_t)((cr[2 * b] & 15) | ((cr[2 * b + 1] & 15) << 4));
    else if (b < logical) val = cr[ns + b - ns / 2];
    to_global(job.packed)[(job.dst_row0 + (row0 + r) * step) * RB + b] = val;
  }
  for (int o = tid; o < nr * NS; o += kRows) {
    const int r = o / NS, g = o - r * NS;
    to_global(job.norms)[(job.dst_row0 + (row0 + r) * step) * NS + g] = g < ng ? scales[r * kMaxGroups + g] : (uint16_t)0;
  }
}

template <int D>
hipError_t launch_d(const EncodeJobDev *jobs, int n_jobs, int src_f32, int64_t max_rows, hipStream_t stream) {
  dim3 grid((unsigned)((max_rows + kRows - 1) / kRows), (unsigned)n_jobs);
  if (src_f32) hipLaunchKernelGGL((encode_kernel<D, true>), grid, dim3(kRows), 0, stream, jobs);
  else hipLaunchKernelGGL((encode_kernel<D, false>), grid, dim3(kRows), 0, stream, jobs);
  return hipGetLastError();
}

// One wave per chunk: lane i copies job i (64 bytes) of the chunk's kernel
// arguments into the table.
// One 16-byte piece of a descriptor per lane, so the chunk moves in a single
// round of kernel-argument loads and stores.
constexpr int kUploadPieces = sizeof(EncodeJobDev) / sizeof(uint4);

__global__ __launch_bounds__(256) void encode_upload_kernel(EncodeLaunch chunk, EncodeJobDev *table, int base) {
  const int i = threadIdx.x;
  if (i < chunk.n_jobs * kUploadPieces) {
    const uint4 v = reinterpret_cast<const uint4 *>(chunk.jobs)[i];
    reinterpret_cast<uint4 *>(table + base)[i] = v;
  }
}

}  // namespace

hipError_t launch_encode_upload(const EncodeLaunch &chunk, EncodeJobDev *table, int base, hipStream_t stream) {
  static_assert(kEncodeJobsPerLaunch * kUploadPieces <= 256, "one lane per 16-byte piece");
  hipLaunchKernelGGL(encode_upload_kernel, dim3(1), dim3(256), 0, stream, chunk, table, base);
  return hipGetLastError();
}

hipError_t launch_encode(const EncodeJobDev *jobs, int n_jobs, int dim, int src_f32, int64_t max_rows,
                         hipStream_t stream) {
  switch (dim) {
    case 16: return launch_d<16>(jobs, n_jobs, src_f32, max_rows, stream);
    case 32: return launch_d<32>(jobs, n_jobs, src_f32, max_rows, stream);
    case 64: return launch_d<64>(jobs, n_jobs, src_f32, max_rows, stream);
    case 128: return launch_d<128>(jobs, n_jobs, src_f32, max_rows, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace bgtq
