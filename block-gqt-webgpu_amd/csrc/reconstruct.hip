// Materialised K for the phase-3 path (CompressedKeys.prepare,
// src/runtime/compressed-keys.ts:51-57; src/webgpu/mixed.wgsl:42-56) and the
// reference reconstruct (src/reference/production_math.py:27-31):
// k[perm[i]] = sum_{j in group(i)} (c_j[code_j] * s_g) R[j, i], accumulated
// as one FMA chain in ascending j. Also the FP32 -> FP16 conversion used for
// FP16 V appends (src/model/append.wgsl:6-10).
#include <hip/hip_fp16.h>

#include "bgtq_internal.h"

namespace bgtq {
namespace {

__global__ void reconstruct_kernel(const DevTables *__restrict__ T, const uint8_t *__restrict__ packed,
                                   const uint16_t *__restrict__ norms, int64_t rows, float *__restrict__ out) {
  const int64_t row = blockIdx.x;
  const int i = threadIdx.x, d = T->dim;
  if (row >= rows || i >= d) return;
  const uint8_t *pr = packed + row * T->row_bytes;
  const uint16_t *nr = norms + row * T->norm_stride;
  const float *books = tables_books(T), *R = tables_rot(T);
  const int g = T->group_of[i], nib = T->nibble_dims, mc = T->max_centroids;
  const float s = __half2float(__ushort_as_half(nr[g]));
  float acc = 0.0f;
  for (int j = T->gstart[g]; j < T->gend[g]; ++j) {
    const int code = j < nib ? (pr[j >> 1] >> ((j & 1) * 4)) & 15 : pr[(nib >> 1) + j - nib];
    const float cs = books[(int)T->pos_book[j] * mc + code] * s;
    acc = __builtin_fmaf(cs, R[j * d + i], acc);
  }
  out[row * d + T->perm[i]] = acc;
}

__global__ void half_convert_kernel(const float *__restrict__ src, uint16_t *__restrict__ dst, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
    dst[i] = __half_as_ushort(__float2half_rn(src[i]));
}

}  // namespace

hipError_t launch_reconstruct(const DevTables *t, const uint8_t *packed, const uint16_t *norms, int64_t rows,
                              float *out, hipStream_t stream) {
  hipLaunchKernelGGL(reconstruct_kernel, dim3((unsigned)rows), dim3(128), 0, stream, t, packed, norms, rows, out);
  return hipGetLastError();
}

hipError_t launch_half_convert(const float *src, uint16_t *dst, int64_t n, hipStream_t stream) {
  const int64_t blocks = std::min<int64_t>((n + 255) / 256, 4096);
  hipLaunchKernelGGL(half_convert_kernel, dim3((unsigned)std::max<int64_t>(blocks, 1)), dim3(256), 0, stream, src, dst, n);
  return hipGetLastError();
}

}  // namespace bgtq
