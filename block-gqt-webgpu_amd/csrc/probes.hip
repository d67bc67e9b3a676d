// Device ceilings measured on the running GPU, for the benchmark's roofline
// context (not part of libbgtq): a streaming HBM read and a dense fp16
// 16x16x32 matrix-core loop. Built into libbgtq_probes.so.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kReadUnroll = 4;

// Grid-stride 16-byte non-temporal loads over the buffer, xor-reduced; the
// store only happens for a value the data never produces, so it keeps the
// loads without adding traffic.
__global__ __launch_bounds__(256) void read_kernel(const u32x4 *__restrict__ src, size_t n16, uint32_t *sink) {
  const size_t stride = (size_t)gridDim.x * 256 * kReadUnroll;
  uint32_t acc = 0;
  for (size_t base = (size_t)blockIdx.x * 256 * kReadUnroll + threadIdx.x; base < n16; base += stride) {
    u32x4 v[kReadUnroll];
#pragma unroll
    for (int u = 0; u < kReadUnroll; ++u) {
      const size_t i = base + (size_t)u * 256;
      v[u] = i < n16 ? __builtin_nontemporal_load(src + i) : u32x4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int u = 0; u < kReadUnroll; ++u) acc ^= v[u][0] ^ v[u][1] ^ v[u][2] ^ v[u][3];
  }
  if (acc == 0x9e3779b9u) sink[blockIdx.x] = acc;
}

// Eight independent accumulation chains per wave keep the matrix core busy.
__global__ __launch_bounds__(256) void mfma_kernel(int iters, float *sink, int store) {
  const int lane = threadIdx.x & 63;
  half8 a, b;
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    a[k] = (_Float16)(0.001f * (lane + k));
    b[k] = (_Float16)(0.002f * (lane - k));
  }
  f32x4 acc[8];
#pragma unroll
  for (int c = 0; c < 8; ++c) acc[c] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  for (int i = 0; i < iters; ++i) {
#pragma unroll
    for (int c = 0; c < 8; ++c) acc[c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, acc[c], 0, 0, 0);
  }
  if (store) {
    float s = 0.0f;
#pragma unroll
    for (int c = 0; c < 8; ++c) s += acc[c][0] + acc[c][1] + acc[c][2] + acc[c][3];
    sink[blockIdx.x * 256 + threadIdx.x] = s;
  }
}

template <typename Launch>
int time_us(Launch launch, int reps, double *us) {
  hipEvent_t a = nullptr, b = nullptr;
  if (hipEventCreate(&a) != hipSuccess || hipEventCreate(&b) != hipSuccess) return 1;
  launch();  // warm up
  hipEventRecord(a, nullptr);
  for (int r = 0; r < reps; ++r) launch();
  hipEventRecord(b, nullptr);
  int rc = hipEventSynchronize(b) == hipSuccess ? 0 : 1;
  float ms = 0.0f;
  if (!rc) rc = hipEventElapsedTime(&ms, a, b) == hipSuccess ? 0 : 1;
  hipEventDestroy(a);
  hipEventDestroy(b);
  if (!rc && hipGetLastError() != hipSuccess) rc = 1;
  *us = (double)ms * 1e3 / reps;
  return rc;
}

}  // namespace

extern "C" {

// Average time of one pass reading `bytes` (a multiple of 16) from `buf` on
// the null stream; returns 0 on success.
int bgtq_probe_read(const void *buf, size_t bytes, int reps, double *us_per_pass) {
  if (!buf || bytes < 16 || bytes % 16 || reps < 1 || !us_per_pass) return 1;
  uint32_t *sink = nullptr;
  const int blocks = 4096;
  if (hipMalloc(&sink, blocks * sizeof(uint32_t)) != hipSuccess) return 1;
  const int rc = time_us([&] { read_kernel<<<blocks, 256>>>(static_cast<const u32x4 *>(buf), bytes / 16, sink); },
                         reps, us_per_pass);
  hipFree(sink);
  return rc;
}

// Dense fp16 matrix-core rate: `waves_per_cu` waves on each of `cus` compute
// units run `iters` x 8 16x16x32 MFMAs; returns the flops of one pass and
// its average time.
int bgtq_probe_mfma(int cus, int iters, int reps, double *flops_per_pass, double *us_per_pass) {
  if (cus < 1 || iters < 1 || reps < 1 || !flops_per_pass || !us_per_pass) return 1;
  const int blocks = cus * 2;  // 256 threads = 4 waves each: 8 waves per compute unit
  float *sink = nullptr;
  if (hipMalloc(&sink, (size_t)blocks * 256 * sizeof(float)) != hipSuccess) return 1;
  *flops_per_pass = (double)blocks * 4 * iters * 8 * (16.0 * 16.0 * 32.0 * 2.0);
  const int rc = time_us([&] { mfma_kernel<<<blocks, 256>>>(iters, sink, 0); }, reps, us_per_pass);
  hipFree(sink);
  return rc;
}

}  // extern "C"
