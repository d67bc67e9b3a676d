// Device scratch of bgtq_decode_noalloc: the decode's workspace (split
// counters, rotated queries, split partials and statistics, laid out as
// bgtq_decode_workspace_size describes) in a file-scope device array, so
// that entry point allocates nothing. Every device the library runs on holds
// its own copy (BGTQ_DECODE_SCRATCH_BYTES) until the process ends.
//
// The array's name is only a host-side stand-in; its address on a device is
// resolved with hipGetSymbolAddress once per device, with that device
// current, and only that address is handed to kernels.
#include <hip/hip_runtime.h>

#include <mutex>

#include "../../include/bgtq.h"

static __device__ __align__(256) uint8_t scratch[BGTQ_DECODE_SCRATCH_BYTES];

namespace bgtq {
namespace {

constexpr int kMaxDevices = 64;
std::mutex g_mutex;
uint8_t *g_scratch[kMaxDevices];

// Grid-stride fill of n 16-byte words with zeros.
__global__ void clear_scratch_kernel(uint4 *p, size_t n) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
    p[i] = uint4{0u, 0u, 0u, 0u};
}

}  // namespace

// The device address of this device's scratch array (device must be current).
// The first call on a device resolves it and clears the array on `stream`,
// waiting for the clear: the split counters must start at zero, and every
// decode leaves them at zero again.
hipError_t decode_scratch_setup(int device, hipStream_t stream, uint8_t **out) {
  if (device < 0 || device >= kMaxDevices || !out) return hipErrorInvalidValue;
  std::lock_guard<std::mutex> lock(g_mutex);
  if (!g_scratch[device]) {
    void *ptr = nullptr;
    hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    if (!ptr || (reinterpret_cast<uintptr_t>(ptr) & 255)) return hipErrorInvalidSymbol;
    static_assert(BGTQ_DECODE_SCRATCH_BYTES % 16 == 0, "whole 16-byte words");
    hipLaunchKernelGGL(clear_scratch_kernel, dim3(256), dim3(256), 0, stream, static_cast<uint4 *>(ptr),
                       (size_t)BGTQ_DECODE_SCRATCH_BYTES / 16);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    if ((e = hipStreamSynchronize(stream)) != hipSuccess) return e;
    g_scratch[device] = static_cast<uint8_t *>(ptr);
  }
  *out = g_scratch[device];
  return hipSuccess;
}

}  // namespace bgtq
