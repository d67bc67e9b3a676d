// Device helpers shared by the matrix-core attention kernels (gfx950):
// buffer descriptors and HBM -> LDS DMA, wave column reductions, the
// 16x16x32 f16 MFMA, fp16 hi/lo operand splitting, device-coherent partial
// stores and explicit memory waits.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace bgtq {
namespace gfx {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef __fp16 fp16x4 __attribute__((__vector_size__(4 * sizeof(__fp16))));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef fp16x4 __attribute__((address_space(3))) lds_fp16x4;
typedef __attribute__((address_space(3))) void lds_void;

constexpr int kLdsLimit = 160 * 1024;  // LDS of one gfx950 CU
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
constexpr float kPScale = 32768.0f;  // P is carried as p * 2^15 so its fp16 lo part stays normal
// Buffer resource word 3 on gfx9: 32-bit dword data format, raw (unswizzled) addressing.
constexpr int kRsrcWord3 = 0x00020000;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void *base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, (int)bytes, kRsrcWord3);
}
// Cache policy of a load: kStream marks data read once (the non-temporal
// bit), so streaming K/V does not displace what the caches hold.
constexpr int kCached = 0;
constexpr int kStream = 2;

// HBM -> LDS without VGPRs: lane i writes 16 (4) bytes at lds + 16 i (4 i).
// Lanes whose offset lies past the descriptor's size write zeros.
template <int POLICY = kCached>
__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t r, uint8_t *lds, uint32_t voff, uint32_t soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void *)lds, 16, (int)voff, (int)soff, 0, POLICY);
}
template <int POLICY = kCached>
__device__ __forceinline__ void dma4(__amdgpu_buffer_rsrc_t r, uint8_t *lds, uint32_t voff, uint32_t soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void *)lds, 4, (int)voff, (int)soff, 0, POLICY);
}

// Reductions over the four 16-lane rows that share a column (lane % 16).
__device__ __forceinline__ float col_max(float v) {
  auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ __forceinline__ float col_sum(float v) {
  auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// This lane's index in its wave, from the mbcnt instructions: it needs no
// input register, so the compiler recomputes it where it is used instead of
// holding a per-lane offset derived from it across a long loop.
__device__ __forceinline__ int lane_id() { return (int)__builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u)); }

// Maximum over the 16 lanes of each row: DPP row rotations by 8, 4, 2 and 1,
// plain VALU operations with no LDS round trip.
__device__ __forceinline__ float row_max(float v) {
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x128, 0xf, 0xf, false)));
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x124, 0xf, 0xf, false)));
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x122, 0xf, 0xf, false)));
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x121, 0xf, 0xf, false)));
  return v;
}

// Minimum over the wave's 64 lanes, in every lane: DPP row rotations, then
// the row swaps (no LDS round trip).
__device__ __forceinline__ int wave_min(int v) {
  v = min(v, __builtin_amdgcn_update_dpp(0, v, 0x128, 0xf, 0xf, false));
  v = min(v, __builtin_amdgcn_update_dpp(0, v, 0x124, 0xf, 0xf, false));
  v = min(v, __builtin_amdgcn_update_dpp(0, v, 0x122, 0xf, 0xf, false));
  v = min(v, __builtin_amdgcn_update_dpp(0, v, 0x121, 0xf, 0xf, false));
  auto a = __builtin_amdgcn_permlane16_swap((uint32_t)v, (uint32_t)v, false, false);
  v = min((int)a[0], (int)a[1]);
  auto c = __builtin_amdgcn_permlane32_swap((uint32_t)v, (uint32_t)v, false, false);
  return min((int)c[0], (int)c[1]);
}

__device__ __forceinline__ f32x4 mfma(half8 a, half8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// x = hi + lo with both halves fp16 (hi rounded toward zero, so lo is exact
// before its own rounding): ~2^-22 relative.
__device__ __forceinline__ void split2(float x0, float x1, uint32_t &hi, uint32_t &lo) {
  const auto h = __builtin_amdgcn_cvt_pkrtz(x0, x1);
  const float r0 = x0 - (float)h[0], r1 = x1 - (float)h[1];
  const auto l = __builtin_amdgcn_cvt_pkrtz(r0, r1);
  hi = __builtin_bit_cast(uint32_t, h);
  lo = __builtin_bit_cast(uint32_t, l);
}

// The same split in four instructions instead of six: lo = fp16(x - hi)
// through the mixed-precision FMA, which reads hi's fp16 halves directly.
// `one` must be 1.0 from a register the compiler cannot see through (an
// empty asm), or it folds the FMA into a subtraction and converts hi back.
__device__ __forceinline__ void split2_mix(float x0, float x1, float one, uint32_t &hi, uint32_t &lo) {
  typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
  const auto h = __builtin_amdgcn_cvt_pkrtz(x0, x1);
  const float r0 = __builtin_fmaf(-(float)h[0], one, x0), r1 = __builtin_fmaf(-(float)h[1], one, x1);
  hi = __builtin_bit_cast(uint32_t, h);
  lo = __builtin_bit_cast(uint32_t, half2_t{(_Float16)r0, (_Float16)r1});
}

// Eight values split with split2_mix.
__device__ __forceinline__ void split8_mix(const float *x, float one, half8 &hi, half8 &lo) {
  u32x4 h4, l4;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    uint32_t h, l;
    split2_mix(x[2 * k], x[2 * k + 1], one, h, l);
    h4[k] = h;
    l4[k] = l;
  }
  hi = __builtin_bit_cast(half8, h4);
  lo = __builtin_bit_cast(half8, l4);
}

// Split of x * sc (sc a power of two) into fp16 hi (rounded toward zero) and lo halves.
__device__ __forceinline__ void split_scaled(const float *x, float sc, half8 &hi, half8 &lo) {
  u32x4 h4, l4;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    uint32_t h, l;
    split2(x[2 * k] * sc, x[2 * k + 1] * sc, h, l);
    h4[k] = h;
    l4[k] = l;
  }
  hi = __builtin_bit_cast(half8, h4);
  lo = __builtin_bit_cast(half8, l4);
}

// Exponent e with max * 2^e near 2^14 (fp16 hi/lo split range); 0 for max 0.
__device__ __forceinline__ int split_exp(float mx) { return mx > 0.0f ? 14 - (int)ceilf(__builtin_log2f(mx)) : 0; }

// Relaxed atomics at device scope: on gfx950 they go to the device-coherent
// level (system-coherent bit) instead of this XCD's L2.
__device__ __forceinline__ void coherent_store(float *ptr, float v) {
  __hip_atomic_store(ptr, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float coherent_load(float *ptr) {
  return __hip_atomic_load(ptr, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// 16- and 8-byte loads at the same level (cache policy sc1), through a
// buffer resource: off is a byte offset inside its range.
constexpr int kPolicySc1 = 16;
__device__ __forceinline__ f32x4 coherent_load4(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, kPolicySc1));
}
__device__ __forceinline__ u32x2 coherent_load2(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(r, (int)off, 0, kPolicySc1));
}

// Waits for all but the newest N vector-memory operations of this wave. The
// LDS writes of buffer_load ... lds are not tracked by the compiler, so ring
// waits are explicit; the memory clobber keeps LDS reads below them.
template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt");
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
__device__ __forceinline__ void wait_lds() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

// Workgroup barrier for LDS traffic only. __syncthreads() also waits for every
// outstanding global load of the wave (its release fence), which would drain
// the HBM -> LDS ring; here the caller has already waited for the DMAs whose
// LDS data the other waves read.
__device__ __forceinline__ void lds_barrier() {
  wait_lds();
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// Two transposed FP16 reads (ds_read_b64_tr_b16: lane i of a 16-lane group
// gets column i of the four rows the group addresses) issued from inline asm.
// The builtin form makes the compiler wait for every vector-memory load in
// flight first (it may alias an LDS DMA), which drains a DMA ring; the caller
// has waited for the DMA that wrote these rows. The compiler's hazard
// recognizer does not look into asm: the s_nop 7 covers the wait states a
// matrix-core instruction that read the destination registers as its
// accumulator input needs before they are written (8-pass XDL). The results
// are not valid until a wait_lds_tied on them.
__device__ __forceinline__ void ds_read_tr16_pair(const uint8_t *lds0, const uint8_t *lds1, u32x2 &a, u32x2 &b) {
  asm volatile("s_nop 7\n\tds_read_b64_tr_b16 %0, %2\n\tds_read_b64_tr_b16 %1, %3"
               : "=&v"(a), "=&v"(b)
               : "v"((uint32_t)(uintptr_t)(lds_void *)lds0), "v"((uint32_t)(uintptr_t)(lds_void *)lds1));
}
// Waits until at most N LDS operations of this wave are in flight; a and b
// are tied to the wait so nothing that reads them is scheduled before it.
// LDS operations complete in order, so with the reads of a and b issued
// before the N newest, they have landed.
template <int N>
__device__ __forceinline__ void wait_lds_tied(u32x2 &a, u32x2 &b) {
  static_assert(N >= 0 && N < 16, "lgkmcnt");
  asm volatile("s_waitcnt lgkmcnt(%2)" : "+v"(a), "+v"(b) : "n"(N));
}

// Wait for transposed read pair dt of DT issued in order (2 (DT - 1 - dt)
// newer reads may still be in flight); dt is a compile-time index after
// unrolling.
template <int DT>
__device__ __forceinline__ void wait_dt(int dt, u32x2 &a, u32x2 &b) {
  if constexpr (DT == 2) {
    if (dt == 0) wait_lds_tied<2>(a, b);
    else wait_lds_tied<0>(a, b);
  } else if constexpr (DT == 4) {
    if (dt == 0) wait_lds_tied<6>(a, b);
    else if (dt == 1) wait_lds_tied<4>(a, b);
    else if (dt == 2) wait_lds_tied<2>(a, b);
    else wait_lds_tied<0>(a, b);
  } else {
    static_assert(DT == 8, "head dim 32, 64 or 128");
    if (dt == 0) wait_lds_tied<14>(a, b);
    else if (dt == 1) wait_lds_tied<12>(a, b);
    else if (dt == 2) wait_lds_tied<10>(a, b);
    else if (dt == 3) wait_lds_tied<8>(a, b);
    else if (dt == 4) wait_lds_tied<6>(a, b);
    else if (dt == 5) wait_lds_tied<4>(a, b);
    else if (dt == 6) wait_lds_tied<2>(a, b);
    else wait_lds_tied<0>(a, b);
  }
}

// 16-byte piece swizzle of an FP16 row of D values in LDS: conflict-free
// transposed (ds_read_b64_tr_b16) and row reads.
template <int D>
__host__ __device__ constexpr int swz(int row) {
  return D == 64 ? (row >> 1) & 7 : row & 15;
}

}  // namespace gfx
}  // namespace bgtq
