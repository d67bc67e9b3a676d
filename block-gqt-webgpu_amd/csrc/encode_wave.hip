// Block-GTQ K encode for gfx950 with one wave per K row: lane j owns dimension
// j (and j + 64 at d=128). The row arithmetic (encode_row.h) is bit-exact with
// the reference encoder (src/reference/production_math.py:4-24) as its torch
// code evaluates on the CPU, the same contract as encode.hip. Latency per row
// is a few microseconds, so appending one decode token per head costs about
// one launch; throughput comes from many rows per wave with the next row's
// inputs loaded while the current one is encoded.
#include "encode_row.h"
#include "gfx950_common.h"

namespace bgtq {
namespace {

using namespace row_enc;

constexpr int kWaves = 4;

// Dynamic LDS of a workgroup: the job's transposed rotation, a copy of its
// table set's first enc_bytes (header, code LUT, books) in whole 1 KB DMA
// pieces, then per-wave scratch.
struct WaveLds {
  int rot_t, tab, scratch, scratch_stride, total;
};
__host__ __device__ inline WaveLds wave_lds(int D, int enc_bytes) {
  WaveLds L;
  L.rot_t = 0;
  L.tab = L.rot_t + D * D * 4;
  L.scratch = L.tab + (enc_bytes + 1023) / 1024 * 1024;
  L.scratch_stride = scratch_bytes(D);
  L.total = L.scratch + kWaves * L.scratch_stride;
  return L;
}

template <int D, bool SRC_F32>
__global__ __launch_bounds__(64 * kWaves) void encode_wave_kernel(EncodeLaunch launch) {
  constexpr int JL = Lane<D>::JL;
  extern __shared__ __align__(16) uint8_t smem[];
  const EncodeJobDev job = launch.jobs[blockIdx.y];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const WaveLds L = wave_lds(D, job.enc_bytes);
  float *rot_t = reinterpret_cast<float *>(smem + L.rot_t);
  const Scratch<D> scr(smem + L.scratch + wave * L.scratch_stride);
  const int64_t nwaves = (int64_t)gridDim.x * kWaves;

  // One round trip: the rotation (d*d*4 bytes, whole 1 KB pieces for d >= 16)
  // and the tables' header, LUT and books go HBM -> LDS (1 KB pieces over the
  // four waves; lanes past a region's size write zeros), the wave's first row
  // is loaded in natural order.
  static_assert(D * D * 4 % 1024 == 0, "rotation in whole DMA pieces");
  {
    const uint8_t *tb = reinterpret_cast<const uint8_t *>(job.t);
    const __amdgpu_buffer_rsrc_t rr = gfx::rsrc(tb + job.off_rot_t, D * D * 4);
    for (int k = wave; k < D * D * 4 / 1024; k += kWaves) gfx::dma16(rr, smem + L.rot_t + k * 1024, k * 1024 + lane * 16, 0);
    const __amdgpu_buffer_rsrc_t rt = gfx::rsrc(tb, job.enc_bytes);
    for (int k = wave; k < (job.enc_bytes + 1023) / 1024; k += kWaves)
      gfx::dma16(rt, smem + L.tab + k * 1024, k * 1024 + lane * 16, 0);
  }
  // Natural-order row values: lane holds element lane + 64 jl (FP16-rounded).
  // Unconditional loads (a row past the job's reads its row 0, an element
  // past D its element 0; both are then zeroed), so the next row's load stays
  // in flight while the current row is encoded instead of being waited for
  // under a branch.
  auto load_row = [&](int64_t r, float (&v)[JL]) {
    const bool row_ok = r < job.rows;
#pragma unroll
    for (int jl = 0; jl < JL; ++jl) {
      const int e = lane + 64 * jl;
      const int64_t at = (row_ok ? r : 0) * job.src_stride + (e < D ? e : 0);
      const float x = SRC_F32 ? f16_bits_to_f32(f32_to_f16_bits(static_cast<const float *>(job.src)[at]))
                              : f16_bits_to_f32(static_cast<const uint16_t *>(job.src)[at]);
      v[jl] = row_ok && e < D ? x : 0.0f;
    }
  };
  int64_t row = (int64_t)blockIdx.x * kWaves + wave;
  float xn[JL];
  load_row(row, xn);
  gfx::wait_vm<0>();
  __syncthreads();

  const DevTables *T = reinterpret_cast<const DevTables *>(smem + L.tab);
  Lane<D> c;
  c.init(T, lane);
  const uint8_t *lut = tables_lut(T);
  const float *books = tables_books(T);
  const int RB = T->row_bytes, ns = T->nibble_dims, NS = T->norm_stride;
  const int logical = ns / 2 + D - ns;
  for (; row < job.rows; row += nwaves) {
    float xnext[JL];
    load_row(row + nwaves, xnext);  // next row's inputs in flight meanwhile
    // head-perm order: x[jl] = row[perm[lane + 64 jl]]
    float x[JL];
#pragma unroll
    for (int jl = 0; jl < JL; ++jl) {
      const int src = c.perm[jl];
      float v = __shfl(xn[0], src & 63, 64);
      if (JL > 1) {
        const float hi = __shfl(xn[JL - 1], src & 63, 64);
        v = src >= 64 ? hi : v;
      }
      x[jl] = c.own[jl] ? v : 0.0f;
    }
    const uint16_t h = encode_row<D>(
        T, c, x, [&](int i, int jl) { return rot_t[i * D + (c.own[jl] ? lane + 64 * jl : 0)]; }, lut, books, scr, lane);
    const int64_t dst = job.dst_row0 + row * job.dst_step;
    // mixed_layout.py:21-27: [nibble bytes][byte codes][zero pad]; FP16 scales zero-padded.
    for (int b = lane; b < RB; b += 64) job.packed[dst * RB + b] = packed_byte(scr.codes, b, ns, logical);
    if (lane < NS) job.norms[dst * NS + lane] = h;
    wave_sync();  // scratch is rewritten by the next row
#pragma unroll
    for (int jl = 0; jl < JL; ++jl) xn[jl] = xnext[jl];
  }
}

template <int D>
hipError_t launch_wave_d(const EncodeLaunch &launch, int src_f32, int wgs_per_job, int lds, hipStream_t stream) {
  dim3 grid((unsigned)std::max(1, wgs_per_job), (unsigned)launch.n_jobs);
  if (src_f32) {
    static const hipError_t ok = hipFuncSetAttribute((const void *)encode_wave_kernel<D, true>,
                                                     hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
    if (ok != hipSuccess) return ok;
    hipLaunchKernelGGL((encode_wave_kernel<D, true>), grid, dim3(64 * kWaves), lds, stream, launch);
  } else {
    static const hipError_t ok = hipFuncSetAttribute((const void *)encode_wave_kernel<D, false>,
                                                     hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
    if (ok != hipSuccess) return ok;
    hipLaunchKernelGGL((encode_wave_kernel<D, false>), grid, dim3(64 * kWaves), lds, stream, launch);
  }
  return hipGetLastError();
}

}  // namespace

int encode_wave_lds_bytes(int dim, int enc_bytes) { return wave_lds(dim, enc_bytes).total; }

hipError_t launch_encode_wave(const EncodeLaunch &launch, int dim, int src_f32, int wgs_per_job, int lds_bytes,
                              hipStream_t stream) {
  switch (dim) {
    case 16: return launch_wave_d<16>(launch, src_f32, wgs_per_job, lds_bytes, stream);
    case 32: return launch_wave_d<32>(launch, src_f32, wgs_per_job, lds_bytes, stream);
    case 64: return launch_wave_d<64>(launch, src_f32, wgs_per_job, lds_bytes, stream);
    case 128: return launch_wave_d<128>(launch, src_f32, wgs_per_job, lds_bytes, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace bgtq
