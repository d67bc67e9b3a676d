// Block-GTQ K encode for gfx950 with one wave per K row: lane j owns dimension
// j (and j + 64 at d=128). The row arithmetic (encode_row.h) is bit-exact with
// the reference encoder (src/reference/production_math.py:4-24) as its torch
// code evaluates on the CPU, the same contract as encode.hip. Latency per row
// is a few microseconds, so appending one decode token per head costs about
// one launch; throughput comes from many rows per wave with the next row's
// inputs loaded while the current one is encoded.
#include "encode_row.h"

namespace bgtq {
namespace {

using namespace row_enc;

constexpr int kWaves = 4;

// Shared tables of a job + per-wave scratch; byte offsets in dynamic LDS.
struct WaveLds {
  int rot_t, lut, books, scratch, scratch_stride, total;
};
__host__ __device__ inline WaveLds wave_lds(int D, int lut_bytes, int book_floats) {
  auto a16 = [](int x) { return (x + 15) & ~15; };
  WaveLds L;
  L.rot_t = 0;
  L.lut = L.rot_t + D * D * 4;
  L.books = L.lut + a16(lut_bytes);
  L.scratch = L.books + a16(book_floats * 4);
  L.scratch_stride = scratch_bytes(D);
  L.total = L.scratch + kWaves * L.scratch_stride;
  return L;
}

template <int D, bool SRC_F32>
__global__ __launch_bounds__(64 * kWaves) void encode_wave_kernel(EncodeLaunch launch) {
  constexpr int JL = Lane<D>::JL;
  extern __shared__ __align__(16) uint8_t smem[];
  const EncodeJobDev job = launch.jobs[blockIdx.y];
  const DevTables *__restrict__ T = job.t;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int mc = T->max_centroids;
  const WaveLds L = wave_lds(D, T->n_codebooks * 256, T->n_books * mc);
  float *rot_t = reinterpret_cast<float *>(smem + L.rot_t);
  uint8_t *lut = smem + L.lut;
  float *books = reinterpret_cast<float *>(smem + L.books);
  const Scratch<D> scr(smem + L.scratch + wave * L.scratch_stride);

  // Stage the job's transposed rotation, code LUT and centroid books.
  {
    const float *src = tables_rot_t(T);
    for (int e = tid; e < D * D; e += 64 * kWaves) rot_t[e] = src[e];
    const uint8_t *ls = tables_lut(T);
    for (int e = tid; e < T->n_codebooks * 256; e += 64 * kWaves) lut[e] = ls[e];
    const float *bs = tables_books(T);
    for (int e = tid; e < T->n_books * mc; e += 64 * kWaves) books[e] = bs[e];
  }
  Lane<D> c;
  c.init(T, lane);
  __syncthreads();

  const int RB = T->row_bytes, ns = T->nibble_dims, NS = T->norm_stride;
  const int logical = ns / 2 + D - ns;
  const int64_t nwaves = (int64_t)gridDim.x * kWaves;
  auto load_row = [&](int64_t r, float (&x)[JL]) {
#pragma unroll
    for (int jl = 0; jl < JL; ++jl) {
      float v = 0.0f;
      if (c.own[jl] && r < job.rows) {
        const int64_t at = r * job.src_stride + c.perm[jl];
        if (SRC_F32) v = f16_bits_to_f32(f32_to_f16_bits(static_cast<const float *>(job.src)[at]));
        else v = f16_bits_to_f32(static_cast<const uint16_t *>(job.src)[at]);
      }
      x[jl] = v;
    }
  };
  int64_t row = (int64_t)blockIdx.x * kWaves + wave;
  float x[JL];
  load_row(row, x);
  for (; row < job.rows; row += nwaves) {
    float xnext[JL];
    load_row(row + nwaves, xnext);  // next row's inputs in flight meanwhile
    const uint16_t h = encode_row<D>(
        T, c, x, [&](int i, int jl) { return rot_t[i * D + (c.own[jl] ? lane + 64 * jl : 0)]; }, lut, books, scr, lane);
    const int64_t dst = job.dst_row0 + row * job.dst_step;
    // mixed_layout.py:21-27: [nibble bytes][byte codes][zero pad]; FP16 scales zero-padded.
    for (int b = lane; b < RB; b += 64) job.packed[dst * RB + b] = packed_byte(scr.codes, b, ns, logical);
    if (lane < NS) job.norms[dst * NS + lane] = h;
    wave_sync();  // scratch is rewritten by the next row
#pragma unroll
    for (int jl = 0; jl < JL; ++jl) x[jl] = xnext[jl];
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

int encode_wave_lds_bytes(int dim, int lut_bytes, int book_floats) { return wave_lds(dim, lut_bytes, book_floats).total; }

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
