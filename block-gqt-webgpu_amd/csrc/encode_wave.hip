// Block-GTQ K encode for gfx950 with one wave per K row: lane j owns dimension
// j (and j + 64 at d=128). Bit-exact with the reference encoder
// (src/reference/production_math.py:4-24) as its torch code evaluates on the
// CPU, the same contract as encode.hip, reached with lane-parallel work:
//  * the FP32 sums of production_math.py:12, :14 and :23 follow ATen's 8-lane
//    inner-sum tree: lane (l, g) forms partial l of group g from the four
//    interleaved accumulators in the tree's order, lane g then adds the eight
//    partials in order; masked-out leaves are exact zeros and are skipped
//    (a + 0 = a for the never-negative-zero accumulators), all groups at once;
//  * y_j = sum_i xn_i R[j][i] (production_math.py:16) is one FMA chain per
//    lane over all i in ascending order from +0, the order of the CPU sgemm;
//    off-group rotation entries are exact zeros, so adding their products
//    changes nothing;
//  * division and square root are IEEE (built with -ffp-contract=off and
//    correctly rounded fp32 division/sqrt).
// Latency per row is a few microseconds, so appending one decode token per
// head costs about one launch; throughput comes from many rows per wave with
// the next row's inputs loaded while the current one is encoded.
#include <hip/hip_fp16.h>

#include "bgtq_internal.h"

namespace bgtq {
namespace {

constexpr int kWaves = 4;

__device__ __forceinline__ float f16_bits_to_f32(uint16_t h) { return __half2float(__ushort_as_half(h)); }
__device__ __forceinline__ uint16_t f32_to_f16_bits(float v) { return __half_as_ushort(__float2half_rn(v)); }

__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

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
  // leaf[D] f32, xn[D] f32, part[64] f32, tot[8] f32, codes[D] u8
  L.scratch_stride = a16(D * 4 * 2 + 64 * 4 + 8 * 4 + D);
  L.total = L.scratch + kWaves * L.scratch_stride;
  return L;
}

// ATen's 8-lane inner sum over leaf[0..D) restricted to each group's positions,
// for all ng groups; lane (l, g) = 8 g + l passes its group's range [gs, ge).
// Every lane then reads tot[g].
template <int D>
__device__ __forceinline__ void group_sums(const float *leaf, float *part, float *tot, int lane, int ng, int gs,
                                           int ge) {
  constexpr int NV = D / 8, SI = NV / 4;
  if (lane < 8 * ng) {
    const int l = lane & 7, g = lane >> 3;
    float a0 = 0.0f, a1 = 0.0f, a2 = 0.0f, a3 = 0.0f;
#pragma unroll
    for (int i = 0; i < SI; ++i) {
      const int p0 = (4 * i + 0) * 8 + l, p1 = (4 * i + 1) * 8 + l, p2 = (4 * i + 2) * 8 + l, p3 = (4 * i + 3) * 8 + l;
      if (p0 >= gs && p0 < ge) a0 += leaf[p0];
      if (p1 >= gs && p1 < ge) a1 += leaf[p1];
      if (p2 >= gs && p2 < ge) a2 += leaf[p2];
      if (p3 >= gs && p3 < ge) a3 += leaf[p3];
    }
#pragma unroll
    for (int v = SI * 4; v < NV; ++v) {
      const int p = v * 8 + l;
      if (p >= gs && p < ge) a0 += leaf[p];
    }
    a0 += a1;
    a0 += a2;
    a0 += a3;
    part[g * 8 + l] = a0;
  }
  wave_sync();
  if (lane < ng) {
    float t = 0.0f;
#pragma unroll
    for (int l = 0; l < 8; ++l) t += part[lane * 8 + l];
    tot[lane] = t;
  }
  wave_sync();
}

template <int D, bool SRC_F32>
__global__ __launch_bounds__(64 * kWaves) void encode_wave_kernel(EncodeLaunch launch) {
  constexpr int JL = D > 64 ? 2 : 1;  // dimensions per lane
  extern __shared__ __align__(16) uint8_t smem[];
  const EncodeJobDev job = launch.jobs[blockIdx.y];
  const DevTables *__restrict__ T = job.t;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int ng = T->groups, mc = T->max_centroids;
  const WaveLds L = wave_lds(D, T->n_codebooks * 256, T->n_books * mc);
  float *rot_t = reinterpret_cast<float *>(smem + L.rot_t);
  uint8_t *lut = smem + L.lut;
  float *books = reinterpret_cast<float *>(smem + L.books);
  uint8_t *scr = smem + L.scratch + wave * L.scratch_stride;
  float *leaf = reinterpret_cast<float *>(scr);
  float *xn = leaf + D;
  float *part = xn + D;
  float *tot = part + 64;
  uint8_t *codes = reinterpret_cast<uint8_t *>(tot + 8);

  // Stage the job's transposed rotation, code LUT and centroid books.
  {
    const float *src = tables_rot_t(T);
    for (int e = tid; e < D * D; e += 64 * kWaves) rot_t[e] = src[e];
    const uint8_t *ls = tables_lut(T);
    for (int e = tid; e < T->n_codebooks * 256; e += 64 * kWaves) lut[e] = ls[e];
    const float *bs = tables_books(T);
    for (int e = tid; e < T->n_books * mc; e += 64 * kWaves) books[e] = bs[e];
  }
  // Group range of this lane's tree partial (lane = 8 g + l).
  const int gs = T->gstart[(lane >> 3) & (kMaxGroups - 1)], ge = T->gend[(lane >> 3) & (kMaxGroups - 1)];
  // Per-lane constants of the dimensions this lane owns.
  int perm[JL], grp[JL], cb[JL], bk[JL];
  float off[JL], inv[JL];
  bool own[JL];
#pragma unroll
  for (int jl = 0; jl < JL; ++jl) {
    const int j = lane + 64 * jl;
    own[jl] = j < D;
    const int jj = own[jl] ? j : 0;
    perm[jl] = T->perm[jj];
    grp[jl] = T->group_of[jj];
    cb[jl] = T->pos_cb[jj];
    bk[jl] = T->pos_book[jj];
    off[jl] = T->lut_off[jj];
    inv[jl] = T->lut_inv[jj];
  }
  __syncthreads();

  const int RB = T->row_bytes, ns = T->nibble_dims, NS = T->norm_stride;
  const int logical = ns / 2 + D - ns;
  const int64_t nwaves = (int64_t)gridDim.x * kWaves;
  auto load_row = [&](int64_t r, float (&x)[JL]) {
#pragma unroll
    for (int jl = 0; jl < JL; ++jl) {
      float v = 0.0f;
      if (own[jl] && r < job.rows) {
        const int64_t at = r * job.src_stride + perm[jl];
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

    // production_math.py:12  n_g = sqrt(sum((x*x)*mask) + 1e-30)
#pragma unroll
    for (int jl = 0; jl < JL; ++jl)
      if (own[jl]) leaf[lane + 64 * jl] = x[jl] * x[jl];
    wave_sync();
    group_sums<D>(leaf, part, tot, lane, ng, gs, ge);
    float nrm[kMaxGroups];
#pragma unroll
    for (int g = 0; g < kMaxGroups; ++g) nrm[g] = g < ng ? __builtin_sqrtf(tot[g] + 1e-30f) : 1.0f;
    // production_math.py:14  raw_g = sum(n_g*mask)/|g| (more than one group)
    float raw[kMaxGroups];
    if (ng > 1) {
      wave_sync();
#pragma unroll
      for (int jl = 0; jl < JL; ++jl) {
        float n = nrm[0];
#pragma unroll
        for (int g = 1; g < kMaxGroups; ++g) n = grp[jl] == g ? nrm[g] : n;
        if (own[jl]) leaf[lane + 64 * jl] = n;
      }
      wave_sync();
      group_sums<D>(leaf, part, tot, lane, ng, gs, ge);
#pragma unroll
      for (int g = 0; g < kMaxGroups; ++g) raw[g] = g < ng ? tot[g] / (float)T->gsize[g] : 0.0f;
    } else {
#pragma unroll
      for (int g = 0; g < kMaxGroups; ++g) raw[g] = nrm[g];
    }
    // production_math.py:15  xn = x / where(n > 1e-10, n, 1)
#pragma unroll
    for (int jl = 0; jl < JL; ++jl) {
      float n = nrm[0];
#pragma unroll
      for (int g = 1; g < kMaxGroups; ++g) n = grp[jl] == g ? nrm[g] : n;
      if (own[jl]) xn[lane + 64 * jl] = x[jl] / (n > 1e-10f ? n : 1.0f);
    }
    wave_sync();
    // production_math.py:16-18  y_j (FMA chain, i ascending), bin, code
    float cent[JL];
#pragma unroll
    for (int jl = 0; jl < JL; ++jl) {
      const int j = own[jl] ? lane + 64 * jl : 0;
      float acc = 0.0f;
#pragma unroll 16
      for (int i = 0; i < D; ++i) acc = __builtin_fmaf(xn[i], rot_t[i * D + j], acc);
      float t = (acc - off[jl]) * inv[jl];
      t = fminf(fmaxf(t, 0.0f), 255.0f);
      const uint8_t code = lut[cb[jl] * 256 + (int)t];
      if (own[jl]) codes[lane + 64 * jl] = code;
      cent[jl] = books[bk[jl] * mc + code];
    }
    // production_math.py:20-23  corrected_g = raw_g / max(sqrt(sum((c*c)*mask)), 1e-10)
    wave_sync();
#pragma unroll
    for (int jl = 0; jl < JL; ++jl)
      if (own[jl]) leaf[lane + 64 * jl] = cent[jl] * cent[jl];
    wave_sync();
    group_sums<D>(leaf, part, tot, lane, ng, gs, ge);
    const int64_t dst = job.dst_row0 + row * job.dst_step;
    // mixed_layout.py:21-27: [nibble bytes][byte codes][zero pad]; FP16 scales zero-padded.
    for (int b = lane; b < RB; b += 64) {
      uint8_t val = 0;
      if (b < ns / 2) val = (uint8_t)((codes[2 * b] & 15) | ((codes[2 * b + 1] & 15) << 4));
      else if (b < logical) val = codes[ns + b - ns / 2];
      job.packed[dst * RB + b] = val;
    }
    if (lane < NS) {
      uint16_t h = 0;
      if (lane < ng) {
        const float c = fmaxf(__builtin_sqrtf(tot[lane]), 1e-10f);
        float rg = raw[0];
#pragma unroll
        for (int g = 1; g < kMaxGroups; ++g) rg = lane == g ? raw[g] : rg;
        h = f32_to_f16_bits(rg / c);
      }
      job.norms[dst * NS + lane] = h;
    }
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
