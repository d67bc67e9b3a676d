// One K row encoded by one wave (lane j owns dimension j, and j + 64 at
// d=128): the arithmetic of src/reference/production_math.py:4-24 as its
// torch code evaluates on the CPU, bit for bit. Shared by the wave encoder
// (encode_wave.hip) and the decode-step append inside the fused decode
// kernel (decode_fast_kernel.h).
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
#pragma once

#include <hip/hip_fp16.h>

#include "bgtq_internal.h"

namespace bgtq {
namespace row_enc {

__device__ __forceinline__ float f16_bits_to_f32(uint16_t h) { return __half2float(__ushort_as_half(h)); }
__device__ __forceinline__ uint16_t f32_to_f16_bits(float v) { return __half_as_ushort(__float2half_rn(v)); }

__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Per-wave LDS scratch of one row: leaf[D] f32, xn[D] f32, part[64] f32,
// tot[8] f32 (unused; kept so the scratch layout is unchanged), codes[D] u8.
__host__ __device__ constexpr int scratch_bytes(int D) { return ((D * 4 * 2 + 64 * 4 + 8 * 4 + D) + 15) & ~15; }

template <int D>
struct Scratch {
  float *leaf, *xn, *part, *tot;
  uint8_t *codes;
  __device__ Scratch() {}
  __device__ explicit Scratch(uint8_t *base) {
    leaf = reinterpret_cast<float *>(base);
    xn = leaf + D;
    part = xn + D;
    tot = part + 64;
    codes = reinterpret_cast<uint8_t *>(tot + 8);
  }
};

// ATen's 8-lane inner sum over leaf[0..D) restricted to each group's positions,
// for all ng groups; lane (l, g) = 8 g + l passes its group's range [gs, ge).
// Lane 8 g returns group g's total; pick() hands it to any lane. The eight
// partials of a group lie in one 16-lane row, so lane 8 g adds them in order
// through row shifts (no LDS round trip).
template <int D>
__device__ __forceinline__ float group_tree(const float *leaf, int lane, int ng, int gs, int ge) {
  constexpr int NV = D / 8, SI = NV / 4;
  // Every leaf of the lane's column is read (one round of LDS reads) and the
  // ones outside the group enter as +0: the leaves are never negative, so the
  // accumulators are never -0 and adding +0 changes nothing.
  const int l = lane & 7;
  float lv[NV];
#pragma unroll
  for (int v = 0; v < NV; ++v) lv[v] = leaf[v * 8 + l];
  const bool act = lane < 8 * ng;
  auto in = [&](int v) { return act && v * 8 + l >= gs && v * 8 + l < ge ? lv[v] : 0.0f; };
  float a0 = 0.0f, a1 = 0.0f, a2 = 0.0f, a3 = 0.0f;
#pragma unroll
  for (int i = 0; i < SI; ++i) {
    a0 += in(4 * i + 0);
    a1 += in(4 * i + 1);
    a2 += in(4 * i + 2);
    a3 += in(4 * i + 3);
  }
#pragma unroll
  for (int v = SI * 4; v < NV; ++v) a0 += in(v);
  a0 += a1;
  a0 += a2;
  a0 += a3;
  // t = part 0 + part 1 + ... + part 7 (lane 8 g + k's part reaches lane 8 g by a row shift of k).
  const int ai = __float_as_int(a0);
  float t = a0;
  t += __int_as_float(__builtin_amdgcn_update_dpp(0, ai, 0x101, 0xf, 0xf, false));
  t += __int_as_float(__builtin_amdgcn_update_dpp(0, ai, 0x102, 0xf, 0xf, false));
  t += __int_as_float(__builtin_amdgcn_update_dpp(0, ai, 0x103, 0xf, 0xf, false));
  t += __int_as_float(__builtin_amdgcn_update_dpp(0, ai, 0x104, 0xf, 0xf, false));
  t += __int_as_float(__builtin_amdgcn_update_dpp(0, ai, 0x105, 0xf, 0xf, false));
  t += __int_as_float(__builtin_amdgcn_update_dpp(0, ai, 0x106, 0xf, 0xf, false));
  t += __int_as_float(__builtin_amdgcn_update_dpp(0, ai, 0x107, 0xf, 0xf, false));
  return t;
}

// Group g's total (g < ng) from group_tree's result, in any lane.
__device__ __forceinline__ float pick(float t, int g) {
  float r = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(t), 0));
#pragma unroll
  for (int k = 1; k < kMaxGroups; ++k) {
    const float v = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(t), 8 * k));
    r = g == k ? v : r;
  }
  return r;
}

// Per-lane constants of the dimensions a lane owns, from the tables.
template <int D>
struct Lane {
  static constexpr int JL = D > 64 ? 2 : 1;  // dimensions per lane
  int perm[JL], grp[JL], cb[JL], bk[JL];
  float off[JL], inv[JL];
  bool own[JL];
  int gs, ge;  // group range of this lane's tree partial (lane = 8 g + l)
  __device__ void init(const DevTables *T, int lane) {
    gs = T->gstart[(lane >> 3) & (kMaxGroups - 1)];
    ge = T->gend[(lane >> 3) & (kMaxGroups - 1)];
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
  }
};

// Encodes ER rows at once (their chains interleaved, each row's arithmetic
// exactly that of a single row): row r's FP16-valued inputs x[r] (head-perm
// order, lane's dimensions), its scratch s[r]; codes land in s[r].codes[0..D),
// and lanes below the norm stride get row r's FP16 scale bits in h[r] (zero
// past the groups, 0 in the other lanes). rot(i, jl) is R[j][i] for the lane's
// dimension j = lane + 64 jl (from LDS, global memory or registers), read once
// for all rows; lut and books may be in LDS or global memory.
template <int D, int ER, typename Rot>
__device__ __forceinline__ void encode_rows(const DevTables *T, const Lane<D> &c, const float (&x)[ER][Lane<D>::JL],
                                            Rot rot, const uint8_t *lut, const float *books,
                                            const Scratch<D> (&s)[ER], int lane, uint16_t (&h)[ER]) {
  constexpr int JL = Lane<D>::JL;
  const int ng = T->groups, mc = T->max_centroids;
  // production_math.py:12  n_g = sqrt(sum((x*x)*mask) + 1e-30): each lane
  // forms the values of its own dimensions' groups and, below ng, of group
  // `lane` (the final scale), so nothing is computed for groups it does not use.
  const int gl = lane < ng ? lane : 0;
#pragma unroll
  for (int r = 0; r < ER; ++r)
#pragma unroll
    for (int jl = 0; jl < JL; ++jl)
      if (c.own[jl]) s[r].leaf[lane + 64 * jl] = x[r][jl] * x[r][jl];
  wave_sync();
  float t1[ER];
#pragma unroll
  for (int r = 0; r < ER; ++r) t1[r] = group_tree<D>(s[r].leaf, lane, ng, c.gs, c.ge);
  float nrm[ER][JL];
#pragma unroll
  for (int r = 0; r < ER; ++r)
#pragma unroll
    for (int jl = 0; jl < JL; ++jl) nrm[r][jl] = __builtin_sqrtf(pick(t1[r], c.grp[jl]) + 1e-30f);
  // production_math.py:14  raw_g = sum(n_g*mask)/|g| (more than one group)
  float raw[ER];
  if (ng > 1) {
    wave_sync();
#pragma unroll
    for (int r = 0; r < ER; ++r)
#pragma unroll
      for (int jl = 0; jl < JL; ++jl)
        if (c.own[jl]) s[r].leaf[lane + 64 * jl] = nrm[r][jl];
    wave_sync();
#pragma unroll
    for (int r = 0; r < ER; ++r) {
      const float t2 = group_tree<D>(s[r].leaf, lane, ng, c.gs, c.ge);
      raw[r] = pick(t2, gl) / (float)T->gsize[gl];
    }
  } else {
#pragma unroll
    for (int r = 0; r < ER; ++r) raw[r] = __builtin_sqrtf(pick(t1[r], 0) + 1e-30f);
  }
  // production_math.py:15  xn = x / where(n > 1e-10, n, 1)
#pragma unroll
  for (int r = 0; r < ER; ++r)
#pragma unroll
    for (int jl = 0; jl < JL; ++jl)
      if (c.own[jl]) s[r].xn[lane + 64 * jl] = x[r][jl] / (nrm[r][jl] > 1e-10f ? nrm[r][jl] : 1.0f);
  wave_sync();
  // production_math.py:16-18  y_j (FMA chain, i ascending), bin, code
  float cent[ER][JL];
#pragma unroll
  for (int jl = 0; jl < JL; ++jl) {
    float acc[ER];
#pragma unroll
    for (int r = 0; r < ER; ++r) acc[r] = 0.0f;
#pragma unroll
    for (int i = 0; i < D; ++i) {
      const float rv = rot(i, jl);
#pragma unroll
      for (int r = 0; r < ER; ++r) acc[r] = __builtin_fmaf(s[r].xn[i], rv, acc[r]);
    }
#pragma unroll
    for (int r = 0; r < ER; ++r) {
      float t = (acc[r] - c.off[jl]) * c.inv[jl];
      t = fminf(fmaxf(t, 0.0f), 255.0f);
      const uint8_t code = lut[c.cb[jl] * 256 + (int)t];
      if (c.own[jl]) s[r].codes[lane + 64 * jl] = code;
      cent[r][jl] = books[c.bk[jl] * mc + code];
    }
  }
  // production_math.py:20-23  corrected_g = raw_g / max(sqrt(sum((c*c)*mask)), 1e-10)
  wave_sync();
#pragma unroll
  for (int r = 0; r < ER; ++r)
#pragma unroll
    for (int jl = 0; jl < JL; ++jl)
      if (c.own[jl]) s[r].leaf[lane + 64 * jl] = cent[r][jl] * cent[r][jl];
  wave_sync();
#pragma unroll
  for (int r = 0; r < ER; ++r) {
    const float t3 = group_tree<D>(s[r].leaf, lane, ng, c.gs, c.ge);
    const float cc = fmaxf(__builtin_sqrtf(pick(t3, gl)), 1e-10f);
    h[r] = lane < T->norm_stride && lane < ng ? f32_to_f16_bits(raw[r] / cc) : (uint16_t)0;
  }
}

// One row (encode_rows of a single row): the row's FP16 scale bits in lanes
// below the norm stride, 0 elsewhere.
template <int D, typename Rot>
__device__ __forceinline__ uint16_t encode_row(const DevTables *T, const Lane<D> &c, const float (&x)[Lane<D>::JL],
                                               Rot rot, const uint8_t *lut, const float *books, const Scratch<D> &s,
                                               int lane) {
  constexpr int JL = Lane<D>::JL;
  float xr[1][JL];
#pragma unroll
  for (int jl = 0; jl < JL; ++jl) xr[0][jl] = x[jl];
  const Scratch<D> sr[1] = {s};
  uint16_t h[1];
  encode_rows<D, 1>(T, c, xr, rot, lut, books, sr, lane, h);
  return h[0];
}

// Byte b of the packed row (src/reference/mixed_layout.py:21-27): nibble
// bytes, then byte codes, then zero padding.
__device__ __forceinline__ uint8_t packed_byte(const uint8_t *codes, int b, int nibble_dims, int logical) {
  // Both code reads unconditional (index 0 past the logical bytes): reads
  // under branches would be one LDS round trip after another.
  const int nb = nibble_dims / 2;
  const bool nib = b < nb;
  const int j = b >= logical ? 0 : nib ? 2 * b : nibble_dims + b - nb;
  const uint32_t c0 = codes[j], c1 = codes[nib ? j + 1 : j];
  return b >= logical ? 0 : nib ? (uint8_t)((c0 & 15) | ((c1 & 15) << 4)) : (uint8_t)c0;
}

}  // namespace row_enc
}  // namespace bgtq
