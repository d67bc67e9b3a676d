// Chunked-prefill attention for gfx950 on the matrix cores.
//
// A chunk of `rows` new query rows of a sequence, at positions start ..
// start+rows-1, attends causally to the sequence's whole history: row r sees
// tokens 0 .. start+r (src/model/compressed-dot.wgsl:28, softmax end of
// src/model/attention.wgsl:19). The queries of one (sequence, KV head) unit are
// its rows x G GQA heads, flattened as qi = row * G + h (the item order of
// src/model/compressed-dot.wgsl:26-27).
//
// Grid (token split, query tile, unit). A workgroup of four waves holds a tile
// of 4 x NCB x 16 queries in registers (each wave NCB 16-query MFMA column
// blocks) and streams one token split of the unit's history through a ring of
// LDS buffers shared by the four waves: packed codes, FP16 scales and FP16 V
// go HBM -> LDS with buffer_load ... lds, each wave issuing a quarter of every
// buffer, four buffers ahead of the one computed on, one barrier per 32-token
// block.
//
// The queries are rotated into the code domain in the prologue, on the matrix
// cores: with k = ((c*s) @ R)[inv_perm] (the reconstruction of
// src/reference/production_math.py:27-31), q.k = sum_g s_g sum_{j in g}
// c_j[code_j] qr_j where qr = Rq q and Rq is R with the head permutation
// folded into its columns. qr^T = Rq q^T comes out of the MFMAs with lane
// (gq, col) holding dims 16 n + 4 gq + r of query col; the QK K-steps use
// that order (MFMA k = 8 gq + jv <-> dim 32 s + 16 (jv / 4) + 4 gq + jv % 4),
// so the rotated queries are QK operands as they stand and the K operand is
// gathered in the same order.
//
// Per 32-token block each wave rebuilds the K operand from LDS lookup tables
// of fp16 (hi, lo) centroid splits once per 16-token x 32-dim step and reuses
// it for its NCB column blocks: QK as 16x16x32 f16 MFMAs (hi*hi + lo*hi +
// hi*lo), per-token group scales, the causal mask, an online softmax in the
// log2 domain and PV as MFMAs with V read transposed (ds_read_b64_tr_b16).
// Splits whose tokens lie past every query of the tile exit at once; a tile
// with one active split writes its output directly, otherwise each split
// stores an (m, l, o) partial and prefill_merge_kernel combines them by
// log-sum-exp. The arithmetic is that of src/reference/attention.py:5-22 with
// causal positions.
#include <hip/hip_fp16.h>

#include <type_traits>

#include "bgtq_internal.h"
#include "gfx950_common.h"

namespace bgtq {
namespace {

using namespace gfx;

constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;
constexpr int kChunk = 32;  // tokens per block: two 16-token MFMA tiles
constexpr int kRing = 6;    // shared LDS buffers: compute one, four in flight, one draining
// Merges of at most this many queries load all splits at once (one wave per
// query, at most two per SIMD of a 256-CU device).
constexpr int64_t kMergeOneRoundQueries = 2048;

// One ring buffer: V block, K block, FP16 scales; every wave DMAs a quarter.
// Packed-code kernels also hold the K-steps' centroid books (fp32) and two
// buffers of built K operands. The ring is as deep as lets two workgroups
// share a compute unit. KF 2 (any packed layout): K rows of up to D bytes,
// up to 8 scales per token, every book (n_books x max_centroids floats).
template <int D, int KF, int NN>
struct PSlot {
  static constexpr int KS = D / 32, DT = D / 16, PR = D / 8;
  static constexpr int VBYTES = kChunk * D * 2;
  static constexpr int VI = VBYTES / 1024;  // 16-byte DMA instructions per V block
  static constexpr int VW = VI / kWaves;    // ... per wave
  static constexpr int RB = KF == 1 ? NN * 16 + (KS - NN) * 32 : KF == 2 ? D : 2 * D;  // K row bytes
  static constexpr int KBYTES = kChunk * RB;
  static constexpr int KQ = KBYTES / kWaves;  // K bytes per wave
  static constexpr int KW = KF >= 1 ? (KQ + 1023) / 1024 : VW;
  static constexpr int KLAST = KF >= 1 ? (KQ - (KW - 1) * 1024) / 16 : 64;  // lanes of the last K instruction
  static constexpr int NBYTES = KF == 1 ? kChunk * 4 : KF == 2 ? kChunk * 16 : 0;
  static constexpr int BYTES = VBYTES + KBYTES + NBYTES;
  static constexpr int LW = VW + KW + (KF >= 1 ? 1 : 0);  // DMA instructions per wave per block
  static constexpr int BOOKS = KF >= 1 ? KS * 1024 * KF : 0;  // KF 1: 256 fp32 centroids per K-step
  static constexpr int KOP = KF >= 1 ? 2 * 2 * KS * 2048 : 0;  // [buffer][u][s]: hi 1 KB, lo 1 KB
  static constexpr int FIXED = BOOKS + KOP;
  static constexpr int RING = 6 * BYTES + FIXED <= kLdsLimit / 2 ? 6 : 4 * BYTES + FIXED <= kLdsLimit / 2 ? 4 : 3;
  static constexpr int AHEAD = RING - 2;
  static constexpr int LDS = RING * BYTES + FIXED;
  static_assert(VI % kWaves == 0 && KQ % 16 == 0 && KBYTES % 16 == 0, "DMA split over four waves");
  static_assert(LDS <= kLdsLimit, "LDS of one workgroup");
  static_assert(AHEAD * LW < 64, "vmcnt range");
};

// Waits until at most `newer` blocks (LW instructions each) of this wave's
// DMAs are still in flight; `newer` is wave-uniform.
template <int LW, int A>
__device__ __forceinline__ void wait_blocks(int newer) {
  if constexpr (A > 0) {
    if (newer >= A) {
      wait_vm<A * LW>();
      return;
    }
    wait_blocks<LW, A - 1>(newer);
  } else {
    wait_vm<0>();
  }
}

__device__ __forceinline__ float wave_max(float v) {
  v = col_max(v);
#pragma unroll
  for (int o = 8; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
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

__device__ __forceinline__ float h2f(uint32_t bits) { return __half2float(__ushort_as_half((uint16_t)bits)); }

// The query's row of [B, rows, Hq] (outputs, partials).
__device__ __forceinline__ int64_t query_row(int b, int rows, int Hq, int kv, int G, int qi) {
  const int row = qi / G, h = qi - row * G;
  return ((int64_t)b * rows + row) * Hq + kv * G + h;
}

// KF: 1 = packed codes of a structured layout, 2 = packed codes of any
// layout, 0 = FP16 K rows. NN: leading nibble K-steps. SG: K-steps in group 0. NCB: 16-query column blocks per wave. At least two
// waves per SIMD (at most 256 registers each), so that one wave's softmax
// overlaps another's matrix-core work; up to four for single-block tiles.
//
// Packed codes: the four waves build each block's K operand once, in LDS,
// one block ahead of the one computed on: K'[t][d] = c_d * s_g(d)(t) *
// 2^(ec - E) with 2^E bounding the block's FP16 scales, split into fp16 hi/lo
// in the MFMA A-operand order. The group scales then ride inside the product
// and a logit is acc * 2^(E - ec - eq) in the log2 domain (the queries carry
// log2(e) / sqrt(d)).
template <int D, int KF, int NN, int SG, int NCB>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2, NCB == 1 ? 4 : 2))) void
prefill_kernel(PrefillParams p, FastLayout fl) {
  using Sl = PSlot<D, KF, NN>;
  constexpr int KS = Sl::KS, DT = Sl::DT, PR = Sl::PR, RB = Sl::RB, AHEAD = Sl::AHEAD;
  constexpr int QW = NCB * 16, QT = kWaves * QW;
  static_assert(NN >= 0 && NN <= KS && SG >= 1 && SG <= KS, "layout");
  extern __shared__ __align__(16) uint8_t smem[];

  // Grid (tile, unit, split), tiles in reverse. Consecutive workgroup ids go
  // to consecutive XCDs, so with the tile fastest every XCD gets an even
  // share of each split's tiles (a split index in the low bits would pin each
  // split to fixed XCDs, and the first splits, active in every tile, would
  // crowd theirs); within a split the heaviest tiles (the last queries, which
  // see the most history) are dispatched first.
  const int tile = p.tiles - 1 - (int)blockIdx.x, unit = blockIdx.y, split = blockIdx.z;
  const int b = unit / p.kv_heads, kv = unit - b * p.kv_heads;
  const int G = p.G, Hq = p.q_heads, rows = p.rows;
  const int tid = threadIdx.x, lane = tid & 63, gq = lane >> 4, col = lane & 15;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int nq = rows * G;
  // The chunk's rows end inside the K/V buffers: start + rows <= max_length.
  const int start = (int)min(p.starts[b], (uint32_t)(p.max_length - rows));
  const int T_b = start + rows;
  const int q0 = tile * QT;
  if (q0 >= nq) return;
  const int n_valid = min(QT, nq - q0);
  const int e_tile = start + (q0 + n_valid - 1) / G + 1;  // exclusive end of the tile's last query
  const int SP = p.split_tokens;
  const int n_act = (e_tile + SP - 1) / SP;
  if (split >= n_act) return;  // workgroup-uniform: before any barrier
  // The tile's history [0, e_tile) is divided evenly (in 32-token blocks)
  // over its n_act splits, so no split is a sliver; each is at most SP long
  // and none is empty ((n_act - 1) * part <= (n_act - 1) * SP < e_tile).
  const int part = ((e_tile + n_act - 1) / n_act + kChunk - 1) / kChunk * kChunk;
  const int t_lo = split * part, t_hi = min(t_lo + part, e_tile);
  const int n_blocks = (t_hi - t_lo + kChunk - 1) / kChunk;
  const DevTables *T = KF >= 1 ? p.tables[kv] : nullptr;
  // Row bytes and scales per token (runtime for KF 2).
  const int rb = KF == 2 ? T->row_bytes : RB;
  const int ns = KF == 2 ? T->norm_stride : 2;
  const int mc = KF == 2 ? T->max_centroids : 0;  // read once, not per block
  float *books = reinterpret_cast<float *>(smem + Sl::RING * Sl::BYTES);
  uint8_t *kop = smem + Sl::RING * Sl::BYTES + Sl::BOOKS;
  auto slot = [&](int i) { return smem + (i % Sl::RING) * Sl::BYTES; };

  // ---------------- streams of this unit ----------------
  const _Float16 *v_base = static_cast<const _Float16 *>(p.v) + b * p.v_seq_stride + kv * p.v_head_stride;
  const uint8_t *k_base = KF >= 1 ? p.packed + b * p.packed_seq_stride + kv * p.packed_head_stride
                                  : reinterpret_cast<const uint8_t *>(static_cast<const _Float16 *>(p.k) +
                                                                      b * p.k_seq_stride + kv * p.k_head_stride);
  const uint16_t *n_base = KF >= 1 ? p.norms + b * p.norms_seq_stride + kv * p.norms_head_stride : nullptr;
  // Swizzled FP16 row pieces of this wave's V (and FP16 K) instructions:
  // instruction k, lane i fills LDS piece 64k + i = (row r, slot c) with
  // global piece c ^ swz(r).
  uint32_t voff_rows[Sl::VW];
#pragma unroll
  for (int kk = 0; kk < Sl::VW; ++kk) {
    const int P = 64 * (wave * Sl::VW + kk) + lane, r = P / PR, c = P % PR;
    voff_rows[kk] = r * (2 * D) + ((c ^ swz<D>(r)) * 16);
  }
  // Block i's descriptors start at its first token and cover its tokens inside
  // the history: the hardware range check returns zeros past the end.
  auto issue = [&](int i) {
    const int c0 = t_lo + i * kChunk;
    const uint32_t rest = (uint32_t)min(T_b - c0, kChunk);  // > 0: c0 < t_hi <= T_b
    uint8_t *sb = slot(i);
    const __amdgpu_buffer_rsrc_t rV = rsrc(v_base + (int64_t)c0 * D, rest * (2 * D));
#pragma unroll
    for (int kk = 0; kk < Sl::VW; ++kk) dma16(rV, sb + (wave * Sl::VW + kk) * 1024, voff_rows[kk], 0);
    uint8_t *kb = sb + Sl::VBYTES;
    if (KF == 1) {
      const __amdgpu_buffer_rsrc_t rK = rsrc(k_base + (int64_t)c0 * RB, rest * RB);
      const __amdgpu_buffer_rsrc_t rN = rsrc(n_base + (int64_t)c0 * 2, rest * 4);
#pragma unroll
      for (int kk = 0; kk < Sl::KW; ++kk) {
        const int off = wave * Sl::KQ + kk * 1024;
        if (kk + 1 < Sl::KW || Sl::KLAST == 64 || lane < Sl::KLAST) dma16(rK, kb + off, off + lane * 16, 0);
      }
      if (lane < kChunk / kWaves) dma4(rN, kb + Sl::KBYTES + wave * 32, wave * 32 + lane * 4, 0);
    } else if (KF == 2) {
      // Ranges end on the access size: the range check zeroes a whole access
      // reaching past the range; the bytes past the last row lie in the same
      // aligned 16 bytes as its end (16-byte aligned bases, c0 a multiple of 32).
      const __amdgpu_buffer_rsrc_t rK = rsrc(k_base + (int64_t)c0 * rb, (rest * rb + 15u) & ~15u);
      const __amdgpu_buffer_rsrc_t rN = rsrc(n_base + (int64_t)c0 * ns, (rest * ns * 2 + 3u) & ~3u);
#pragma unroll
      for (int kk = 0; kk < Sl::KW; ++kk) {
        const int off = wave * Sl::KQ + kk * 1024;
        if (kk + 1 < Sl::KW || Sl::KLAST == 64 || lane < Sl::KLAST) dma16(rK, kb + off, off + lane * 16, 0);
      }
      if (lane < Sl::NBYTES / kWaves / 4)
        dma4(rN, kb + Sl::KBYTES + wave * (Sl::NBYTES / kWaves), wave * (Sl::NBYTES / kWaves) + lane * 4, 0);
    } else {
      const __amdgpu_buffer_rsrc_t rK = rsrc(k_base + (int64_t)c0 * (2 * D), rest * (2 * D));
#pragma unroll
      for (int kk = 0; kk < Sl::VW; ++kk) dma16(rK, kb + (wave * Sl::VW + kk) * 1024, voff_rows[kk], 0);
    }
  };
#pragma unroll
  for (int i = 0; i < AHEAD; ++i)
    if (i < n_blocks) issue(i);

  // ---------------- prologue ----------------
  // Centroid books of the K-steps into LDS (wave 0, 256 floats per step);
  // this wave's queries rotated, scaled by log2(e) / sqrt(d) and split into QK
  // operands. B operand of QK step s for column block cb: lane holds query
  // col's dims 32 s + 4 gq + 0..3 and 32 s + 16 + 4 gq + 0..3.
  const int ec = KF >= 1 ? T->cent_exp : 0;
  if (KF == 2 && wave == 0) {  // every book's centroids, [n_books][max_centroids] floats
    const uint32_t nbytes = (uint32_t)(T->n_books * T->max_centroids * 4);
    const __amdgpu_buffer_rsrc_t rb_ = rsrc(tables_books(T), nbytes);
#pragma unroll
    for (int k = 0; k < Sl::BOOKS / 256; ++k)
      if ((uint32_t)k * 256 < nbytes) dma4(rb_, reinterpret_cast<uint8_t *>(books) + 256 * k, 256 * k + lane * 4, 0);
  }
  // KF 2: descriptors of the build's positions 32 s + 4 gq + 0..3 and
  // 32 s + 16 + 4 gq + 0..3 (byte offset | nibble shift << 8 | nibble flag
  // << 11 | book << 12 | group << 16).
  constexpr int KS2 = KF == 2 ? KS : 1;
  u32x4 gdl[KS2][2];
  if (KF == 2) {
    const u32x4 *gd = reinterpret_cast<const u32x4 *>(reinterpret_cast<const uint8_t *>(T) + T->off_gdesc);
#pragma unroll
    for (int s = 0; s < KS2; ++s) {
      gdl[s][0] = gd[8 * s + gq];
      gdl[s][1] = gd[8 * s + 4 + gq];
    }
  }
  if (KF == 1 && wave == 0) {
    const int mc = T->max_centroids;
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      const __amdgpu_buffer_rsrc_t rb = rsrc(tables_books(T) + fl.book[s] * mc, (uint32_t)(min(mc, 256) * 4));
#pragma unroll
      for (int k = 0; k < 4; ++k) dma4(rb, reinterpret_cast<uint8_t *>(books + s * 256 + 64 * k), 256 * k + lane * 4, 0);
    }
  }
  const float qscale = kLog2e * p.inv_sqrt_d;
  // A query already in the code domain (q_rotated) loads in the QK order.
  const bool rotate = KF >= 1 && !p.q_rotated;
  bool valid[NCB];
  half8 qhi[NCB][KS], qlo[NCB][KS];
  int eqs[NCB];   // logit = acc * 2^(E - ec - eqs)
  int lim[NCB];   // exclusive token end of this lane's column query inside the split
  int lim_min = t_hi;
#pragma unroll
  for (int cb = 0; cb < NCB; ++cb) {
    const int qi = q0 + wave * QW + cb * 16 + col;
    valid[cb] = qi < nq;
    const f32x4 *src = reinterpret_cast<const f32x4 *>(p.q + query_row(b, rows, Hq, kv, G, valid[cb] ? qi : 0) * D);
    float qv[D / 4];  // this lane's share of the query row
    float qmax = 0.0f;
#pragma unroll
    for (int s = 0; s < KS; ++s)
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        // Rotated in the kernel: natural order 32 s + 8 gq + 4 hh + 0..3 (the
        // rotation's k order); otherwise QK order 32 s + 16 hh + 4 gq + 0..3.
        const f32x4 v = valid[cb] ? src[rotate ? 8 * s + 2 * gq + hh : 8 * s + 4 * hh + gq]
                                  : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          qv[8 * s + 4 * hh + k] = v[k] * qscale;
          qmax = fmaxf(qmax, fabsf(qv[8 * s + 4 * hh + k]));
        }
      }
    int eq = split_exp(col_max(qmax));
    if (rotate) {
      // qr^T = Rq q^T on the matrix cores (q and Rq split hi/lo, three MFMAs
      // per step): D layout, lane holds rows j = 16 n + 4 gq + r of query col.
      half8 bh[KS], bl[KS];
#pragma unroll
      for (int s = 0; s < KS; ++s) split_scaled(qv + 8 * s, __builtin_ldexpf(1.0f, eq), bh[s], bl[s]);
      const u32x4 *rq = reinterpret_cast<const u32x4 *>(tables_rot_q(T));
      f32x4 qr[DT];
#pragma unroll
      for (int n = 0; n < DT; ++n) {
        qr[n] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int s = 0; s < KS; ++s) {
          const u32x4 *op = rq + ((n * KS + s) * 64 + lane) * 2;
          const half8 ah = __builtin_bit_cast(half8, op[0]), al = __builtin_bit_cast(half8, op[1]);
          qr[n] = mfma(ah, bh[s], qr[n]);
          qr[n] = mfma(al, bh[s], qr[n]);
          qr[n] = mfma(ah, bl[s], qr[n]);
        }
      }
      float rmax = 0.0f;
#pragma unroll
      for (int n = 0; n < DT; ++n)
#pragma unroll
        for (int r = 0; r < 4; ++r) rmax = fmaxf(rmax, fabsf(qr[n][r]));
      const int e2 = split_exp(col_max(rmax));
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        float x[8];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          x[r] = qr[2 * s][r];
          x[4 + r] = qr[2 * s + 1][r];
        }
        split_scaled(x, __builtin_ldexpf(1.0f, e2), qhi[cb][s], qlo[cb][s]);
      }
      eq += e2;
    } else {
#pragma unroll
      for (int s = 0; s < KS; ++s) split_scaled(qv + 8 * s, __builtin_ldexpf(1.0f, eq), qhi[cb][s], qlo[cb][s]);
    }
    eqs[cb] = eq + ec;
    lim[cb] = valid[cb] ? min(start + qi / G + 1, t_hi) : t_hi;
    lim_min = min(lim_min, lim[cb]);
  }
  // Wave-uniform: blocks reaching past lim_min need the per-query mask.
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) lim_min = min(lim_min, __shfl_xor(lim_min, o, 64));
  wait_vm<0>();
  __syncthreads();

  // Builds block i's K operand into buffer i & 1; returns E (2^E >= every
  // FP16 scale of the block). Thread (wave w, lane) builds the (u, s) steps
  // w + 4 k: token 16 u + col, dims 32 s + 4 gq + 0..3 and 32 s + 16 + 4 gq + 0..3.
  auto build = [&](int i) -> int {
    if constexpr (KF == 1) {
      const uint8_t *kraw = slot(i) + Sl::VBYTES;
      const uint32_t *nrm = reinterpret_cast<const uint32_t *>(kraw + Sl::KBYTES);
      const uint32_t nw = nrm[lane & 31];
      const float smax = wave_max(SG < KS ? fmaxf(h2f(nw & 0xffffu), h2f(nw >> 16)) : h2f(nw & 0xffffu));
      const int E = smax > 0.0f ? (int)ceilf(__builtin_log2f(smax)) : 0;
      uint8_t *kb = kop + (i & 1) * (2 * KS * 2048);
#pragma unroll
      for (int k = 0; k < 2 * KS / kWaves; ++k) {
        const int combo = wave + kWaves * k, u = combo / KS, s = combo - u * KS;
        const int t = 16 * u + col;
        const uint32_t nt = nrm[t];
        const float F = __builtin_ldexpf(s < SG ? h2f(nt & 0xffffu) : h2f(nt >> 16), ec - E);
        uint32_t e[8];
        if (s < NN) {
          const uint8_t *row = kraw + t * RB + 16 * s + 2 * gq;
          const uint32_t w = (uint32_t)*reinterpret_cast<const uint16_t *>(row) |
                             ((uint32_t)*reinterpret_cast<const uint16_t *>(row + 8) << 16);
#pragma unroll
          for (int k2 = 0; k2 < 8; ++k2) e[k2] = (w >> (4 * k2)) & 15u;
        } else {
          const uint8_t *row = kraw + t * RB + 16 * NN + 32 * (s - NN) + 4 * gq;
          const uint32_t w0 = *reinterpret_cast<const uint32_t *>(row), w1 = *reinterpret_cast<const uint32_t *>(row + 16);
#pragma unroll
          for (int k2 = 0; k2 < 4; ++k2) {
            e[k2] = (w0 >> (8 * k2)) & 255u;
            e[4 + k2] = (w1 >> (8 * k2)) & 255u;
          }
        }
        float v[8];
#pragma unroll
        for (int k2 = 0; k2 < 8; ++k2) v[k2] = books[s * 256 + e[k2]] * F;
        half8 hi, lo;
        split_scaled(v, 1.0f, hi, lo);
        uint8_t *dst = kb + (u * KS + s) * 2048 + lane * 16;
        *reinterpret_cast<half8 *>(dst) = hi;
        *reinterpret_cast<half8 *>(dst + 1024) = lo;
      }
      return E;
    } else if constexpr (KF == 2) {
      // Any layout: each element's code through its descriptor, times its
      // book's centroid and its group's scale of the token, 2^(ec - E).
      const uint8_t *kraw = slot(i) + Sl::VBYTES;
      const uint16_t *nrm = reinterpret_cast<const uint16_t *>(kraw + Sl::KBYTES);
      // E bounds the scales of the block's tokens inside the history only: the
      // scale DMA's range is rounded up to 4 bytes, so with rest * ns odd the
      // slot also holds the first scale of the token after the history.
      const int n_in = min(T_b - (t_lo + i * kChunk), kChunk) * ns;
      float smax = 0.0f;
#pragma unroll
      for (int k = 0; k < Sl::NBYTES / 2 / 64; ++k) {
        const int e = lane + 64 * k;
        if (e < n_in) smax = fmaxf(smax, fabsf(h2f(nrm[e])));
      }
      smax = wave_max(smax);
      const int E = smax > 0.0f ? (int)ceilf(__builtin_log2f(smax)) : 0;
      uint8_t *kb = kop + (i & 1) * (2 * KS * 2048);
#pragma unroll
      for (int k = 0; k < 2 * KS / kWaves; ++k) {
        const int combo = wave + kWaves * k, u = combo / KS, s = combo - u * KS;
        const int t = 16 * u + col;
        float v[8];
#pragma unroll
        for (int k2 = 0; k2 < 8; ++k2) {
          uint32_t dsc = 0;
#pragma unroll
          for (int ss = 0; ss < KS2; ++ss)  // static register indices
            if (ss == s) dsc = gdl[ss][k2 >> 2][k2 & 3];
          const uint32_t byte = kraw[t * rb + (int)(dsc & 255u)];
          const uint32_t code = (dsc >> 11) & 1u ? (byte >> ((dsc >> 8) & 7u)) & 15u : byte;
          const float c = books[(int)((dsc >> 12) & 15u) * mc + (int)code];
          const float sc = h2f(nrm[t * ns + (int)((dsc >> 16) & 15u)]);
          v[k2] = c * __builtin_ldexpf(sc, ec - E);
        }
        half8 hi, lo;
        split_scaled(v, 1.0f, hi, lo);
        uint8_t *dst = kb + (u * KS + s) * 2048 + lane * 16;
        *reinterpret_cast<half8 *>(dst) = hi;
        *reinterpret_cast<half8 *>(dst + 1024) = lo;
      }
      return E;
    } else {
      return 0;
    }
  };
  int E_cur = n_blocks > 0 ? build(0) : 0;

  float m_run[NCB], l_run[NCB];
  f32x4 O[NCB][DT];
#pragma unroll
  for (int cb = 0; cb < NCB; ++cb) {
    m_run[cb] = -INFINITY;
    l_run[cb] = 0.0f;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) O[cb][dt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  }
  const int trow = 4 * gq + (col >> 2);
  const int tpiece = (col & 3) >> 1, thalf = (col & 1) * 8;

  // One 32-token block: QK, mask (tail blocks only), online softmax, PV.
  auto compute = [&](int i, auto masked) {
    constexpr bool MASK = decltype(masked)::value;
    const int c0 = t_lo + i * kChunk;
    const uint8_t *sb = slot(i);
    f32x4 acc[NCB][2];
#pragma unroll
    for (int cb = 0; cb < NCB; ++cb) acc[cb][0] = acc[cb][1] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int u = 0; u < 2; ++u) {
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        if constexpr (KF >= 1) {
          const uint8_t *src = kop + (i & 1) * (2 * KS * 2048) + (u * KS + s) * 2048 + lane * 16;
          const half8 ah = *reinterpret_cast<const half8 *>(src), al = *reinterpret_cast<const half8 *>(src + 1024);
#pragma unroll
          for (int cb = 0; cb < NCB; ++cb) {
            acc[cb][u] = mfma(ah, qhi[cb][s], acc[cb][u]);
            acc[cb][u] = mfma(al, qhi[cb][s], acc[cb][u]);
            acc[cb][u] = mfma(ah, qlo[cb][s], acc[cb][u]);
          }
        } else {
          // FP16 K rows: 8-byte halves of swizzled 16-byte pieces
          const uint8_t *kbuf = sb + Sl::VBYTES;
          const int t = 16 * u + col;
          const int p0 = 4 * s + (gq >> 1), p1 = p0 + 2, off = (gq & 1) * 8;
          const u32x2 a0 = *reinterpret_cast<const u32x2 *>(kbuf + t * (2 * D) + ((p0 ^ swz<D>(t)) * 16) + off);
          const u32x2 a1 = *reinterpret_cast<const u32x2 *>(kbuf + t * (2 * D) + ((p1 ^ swz<D>(t)) * 16) + off);
          const half8 ah = __builtin_bit_cast(half8, u32x4{a0[0], a0[1], a1[0], a1[1]});
#pragma unroll
          for (int cb = 0; cb < NCB; ++cb) {
            acc[cb][u] = mfma(ah, qhi[cb][s], acc[cb][u]);
            acc[cb][u] = mfma(ah, qlo[cb][s], acc[cb][u]);
          }
        }
      }
    }
    // V of this block, read transposed for the PV B operands (lane: V[tokens
    // of its P slots][16 dt + col]). At d=64 issued before the softmax, so
    // the LDS latency hides under it; at d=128 just before PV (the 32 more
    // live registers across the softmax would spill).
    u32x2 vt[DT][2];
    auto read_v = [&]() {
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        const int piece = 2 * dt + tpiece;
        ds_read_tr16_pair(sb + trow * (2 * D) + ((piece ^ swz<D>(trow)) * 16) + thalf,
                          sb + (16 + trow) * (2 * D) + ((piece ^ swz<D>(16 + trow)) * 16) + thalf, vt[dt][0],
                          vt[dt][1]);
      }
    };
    if constexpr (D == 64) read_v();
    half8 pha[NCB], pla[NCB];
#pragma unroll
    for (int cb = 0; cb < NCB; ++cb) {
      // raw logits of query col: tokens c0 + 16u + 4gq + r
      float xr[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        xr[j] = acc[cb][j >> 2][j & 3];
        if constexpr (MASK) {
          const int tok = c0 + 16 * (j >> 2) + 4 * gq + (j & 3);
          xr[j] = tok < lim[cb] ? xr[j] : -INFINITY;
        }
      }
      const float C = __builtin_ldexpf(1.0f, E_cur - eqs[cb]);
      const float mloc = fmaxf(fmaxf(fmaxf(xr[0], xr[1]), fmaxf(xr[2], xr[3])),
                               fmaxf(fmaxf(xr[4], xr[5]), fmaxf(xr[6], xr[7])));
      const float m_new = fmaxf(m_run[cb], col_max(mloc) * C);
      const float alpha = m_new == -INFINITY ? 1.0f : __builtin_amdgcn_exp2f(m_run[cb] - m_new);
      const float nmb = 15.0f - (m_new == -INFINITY ? 0.0f : m_new);
      float pr[8], psum = 0.0f;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        pr[j] = __builtin_amdgcn_exp2f(__builtin_fmaf(xr[j], C, nmb));
        psum += pr[j];
      }
      l_run[cb] = __builtin_fmaf(l_run[cb], alpha, psum);
      m_run[cb] = m_new;
      u32x4 ph, pl;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        uint32_t h, l;
        split2(pr[2 * k], pr[2 * k + 1], h, l);
        ph[k] = h;
        pl[k] = l;
      }
      pha[cb] = __builtin_bit_cast(half8, ph);
      pla[cb] = __builtin_bit_cast(half8, pl);
      if (__builtin_amdgcn_ballot_w64(alpha != 1.0f)) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float ar = __shfl(alpha, 4 * gq + r, 64);
#pragma unroll
          for (int dt = 0; dt < DT; ++dt) O[cb][dt][r] *= ar;
        }
      }
    }
    // PV: B operand = the transposed V reads; dt's pair has landed once at
    // most the 2 (DT - 1 - dt) newer reads are in flight.
    if constexpr (D != 64) read_v();
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
      wait_dt<DT>(dt, vt[dt][0], vt[dt][1]);
      const u32x2 a0 = vt[dt][0], a1 = vt[dt][1];
      const half8 vb = __builtin_bit_cast(half8, u32x4{a0[0], a0[1], a1[0], a1[1]});
#pragma unroll
      for (int cb = 0; cb < NCB; ++cb) {
        O[cb][dt] = mfma(pha[cb], vb, O[cb][dt]);
        O[cb][dt] = mfma(pla[cb], vb, O[cb][dt]);
      }
    }
  };

  for (int i = 0; i < n_blocks; ++i) {
    // Block i + AHEAD goes to the buffer of block i - 2, whose V every wave
    // read before the barrier of iteration i - 1. Wait for block i + 1
    // (built below); block i has landed already.
    if (i + AHEAD < n_blocks) issue(i + AHEAD);
    if (i + 1 < n_blocks) wait_blocks<Sl::LW, AHEAD - 1>(min(n_blocks - 2 - i, AHEAD - 1));
    // Block i + 1 visible to all waves; block i's K operand (built last
    // iteration) complete; every wave done with the operand buffer of i - 1.
    // An LDS-only barrier: the wait above covers the DMAs of block i + 1, and
    // __syncthreads() would also wait for those of the blocks still in flight.
    lds_barrier();
    const int E_next = i + 1 < n_blocks ? build(i + 1) : 0;
    if (t_lo + i * kChunk + kChunk > lim_min) compute(i, std::true_type{});
    else compute(i, std::false_type{});
    E_cur = E_next;
  }

  // ---------------- epilogue ----------------
  // O row 4 gq + r of block cb is query (cb, 4 gq + r); its (m, l) live in
  // column lane 4 gq + r. One active split: the output; else the partial
  // (m, l) at part[(row * S + split) * 2] and o at part_o[(row * S + split) * D].
  const int S = p.splits;
  float *part_o = p.part + (int64_t)p.batch * rows * Hq * S * 2;
#pragma unroll
  for (int cb = 0; cb < NCB; ++cb) {
    const float l_tot = col_sum(l_run[cb]);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int qr_lane = 4 * gq + r;
      const float lr = __shfl(l_tot, qr_lane, 64);
      const int qi = q0 + wave * QW + cb * 16 + qr_lane;
      if (qi >= nq) continue;
      const int64_t g_row = query_row(b, rows, Hq, kv, G, qi);
      if (n_act == 1) {
        const float inv = 1.0f / lr;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) p.out[g_row * D + 16 * dt + col] = O[cb][dt][r] * inv;
      } else {
        float *po = part_o + (g_row * S + split) * D;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) po[16 * dt + col] = O[cb][dt][r] * (1.0f / kPScale);
      }
    }
    if (n_act > 1 && gq == 0 && valid[cb]) {
      const int64_t g_row = query_row(b, rows, Hq, kv, G, q0 + wave * QW + cb * 16 + col);
      float *pm = p.part + (g_row * S + split) * 2;
      pm[0] = m_run[cb];
      pm[1] = l_tot * (1.0f / kPScale);
    }
  }
}

// One query's merge: every active split's o row is loaded in one round (split
// k < SMAX reads split min(k, n_act - 1), whose weight is zero past n_act), then
// combined with the log-sum-exp weights of the (m, l) pairs (lane s: split s).
template <int D, int SMAX>
__device__ __forceinline__ void merge_query(const float *part_o, float2 ml, int n_act, int lane, float *out) {
  constexpr int DL = D / 64;  // output dims per lane
  float o[SMAX][DL];
#pragma unroll
  for (int k = 0; k < SMAX; ++k)
#pragma unroll
    for (int e = 0; e < DL; ++e) o[k][e] = part_o[min(k, n_act - 1) * D + lane + 64 * e];
  float M = ml.x;
#pragma unroll
  for (int s = 32; s >= 1; s >>= 1) M = fmaxf(M, __shfl_xor(M, s, 64));
  float w = ml.x == -INFINITY ? 0.0f : exp2f(ml.x - M);
  float L = w * ml.y;
#pragma unroll
  for (int s = 32; s >= 1; s >>= 1) L += __shfl_xor(L, s, 64);
  w = w / L;
  float acc[DL];
#pragma unroll
  for (int e = 0; e < DL; ++e) acc[e] = 0.0f;
#pragma unroll
  for (int k = 0; k < SMAX; ++k) {
    const float wk = __shfl(w, k, 64);
#pragma unroll
    for (int e = 0; e < DL; ++e) acc[e] = __builtin_fmaf(o[k][e], wk, acc[e]);
  }
#pragma unroll
  for (int e = 0; e < DL; ++e) out[lane + 64 * e] = acc[e];
}

// The same in rounds of eight splits: fewer registers, for launches with
// enough queries that occupancy, not one query's latency, sets the time.
template <int D>
__device__ __forceinline__ void merge_query_rounds(const float *part_o, float2 ml, int n_act, int lane, float *out) {
  constexpr int DL = D / 64;
  float M = ml.x;
#pragma unroll
  for (int s = 32; s >= 1; s >>= 1) M = fmaxf(M, __shfl_xor(M, s, 64));
  float w = ml.x == -INFINITY ? 0.0f : exp2f(ml.x - M);
  float L = w * ml.y;
#pragma unroll
  for (int s = 32; s >= 1; s >>= 1) L += __shfl_xor(L, s, 64);
  w = w / L;
  float acc[DL];
#pragma unroll
  for (int e = 0; e < DL; ++e) acc[e] = 0.0f;
  for (int s0 = 0; s0 < n_act; s0 += 8) {
    float o[8][DL];
#pragma unroll
    for (int k = 0; k < 8; ++k)
#pragma unroll
      for (int e = 0; e < DL; ++e) o[k][e] = s0 + k < n_act ? part_o[(s0 + k) * D + lane + 64 * e] : 0.0f;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const float wk = __shfl(w, min(s0 + k, 63), 64);
#pragma unroll
      for (int e = 0; e < DL; ++e) acc[e] = __builtin_fmaf(o[k][e], wk, acc[e]);
    }
  }
#pragma unroll
  for (int e = 0; e < DL; ++e) out[lane + 64 * e] = acc[e];
}

// LSE merge of the split partials of tiles with more than one active split:
// one wave per query, lane s holding split s's (m, l). ONE_ROUND: the o rows
// of all active splits read at once (small launches, where each query's
// latency is the time); else in rounds of eight.
template <int D, bool ONE_ROUND>
__global__ __launch_bounds__(kThreads) void prefill_merge_kernel(PrefillParams p, int tile_queries) {
  const int unit = blockIdx.y;
  const int b = unit / p.kv_heads, kv = unit - b * p.kv_heads;
  const int G = p.G, Hq = p.q_heads, rows = p.rows, nq = rows * G;
  const int lane = threadIdx.x & 63;
  const int qi = blockIdx.x * kWaves + (threadIdx.x >> 6);
  if (qi >= nq) return;
  const int start = (int)min(p.starts[b], (uint32_t)(p.max_length - rows));
  const int tile = qi / tile_queries;
  const int q_last = min(nq, (tile + 1) * tile_queries) - 1;
  const int e_tile = start + q_last / G + 1;
  const int n_act = (e_tile + p.split_tokens - 1) / p.split_tokens;
  if (n_act == 1) return;
  const int S = p.splits;
  const int64_t g_row = query_row(b, rows, Hq, kv, G, qi);
  const float *part_o = p.part + (int64_t)p.batch * rows * Hq * S * 2 + g_row * S * D;
  const float2 ml = lane < n_act ? reinterpret_cast<const float2 *>(p.part)[g_row * S + lane]
                                 : float2{-INFINITY, 0.0f};
  if (!ONE_ROUND) merge_query_rounds<D>(part_o, ml, n_act, lane, p.out + g_row * D);
  else if (n_act <= 8) merge_query<D, 8>(part_o, ml, n_act, lane, p.out + g_row * D);
  else if (n_act <= 16) merge_query<D, 16>(part_o, ml, n_act, lane, p.out + g_row * D);
  else if (n_act <= 32) merge_query<D, 32>(part_o, ml, n_act, lane, p.out + g_row * D);
  else merge_query<D, kPrefillMaxSplits>(part_o, ml, n_act, lane, p.out + g_row * D);
}

template <int D, int KF, int NN, int SG, int NCB>
hipError_t launch_ncb(const PrefillParams &p, const FastLayout &fl, hipStream_t stream) {
  constexpr int lds = PSlot<D, KF, NN>::LDS;
  static const hipError_t allowed = hipFuncSetAttribute((const void *)prefill_kernel<D, KF, NN, SG, NCB>,
                                                        hipFuncAttributeMaxDynamicSharedMemorySize, lds);
  if (allowed != hipSuccess) {
    (void)hipGetLastError();  // do not leave the failure behind for the caller's next HIP call
    return allowed;
  }
  const unsigned units = (unsigned)(p.batch * p.kv_heads);
  hipLaunchKernelGGL((prefill_kernel<D, KF, NN, SG, NCB>), dim3((unsigned)p.tiles, units, (unsigned)p.splits),
                     dim3(kThreads), lds, stream, p, fl);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess || p.splits == 1) return e;
  const int nq = p.rows * p.G;
  const dim3 grid((unsigned)((nq + kWaves - 1) / kWaves), units);
  if ((int64_t)nq * units <= kMergeOneRoundQueries)
    hipLaunchKernelGGL((prefill_merge_kernel<D, true>), grid, dim3(kThreads), 0, stream, p, kWaves * 16 * NCB);
  else
    hipLaunchKernelGGL((prefill_merge_kernel<D, false>), grid, dim3(kThreads), 0, stream, p, kWaves * 16 * NCB);
  return hipGetLastError();
}

template <int D, int KF, int NN, int SG>
hipError_t launch_one(const PrefillParams &p, const FastLayout &fl, hipStream_t stream) {
  constexpr int NCB = prefill_column_blocks(D);
  if (p.tile_queries == kWaves * 16) return launch_ncb<D, KF, NN, SG, 1>(p, fl, stream);
  if (p.tile_queries == kWaves * 16 * NCB) return launch_ncb<D, KF, NN, SG, NCB>(p, fl, stream);
  return hipErrorInvalidValue;
}

}  // namespace

int prefill_general_book_bytes(int dim) { return dim == 64 ? PSlot<64, 2, 0>::BOOKS : PSlot<128, 2, 0>::BOOKS; }

hipError_t launch_prefill(const PrefillParams &p, const FastLayout &fl, int nn, int sg, hipStream_t stream) {
  const int D = p.dim;
  if (nn < 0) return D == 64 ? launch_one<64, 2, 0, 1>(p, fl, stream) : launch_one<128, 2, 0, 1>(p, fl, stream);
  if (p.key_format == 0) return D == 64 ? launch_one<64, 0, 0, 2>(p, fl, stream) : launch_one<128, 0, 0, 4>(p, fl, stream);
#define BGTQ_PREFILL(DD, N, S) \
  if (D == DD && nn == N && sg == S) return launch_one<DD, 1, N, S>(p, fl, stream);
  BGTQ_PREFILL(64, 1, 1)
  BGTQ_PREFILL(64, 2, 2)
  BGTQ_PREFILL(64, 0, 2)
  BGTQ_PREFILL(64, 2, 1)
  BGTQ_PREFILL(64, 0, 1)
  BGTQ_PREFILL(128, 2, 2)
  BGTQ_PREFILL(128, 4, 4)
  BGTQ_PREFILL(128, 0, 4)
  BGTQ_PREFILL(128, 4, 2)
  BGTQ_PREFILL(128, 0, 2)
#undef BGTQ_PREFILL
  return hipErrorInvalidValue;
}

}  // namespace bgtq
