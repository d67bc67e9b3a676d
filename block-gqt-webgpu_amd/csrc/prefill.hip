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
// block. Each wave rebuilds the K operand from LDS lookup tables of fp16
// (hi, lo) centroid splits once per 16-token x 32-dim step and reuses it for
// its NCB column blocks: QK as 16x16x32 f16 MFMAs (hi*hi + lo*hi + hi*lo),
// per-token group scales, the causal mask, an online softmax in the log2
// domain and PV as MFMAs with V read transposed (ds_read_b64_tr_b16).
// Splits whose tokens lie past every query of the tile exit at once; a tile
// with one active split writes its output directly, otherwise the last
// workgroup of the tile to arrive merges the (m, l, o) partials by
// log-sum-exp.
//
// Queries arrive rotated into the code domain and scaled by 1/sqrt(d)
// (rotate_q_kernel): with k = ((c*s) @ R)[inv_perm] (the reconstruction of
// src/reference/production_math.py:27-31), q.k = sum_g s_g sum_{j in g}
// c_j[code_j] (R q[perm])_j. The arithmetic is that of
// src/reference/attention.py:5-22 with causal positions.
#include <hip/hip_fp16.h>

#include "bgtq_internal.h"
#include "gfx950_common.h"

namespace bgtq {
namespace {

using namespace gfx;

constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;
constexpr int kChunk = 32;  // tokens per block: two 16-token MFMA tiles
constexpr int kRing = 6;    // shared LDS buffers: compute one, four in flight, one draining

// One ring buffer: V block, K block, FP16 scales; every wave DMAs a quarter.
template <int D, int KF, int NN>
struct PSlot {
  static constexpr int KS = D / 32, DT = D / 16, PR = D / 8;
  static constexpr int VBYTES = kChunk * D * 2;
  static constexpr int VI = VBYTES / 1024;  // 16-byte DMA instructions per V block
  static constexpr int VW = VI / kWaves;    // ... per wave
  static constexpr int RB = KF == 1 ? NN * 16 + (KS - NN) * 32 : 2 * D;  // K row bytes
  static constexpr int KBYTES = kChunk * RB;
  static constexpr int KQ = KBYTES / kWaves;  // K bytes per wave
  static constexpr int KW = KF == 1 ? (KQ + 1023) / 1024 : VW;
  static constexpr int KLAST = KF == 1 ? (KQ - (KW - 1) * 1024) / 16 : 64;  // lanes of the last K instruction
  static constexpr int NBYTES = KF == 1 ? kChunk * 4 : 0;
  static constexpr int BYTES = VBYTES + KBYTES + NBYTES;
  static constexpr int LW = VW + KW + (KF == 1 ? 1 : 0);  // DMA instructions per wave per block
  static constexpr int RING = kRing;
  static constexpr int AHEAD = RING - 2;
  static constexpr int TABLES = KF == 1 ? KS * 2048 : 0;
  static constexpr int LDS = RING * BYTES + TABLES;
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

// KF: 1 = packed codes, 0 = FP16 K rows. NN: leading nibble K-steps. SG:
// K-steps in group 0. NCB: 16-query column blocks per wave.
// Two waves per SIMD (at most 256 registers each): one wave's softmax overlaps
// the other's matrix-core work.
template <int D, int KF, int NN, int SG, int NCB>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2, 2))) void prefill_kernel(
    PrefillParams p, FastLayout fl) {
  using Sl = PSlot<D, KF, NN>;
  constexpr int KS = Sl::KS, DT = Sl::DT, PR = Sl::PR, RB = Sl::RB, AHEAD = Sl::AHEAD;
  constexpr int QW = NCB * 16, QT = kWaves * QW;
  static_assert(NN >= 0 && NN <= KS && SG >= 1 && SG <= KS, "layout");
  extern __shared__ __align__(16) uint8_t smem[];

  const int split = blockIdx.x, tile = blockIdx.y, unit = blockIdx.z;
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
  const int t_lo = split * SP, t_hi = min(t_lo + SP, e_tile);
  const int n_blocks = (t_hi - t_lo + kChunk - 1) / kChunk;
  const DevTables *T = KF == 1 ? p.tables[kv] : nullptr;
  uint8_t *tabs = smem + Sl::RING * Sl::BYTES;

  // ---------------- streams of this unit ----------------
  const _Float16 *v_base = static_cast<const _Float16 *>(p.v) + b * p.v_seq_stride + kv * p.v_head_stride;
  const uint8_t *k_base = KF == 1 ? p.packed + b * p.packed_seq_stride + kv * p.packed_head_stride
                                  : reinterpret_cast<const uint8_t *>(static_cast<const _Float16 *>(p.k) +
                                                                      b * p.k_seq_stride + kv * p.k_head_stride);
  const uint16_t *n_base = KF == 1 ? p.norms + b * p.norms_seq_stride + kv * p.norms_head_stride : nullptr;
  // Swizzled FP16 row pieces of this wave's V (and FP16 K) instructions:
  // instruction k, lane i fills LDS piece 64k + i = (row r, slot c) with
  // global piece c ^ swz(r).
  uint32_t voff_rows[Sl::VW];
#pragma unroll
  for (int kk = 0; kk < Sl::VW; ++kk) {
    const int P = 64 * (wave * Sl::VW + kk) + lane, r = P / PR, c = P % PR;
    voff_rows[kk] = r * (2 * D) + ((c ^ swz<D>(r)) * 16);
  }
  auto issue = [&](int i) {
    const int c0 = t_lo + i * kChunk;
    const uint32_t rest = (uint32_t)min(T_b - c0, kChunk);  // tokens of the block inside the history (> 0)
    uint8_t *sb = smem + (i % Sl::RING) * Sl::BYTES;
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
  // MFMA lookup tables of the K-steps' books into LDS (wave 0), this wave's
  // query operands into registers, then one wait for everything.
  if (KF == 1 && wave == 0) {
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      const uint8_t *src = tables_mfma(T) + fl.book[s] * kMfmaTableBytes + (s < NN ? 0 : 2048);
      const __amdgpu_buffer_rsrc_t rt = rsrc(src, s < NN ? 2048 : 1024);
      dma16(rt, tabs + s * 2048, lane * 16, 0);
      if (s < NN) dma16(rt, tabs + s * 2048 + 1024, 1024 + lane * 16, 0);
    }
  }
  // B operand of QK for column block cb: lane holds qr[query col][32 s + 8 gq + 0..7].
  bool valid[NCB];
  int64_t gqi[NCB];  // global query row of this lane's column query
  f32x4 qv[NCB][KS][2];
#pragma unroll
  for (int cb = 0; cb < NCB; ++cb) {
    const int qi = q0 + wave * QW + cb * 16 + col;
    valid[cb] = qi < nq;
    const int row = valid[cb] ? qi / G : 0, h = valid[cb] ? qi - row * G : 0;
    gqi[cb] = ((int64_t)b * rows + row) * Hq + kv * G + h;
    const f32x4 *src = reinterpret_cast<const f32x4 *>(p.qr + gqi[cb] * D);
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      qv[cb][s][0] = valid[cb] ? src[8 * s + 2 * gq] : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
      qv[cb][s][1] = valid[cb] ? src[8 * s + 2 * gq + 1] : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    }
  }
  const int ec = KF == 1 ? T->cent_exp : 0;
  half8 qhi[NCB][KS], qlo[NCB][KS];
  float kq[NCB];  // log2-domain logit = (sum_g s_g acc_g) * kq
  int lim[NCB];   // exclusive token end of this lane's column query inside the split
  int lim_min = t_hi;
#pragma unroll
  for (int cb = 0; cb < NCB; ++cb) {
    float qmax = 0.0f;
#pragma unroll
    for (int s = 0; s < KS; ++s)
#pragma unroll
      for (int k = 0; k < 4; ++k) qmax = fmaxf(qmax, fmaxf(fabsf(qv[cb][s][0][k]), fabsf(qv[cb][s][1][k])));
    qmax = col_max(qmax);
    const int eq = qmax > 0.0f ? 14 - (int)ceilf(__builtin_log2f(qmax)) : 0;
    const float qsc = __builtin_ldexpf(1.0f, eq);
#pragma unroll
    for (int s = 0; s < KS; ++s)
#pragma unroll
      for (int jv = 0; jv < 8; ++jv) {
        const float x = qv[cb][s][jv >> 2][jv & 3] * qsc;
        qhi[cb][s][jv] = (_Float16)x;
        qlo[cb][s][jv] = (_Float16)(x - (float)qhi[cb][s][jv]);
      }
    kq[cb] = __builtin_ldexpf(kLog2e, -(eq + ec));
    const int qi = q0 + wave * QW + cb * 16 + col;
    lim[cb] = valid[cb] ? min(start + qi / G + 1, t_hi) : t_hi;
    lim_min = min(lim_min, lim[cb]);
  }
  // Wave-uniform: blocks reaching past lim_min need the per-query mask.
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) lim_min = min(lim_min, __shfl_xor(lim_min, o, 64));
  wait_vm<0>();
  __syncthreads();

  const uint32_t *tn = reinterpret_cast<const uint32_t *>(tabs);
  const _Float16 *tb = reinterpret_cast<const _Float16 *>(tabs);
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

  for (int i = 0; i < n_blocks; ++i) {
    const int c0 = t_lo + i * kChunk;
    // Block i + AHEAD goes to the buffer of block i - 2, which every wave
    // finished before the barrier of iteration i - 1.
    if (i + AHEAD < n_blocks) issue(i + AHEAD);
    wait_blocks<Sl::LW, AHEAD>(min(n_blocks - 1 - i, AHEAD));
    __syncthreads();  // every wave's quarter of block i has landed
    const uint8_t *sb = smem + (i % Sl::RING) * Sl::BYTES;
    const uint8_t *kbuf = sb + Sl::VBYTES;

    float x[NCB][8];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      f32x4 acc[NCB][2];
#pragma unroll
      for (int cb = 0; cb < NCB; ++cb) {
        acc[cb][0] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        acc[cb][1] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
      }
      const int t = 16 * u + col;  // A-operand row (token) of this lane
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        const int g = s < SG ? 0 : 1;
        if (KF == 1) {
          u32x4 hi, lo;
          if (s < NN) {
            const uint32_t w = *reinterpret_cast<const uint32_t *>(kbuf + t * RB + 16 * s + 4 * gq);
            const uint32_t *t32 = tn + s * 512;
#pragma unroll
            for (int k = 0; k < 4; ++k) {
              const uint32_t e = (w >> (8 * k)) & 255u;
              hi[k] = t32[e];
              lo[k] = t32[256 + e];
            }
          } else {
            const u32x2 w = *reinterpret_cast<const u32x2 *>(kbuf + t * RB + 16 * NN + 32 * (s - NN) + 8 * gq);
            const _Float16 *t16 = tb + s * 1024;
            half8 h8, l8;
#pragma unroll
            for (int k = 0; k < 8; ++k) {
              const uint32_t e = (w[k >> 2] >> (8 * (k & 3))) & 255u;
              h8[k] = t16[e];
              l8[k] = t16[256 + e];
            }
            hi = __builtin_bit_cast(u32x4, h8);
            lo = __builtin_bit_cast(u32x4, l8);
          }
          const half8 ah = __builtin_bit_cast(half8, hi), al = __builtin_bit_cast(half8, lo);
#pragma unroll
          for (int cb = 0; cb < NCB; ++cb) {
            acc[cb][g] = mfma(ah, qhi[cb][s], acc[cb][g]);
            acc[cb][g] = mfma(al, qhi[cb][s], acc[cb][g]);
            acc[cb][g] = mfma(ah, qlo[cb][s], acc[cb][g]);
          }
        } else {
          const int piece = 4 * s + gq;
          const half8 a = *reinterpret_cast<const half8 *>(kbuf + t * (2 * D) + ((piece ^ swz<D>(t)) * 16));
#pragma unroll
          for (int cb = 0; cb < NCB; ++cb) {
            acc[cb][0] = mfma(a, qhi[cb][s], acc[cb][0]);
            acc[cb][0] = mfma(a, qlo[cb][s], acc[cb][0]);
          }
        }
      }
      // logits of this lane: query col of each block, tokens c0 + 16u + 4gq + r
      u32x4 nr{0u, 0u, 0u, 0u};
      if (KF == 1) nr = *reinterpret_cast<const u32x4 *>(kbuf + Sl::KBYTES + (16 * u + 4 * gq) * 4);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        float s0 = 1.0f, s1 = 1.0f;
        if (KF == 1) {
          s0 = __half2float(__ushort_as_half((uint16_t)(nr[r] & 0xffffu)));
          s1 = __half2float(__ushort_as_half((uint16_t)(nr[r] >> 16)));
        }
#pragma unroll
        for (int cb = 0; cb < NCB; ++cb) {
          float v;
          if (KF == 1 && SG < KS) v = __builtin_fmaf(s1, acc[cb][1][r], s0 * acc[cb][0][r]);
          else v = s0 * acc[cb][0][r];
          x[cb][4 * u + r] = v * kq[cb];
        }
      }
    }
    if (c0 + kChunk > lim_min) {
#pragma unroll
      for (int cb = 0; cb < NCB; ++cb)
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const int tok = c0 + 16 * (j >> 2) + 4 * gq + (j & 3);
          x[cb][j] = tok < lim[cb] ? x[cb][j] : -INFINITY;
        }
    }
    // online softmax (log2 domain) per column query, then P as hi/lo A operands
    half8 pha[NCB], pla[NCB];
#pragma unroll
    for (int cb = 0; cb < NCB; ++cb) {
      const float *xc = x[cb];
      const float mloc = fmaxf(fmaxf(fmaxf(xc[0], xc[1]), fmaxf(xc[2], xc[3])),
                               fmaxf(fmaxf(xc[4], xc[5]), fmaxf(xc[6], xc[7])));
      const float m_new = fmaxf(m_run[cb], col_max(mloc));
      const float alpha = m_new == -INFINITY ? 1.0f : __builtin_amdgcn_exp2f(m_run[cb] - m_new);
      const float mb = (m_new == -INFINITY ? 0.0f : m_new) - 15.0f;
      float pr[8], psum = 0.0f;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        pr[j] = __builtin_amdgcn_exp2f(xc[j] - mb);
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
    // PV: B operand = V[tokens of this lane's P slots][16 dt + col], read transposed.
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
      const int piece = 2 * dt + tpiece;
      const fp16x4 v0 = __builtin_amdgcn_ds_read_tr16_b64_v4f16(
          (lds_fp16x4 *)(sb + trow * (2 * D) + ((piece ^ swz<D>(trow)) * 16) + thalf));
      const fp16x4 v1 = __builtin_amdgcn_ds_read_tr16_b64_v4f16(
          (lds_fp16x4 *)(sb + (16 + trow) * (2 * D) + ((piece ^ swz<D>(16 + trow)) * 16) + thalf));
      const u32x2 a0 = __builtin_bit_cast(u32x2, v0), a1 = __builtin_bit_cast(u32x2, v1);
      const half8 vb = __builtin_bit_cast(half8, u32x4{a0[0], a0[1], a1[0], a1[1]});
#pragma unroll
      for (int cb = 0; cb < NCB; ++cb) {
        O[cb][dt] = mfma(pha[cb], vb, O[cb][dt]);
        O[cb][dt] = mfma(pla[cb], vb, O[cb][dt]);
      }
    }
  }

  // ---------------- epilogue ----------------
  // O row 4 gq + r of block cb is query (cb, 4 gq + r); its (m, l) live in
  // column lane 4 gq + r.
  const int S = p.splits;
#pragma unroll
  for (int cb = 0; cb < NCB; ++cb) {
    const float l_tot = col_sum(l_run[cb]);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int qr_lane = 4 * gq + r;
      const float lr = __shfl(l_tot, qr_lane, 64);
      const bool ok = __shfl((int)valid[cb], qr_lane, 64) != 0;
      const int64_t g_row = __shfl(gqi[cb], qr_lane, 64);
      if (!ok) continue;
      if (n_act == 1) {
        const float inv = 1.0f / lr;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) p.out[g_row * D + 16 * dt + col] = O[cb][dt][r] * inv;
      } else {
        float *pp = p.part + (g_row * S + split) * (D + 2);
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) coherent_store(pp + 2 + 16 * dt + col, O[cb][dt][r] * (1.0f / kPScale));
      }
    }
    if (n_act > 1 && gq == 0 && valid[cb]) {
      float *pp = p.part + (gqi[cb] * S + split) * (D + 2);
      coherent_store(pp, m_run[cb]);
      coherent_store(pp + 1, l_tot * (1.0f / kPScale));
    }
  }
  if (n_act == 1) return;
  // Last workgroup of this tile to finish merges its splits. Every thread
  // waits for its partial stores before the arrival is counted.
  __shared__ int last;
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  uint32_t *counter = p.counters + (int64_t)unit * p.tiles + tile;
  if (tid == 0)
    last = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == (unsigned)(n_act - 1);
  __syncthreads();
  if (!last) return;
  // One wave per query: lane s holds split s's (m, l); the o rows are read
  // coalesced, eight splits at a time.
  constexpr int DL = D / 64;  // output dims per lane
  for (int qq = wave; qq < n_valid; qq += kWaves) {
    const int qi = q0 + qq, row = qi / G, h = qi - row * G;
    const int64_t g_row = ((int64_t)b * rows + row) * Hq + kv * G + h;
    float *pp = p.part + g_row * S * (D + 2);
    const float ms = lane < n_act ? coherent_load(pp + lane * (D + 2)) : -INFINITY;
    const float ls = lane < n_act ? coherent_load(pp + lane * (D + 2) + 1) : 0.0f;
    float M = ms;
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) M = fmaxf(M, __shfl_xor(M, o, 64));
    float w = ms == -INFINITY ? 0.0f : exp2f(ms - M);
    float L = w * ls;
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) L += __shfl_xor(L, o, 64);
    w = w / L;
    float acc[DL];
#pragma unroll
    for (int k = 0; k < DL; ++k) acc[k] = 0.0f;
    for (int s0 = 0; s0 < n_act; s0 += 8) {
      float o[8][DL];
#pragma unroll
      for (int k = 0; k < 8; ++k)
#pragma unroll
        for (int e = 0; e < DL; ++e)
          o[k][e] = s0 + k < n_act ? coherent_load(pp + (s0 + k) * (D + 2) + 2 + lane + 64 * e) : 0.0f;
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const float wk = __shfl(w, min(s0 + k, 63), 64);
#pragma unroll
        for (int e = 0; e < DL; ++e) acc[e] = __builtin_fmaf(o[k][e], s0 + k < n_act ? wk : 0.0f, acc[e]);
      }
    }
#pragma unroll
    for (int e = 0; e < DL; ++e) p.out[g_row * D + lane + 64 * e] = acc[e];
  }
  if (tid == 0) __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <int D, int KF, int NN, int SG>
hipError_t launch_one(const PrefillParams &p, const FastLayout &fl, hipStream_t stream) {
  constexpr int NCB = prefill_column_blocks(D);
  constexpr int lds = PSlot<D, KF, NN>::LDS;
  static const hipError_t allowed = hipFuncSetAttribute((const void *)prefill_kernel<D, KF, NN, SG, NCB>,
                                                        hipFuncAttributeMaxDynamicSharedMemorySize, lds);
  if (allowed != hipSuccess) {
    (void)hipGetLastError();
    return allowed;
  }
  dim3 grid((unsigned)p.splits, (unsigned)p.tiles, (unsigned)(p.batch * p.kv_heads));
  hipLaunchKernelGGL((prefill_kernel<D, KF, NN, SG, NCB>), grid, dim3(kThreads), lds, stream, p, fl);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_prefill(const PrefillParams &p, const FastLayout &fl, int nn, int sg, hipStream_t stream) {
  const int D = p.dim;
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
