// Chunked-prefill attention for gfx950 on the matrix cores.
//
// A chunk of `rows` new query rows of a sequence, at positions start ..
// start+rows-1, attends causally to the sequence's whole history: row r sees
// tokens 0 .. start+r (src/model/compressed-dot.wgsl:28, softmax end of
// src/model/attention.wgsl:19). The queries of one (sequence, KV head) unit are
// its rows x G GQA heads, flattened as qi = row * G + h (the item order of
// src/model/compressed-dot.wgsl:26-27).
//
// Grid: `ranges` workgroups, each taking an equal range of the work (every
// (KV head, sequence, query tile)'s causal history in 32-token blocks,
// flattened), so they all end together however unequal the tiles' histories
// are. A workgroup of four waves holds a tile of 4 x NCB x 16 queries in
// registers (each wave NCB 16-query MFMA column blocks) and streams the
// tile's blocks of its range through a ring of LDS buffers shared by the four
// waves: packed codes, FP16 scales and FP16 V go HBM -> LDS with
// buffer_load ... lds, each wave issuing a quarter of every buffer, four
// buffers ahead of the one computed on, one barrier per 32-token block. A
// range crossing tiles handles them one after the other.
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
// A tile inside one range writes its output directly; a tile shared by
// several ranges leaves an (m, l, o) partial per range and
// prefill_merge_kernel combines them by log-sum-exp. The arithmetic is that
// of src/reference/attention.py:5-22 with causal positions.
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
// Online softmax with lazy rescaling: a query's running maximum m moves only
// when a block's maximum exceeds it by more than kTau (log2 units), and
// P = 2^(x - m + kPBias) stays within 2^15, so its fp16 lo part stays normal
// for the largest terms. Partials carry o and l scaled by kPOut = 2^kPBias.
constexpr int kSegmentCost = kPrefillSegmentCost;  // a segment's set-up, in 32-token blocks' worth of time
constexpr int kTauLog2 = 8;
constexpr float kTau = kTauLog2;
constexpr float kPBias = 15 - kTauLog2;
constexpr float kPOut = 1 << (15 - kTauLog2);

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
  // Packed K and its scales move as 4-byte DMAs with every lane of every wave
  // busy (no lane-masked instructions, so the compiler's waits for register
  // loads issued before the ring stay exact): the K block padded to a
  // multiple of 1 KB, the scales to 1 KB (past the block's tokens the range
  // check reads zeros).
  static constexpr int KPAD = KF >= 1 ? (KBYTES + 1023) / 1024 * 1024 : KBYTES;
  static constexpr int KW = KF >= 1 ? KPAD / 1024 : VW;  // K DMA instructions per wave
  static constexpr int NUSED = KF == 1 ? kChunk * 4 : KF == 2 ? kChunk * 16 : 0;  // scale bytes of a block
  static constexpr int NBYTES = KF >= 1 ? 1024 : 0;
  static constexpr int BYTES = VBYTES + KPAD + NBYTES;
  static constexpr int LW = VW + KW + (KF >= 1 ? 1 : 0);  // DMA instructions per wave per block
  static constexpr int BOOKS = KF >= 1 ? KS * 1024 * KF : 0;  // KF 1: 256 fp32 centroids per K-step
  static constexpr int KOP = KF >= 1 ? 2 * 2 * KS * 2048 : 0;  // [buffer][u][s]: hi 1 KB, lo 1 KB
  static constexpr int CURSOR = kWaves * 32;  // each wave's segment cursor (8 ints), after the operands
  static constexpr int FIXED = BOOKS + KOP + CURSOR;
  static constexpr int RING = 6 * BYTES + FIXED <= kLdsLimit / 2 ? 6 : 4 * BYTES + FIXED <= kLdsLimit / 2 ? 4 : 3;
  static constexpr int AHEAD = RING - 2;
  static constexpr int LDS = RING * BYTES + FIXED;
  static_assert(VI % kWaves == 0 && KBYTES % 16 == 0 && NUSED <= NBYTES, "DMA split over four waves");
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

__device__ __forceinline__ float wave_max(float v) { return col_max(row_max(v)); }

// Clamped start of sequence b's chunk: its rows end inside the K/V buffers.
__device__ __forceinline__ int seq_start(const PrefillParams &p, int b) {
  return (int)min(p.starts[b], (uint32_t)(p.max_length - p.rows));
}
// History end of query tile t's last query, relative to the chunk start.
__device__ __forceinline__ int tile_end(int nq, int QT, int G, int t) { return (min(nq, (t + 1) * QT) - 1) / G + 1; }

// Tile at position k of a sequence's tile order 0, T-1, 1, T-2, ...: the
// causal histories grow with the tile, so consecutive work ranges mix long and
// short tiles instead of one range taking many short tiles (each of which
// costs a segment's set-up).
__device__ __forceinline__ int tile_at(int k, int T) { return (k & 1) ? T - 1 - (k >> 1) : k >> 1; }

// Inclusive scan of x over the workgroup's threads; total (wave-uniform) is
// the sum over all of them. red: kWaves ints of LDS. Two workgroup barriers.
__device__ int block_incl_scan(int x, int *red, int lane, int wave, int &total) {
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int y = __shfl_up(x, o, 64);
    if (lane >= o) x += y;
  }
  if (lane == 63) red[wave] = x;
  __syncthreads();
  int off = 0, sum = 0;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) {
    const int v = red[w];
    off += w < wave ? v : 0;
    sum += v;
  }
  __syncthreads();
  total = __builtin_amdgcn_readfirstlane(sum);
  return x + off;
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

  const int G = p.G, Hq = p.q_heads, rows = p.rows;
  const int tid = threadIdx.x, lane = tid & 63, gq = lane >> 4, col = lane & 15;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int nq = rows * G;
  const int n_tiles = p.tiles, B = p.batch, KV = p.kv_heads;

  // ---------------- this workgroup's range of the work ----------------
  // The work is every (KV head, sequence, query tile)'s causal history in
  // 32-token blocks, flattened in that order (tiles in the order of
  // tile_at), each tile costing kSegmentCost blocks' worth of set-up (loading
  // and rotating its queries, filling the ring, writing its result) before
  // its blocks(b, t) = ceil((start_b + e_off(t)) / 32) blocks. Workgroup w
  // takes cost units [w R, (w + 1) R): equal shares however long the tiles
  // and however many of them a share touches, so the grid of about two
  // workgroups per compute unit ends together. Each tile a share touches is
  // a segment (queries loaded, history streamed, output or partial written);
  // only the first and the last can hold part of a tile, and their partials
  // go to the workgroup's two records. The starts are device values, so the
  // work is counted here, by all threads, before the LDS ring is in use.
  int *red = reinterpret_cast<int *>(smem);
  const int pairs = B * n_tiles;
  auto pair_blocks = [&](int k) {
    const int b = k / n_tiles, t = tile_at(k - b * n_tiles, n_tiles);
    return (seq_start(p, b) + tile_end(nq, QT, G, t) + kChunk - 1) / kChunk;
  };
  // Costs fit 31 bits (the host refuses more work).
  int w1 = 0;  // cost of one KV head over every sequence and tile
  int x1 = 0, incl1 = 0;  // this thread's pair and prefix when one round holds every pair
  for (int k0 = 0; k0 < pairs; k0 += kThreads) {
    const int x = k0 + tid < pairs ? kSegmentCost + pair_blocks(k0 + tid) : 0;
    int total;
    const int incl = block_incl_scan(x, red, lane, wave, total);
    x1 = x;
    incl1 = incl;
    w1 += total;
  }
  const int W = w1 * KV;
  // Range lengths: R for every workgroup, or, with p.first_round set (two
  // workgroups per compute unit), 3 R' for the first p.first_round workgroups
  // and 2 R' for the rest: the first workgroup dispatched to a compute unit
  // gets the larger share of its issue slots.
  const int H = p.first_round, NW = (int)gridDim.x;
  const int R = p.range_blocks > 0 ? p.range_blocks
                : H > 0          ? max((W + 3 * H + 2 * (NW - H) - 1) / (3 * H + 2 * (NW - H)), 1)
                                 : max((W + NW - 1) / NW, kPrefillMinRange);
  const int w = (int)blockIdx.x;
  const int j0 = H > 0 ? (w < H ? 3 * R * w : 3 * R * H + 2 * R * (w - H)) : w * R;
  if (j0 >= W) return;  // workgroup-uniform: before any barrier of the segments
  const int j1 = min(j0 + (H > 0 ? (w < H ? 3 * R : 2 * R) : R), W);
  // The range holding cost unit c.
  auto range_of = [&](int c) { return H > 0 ? (c < 3 * R * H ? c / (3 * R) : H + (c - 3 * R * H) / (2 * R)) : c / R; };
  int kv = j0 / w1;
  const int rem = j0 - kv * w1;
  // The (sequence, tile) pair holding cost unit rem of KV head kv, and the
  // unit's offset in that tile's cost.
  int b = 0, t = 0, off = 0;
  if (pairs <= kThreads) {  // the one round's prefixes are at hand
    const int excl = incl1 - x1;
    if (x1 > 0 && excl <= rem && rem < excl + x1) {
      red[kWaves] = tid;
      red[kWaves + 1] = rem - excl;
    }
    __syncthreads();
    const int k_hit = __builtin_amdgcn_readfirstlane(red[kWaves]);
    b = k_hit / n_tiles;
    t = k_hit - b * n_tiles;
    off = __builtin_amdgcn_readfirstlane(red[kWaves + 1]);
    __syncthreads();  // every wave has read the cursor before the ring reuses the LDS
  }
  for (int k0 = 0, base = 0; pairs > kThreads && k0 < pairs; k0 += kThreads) {
    const int k = k0 + tid;
    const int x = k < pairs ? kSegmentCost + pair_blocks(k) : 0;
    int total;
    const int excl = base + block_incl_scan(x, red, lane, wave, total) - x;
    if (x > 0 && excl <= rem && rem < excl + x) {
      red[kWaves] = k;
      red[kWaves + 1] = rem - excl;
    }
    __syncthreads();
    if (base + total > rem) {  // workgroup-uniform
      const int k_hit = __builtin_amdgcn_readfirstlane(red[kWaves]);
      b = k_hit / n_tiles;
      t = k_hit - b * n_tiles;  // position in the tile order
      off = __builtin_amdgcn_readfirstlane(red[kWaves + 1]);
      __syncthreads();  // every wave has read the cursor before the ring reuses the LDS
      break;
    }
    base += total;
  }

  // Per-wave cursor words (8 ints each) after the operand buffers.
  int *const cur_base = reinterpret_cast<int *>(smem + Sl::RING * Sl::BYTES + Sl::BOOKS + Sl::KOP);

  // One segment: blocks [blk_lo, blk_lo + n_blocks) of tile `tile` of
  // sequence b's KV head kv; whole: the tile's entire history (the output is
  // written), else the partial goes to record rec_slot of this workgroup.
  auto segment = [&](const PrefillParams &p, const int tid, const int b, const int kv, const int tile, const int blk_lo,
                     const int n_blocks, const int bt, const int rec_slot) {
    const bool whole = blk_lo == 0 && n_blocks == bt;
    const int lane = tid & 63, gq = lane >> 4, col = lane & 15;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    float one = 1.0f;  // opaque 1.0 for the mixed-precision splits
    asm volatile("" : "+s"(one));
    const int start = seq_start(p, b);  // the chunk's rows end inside the K/V buffers
    const int T_b = start + rows;
    const int q0 = tile * QT;
    const int n_valid = min(QT, nq - q0);
    const int e_tile = start + (q0 + n_valid - 1) / G + 1;  // exclusive end of the tile's last query
    const int t_lo = blk_lo * kChunk, t_hi = min(t_lo + n_blocks * kChunk, e_tile);
    const DevTables *T = KF >= 1 ? p.tables[kv] : nullptr;
    // Row bytes and scales per token (runtime for KF 2).
    // Table fields are wave-uniform: scalar values, so buffer descriptors built
    // from them need no per-lane loop.
    const int rb = KF == 2 ? __builtin_amdgcn_readfirstlane(T->row_bytes) : RB;
    const int ns = KF == 2 ? __builtin_amdgcn_readfirstlane(T->norm_stride) : 2;
    const int mc = KF == 2 ? __builtin_amdgcn_readfirstlane(T->max_centroids) : 0;  // read once, not per block
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
      const int ln = lane_id();  // recomputed here: the DMA offsets stay out of the loop's registers
      const int c0 = t_lo + i * kChunk;
      const uint32_t rest = (uint32_t)min(T_b - c0, kChunk);  // > 0: c0 < t_hi <= T_b
      uint8_t *sb = slot(i);
      const __amdgpu_buffer_rsrc_t rV = rsrc(v_base + (int64_t)c0 * D, rest * (2 * D));
#pragma unroll
      for (int kk = 0; kk < Sl::VW; ++kk) dma16(rV, sb + (wave * Sl::VW + kk) * 1024, voff_rows[kk], 0);
      uint8_t *kb = sb + Sl::VBYTES;
      if (KF >= 1) {
        // Ranges end on the access size: the range check zeroes a whole access
        // reaching past the range; the bytes past the last row lie in the same
        // aligned 4 bytes as its end (16-byte aligned bases, c0 a multiple of 32).
        const int rbk = KF == 1 ? RB : rb, nsk = KF == 1 ? 2 : ns;
        const __amdgpu_buffer_rsrc_t rK = rsrc(k_base + (int64_t)c0 * rbk, (rest * rbk + 3u) & ~3u);
        const __amdgpu_buffer_rsrc_t rN = rsrc(n_base + (int64_t)c0 * nsk, (rest * nsk * 2 + 3u) & ~3u);
#pragma unroll
        for (int kk = 0; kk < Sl::KW; ++kk) {
          const int off = (kk * kWaves + wave) * 256;
          dma4(rK, kb + off, off + ln * 4, 0);
        }
        dma4(rN, kb + Sl::KPAD + wave * 256, wave * 256 + ln * 4, 0);
      } else {
        const __amdgpu_buffer_rsrc_t rK = rsrc(k_base + (int64_t)c0 * (2 * D), rest * (2 * D));
#pragma unroll
        for (int kk = 0; kk < Sl::VW; ++kk) dma16(rK, kb + (wave * Sl::VW + kk) * 1024, voff_rows[kk], 0);
      }
    };

    // ---------------- prologue ----------------
    // Centroid books of the K-steps into LDS (wave 0, 256 floats per step);
    // this wave's queries rotated, scaled by log2(e) / sqrt(d) and split into QK
    // operands. B operand of QK step s for column block cb: lane holds query
    // col's dims 32 s + 4 gq + 0..3 and 32 s + 16 + 4 gq + 0..3.
    const int ec = KF >= 1 ? __builtin_amdgcn_readfirstlane(T->cent_exp) : 0;
    const float *tbooks =
        KF >= 1 ? reinterpret_cast<const float *>(reinterpret_cast<const uint8_t *>(T) +
                                                  __builtin_amdgcn_readfirstlane((int)T->off_books))
                : nullptr;
    // Read with the other table fields, before the query loads, whose wait it
    // would otherwise join.
    const u32x4 *rq = reinterpret_cast<const u32x4 *>(
        reinterpret_cast<const uint8_t *>(T) + (KF >= 1 ? __builtin_amdgcn_readfirstlane((int)T->off_rot_q) : 0));
    if (KF == 2 && wave == 0) {  // every book's centroids, [n_books][max_centroids] floats
      const uint32_t nbytes = (uint32_t)__builtin_amdgcn_readfirstlane(T->n_books * T->max_centroids * 4);
      const __amdgpu_buffer_rsrc_t rb_ = rsrc(tbooks, nbytes);
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
      const int mc = __builtin_amdgcn_readfirstlane(T->max_centroids);
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        const __amdgpu_buffer_rsrc_t rb = rsrc(tbooks + fl.book[s] * mc, (uint32_t)(min(mc, 256) * 4));
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
    int lim[NCB];   // exclusive token end of this lane's column query inside the segment
    int lim_min = t_hi;
    // Every column block's query loads go out together, before the ring's
    // DMAs, so the waits for them (and for the rotation operands) are not
    // held up behind the ring: a segment starts in a few memory round trips.
    f32x4 qraw[NCB][2 * KS];
#pragma unroll
    for (int cb = 0; cb < NCB; ++cb) {
      const int qi = q0 + wave * QW + cb * 16 + col;
      valid[cb] = qi < nq;
      const f32x4 *src = reinterpret_cast<const f32x4 *>(p.q + query_row(b, rows, Hq, kv, G, valid[cb] ? qi : 0) * D);
#pragma unroll
      for (int s = 0; s < KS; ++s)
#pragma unroll
        for (int hh = 0; hh < 2; ++hh)
          // Rotated in the kernel: natural order 32 s + 8 gq + 4 hh + 0..3 (the
          // rotation's k order); otherwise QK order 32 s + 16 hh + 4 gq + 0..3.
        {
          // Loaded unconditionally (an invalid query reads row 0) and then
          // selected: no lane-masked load, so the waits stay exact.
          const f32x4 v = src[rotate ? 8 * s + 2 * gq + hh : 8 * s + 4 * hh + gq];
          qraw[cb][2 * s + hh] = valid[cb] ? v : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        }
      lim[cb] = valid[cb] ? min(start + qi / G + 1, t_hi) : t_hi;
      lim_min = min(lim_min, lim[cb]);
    }
    // At d=64 the rotation operands (64 registers) load with the queries and
    // the ring's first blocks follow at once, so all those round trips
    // overlap (the DMAs are unmasked and straight-line, so the waits for the
    // loads count exactly the DMAs after them). At d=128 the operands are too
    // many to hold: they load during the rotation, and the ring starts after
    // it (a wait for a load issued after the DMAs would wait for them too).
    constexpr int RQ = D == 64 ? DT * KS * 2 : 1;
    u32x4 rqo[RQ];
    if constexpr (D == 64) {
      if (rotate) {
#pragma unroll
        for (int i = 0; i < RQ; ++i) rqo[i] = rq[((i >> 1) * 64 + lane) * 2 + (i & 1)];
      }
#pragma unroll
      for (int i = 0; i < AHEAD; ++i)
        if (i < n_blocks) issue(i);
    }
    // Scaled by log2(e) / sqrt(d) and split hi/lo with a per-query exponent:
    // the QK operands directly, or the rotation's B operands.
    int eq[NCB];
    half8 bh[NCB][KS], bl[NCB][KS];
#pragma unroll
    for (int cb = 0; cb < NCB; ++cb) {
      float qv[D / 4];  // this lane's share of the query row
      float qmax = 0.0f;
#pragma unroll
      for (int k = 0; k < D / 4; ++k) {
        qv[k] = qraw[cb][k >> 2][k & 3] * qscale;
        qmax = fmaxf(qmax, fabsf(qv[k]));
      }
      eq[cb] = split_exp(col_max(qmax));
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        if (rotate) split_scaled(qv + 8 * s, __builtin_ldexpf(1.0f, eq[cb]), bh[cb][s], bl[cb][s]);
        else split_scaled(qv + 8 * s, __builtin_ldexpf(1.0f, eq[cb]), qhi[cb][s], qlo[cb][s]);
      }
    }
    if (rotate) {
      // qr^T = Rq q^T on the matrix cores (q and Rq split hi/lo, three MFMAs
      // per step), each operand pair of Rq loaded once for all column blocks:
      // D layout, lane holds rows j = 16 n + 4 gq + r of query col.
      f32x4 qr[NCB][DT];
#pragma unroll
      for (int n = 0; n < DT; ++n) {
#pragma unroll
        for (int cb = 0; cb < NCB; ++cb) qr[cb][n] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int s = 0; s < KS; ++s) {
          const int io = (n * KS + s) * 2;
          const u32x4 *op = rq + ((n * KS + s) * 64 + lane) * 2;
          const half8 ah = __builtin_bit_cast(half8, D == 64 ? rqo[min(io, RQ - 1)] : op[0]);
          const half8 al = __builtin_bit_cast(half8, D == 64 ? rqo[min(io + 1, RQ - 1)] : op[1]);
#pragma unroll
          for (int cb = 0; cb < NCB; ++cb) {
            qr[cb][n] = mfma(ah, bh[cb][s], qr[cb][n]);
            qr[cb][n] = mfma(al, bh[cb][s], qr[cb][n]);
            qr[cb][n] = mfma(ah, bl[cb][s], qr[cb][n]);
          }
        }
      }
#pragma unroll
      for (int cb = 0; cb < NCB; ++cb) {
        float rmax = 0.0f;
#pragma unroll
        for (int n = 0; n < DT; ++n)
#pragma unroll
          for (int r = 0; r < 4; ++r) rmax = fmaxf(rmax, fabsf(qr[cb][n][r]));
        const int e2 = split_exp(col_max(rmax));
#pragma unroll
        for (int s = 0; s < KS; ++s) {
          float x[8];
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            x[r] = qr[cb][2 * s][r];
            x[4 + r] = qr[cb][2 * s + 1][r];
          }
          split_scaled(x, __builtin_ldexpf(1.0f, e2), qhi[cb][s], qlo[cb][s]);
        }
        eq[cb] += e2;
      }
    }
#pragma unroll
    for (int cb = 0; cb < NCB; ++cb) eqs[cb] = eq[cb] + ec;
    if constexpr (D != 64) {
#pragma unroll
      for (int i = 0; i < AHEAD; ++i)
        if (i < n_blocks) issue(i);
    }
    // Wave-uniform: blocks reaching past lim_min need the per-query mask.
    lim_min = wave_min(lim_min);
    // Block 0 (and the books before it) landed for every wave; the later
    // blocks stay in flight.
    wait_blocks<Sl::LW, AHEAD - 1>(min(n_blocks, AHEAD) - 1);
    lds_barrier();

    // Builds block i's K operand into buffer i & 1; returns E (2^E >= every
    // FP16 scale of the block). Thread (wave w, lane) builds the (u, s) steps
    // w + 4 k: token 16 u + col, dims 32 s + 4 gq + 0..3 and 32 s + 16 + 4 gq + 0..3.
    auto build = [&](int i, auto nib_c) -> int {
      if constexpr (KF == 1) {
        // NIB: this wave's K-steps hold nibble codes (every combo of a wave has
        // the same step s = wave % KS).
        constexpr bool NIB = decltype(nib_c)::value;
        const uint8_t *kraw = slot(i) + Sl::VBYTES;
        const uint32_t *nrm = reinterpret_cast<const uint32_t *>(kraw + Sl::KPAD);
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
          if constexpr (NIB) {
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
          split8_mix(v, one, hi, lo);
          uint8_t *dst = kb + (u * KS + s) * 2048 + lane * 16;
          *reinterpret_cast<half8 *>(dst) = hi;
          *reinterpret_cast<half8 *>(dst + 1024) = lo;
        }
        return E;
      } else if constexpr (KF == 2) {
        // Any layout: each element's code through its descriptor, times its
        // book's centroid and its group's scale of the token, 2^(ec - E).
        const uint8_t *kraw = slot(i) + Sl::VBYTES;
        const uint16_t *nrm = reinterpret_cast<const uint16_t *>(kraw + Sl::KPAD);
        // E bounds the scales of the block's tokens inside the history only: the
        // scale DMA's range is rounded up to 4 bytes, so with rest * ns odd the
        // slot also holds the first scale of the token after the history.
        const int n_in = min(T_b - (t_lo + i * kChunk), kChunk) * ns;
        float smax = 0.0f;
#pragma unroll
        for (int k = 0; k < Sl::NUSED / 2 / 64; ++k) {
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
          split8_mix(v, one, hi, lo);
          uint8_t *dst = kb + (u * KS + s) * 2048 + lane * 16;
          *reinterpret_cast<half8 *>(dst) = hi;
          *reinterpret_cast<half8 *>(dst + 1024) = lo;
        }
        return E;
      } else {
        return 0;
      }
    };
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

    // One 32-token block with E_blk its scale exponent; returns block i + 1's.
    // Branch-free phases, so the scheduler can overlap a wave's matrix-core and
    // vector work: QK of block i with the K-operand build of block i + 1 (into
    // the other operand buffer; built past the last block too, from a stale but
    // in-bounds ring slot) and the block maxima; a rescale of the running sums
    // only when a query's maximum grew by more than 2^kTau (one wave-uniform
    // branch per block); then per column block the exponentials, their fp16
    // split and its PV products.
    auto step = [&](int i, int E_blk, auto masked, auto nib_c) -> int {
      constexpr bool MASK = decltype(masked)::value;
      const int c0 = t_lo + i * kChunk;
      const uint8_t *sb = slot(i);
      // V of this block, read transposed for the PV B operands (lane: V[tokens
      // of its P slots][16 dt + col]). At d=64 issued after QK, so the latency
      // hides under the build and the maxima; at d=128 after the rescale (32
      // more registers live across the maxima would spill).
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
      if constexpr (D == 64) read_v();
      const int E_next = build(i + 1, nib_c);
      // Raw logits of query col (tokens c0 + 16u + 4gq + r) and each query's
      // block maximum in the scaled log2 domain.
      float xr[NCB][8], Cb[NCB], bmax[NCB];
      bool grow = false;
#pragma unroll
      for (int cb = 0; cb < NCB; ++cb) {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          xr[cb][j] = acc[cb][j >> 2][j & 3];
          if constexpr (MASK) {
            const int tok = c0 + 16 * (j >> 2) + 4 * gq + (j & 3);
            xr[cb][j] = tok < lim[cb] ? xr[cb][j] : -INFINITY;
          }
        }
        Cb[cb] = __builtin_ldexpf(1.0f, E_blk - eqs[cb]);
        const float mloc = fmaxf(fmaxf(fmaxf(xr[cb][0], xr[cb][1]), fmaxf(xr[cb][2], xr[cb][3])),
                                 fmaxf(fmaxf(xr[cb][4], xr[cb][5]), fmaxf(xr[cb][6], xr[cb][7])));
        bmax[cb] = col_max(mloc) * Cb[cb];
        grow |= bmax[cb] > m_run[cb] + kTau;
      }
      if (__builtin_amdgcn_ballot_w64(grow)) {
#pragma unroll
        for (int cb = 0; cb < NCB; ++cb) {
          const float m_new = bmax[cb] > m_run[cb] + kTau ? bmax[cb] : m_run[cb];
          const float alpha = m_new == m_run[cb] ? 1.0f : __builtin_amdgcn_exp2f(m_run[cb] - m_new);
          l_run[cb] *= alpha;
          m_run[cb] = m_new;
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const float ar = __shfl(alpha, 4 * gq + r, 64);
#pragma unroll
            for (int dt = 0; dt < DT; ++dt) O[cb][dt][r] *= ar;
          }
        }
      }
      if constexpr (D != 64) read_v();
      // P = 2^(x C - m + kPBias) <= 2^15: no logit exceeds its running maximum
      // by more than kTau. PV: B operand = the transposed V reads; dt's pair has
      // landed once at most the 2 (DT - 1 - dt) newer reads are in flight.
#pragma unroll
      for (int cb = 0; cb < NCB; ++cb) {
        const float nmb = kPBias - (m_run[cb] == -INFINITY ? 0.0f : m_run[cb]);
        float pr[8], psum = 0.0f;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          pr[j] = __builtin_amdgcn_exp2f(__builtin_fmaf(xr[cb][j], Cb[cb], nmb));
          psum += pr[j];
        }
        l_run[cb] += psum;
        u32x4 ph, pl;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          uint32_t h, l;
          split2_mix(pr[2 * k], pr[2 * k + 1], one, h, l);
          ph[k] = h;
          pl[k] = l;
        }
        const half8 pha = __builtin_bit_cast(half8, ph), pla = __builtin_bit_cast(half8, pl);
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
          if (cb == 0) wait_dt<DT>(dt, vt[dt][0], vt[dt][1]);
          const u32x2 a0 = vt[dt][0], a1 = vt[dt][1];
          const half8 vb = __builtin_bit_cast(half8, u32x4{a0[0], a0[1], a1[0], a1[1]});
          O[cb][dt] = mfma(pha, vb, O[cb][dt]);
          O[cb][dt] = mfma(pla, vb, O[cb][dt]);
        }
      }
      return E_next;
    };

    // The main loop, specialised for this wave's build kind.
    auto run = [&](auto nib_c) {
      int E_cur = build(0, nib_c);
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
        if (t_lo + i * kChunk + kChunk > lim_min) E_cur = step(i, E_cur, std::true_type{}, nib_c);
        else E_cur = step(i, E_cur, std::false_type{}, nib_c);
      }
    };
    if constexpr (KF == 1) {
      static_assert(kWaves % KS == 0, "one K-step per wave in the build");
      if (wave % KS < NN) run(std::true_type{});
      else run(std::false_type{});
    } else {
      run(std::false_type{});
    }

    // ---------------- epilogue ----------------
    // O row 4 gq + r of block cb is query (cb, 4 gq + r); its (m, l) live in
    // column lane 4 gq + r. A whole tile: the output; else the partial, per
    // query of the tile (m, l, o[D]) in record rec_slot of this workgroup.
    float *rec = p.part + ((int64_t)blockIdx.x * 2 + rec_slot) * QT * (D + 2);
#pragma unroll
    for (int cb = 0; cb < NCB; ++cb) {
      const float l_tot = col_sum(l_run[cb]);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int qr_lane = 4 * gq + r;
        const float lr = __shfl(l_tot, qr_lane, 64);
        const int qt = wave * QW + cb * 16 + qr_lane;
        if (q0 + qt >= nq) continue;
        if (whole) {
          const int64_t g_row = query_row(b, rows, Hq, kv, G, q0 + qt);
          const float inv = 1.0f / lr;
#pragma unroll
          for (int dt = 0; dt < DT; ++dt) p.out[g_row * D + 16 * dt + col] = O[cb][dt][r] * inv;
        } else {
#pragma unroll
          for (int dt = 0; dt < DT; ++dt) rec[qt * (D + 2) + 2 + 16 * dt + col] = O[cb][dt][r] * (1.0f / kPOut);
        }
      }
      if (!whole && gq == 0 && valid[cb]) {
        float *pm = rec + (wave * QW + cb * 16 + col) * (D + 2);
        pm[0] = m_run[cb];
        pm[1] = l_tot * (1.0f / kPOut);
      }
    }
  };

  // ---------------- segments ----------------
  // The cursor lives in this wave's LDS words rather than in registers, so
  // nothing of it is held across a segment.
  int *cur = cur_base + 8 * wave;
  if (lane == 0) {
    cur[0] = j0;
    cur[1] = b;
    cur[2] = t;
    cur[3] = kv;
    cur[4] = off;
  }
  for (bool first = true;;) {
    const int j = __builtin_amdgcn_readfirstlane(cur[0]);
    if (j >= j1) break;  // workgroup-uniform
    const int sb = __builtin_amdgcn_readfirstlane(cur[1]), sk = __builtin_amdgcn_readfirstlane(cur[2]);
    const int skv = __builtin_amdgcn_readfirstlane(cur[3]), soff = __builtin_amdgcn_readfirstlane(cur[4]);
    const int st = tile_at(sk, n_tiles);
    const int bt = (seq_start(p, sb) + tile_end(nq, QT, G, st) + kChunk - 1) / kChunk;
    // This range's part of the tile's cost, [soff, cend), and its blocks.
    const int cend = min(kSegmentCost + bt, soff + (j1 - j));
    const int blk = max(soff - kSegmentCost, 0), n = max(cend - kSegmentCost, 0) - blk;
    const int slot = first ? 0 : 1;
    if (n > 0 && blk == 0 && tid == 0 && gridDim.x > 1) {
      // The merge finds a tile's partials from here: workgroups w_first ..
      // w_last (those holding the tile's first and last block), the first
      // one's in its record slot, the others' in slot 0.
      const int c_first = j - soff + kSegmentCost;  // cost unit of the tile's block 0
      int4 *info = reinterpret_cast<int4 *>(p.tile_info) + ((int64_t)skv * B + sb) * n_tiles + st;
      *info = int4{(int)blockIdx.x, range_of(c_first + bt - 1), slot, 0};
    }
    if (lane == 0) {  // the next segment: the following tile, from its start
      const bool wrap_t = sk + 1 == n_tiles, wrap_b = wrap_t && sb + 1 == B;
      cur[0] = j + (cend - soff);
      cur[1] = wrap_t ? (wrap_b ? 0 : sb + 1) : sb;
      cur[2] = wrap_t ? 0 : sk + 1;
      cur[3] = wrap_b ? skv + 1 : skv;
      cur[4] = 0;
    }
    if (n > 0) {  // a range can end inside a tile's set-up share, holding none of its blocks
      // Every wave is done with the previous segment's ring, books and operands.
      if (!first) lds_barrier();
      // The thread index goes in through an opaque copy, so per-lane offsets
      // are recomputed per segment rather than held in registers across it.
      int tid_s = tid;
      asm volatile("" : "+v"(tid_s));
      segment(p, tid_s, sb, skv, st, blk, n, bt, slot);
      first = false;
    }
  }
}

// LSE merge of the tiles whose history several ranges shared. Grid (unit,
// tile x QT / 16): a workgroup takes 16 queries of a tile, a thread one
// query's four consecutive dims per 64, every record's loads in flight at
// once in rounds of four, merged online (a running maximum rescales what came
// before). The tile's records are those of workgroups w_first .. w_last, the
// first one's in the slot the tile table names, the others' in slot 0, each
// (m, l, o[D]) per query of the tile with o and l scaled by 2^-kPBias. Tiles
// one workgroup held whole were written by it: their workgroups exit.
template <int D>
__global__ __launch_bounds__(kThreads) void prefill_merge_kernel(PrefillParams p) {
  constexpr int QPW = kThreads / 16;  // queries per workgroup: 16 threads each
  constexpr int DL = D / 64;          // float4 pieces per thread
  const int QT = p.tile_queries, groups = QT / QPW;
  const int unit = blockIdx.y, tile = blockIdx.x / groups;
  const int b = unit / p.kv_heads, kv = unit - b * p.kv_heads;
  const int G = p.G, rows = p.rows, nq = rows * G;
  const int4 info = reinterpret_cast<const int4 *>(p.tile_info)[((int64_t)kv * p.batch + b) * p.tiles + tile];
  const int n = info.y - info.x + 1;
  if (n == 1) return;
  const int qt = (blockIdx.x - tile * groups) * QPW + (threadIdx.x >> 4), c = threadIdx.x & 15;
  const int qi = tile * QT + qt;
  if (qi >= nq) return;
  const int64_t rs = (int64_t)QT * (D + 2);  // floats per record
  const float *first = p.part + ((int64_t)info.x * 2 + info.z) * rs + (int64_t)qt * (D + 2);
  const float *rest = p.part + ((int64_t)info.x + 1) * 2 * rs + (int64_t)qt * (D + 2);
  float M = -INFINITY, L = 0.0f;
  f32x4 acc[DL];
#pragma unroll
  for (int e = 0; e < DL; ++e) acc[e] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  for (int k0 = 0; k0 < n; k0 += 4) {
    float m[4], l[4];
    f32x4 o[4][DL];
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      const int k = min(k0 + kk, n - 1);
      const float *r = k == 0 ? first : rest + (int64_t)(k - 1) * 2 * rs;
      m[kk] = k0 + kk < n ? r[0] : -INFINITY;
      l[kk] = r[1];
#pragma unroll
      for (int e = 0; e < DL; ++e) {  // dims 64 e + 4 c .. + 3 (the row's o starts 8 bytes in)
        const float *src = r + 2 + 64 * e + 4 * c;
        o[kk][e] = f32x4{src[0], src[1], src[2], src[3]};
      }
    }
    float Mn = M;
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) Mn = fmaxf(Mn, m[kk]);
    const float sc = M == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(M - Mn);
    L *= sc;
#pragma unroll
    for (int e = 0; e < DL; ++e) acc[e] *= sc;
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      const float w = m[kk] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m[kk] - Mn);
      L = __builtin_fmaf(w, l[kk], L);
#pragma unroll
      for (int e = 0; e < DL; ++e) acc[e] += o[kk][e] * w;
    }
    M = Mn;
  }
  const float inv_l = 1.0f / L;
  float *out = p.out + query_row(b, rows, p.q_heads, kv, G, qi) * D;
#pragma unroll
  for (int e = 0; e < DL; ++e) *reinterpret_cast<f32x4 *>(out + 64 * e + 4 * c) = acc[e] * inv_l;
}

// The same merge for launches with few queries: one wave per query, every
// record's (m, l) pair in one lane and every record's o row loaded in one
// round (record k < SMAX reads record min(k, n - 1), whose weight is zero
// past n); tiles with more than SMAX records take the rounds above instead.
template <int D, int SMAX>
__global__ __launch_bounds__(kThreads) void prefill_merge_one_round_kernel(PrefillParams p) {
  constexpr int DL = D / 64;
  const int unit = blockIdx.y;
  const int b = unit / p.kv_heads, kv = unit - b * p.kv_heads;
  const int G = p.G, rows = p.rows, nq = rows * G, QT = p.tile_queries;
  const int lane = threadIdx.x & 63;
  const int qi = blockIdx.x * kWaves + (threadIdx.x >> 6);
  if (qi >= nq) return;
  const int tile = qi / QT, qt = qi - tile * QT;
  const int4 info = reinterpret_cast<const int4 *>(p.tile_info)[((int64_t)kv * p.batch + b) * p.tiles + tile];
  const int n = info.y - info.x + 1;
  if (n == 1) return;
  const int64_t rs = (int64_t)QT * (D + 2);  // floats per record
  const float *first = p.part + ((int64_t)info.x * 2 + info.z) * rs + (int64_t)qt * (D + 2);
  const float *rest = p.part + ((int64_t)info.x + 1) * 2 * rs + (int64_t)qt * (D + 2);
  auto rec = [&](int k) { return k == 0 ? first : rest + (int64_t)(k - 1) * 2 * rs; };
  float *out = p.out + query_row(b, rows, p.q_heads, kv, G, qi) * D;
  if (n > SMAX) {  // wave-uniform: online rounds of eight records
    float M = -INFINITY, L = 0.0f, acc[DL];
#pragma unroll
    for (int e = 0; e < DL; ++e) acc[e] = 0.0f;
    for (int k0 = 0; k0 < n; k0 += 8) {
      float m[8], l[8], o[8][DL];
#pragma unroll
      for (int kk = 0; kk < 8; ++kk) {
        const float *r = rec(min(k0 + kk, n - 1));
        m[kk] = k0 + kk < n ? r[0] : -INFINITY;
        l[kk] = r[1];
#pragma unroll
        for (int e = 0; e < DL; ++e) o[kk][e] = r[2 + lane + 64 * e];
      }
      float Mn = M;
#pragma unroll
      for (int kk = 0; kk < 8; ++kk) Mn = fmaxf(Mn, m[kk]);
      const float sc = M == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(M - Mn);
      L *= sc;
#pragma unroll
      for (int e = 0; e < DL; ++e) acc[e] *= sc;
#pragma unroll
      for (int kk = 0; kk < 8; ++kk) {
        const float w = m[kk] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m[kk] - Mn);
        L = __builtin_fmaf(w, l[kk], L);
#pragma unroll
        for (int e = 0; e < DL; ++e) acc[e] = __builtin_fmaf(o[kk][e], w, acc[e]);
      }
      M = Mn;
    }
#pragma unroll
    for (int e = 0; e < DL; ++e) out[lane + 64 * e] = acc[e] / L;
    return;
  }
  float o[SMAX][DL];
#pragma unroll
  for (int k = 0; k < SMAX; ++k)
#pragma unroll
    for (int e = 0; e < DL; ++e) o[k][e] = rec(min(k, n - 1))[2 + lane + 64 * e];
  const float *rl = rec(min(lane, n - 1));
  const float ml = lane < n ? rl[0] : -INFINITY, ll = rl[1];
  float M = ml;
#pragma unroll
  for (int s = 32; s >= 1; s >>= 1) M = fmaxf(M, __shfl_xor(M, s, 64));
  float w = ml == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(ml - M);
  float L = w * ll;
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

// Launches with at most this many queries merge one query per wave in one
// round of loads (latency bound: few queries, many records each).
constexpr int64_t kMergeOneRoundQueries = 2048;

template <int D, int KF, int NN, int SG, int NCB>
hipError_t launch_ncb(const PrefillParams &p, const FastLayout &fl, hipStream_t stream) {
  constexpr int lds = PSlot<D, KF, NN>::LDS;
  static const hipError_t allowed = hipFuncSetAttribute((const void *)prefill_kernel<D, KF, NN, SG, NCB>,
                                                        hipFuncAttributeMaxDynamicSharedMemorySize, lds);
  if (allowed != hipSuccess) {
    (void)hipGetLastError();  // do not leave the failure behind for the caller's next HIP call
    return allowed;
  }
  hipLaunchKernelGGL((prefill_kernel<D, KF, NN, SG, NCB>), dim3((unsigned)p.ranges), dim3(kThreads), lds, stream, p, fl);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess || p.ranges == 1) return e;
  const unsigned units = (unsigned)(p.batch * p.kv_heads);
  const int nq = p.rows * p.G;
  if ((int64_t)nq * units <= kMergeOneRoundQueries)
    hipLaunchKernelGGL((prefill_merge_one_round_kernel<D, 64>), dim3((unsigned)((nq + kWaves - 1) / kWaves), units),
                       dim3(kThreads), 0, stream, p);
  else
    hipLaunchKernelGGL((prefill_merge_kernel<D>), dim3((unsigned)(p.tiles * (p.tile_queries / (kThreads / 16))), units),
                       dim3(kThreads), 0, stream, p);
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
