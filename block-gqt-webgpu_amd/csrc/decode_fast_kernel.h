// Fused single-launch decode attention for gfx950 on the matrix cores: the
// kernel template and its launch helpers. The instances are compiled in
// decode_fast_any64.hip, decode_fast_any64_append.hip,
// decode_fast_any64_prefill.hip, decode_fast_any128.hip (any packed layout), decode_fast_d64.hip, decode_fast_d64_append.hip,
// decode_fast_d64_prefill.hip and decode_fast_d128.hip (structured layouts
// and FP16 K), so they build in parallel and each kind of launch can take its
// own scheduling options; decode_fast.hip dispatches to them.
//
// One workgroup (4 waves) per (sequence, KV head, token split). Everything a
// decode step of one layer needs happens in this one launch:
//   prologue  the KV head's G query rows are rotated into the code domain
//             (qr = R q[perm] / sqrt(d), a dense d x d product whose
//             off-group entries are exact zeros) and split into fp16 hi/lo
//             MFMA operands; the centroid books are expanded into LDS lookup
//             tables of fp16 (hi, lo) pairs: for nibble K-steps one entry per
//             packed byte (two dims), for byte K-steps one entry per code.
//   main loop each wave streams 32-token chunks of packed codes, FP16 scales
//             and FP16 V straight from HBM into a two-slot ring of LDS
//             buffers with buffer_load ... lds (no VGPR staging, non-temporal:
//             every byte is read once): the chunk issued at the top of an
//             iteration lands while the wave computes QK and the softmax of
//             the previous one. Reads past the sequence's length return zeros, so
//             the tail needs no clamping. From LDS it rebuilds the K
//             operand through the tables, runs QK as 16x16x32
//             f16 MFMAs (hi*hi + lo*hi + hi*lo, FP32-level logits), an online
//             softmax in the log2 domain, and PV as MFMAs with the V operand
//             read transposed by ds_read_b64_tr_b16. V rows (and FP16 K rows)
//             land in LDS with their 16-byte pieces XOR-swizzled by row, so
//             the transposed and row reads are free of bank conflicts.
//   epilogue  the four waves merge in LDS; with several splits each
//             workgroup stores an (m, l, o) partial and the last workgroup of
//             its (sequence, KV head) to arrive (a device-scope counter)
//             merges them by log-sum-exp and resets the counter to zero.
//
// The arithmetic is that of src/reference/attention.py:5-22 on the
// reconstructed K of src/reference/production_math.py:27-31: with
// k = ((c*s) @ R)[inv_perm], q.k = sum_g s_g sum_{j in g} c_j[code_j] (R q[perm])_j.
// The reference computes the same product as an on-chip group rebuild
// (src/model/compressed-dot.wgsl:14-31) followed by separate softmax and
// weighted passes (src/model/attention.wgsl:24-39).
#pragma once

#include <hip/hip_fp16.h>

#include "bgtq_internal.h"
#include "encode_row.h"
#include "gfx950_common.h"

namespace bgtq {
namespace {

using namespace gfx;

constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;
constexpr int kChunk = 32;  // tokens per wave iteration: two 16-token MFMA tiles
constexpr int kRing = 2;    // LDS chunk buffers per wave: compute one, the next in flight
constexpr bool kInterleaved = true;
constexpr int kMergeOneRound = 40;  // split counts merged with a single round of loads

// Kinds of launch of the fused kernel. Each kind's instances can sit in a
// translation unit of their own, compiled with the scheduling options that
// measured best for that kind.
constexpr int kKindDecode = 1;   // decode, no appended rows (FP32 V included)
constexpr int kKindAppend = 2;   // decode with an appended token (bgtq_decode_append)
constexpr int kKindPrefill = 4;  // row-wise prefill (p.starts), with or without appended rows
constexpr int kKindAll = 7;

inline int decode_fast_launch_kind(const DecodeParams &p) {
  return p.starts ? kKindPrefill : p.k_new ? kKindAppend : kKindDecode;
}

template <int D>
struct Geo {
  static constexpr int KS = D / 32;  // K-steps of QK
  static constexpr int DT = D / 16;  // 16-dim tiles of PV
  static constexpr int PR = D / 8;   // 16-byte pieces per FP16 row
  static constexpr int KRI = kChunk * D * 2 / 1024;  // 16-byte DMA instructions per chunk of FP16 rows
};

// One ring buffer: V chunk, FP16 scales (32 x 4 bytes), K chunk. Every DMA
// instruction runs on all 64 lanes (lanes past the data read zeros into the
// padding: scales to 256 bytes per scale DMA, K to whole 1 KB pieces), so the compiler's
// count of loads in flight matches the hardware's and its own waits for
// register loads never wait for ring data. Two workgroups of the layout-B
// d=64 kernel still fit one CU's 160 KB.
// KF 2 (any packed layout): RB is the largest row a layout can have, NN the
// scale DMAs (one for norm strides up to 4, two up to 8; at d=64 the second
// covers 128 bytes, norm strides up to 6, and the book tables get 3.5 KB, so
// that two workgroups still share a CU).
// 16-byte piece swizzle of an FP32 row of D >= 64 values in LDS: rows
// 4 g + 0..3 (mod 16) XOR their piece index with 4 g, so the PV reads of the
// four lane groups (rows 4 apart, the same 16 values) hit different banks.
__host__ __device__ constexpr int swz32(int row) { return ((row >> 2) & 3) << 2; }

// Row-wise prefill stages its rotated queries (16 heads, rows padded to D + 4
// floats) in dynamic LDS after the ring: no ring slot waits for the staging
// to be read, and an append workgroup's slots keep its encoders' data.
__host__ __device__ constexpr int prefill_stage_bytes(int D) { return 16 * (D + 4) * 4; }

// VF: the V rows' format, 0 = FP16 (2 bytes per value), 1 = FP32 (4 bytes;
// a ring of one slot per wave where two do not fit). NW: waves per workgroup.
template <int D, int KF, int NN, int VF = 0, int NW = kWaves>
struct Slot {
  static constexpr int KS = D / 32;
  static constexpr int RB = KF == 1 ? NN * 16 + (KS - NN) * 32 : KF == 2 ? D : 2 * D;  // K row bytes
  static constexpr int KBYTES = kChunk * RB;
  static constexpr int KI = (KBYTES + 1023) / 1024;  // 16-byte DMA instructions per K chunk
  static constexpr int NSC = KF == 1 ? 1 : KF == 2 ? NN : 0;  // scale DMAs per chunk
  static constexpr bool SMALL2 = KF == 2 && NN == 2 && D == 64;
  static constexpr int NBYTES = SMALL2 ? 384 : NSC * 64 * 4;
  static constexpr int VBYTES = kChunk * D * (VF ? 4 : 2);
  static constexpr int VI = VBYTES / 1024;    // 16-byte DMA instructions per V chunk
  static constexpr int NOFF = VBYTES;         // scales
  static constexpr int KOFF = NOFF + NBYTES;  // K
  static constexpr int BYTES = KOFF + KI * 1024;
  static constexpr int L = VI + KI + NSC;  // DMA instructions per chunk
  // Lookup tables (static LDS): KF 1, the K-steps' books; KF 2, the books'
  // code tables (CTABLES bytes), then kPairSlots pair tables of 2 KB.
  static constexpr int CTABLES = KF == 2 && D == 64 ? 3584 : KF >= 1 ? KS * 2048 : 0;
  static constexpr int TABLES = CTABLES + (KF == 2 ? kPairSlots * 2048 : 0);
  static constexpr int RING = VF && kRing * NW * BYTES + TABLES > kLdsLimit ? 1 : kRing;
  static constexpr int AHEAD = RING - 1;
  static constexpr int DYN = RING * NW * BYTES;  // dynamic LDS: the ring (the tables are static)
  // Decode-step append: the new token's wave encodes it with its last ring
  // slot as scratch (from offset 0) and a copy of its KV head's tables header,
  // code LUT and centroid books (from ENC_OFF, ENC_DMAS 1 KB pieces).
  static constexpr int ENC_OFF = KF >= 1 ? (row_enc::scratch_bytes(D) + 1023) / 1024 * 1024 : 0;
  static constexpr int ENC_DMAS = KF >= 1 ? (BYTES - ENC_OFF) / 1024 : 0;
  static_assert(DYN + TABLES <= kLdsLimit, "LDS of one workgroup");
  static_assert(VF || NW != kWaves || !SMALL2 || 2 * (DYN + TABLES) <= kLdsLimit, "two workgroups per CU");
  static_assert(AHEAD >= (VF ? 0 : 1) && AHEAD <= 3, "ring waits cover up to three chunks in flight");
};

// Split merge in one round trip, one wave per query head (heads wave,
// wave + 4, ..., two at a time): lane s loads split s's (m, l), and every lane
// loads each split's o at its DL dimensions, all loads in flight at once
// (S <= SMAX).
// The weights w_s = 2^(m_s - M) come from wave reductions and reach every
// lane through lane reads. Instantiated for a few SMAX and inlined: as a
// called function it saved the caller's registers it reuses to scratch
// memory and reloaded them on return, a memory round trip at the end of
// every merge.
// Rows of a row-wise unit's columns: column g's partials at row pbase + g of
// the partial array; its output at row obase + (j / G) * Hq + j % G, with
// j = jbase + g its query in the chunk's rows x G heads.
struct MergeRows {
  int64_t pbase, obase;
  int jbase, G, Hq, ncol;
  int sp;  // partial rows per column (the launch's most partials per unit)
  __device__ int64_t out_row(int g) const {
    const int j = jbase + g, r = j / G;
    return obase + (int64_t)r * Hq + (j - r * G);
  }
};

template <int D, int SMAX, int NW>
__device__ __forceinline__ void merge_one_round(float *part, float *out, float *stats, int64_t head0, int G, int S,
                                             int wave, int lane) {
  constexpr int kWaves = NW;
  static_assert(SMAX <= 64, "one split per lane");
  constexpr int DL = D / 64;  // dimensions per lane
  constexpr int NH = 2;       // heads of one wave merged together (heads g and g + 4)
  for (int g0 = wave; g0 < G; g0 += NH * kWaves) {
    float ms[NH], ls[NH], o[NH][SMAX][DL];
#pragma unroll
    for (int h = 0; h < NH; ++h) {
      const int g = g0 + h * kWaves;
      ms[h] = -INFINITY;
      ls[h] = 0.0f;
      if (g >= G) continue;
      float *pp = part + (head0 + g) * S * (D + 2);
      if (lane < S) {
        ms[h] = coherent_load(pp + lane * (D + 2));
        ls[h] = coherent_load(pp + lane * (D + 2) + 1);
      }
#pragma unroll
      for (int s = 0; s < SMAX; ++s) {
        if (s < S) {
          if (DL == 2) {
            const uint64_t v = __hip_atomic_load(reinterpret_cast<uint64_t *>(pp + s * (D + 2) + 2 + 2 * lane),
                                                 __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            o[h][s][0] = __uint_as_float((uint32_t)v);
            o[h][s][DL - 1] = __uint_as_float((uint32_t)(v >> 32));
          } else {
            o[h][s][0] = coherent_load(pp + s * (D + 2) + 2 + lane);
          }
        }
      }
    }
#pragma unroll
    for (int h = 0; h < NH; ++h) {
      const int g = g0 + h * kWaves;
      if (g >= G) continue;
      const int64_t head = head0 + g;
      const float M = col_max(row_max(ms[h]));
      const float w = ms[h] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(ms[h] - M);
      float lw = ls[h] * w;
      lw += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(lw), 0x128, 0xf, 0xf, false));
      lw += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(lw), 0x124, 0xf, 0xf, false));
      lw += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(lw), 0x122, 0xf, 0xf, false));
      lw += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(lw), 0x121, 0xf, 0xf, false));
      const float Lsum = col_sum(lw);
      float acc[DL];
#pragma unroll
      for (int dl = 0; dl < DL; ++dl) acc[dl] = 0.0f;
#pragma unroll
      for (int s = 0; s < SMAX; ++s) {
        if (s < S) {
          const float ws = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(w), s));
#pragma unroll
          for (int dl = 0; dl < DL; ++dl) acc[dl] = __builtin_fmaf(o[h][s][dl], ws, acc[dl]);
        }
      }
#pragma unroll
      for (int dl = 0; dl < DL; ++dl) out[head * D + DL * lane + dl] = acc[dl] / Lsum;
      if (lane == 0 && stats) {
        stats[head * 2] = M * kLn2;
        stats[head * 2 + 1] = Lsum;
      }
    }
  }
}

// Row-wise prefill split merge (PF). Wave w of NW merges the unit's columns
// w, w + NW, ... (NH of them), all their loads in flight at once. Partial rows are
// o[D], m, l, pad (16-byte aligned). A lane is (split group sg, dimension
// quad dq): it loads the o quads of splits sg, sg + SG, ... as 16-byte loads
// and lane s the (m, l) of split s; the weights reach the lanes by lane
// reads and the split groups' sums meet through lane swaps. Inlined, so the
// buffer resource's base stays in scalar registers.
template <int D, int SMAX, int NH, int NW>
__device__ __forceinline__ void merge_rows(float *part, float *out, const MergeRows mr, int S, int wave, int lane) {
  constexpr int DQ = D / 4;                // dimension quads
  constexpr int SG = 64 / DQ;              // split groups (4 at d=64, 2 at d=128)
  constexpr int J = (SMAX + SG - 1) / SG;  // splits per lane at most
  constexpr uint32_t ROWB = (D + 4) * 4;   // bytes per partial row
  S = __builtin_amdgcn_readfirstlane(S);
  const int G = mr.ncol;
  if (wave >= G) return;
  const int sg = lane / DQ, dq = lane - sg * DQ;
  const int sl = min(lane, S - 1);
  // The unit's partials: NW NH columns x S rows.
  // The unit's partials: NW NH columns x mr.sp rows (its first S used).
  const __amdgpu_buffer_rsrc_t r = rsrc(part + mr.pbase * mr.sp * (D + 4), (uint32_t)(NW * NH) * (uint32_t)mr.sp * ROWB);
  u32x2 ml[NH];
  f32x4 o[NH][J];
#pragma unroll
  for (int h = 0; h < NH; ++h) {
    const int g = wave + NW * h;
    const uint32_t col = (uint32_t)(g < G ? g : wave) * (uint32_t)mr.sp * ROWB;
    ml[h] = coherent_load2(r, col + (uint32_t)sl * ROWB + D * 4);
#pragma unroll
    for (int j = 0; j < J; ++j) {
      const int s = min(sg + SG * j, S - 1);
      o[h][j] = coherent_load4(r, col + (uint32_t)s * ROWB + 16u * dq);
    }
  }
  // The columns step by step side by side (no branch between them), so
  // their chains of lane reductions overlap; only the stores are predicated.
  float m[NH], w[NH], Lsum[NH];
#pragma unroll
  for (int h = 0; h < NH; ++h) m[h] = lane < S ? __uint_as_float(ml[h][0]) : -INFINITY;
  float M[NH];
#pragma unroll
  for (int h = 0; h < NH; ++h) M[h] = row_max(m[h]);
#pragma unroll
  for (int h = 0; h < NH; ++h) M[h] = col_max(M[h]);
#pragma unroll
  for (int h = 0; h < NH; ++h) {
    w[h] = m[h] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m[h] - M[h]);
    Lsum[h] = (lane < S ? __uint_as_float(ml[h][1]) : 0.0f) * w[h];
  }
  // Row sums: rotations by 8, 4, 2, 1 lanes (DPP row_ror).
#pragma unroll
  for (int h = 0; h < NH; ++h)
    Lsum[h] += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(Lsum[h]), 0x128, 0xf, 0xf, false));
#pragma unroll
  for (int h = 0; h < NH; ++h)
    Lsum[h] += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(Lsum[h]), 0x124, 0xf, 0xf, false));
#pragma unroll
  for (int h = 0; h < NH; ++h)
    Lsum[h] += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(Lsum[h]), 0x122, 0xf, 0xf, false));
#pragma unroll
  for (int h = 0; h < NH; ++h)
    Lsum[h] += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(Lsum[h]), 0x121, 0xf, 0xf, false));
#pragma unroll
  for (int h = 0; h < NH; ++h) Lsum[h] = col_sum(Lsum[h]);
  f32x4 acc[NH];
#pragma unroll
  for (int h = 0; h < NH; ++h) {
    acc[h] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int j = 0; j < J; ++j) {
      const int s = sg + SG * j;
      const float ws = __shfl(w[h], s < 64 ? s : 0, 64);
      acc[h] = s < S ? acc[h] + o[h][j] * ws : acc[h];
    }
  }
  // Sum over the split groups: lanes dq + DQ k.
#pragma unroll
  for (int h = 0; h < NH; ++h)
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      float v = acc[h][k];
      if (SG == 4) {
        auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
        v = __uint_as_float(a[0]) + __uint_as_float(a[1]);
      }
      auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
      acc[h][k] = __uint_as_float(b[0]) + __uint_as_float(b[1]);
    }
#pragma unroll
  for (int h = 0; h < NH; ++h) {
    const int g = wave + NW * h;
    // One reciprocal per column (within an ulp; the outputs' tolerance is 1e-4 relative).
    const float inv = __builtin_amdgcn_rcpf(Lsum[h]);
    if (g < G && sg == 0)
      *reinterpret_cast<f32x4 *>(out + mr.out_row(g) * D + 4 * dq) = acc[h] * inv;
  }
}

// KF: 1 = packed codes of a structured layout, 2 = packed codes of any
// layout, 0 = FP16 K rows. NN: leading nibble K-steps (KF 2: scale DMAs).
// SG: K-steps in group 0 (== KS: one scale per token; unused by KF 2).
// PK (KF 2): leading pair K-steps of every head (two codes per packed byte).
// PF (8 or 16): row-wise chunked prefill (p.starts set). A unit is PF query
// columns of one (sequence, KV head): the chunk's rows x G heads flattened
// row-major (query j = row * G + head), so a unit fills its MFMA columns
// whatever G is and the chunk's history is streamed once per PF queries
// (16: least streaming; 8: twice the units, each with half the epilogue and
// merge, which is shorter on the latency-bound small launches). Column j sees
// the first min(starts[b], max_length - rows) + row + 1 tokens. A unit uses
// only as many of its splits as its history needs (p.split_floor tokens per
// split at least); the others exit before their first chunk.
// VF: V rows of FP32 values (1; decode without an appended token) or FP16
// (0). FP32 V enters the PV MFMAs as three FP16 parts per value.
// NW: waves per workgroup (4; row-wise prefill at d=64, 8: a unit's splits
// then cover twice the tokens each and half as many partials are merged).
// Every kernel argument the set-up reads, loaded at once (one asm statement,
// whose operands' wait is the only one): left to itself the compiler loads
// them a basic block at a time, a chain of dependent scalar round trips ahead
// of the first DMA. Needs p, fl and kv.
#define BGTQ_ARGS                                                                                              \
  "s"(p.kv_heads), "s"(p.rows), "s"(p.starts), "s"(p.lengths), "s"(p.max_length), "s"(p.G), "s"(p.q_heads), \
      "s"(p.splits), "s"(p.ends), "s"(p.k_new), "s"(p.q_rotated), "s"(p.q), "s"(p.v), "s"(p.packed),         \
      "s"(p.norms), "s"(p.k), "s"(p.logits), "s"(p.qgroups), "s"(p.split_floor)
#define BGTQ_LOAD_ARGS                                                                                         \
  if constexpr (KF == 0) asm volatile("" ::BGTQ_ARGS);                                                         \
  if constexpr (KF == 1)                                                                                       \
  asm volatile("" ::BGTQ_ARGS, "s"(fl.mfma[kv]), "s"(fl.rot_q[kv]), "s"(fl.cent_exp[kv]), "s"(fl.book[0]),     \
  "s"(fl.book[1]), "s"(fl.book[Gm::KS - 2]), "s"(fl.book[Gm::KS - 1]));                                        \
  if constexpr (KF == 2)                                                                                       \
  asm volatile("" ::BGTQ_ARGS, "s"(fl.mfma[kv]), "s"(fl.rot_q[kv]), "s"(fl.cent_exp[kv]), "s"(fl.glane[kv]),   \
  "s"((int)fl.gnb[kv]), "s"((int)fl.gbstride[kv]), "s"((int)fl.gbnib[kv]), "s"(fl.gpair[kv]),                  \
  "s"((int)fl.grb[kv]), "s"((int)fl.gns[kv]));

// AP: the launch's extra outputs, compiled in only where used: 0 none, 1 the
// appended rows (decode or prefill append), 2 materialised logits (inspect()).
// RL: the workgroup's role in a launch with appended rows and packed K, known
// from its split index before anything else: 1 a history split, 2 an append
// workgroup; 0 either (decided at run time). The kernel below picks it.
template <int D, int KF, int NN, int SG, int PK = 0, int PF = 0, int VF = 0, int NW = kWaves, int AP = 1, int RL = 0>
__device__ __forceinline__ void decode_fast_body(const DecodeParams &p, const FastLayout &fl, uint8_t *tabs) {
  using Gm = Geo<D>;
  using Sl = Slot<D, KF, NN, VF, NW>;
  static_assert(VF == 0 || PF == 0, "FP32 V: decode only");
  static_assert(NW == 4 || NW == 8, "waves per workgroup");
  constexpr int kWaves = NW, kThreads = 64 * NW;
  static_assert(PF == 0 || PF == 8 || PF == 16, "row-wise unit width");
  constexpr int UC = PF ? PF : 16;  // columns of a row-wise unit
  static_assert(KF == 0 || row_enc::scratch_bytes(D) <= Sl::BYTES, "append scratch fits a ring slot");
  constexpr int KS = Gm::KS, DT = Gm::DT, PR = Gm::PR, VI = Sl::VI, KRI = Gm::KRI;
  constexpr int VB = VF ? 4 : 2;  // bytes per V value
  constexpr int RB = Sl::RB, KI = Sl::KI, L = Sl::L, AHEAD = Sl::AHEAD;
  static_assert(NN >= 0 && NN <= KS && SG >= 1 && SG <= KS, "layout");
  static_assert(Sl::BYTES >= 16 * (D + 4) * 4, "q staging fits one ring slot");
  static_assert(KF == 0 || Gm::DT % kWaves == 0 || kWaves % Gm::DT == 0, "rotation tiles split evenly over the waves");
  static_assert(KF != 2 || (NN >= 1 && NN <= 2), "one or two scale DMAs");
  static_assert(Sl::RING * kWaves * Sl::BYTES >= kWaves * 16 * (D + 2) * 4, "wave merge fits the ring");
  static_assert(Sl::RING * kWaves * Sl::BYTES >= 2 * 16 * 257 * 4, "split merge (<= 256 splits + append) fits the ring");
  extern __shared__ __align__(16) uint8_t smem[];

  // Grid (split, KV head, sequence); PF: (KV head, query group, split). The
  // head's layout words are loaded with the kernel arguments, with no
  // division ahead of them. Workgroups go to the XCDs round-robin by linear
  // index, so PF puts the split slowest: the units' first splits, the ones
  // every history has, spread over all XCDs (split fastest put every unit's
  // split 0 on one XCD), and an XCD's units share one KV head's history.
  // qrow: the sequence (PF: b * qgroups + query group).
  const int split = PF ? blockIdx.z : blockIdx.x, kv = PF ? blockIdx.x : blockIdx.y,
            qrow = PF ? blockIdx.y : blockIdx.z;
  // Every kernel argument the set-up reads, in one round trip (with the
  // role chosen by the kernel, already loaded there).
  BGTQ_LOAD_ARGS
  __builtin_amdgcn_sched_barrier(0);
  const int unit = qrow * p.kv_heads + kv;
  uint32_t *const counter = p.counters + (int64_t)unit * (p.counter_stride > 0 ? p.counter_stride : 1);
  constexpr bool rowwise = PF != 0;
  const int rows = rowwise ? p.rows : 1;
  // PF: qrow = b * qgroups + qg (query group qg of sequence b).
  const int ngroups = rowwise ? p.qgroups : 1;
  const int b = rowwise ? qrow / ngroups : qrow;
  const int qg = rowwise ? qrow - b * ngroups : 0;
  // A scalar load (constant address space): its wait goes where the value is
  // first used, after the loads below are issued.
  typedef const __attribute__((address_space(4))) uint32_t const_u32;
  const uint32_t len_b = reinterpret_cast<const_u32 *>(
      reinterpret_cast<uintptr_t>(rowwise ? p.starts : p.lengths))[b];
  const int G = p.G, Hq = p.q_heads, hq0 = kv * G;
  const int tid = threadIdx.x, lane = tid & 63, gq = lane >> 4, col = lane & 15;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: scalar loop control
  // The unit's query columns: decode, its G heads; PF, flattened queries
  // j = 16 qg + col of the chunk's rows x G heads.
  const int ncol = rowwise ? min(UC, rows * G - UC * qg) : G;
  const bool head_ok = col < ncol;
  // This lane's column (columns past ncol read column 0's query): its query
  // row of the chunk and head, and the row of q / out it indexes.
  const int jq = rowwise ? UC * qg + (head_ok ? col : 0) : 0;
  const int row_c = rowwise ? jq / G : 0;
  const int head_c = rowwise ? jq - row_c * G : (head_ok ? col : 0);
  const int64_t qidx = rowwise ? ((int64_t)b * rows + row_c) * Hq + hq0 + head_c : (int64_t)qrow * Hq + hq0 + head_c;
  // Rows of out and of the split partials of column g.
  auto out_row = [&](int g) -> int64_t {
    if (!rowwise) return (int64_t)qrow * Hq + hq0 + g;
    const int j = UC * qg + g, r = j / G;
    return ((int64_t)b * rows + r) * Hq + hq0 + (j - r * G);
  };
  const int64_t pbase = rowwise ? (int64_t)unit * UC : (int64_t)qrow * Hq + hq0;
  // The K-steps' lookup tables are static LDS (an address fixed at compile
  // time, so a lookup's address is the code byte shifted: one instruction);
  // the ring is the dynamic LDS.
  // KF 2: the code tables of the KV head's books, 1 KB each (tabs, declared
  // by the kernel).
  uint8_t *ring = smem;
  auto slot_base = [&](int s) { return ring + (s * kWaves + wave) * Sl::BYTES; };

  // ---------------- streams of this (sequence, KV head) ----------------
  // Each chunk's loads use buffer descriptors based at the chunk's first token
  // and sized to the chunk's tokens inside the sequence: the hardware range
  // check (which covers the per-lane offset) returns zeros past the length.
  // V strides count values.
  const uint8_t *v_rows =
      static_cast<const uint8_t *>(p.v) + ((int64_t)b * p.v_seq_stride + (int64_t)kv * p.v_head_stride) * VB;
  const _Float16 *v_base = reinterpret_cast<const _Float16 *>(v_rows);  // FP16 V: the appended row's store
  const uint8_t *k_base = KF >= 1 ? p.packed + b * p.packed_seq_stride + kv * p.packed_head_stride
                                  : reinterpret_cast<const uint8_t *>(static_cast<const _Float16 *>(p.k) +
                                                                      b * p.k_seq_stride + kv * p.k_head_stride);
  const uint16_t *n_base = KF >= 1 ? p.norms + b * p.norms_seq_stride + kv * p.norms_head_stride : nullptr;
  // Packed row bytes and scales per row (runtime for KF 2).
  const int rb = KF == 2 ? fl.grb[kv] : RB;
  const int ns = KF == 2 ? fl.gns[kv] : 2;
  // Per-lane source offsets of the swizzled FP16 row pieces: DMA instruction k,
  // lane i fills LDS piece 64k + i = (row r, slot c) with global piece c ^ swz(r).
  // FP32 V rows (D / 4 pieces) swizzle with swz32.
  uint32_t voff_rows[VI], koff_rows[KF == 0 ? KRI : 1];
#pragma unroll
  for (int k = 0; k < VI; ++k) {
    const int P = 64 * k + lane, r = P / (VF ? D / 4 : PR), c = P % (VF ? D / 4 : PR);
    voff_rows[k] = VF ? r * (4 * D) + ((c ^ swz32(r)) * 16) : r * (2 * D) + ((c ^ swz<D>(r)) * 16);
  }
#pragma unroll
  for (int k = 0; k < (KF == 0 ? KRI : 0); ++k) {
    const int P = 64 * k + lane, r = P / PR, c = P % PR;
    koff_rows[k] = r * (2 * D) + ((c ^ swz<D>(r)) * 16);
  }

  // ---------------- prologue ----------------
  // One round trip: wave 0 DMAs the MFMA lookup tables of the K-steps' books
  // into LDS; every wave loads its lanes' query values (lane (gq, col): head
  // col, dims 32 s + 8 gq + 0..7) and, for packed K, the MFMA operands of its
  // tiles of the permuted rotation. The first AHEAD chunks are issued behind
  // these loads and stay in flight through the prologue.
  if (KF == 1 && wave == 0) {
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      const uint8_t *src = fl.mfma[kv] + fl.book[s] * kMfmaTableBytes + (s < NN ? 0 : 2048);
      const __amdgpu_buffer_rsrc_t rt = rsrc(src, s < NN ? 2048 : 1024);
      dma16(rt, tabs + s * 2048, lane * 16, 0);
      if (s < NN) dma16(rt, tabs + s * 2048 + 1024, 1024 + lane * 16, 0);
    }
  }
  if (KF == 2 && wave == 0) {
    // The code table ([code]: hi | lo << 16) of every book: the first
    // gbstride bytes (max_centroids entries, whole 256-byte pieces) at
    // book * (gbstride + 32) + field width.
    const int nb = fl.gnb[kv], pieces = fl.gbstride[kv] / 256, span = fl.gbstride[kv] + 32;
    const uint32_t nibble_books = (uint32_t)fl.gbnib[kv];
#pragma unroll
    for (int bk = 0; bk < 8; ++bk) {
#pragma unroll
      for (int pc = 0; pc < 4; ++pc) {
        if (bk < nb && pc < pieces) {
          const __amdgpu_buffer_rsrc_t rt = rsrc(fl.mfma[kv] + bk * kMfmaTableBytes + 2048 + pc * 256, 256);
          dma4(rt, tabs + bk * span + ((nibble_books >> bk) & 1u ? 4 : 8) + pc * 256, lane * 4, 0);
        }
      }
    }
    // The pair tables ([byte]: hi pair, lo pair, 8 bytes) of the pair
    // K-steps' books, 2 KB each: one 8-byte read per packed byte.
    const uint32_t pair_books = fl.gpair[kv];
#pragma unroll
    for (int ps = 0; ps < (PK > 0 ? kPairSlots : 0); ++ps) {
      const uint32_t bk = (pair_books >> (8 * ps)) & 0xffu;
      if (bk != 0xffu) {
        const __amdgpu_buffer_rsrc_t rt = rsrc(fl.mfma[kv] + bk * kMfmaTableBytes, 2048);
#pragma unroll
        for (int q = 0; q < 2; ++q) dma16(rt, tabs + Sl::CTABLES + ps * 2048 + q * 1024, q * 1024 + lane * 16, 0);
      }
    }
  }
  // 16-row tiles of the rotation per wave (more waves than tiles: the first DT
  // waves take one each; row-wise prefill, the first DT / 2 two each, so
  // fewer waves load the queries).
  constexpr int NT = KF >= 1 && DT >= kWaves ? DT / kWaves : PF && DT >= 2 ? 2 : 1;
  const bool rot_wave = KF >= 1 && wave * NT < DT;
  // A query already in the code domain (q_rotated) is the QK operand as loaded.
  const bool rotate = KF >= 1 && !p.q_rotated;
  // Loads of a valid row (heads past G are zeroed after the chunk issue).
  // Row-wise prefill: waves that neither rotate nor use the query as loaded
  // (they read the rotated one from LDS) load none (a wave-uniform test;
  // 32-row chunks 33.42 -> 32.70 ms of attention per prompt). Decode loads
  // unconditionally: there the wait a branch puts where it joins (before the
  // prologue's later loads go out) cost more than the loads (C2 step +8 us).
  f32x4 qload[KS][2] = {};
  if (PF == 0 || !rotate || rot_wave) {
    const f32x4 *src = reinterpret_cast<const f32x4 *>(p.q + qidx * D);
#pragma unroll
    for (int s = 0; s < KS; ++s)
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) qload[s][hh] = src[8 * s + 2 * gq + hh];
  }
  u32x4 rq[NT][KS][2];
  // (wave-uniform: waves past the tiles load none)
  if (rotate && rot_wave) {
    const u32x4 *op = reinterpret_cast<const u32x4 *>(fl.rot_q[kv]);  // [tile][K-step][lane][hi, lo]
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        const int at = (((wave * NT + t) * KS + s) * 64 + lane) * 2;
        rq[t][s][0] = op[at];
        rq[t][s][1] = op[at + 1];
      }
  }
  const int ec = KF >= 1 ? fl.cent_exp[kv] : 0;
  // KF 2: this lane's code-lookup record of each K-step (built with the
  // tables, one per K-step and lane group gq): koff, hib, glo, nsl, ext[8],
  // tbo[8], gmask[4][4] (36 words, described where they are used).
  constexpr int KS2 = KF == 2 ? KS : 1;
  constexpr int RW = kLaneRecordWords / 4;
  u32x4 grec[KS2][RW];
  if (KF == 2) {
    const u32x4 *gr = reinterpret_cast<const u32x4 *>(fl.glane[kv]);
#pragma unroll
    for (int s = 0; s < KS2; ++s)
#pragma unroll
      for (int m = 0; m < RW; ++m)
        if (m < 9 || s < PK) grec[s][m] = gr[(s * 4 + gq) * RW + m];
  }
  // The sequence's length arrives while the loads above are in flight: what
  // depends on it comes after them.
  // PF: the chunk starts at min(starts[b], max_length - rows) (rows <= max_length);
  // the unit's history ends after its last column's row.
  const int start_c = rowwise ? (int)min(len_b, (uint32_t)(p.max_length - rows)) : 0;
  const int T_b = rowwise ? start_c + (UC * qg + ncol - 1) / G + 1 : (int)min(len_b, (uint32_t)p.max_length);
  // PF: the splits this unit's history needs (every workgroup of the unit
  // computes the same number); the others leave before their first chunk,
  // once the prologue's DMAs into their LDS have landed.
  // Appended rows with packed K (p.k_new): decode, the sequence's new token
  // (row T_b - 1); row-wise prefill, the chunk's rows (start_c .. T_b - 1 of
  // the unit's last column). They belong to p.app_parts more workgroups of
  // the (sequence, KV head) or unit, after its splits (the append
  // workgroups): decode, one, which encodes and stores the token and its V
  // row and leaves the token's partial (m, l, o) like a split; prefill, one
  // per kWaves rows, each wave encoding one row, and the part's rows then
  // attended to as one chunk. The history splits attend to the tokens
  // before them and never wait for an encode.
  const bool app = RL != 0 || (KF >= 1 && AP == 1 && p.k_new != nullptr);
  const bool lg = AP == 2 && p.logits != nullptr;  // materialised logits (inspect())
  const int part = split - p.splits;
  const bool app_wg = RL == 2 || (RL == 0 && app && part >= 0);
  const int sf = p.split_floor;
  const int S_hist = !rowwise ? p.splits
                     : app    ? min(p.splits, (start_c + sf - 1) / sf)
                              : min(p.splits, max(1, (T_b + sf - 1) / sf));
  if (rowwise && !app_wg && split >= S_hist) {
    wait_vm<0>();
    return;
  }
  const int S = S_hist + (app ? p.app_parts : 0);  // partials merged per (sequence, KV head) or unit
  // Partial rows per query column: the launch's most (row-wise units of one
  // launch use different split counts; each column's rows start at the same
  // stride, so units never share rows).
  const int SP = p.splits + (app ? p.app_parts : 0);
  const int pslot = app_wg ? S_hist + part : split;  // this workgroup's partial
  // Prefill append workgroup: its rows r_a .. r_a + n_a - 1 of the chunk.
  // (ER rows per wave: a wave encodes them side by side)
  constexpr int ER = PF ? kPrefillAppendRowsPerWave : 1;
  const int r_a = rowwise ? part * kWaves * ER : 0;
  const int n_a = rowwise ? min(kWaves * ER, rows - r_a) : 0;
  // Tokens the history splits attend to; the append workgroup's range ends
  // after its rows (decode: all tokens, so the new one lies inside the causal
  // limits).
  const int T_att = !app ? T_b : app_wg ? (rowwise ? start_c + r_a + n_a : T_b) : rowwise ? start_c : T_b - 1;
  // Splits of one (sequence, KV head) interleave at chunk granularity: wave w
  // of split s takes chunks (s * 4 + w) + 4 S i, so the waves working on a
  // sequence at any moment sweep adjacent memory.
  const int t_end = kInterleaved ? T_att : min(T_att, split * p.split_tokens + p.split_tokens);
  const int stride = kInterleaved ? max(S_hist, 1) * kWaves * kChunk : kWaves * kChunk;
  // This wave's chunks start at first + 128 i (a prefill append workgroup's
  // wave 0: its rows, assembled in its ring slot 0).
  const int first = app_wg && rowwise ? start_c + r_a
                    : kInterleaved    ? (split * kWaves + wave) * kChunk
                                      : split * p.split_tokens + wave * kChunk;
  const int n_chunks = app_wg ? (rowwise && wave == 0 ? 1 : 0)
                       : first < t_end ? (t_end - first + stride - 1) / stride : 0;
  // Decode reads every byte once (non-temporal, nothing cached is displaced);
  // a row-wise prefill chunk's history is read by every unit of its KV head,
  // so those loads keep the default policy and the units share it in L2.
  constexpr int kPol = PF ? kCached : kStream;
  auto issue = [&](int i) {
    const int c0 = first + i * stride;
    // Tokens of the chunk inside the sequence; none for a chunk past the end
    // (a zero-sized descriptor: the DMA only writes zeros to LDS). A history
    // split's range ends before the appended token, so its row arrives as
    // zeros; the append workgroup streams nothing.
    const int in_seq = app_wg ? 0 : min(T_att - c0, kChunk);
    const uint32_t rest = __builtin_amdgcn_readfirstlane(in_seq > 0 ? in_seq : 0);  // wave-uniform: SGPR descriptor
    uint8_t *sb = slot_base(i % Sl::RING);
    const __amdgpu_buffer_rsrc_t rV = rsrc(v_rows + (int64_t)c0 * D * VB, rest * (VB * D));
#pragma unroll
    for (int k = 0; k < VI; ++k) dma16<kPol>(rV, sb + k * 1024, voff_rows[k], 0);
    uint8_t *kb = sb + Sl::KOFF;
    if (KF == 1) {
      const __amdgpu_buffer_rsrc_t rK = rsrc(k_base + (int64_t)c0 * RB, rest * RB);
      const __amdgpu_buffer_rsrc_t rN = rsrc(n_base + (int64_t)c0 * 2, rest * 4);
#pragma unroll
      for (int k = 0; k < KI; ++k) dma16<kPol>(rK, kb + k * 1024, k * 1024 + lane * 16, 0);
      dma4<kPol>(rN, sb + Sl::NOFF, lane * 4, 0);
    } else if (KF == 2) {
      // Rows of rb bytes and ns scales, packed back to back: the chunk's rows
      // fill the K area's front, its scale rows the scale area's. The range
      // check zeroes a whole access that reaches past the range, so the ranges
      // end on the access size (16 and 4 bytes): the last row's bytes arrive,
      // and the few bytes past it lie in the same aligned 16 bytes as the row's
      // end (both bases are 16-byte aligned, c0 a multiple of 32).
      const __amdgpu_buffer_rsrc_t rK = rsrc(k_base + (int64_t)c0 * rb, (rest * rb + 15u) & ~15u);
      const __amdgpu_buffer_rsrc_t rN = rsrc(n_base + (int64_t)c0 * ns, (rest * ns * 2 + 3u) & ~3u);
#pragma unroll
      for (int k = 0; k < KI; ++k) dma16<kPol>(rK, kb + k * 1024, k * 1024 + lane * 16, 0);
#pragma unroll
      for (int k = 0; k < Sl::NSC; ++k)
        if (k * 256 + lane * 4 < Sl::NBYTES) dma4<kPol>(rN, sb + Sl::NOFF + k * 256, k * 256 + lane * 4, 0);
    } else {
      const __amdgpu_buffer_rsrc_t rK = rsrc(k_base + (int64_t)c0 * (2 * D), rest * (2 * D));
#pragma unroll
      for (int k = 0; k < KI; ++k) dma16<kPol>(rK, kb + k * 1024, koff_rows[k], 0);
    }
  };
  // Per-head causal limits.
  // The causal end is read for every lane (heads past G read head 0's) and
  // then selected: a load under the lane test would be waited for at once.
  const int end_any = rowwise ? start_c + row_c + 1 : p.ends ? p.ends[qidx] : T_b;
  const int end_h = head_ok ? min(end_any, T_b) : 0;
  int lim = min(end_h, t_end);
  // Wave-uniform: chunks reaching past lim_min need the per-head mask.
  int lim_min = head_ok ? lim : t_end;
  lim_min = wave_min(lim_min);

  // ---------------- decode-step append ----------------
  // With p.k_new the sequence's newest token (row T_b - 1) arrives in this
  // launch. FP16 K: the wave whose chunk holds it (the owner) loads the new
  // K and V rows with the prologue's loads, converts them, stores them to
  // the caches for the later steps and, after that chunk's loads land,
  // writes them over the chunk's LDS copy (whose loads may have read the
  // rows before they were stored). Packed K takes longer to encode, so the
  // token goes to the append workgroup: its wave 0 (the owner) stores the
  // new V row, and its wave 2 (the encoder) loads the new K (and, at d=64,
  // its column of the transposed rotation) and V, encodes and stores the K
  // row before the query rotation (the workgroup's other waves have no
  // chunks to wait for), then starts its attention state with the new token
  // (its logit from the row it encoded); the workgroup's merge of its waves'
  // states gives the token's partial.
  constexpr int JL = D > 64 ? 2 : 1;
  // Prefill append workgroup: wave w encodes chunk rows r_a + ER w + e
  // (cache rows start_c + r_a + ER w + e), e < ER, those the chunk has.
  const int t_new = rowwise ? start_c + r_a + ER * wave : T_b - 1;
  const int c_new = t_new >= 0 ? t_new / kChunk : 0;
  const int own_w = VF || rowwise || AP != 1 || p.k_new == nullptr || t_new < 0 ? -1
                    : app                                             ? (app_wg ? 0 : -1)
                                                                      : c_new % (p.splits * kWaves) - split * kWaves;
  const bool owner = own_w == wave;
  const bool encoder = rowwise ? app_wg && ER * wave < n_a
                               : KF >= 1 && own_w >= 0 && own_w < kWaves && wave == (own_w + 2) % kWaves;
  const int i_new = owner ? c_new / (p.splits * kWaves) : -1;  // the owner's loop iteration of that chunk
  // The q rotation stages through the last ring slot of a wave other than
  // the encoder, whose slot receives the encoder's tables meanwhile.
  const int stage_w = own_w >= 0 && own_w < kWaves ? (own_w + 1) % kWaves : 0;
  if (owner && KF >= 1) {  // the owner's chunk pass leaves the new token to the encoder
    lim = min(lim, t_new);
    lim_min = min(lim_min, t_new);
  }
  const int t_logit = owner && KF >= 1 ? t_new : t_end;  // logits this wave materialises: tokens below
  // Row e of this wave's encoded rows (ER of them, decode: the one new token):
  uint32_t pk_new[ER][JL] = {};                // packed K bytes lane, lane + 64
  uint16_t h_new[ER] = {};                     // FP16 scale bits (lanes below the norm stride)
  u32x4 v_new16{0u, 0u, 0u, 0u}, k_new16{0u, 0u, 0u, 0u};  // FP16 pieces of the V / K row (lanes below D / 8)
  uint32_t v_raw[ER][8] = {}, k_raw[8] = {};   // lane's 8 values of the new V / K row: FP32 bits, or FP16 pairs
  uint32_t k_nat[ER][JL] = {};                 // packed K: new K element lane + 64 jl (FP32 or FP16 bits)
  float rt_col[D == 64 ? D : 1];               // d=64: R[lane][i] for every i
  row_enc::Lane<D> lc;
  // Source offsets of row e (prefill: chunk row r_a + ER wave + e, clamped to
  // the part's rows; the rows past it are loaded but not used).
  auto new_off = [&](int e, int64_t seq_stride, int64_t row_stride, int64_t head_stride) {
    const int r_new = rowwise ? r_a + min(ER * wave + e, n_a - 1) : 0;
    return (int64_t)b * seq_stride + (int64_t)r_new * row_stride + kv * head_stride;
  };
  const int64_t v_off = new_off(0, p.v_new_seq_stride, p.v_new_row_stride, p.v_new_head_stride);
  const int64_t k_off = new_off(0, p.k_new_seq_stride, p.k_new_row_stride, p.k_new_head_stride);
  // The new rows' loads carry no branch (a load under a lane test or a
  // format select compiles to a branch whose join waits for it, holding back
  // every load after it). Lane i < D / 8 gets elements 8 i .. 8 i + 7: FP32
  // as eight words, FP16 as four words of two halves; the other lanes re-read
  // lane 0's piece. The rows are 4-byte aligned (checked on the host).
  auto load_piece = [&](const void *src, int f32, int64_t off, uint32_t (&r)[8]) {
    const int pl = lane < PR ? lane : 0;
    const uint8_t *base = static_cast<const uint8_t *>(src) + (off + 8 * pl) * (f32 ? 4 : 2);
    const uint32_t *p0 = reinterpret_cast<const uint32_t *>(base);
    const uint32_t *p1 = reinterpret_cast<const uint32_t *>(base + (f32 ? 16 : 0));
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      r[k] = p0[k];
      r[4 + k] = p1[k];
    }
  };
  auto half_piece = [&](int f32, const uint32_t (&r)[8]) {
    u32x4 h;
#pragma unroll
    for (int k = 0; k < 4; ++k)
      h[k] = f32 ? (uint32_t)row_enc::f32_to_f16_bits(__uint_as_float(r[2 * k])) |
                       ((uint32_t)row_enc::f32_to_f16_bits(__uint_as_float(r[2 * k + 1])) << 16)
                 : r[k];
    return h;
  };
  if (encoder) {
    // The tables' header, code LUT and books (contiguous from the start of
    // the table set, fl.enc_bytes[kv] bytes) into this wave's last ring
    // slot, first of this wave's loads: the prologue's wait covers them.
    const __amdgpu_buffer_rsrc_t rt =
        rsrc(reinterpret_cast<const uint8_t *>(p.tables[kv]) + fl.enc_from[kv], fl.enc_bytes[kv]);
    uint8_t *dst = ring + ((Sl::RING - 1) * kWaves + wave) * Sl::BYTES + Sl::ENC_OFF;
#pragma unroll
    for (int k = 0; k < Sl::ENC_DMAS; ++k) dma16(rt, dst + k * 1024, k * 1024 + lane * 16, 0);
#pragma unroll
    for (int e = 0; e < ER; ++e) {
      load_piece(p.v_new, p.v_new_f32, new_off(e, p.v_new_seq_stride, p.v_new_row_stride, p.v_new_head_stride),
                 v_raw[e]);
      const int64_t ko = new_off(e, p.k_new_seq_stride, p.k_new_row_stride, p.k_new_head_stride);
#pragma unroll
      for (int jl = 0; jl < JL; ++jl) {
        // FP16: the word holding the element (the row offset is even).
        const int64_t idx = ko + lane + 64 * jl;
        const uint32_t *w = p.k_new_f32 ? static_cast<const uint32_t *>(p.k_new) + idx
                                        : reinterpret_cast<const uint32_t *>(static_cast<const uint16_t *>(p.k_new) +
                                                                             (idx & ~(int64_t)1));
        const uint32_t kw = *w;
        k_nat[e][jl] = p.k_new_f32 ? kw : (kw >> (16 * (uint32_t)(idx & 1))) & 0xffffu;
      }
    }
    if (D == 64) {
#pragma unroll
      for (int i = 0; i < D; ++i) rt_col[i] = fl.rot_t[kv][i * D + lane];
    }
  }
  if (owner) {
    load_piece(p.v_new, p.v_new_f32, v_off, v_raw[0]);
    if (KF == 0) load_piece(p.k_new, p.k_new_f32, k_off, k_raw);
  }

  // Unconditional, so every wave has exactly AHEAD * L chunk loads in flight
  // behind its prologue loads (chunks past the end are zero-sized). The
  // scheduling barriers keep the prologue's loads ahead of them, so waiting
  // for those loads never waits for the chunks.
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int i = 0; i < AHEAD; ++i)
    if (!app_wg) issue(i);
  __builtin_amdgcn_sched_barrier(0);
  float qv[KS][8];
#pragma unroll
  for (int s = 0; s < KS; ++s)
#pragma unroll
    for (int k = 0; k < 8; ++k) qv[s][k] = head_ok ? qload[s][k >> 2][k & 3] : 0.0f;
  // Encodes this wave's ER rows: codes and scales (pk_new, h_new) to
  // registers; decode, also the new row in the code domain (k_j = c_j
  // s_g(j), positions j in head-perm order) and its FP16-rounded V row into
  // the scratch for the token's logits and output. Scratch of row e: row 0,
  // the start of this wave's last ring slot (its tables from Sl::ENC_OFF);
  // rows 1 .. ER - 1 (prefill), its slot 0 from the start (the query
  // rotation stages through the end of wave 0's).
  // src/model/codec.wgsl:14: the FP32 K is rounded to FP16 first; x in head-perm order.
  // T, lut, books: the LDS copy of the tables (header, LUT, books) loaded in
  // the prologue; for KF 2 tables larger than the slot holds, the header in
  // device memory with an LDS copy of the LUT and books, or (larger still)
  // all three in device memory.
  static_assert(KF == 0 || (ER - 1) * row_enc::scratch_bytes(D) <= Sl::BYTES, "encoder scratch fits a ring slot");
  auto enc_scratch = [&](int e) {
    return row_enc::Scratch<D>(e == 0 ? ring + ((Sl::RING - 1) * kWaves + wave) * Sl::BYTES
                                      : ring + wave * Sl::BYTES + (e - 1) * row_enc::scratch_bytes(D));
  };
  auto encode_block = [&]() {
    const uint8_t *enc_lds = ring + ((Sl::RING - 1) * kWaves + wave) * Sl::BYTES + Sl::ENC_OFF;
    const DevTables *T_dev = reinterpret_cast<const DevTables *>(p.tables[kv]);
    const DevTables *T_use = reinterpret_cast<const DevTables *>(enc_lds);
    const uint8_t *lut_use = tables_lut(T_use);
    const float *books_use = tables_books(T_use);
    if (KF == 2 && fl.enc_bytes[kv] == 0) {
      T_use = T_dev;
      lut_use = tables_lut(T_dev);
      books_use = tables_books(T_dev);
    } else if (KF == 2 && fl.enc_from[kv] != 0) {
      T_use = T_dev;
      lut_use = enc_lds;
      books_use = reinterpret_cast<const float *>(enc_lds + (T_dev->off_books - T_dev->off_lut));
    }
    const DevTables *T = T_use;
    const uint8_t *lut = lut_use;
    const float *books = books_use;
    lc.init(T, lane);
    const int ndims = __builtin_amdgcn_readfirstlane(T->nibble_dims);  // read with the lane set-up
    float x[ER][JL];
#pragma unroll
    for (int e = 0; e < ER; ++e)
#pragma unroll
      for (int jl = 0; jl < JL; ++jl) {
        const int src = lc.perm[jl];
        uint32_t raw = __shfl(k_nat[e][0], src & 63, 64);
        if (JL > 1) {
          const uint32_t hi = __shfl(k_nat[e][JL - 1], src & 63, 64);
          raw = src >= 64 ? hi : raw;
        }
        const uint16_t h16 = p.k_new_f32 ? row_enc::f32_to_f16_bits(__uint_as_float(raw)) : (uint16_t)raw;
        x[e][jl] = lc.own[jl] ? row_enc::f16_bits_to_f32(h16) : 0.0f;
      }
    row_enc::Scratch<D> scr[ER];
#pragma unroll
    for (int e = 0; e < ER; ++e) scr[e] = enc_scratch(e);
    const float *rt = fl.rot_t[kv];
    row_enc::encode_rows<D, ER>(
        T, lc, x,
        [&](int i, int jl) { return D == 64 ? rt_col[D == 64 ? i : 0] : rt[i * D + (lc.own[jl] ? lane + 64 * jl : 0)]; },
        lut, books, scr, lane, h_new);
    // The packed rows' bytes; they are stored after the rotation, so the
    // rotation's wait for this wave's loads does not wait for the stores.
    const int logical = ndims / 2 + D - ndims;
#pragma unroll
    for (int e = 0; e < ER; ++e)
#pragma unroll
      for (int jl = 0; jl < JL; ++jl) pk_new[e][jl] = row_enc::packed_byte(scr[e].codes, lane + 64 * jl, ndims, logical);
    if constexpr (!PF) {
      const row_enc::Scratch<D> &s0 = scr[0];
#pragma unroll
      for (int jl = 0; jl < JL; ++jl) {
        const float sc = row_enc::f16_bits_to_f32((uint16_t)__shfl((int)h_new[0], lc.grp[jl], 64));
        if (lc.own[jl]) s0.xn[lane + 64 * jl] = books[lc.bk[jl] * T->max_centroids + s0.codes[lane + 64 * jl]] * sc;
      }
      if (lane < PR) reinterpret_cast<u32x4 *>(s0.leaf)[lane] = half_piece(p.v_new_f32, v_raw[0]);
    }
    row_enc::wave_sync();
  };
  if (encoder) {
    // An append workgroup's encoders encode their rows as soon as their own
    // loads have landed (the tables' header, LUT and books in the last ring
    // slot, the new K and V rows, the rotation column), ahead of the query
    // rotation: the workgroup's other waves have no chunks, so the rotation's
    // barriers cost them nothing.
    wait_vm<0>();  // no chunk DMAs behind the prologue's loads
    encode_block();
  }
  if (rotate) {
    // qr^T = Rq q^T, Rq = R with the head permutation folded into its
    // columns, on the matrix cores (q and Rq split hi/lo, three MFMAs per
    // K-step, off-group entries exact zeros). Tile n leaves rows
    // j = 16 n + 4 gq + 0..3 of head col in this lane; they go through LDS
    // (the last ring slot, rows padded to D + 4 floats) to the QK layout.
    float qmax = 0.0f;
#pragma unroll
    for (int s = 0; s < KS; ++s)
#pragma unroll
      for (int jv = 0; jv < 8; ++jv) qmax = fmaxf(qmax, fabsf(qv[s][jv]));
    const int e0 = split_exp(col_max(qmax));
    half8 bh[KS], bl[KS];
#pragma unroll
    for (int s = 0; s < KS; ++s) split_scaled(qv[s], __builtin_ldexpf(1.0f, e0), bh[s], bl[s]);
    // (row-wise prefill: its staging area after the ring)
    float *qs = reinterpret_cast<float *>(PF ? ring + Sl::DYN : ring + ((Sl::RING - 1) * kWaves + stage_w) * Sl::BYTES);
    const float unscale = __builtin_ldexpf(1.0f, -e0);
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      if (!rot_wave) break;  // wave-uniform: waves past the tiles only read the result
      f32x4 acc = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        const half8 ah = __builtin_bit_cast(half8, rq[t][s][0]), al = __builtin_bit_cast(half8, rq[t][s][1]);
        acc = mfma(ah, bh[s], acc);
        acc = mfma(al, bh[s], acc);
        acc = mfma(ah, bl[s], acc);
      }
      *reinterpret_cast<f32x4 *>(qs + col * (D + 4) + 16 * (wave * NT + t) + 4 * gq) = acc * unscale;
    }
    if (app_wg) wait_vm<0>();  // the table DMAs (append workgroups issue no chunks)
    else wait_vm<AHEAD * L>();  // the table DMAs, which precede the chunks
    lds_barrier();
#pragma unroll
    for (int s = 0; s < KS; ++s)
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        const f32x4 v = *reinterpret_cast<const f32x4 *>(qs + col * (D + 4) + 32 * s + 8 * gq + 4 * hh);
#pragma unroll
        for (int k = 0; k < 4; ++k) qv[s][4 * hh + k] = v[k];
      }
  } else if (KF >= 1) {
    if (app_wg) wait_vm<0>();  // the table DMAs (append workgroups issue no chunks)
    else wait_vm<AHEAD * L>();  // the table DMAs, which precede the chunks
    lds_barrier();
  }
  // B operand of QK: lane holds qr[head = col][32 s + 8 gq + 0..7], split hi/lo
  // after scaling the head's row so its largest entry is near 2^14.
  half8 qhi[KS], qlo[KS];
  float kq;  // log2-domain logit = (sum_g s_g acc_g) * kq
  {
    float qmax = 0.0f;
#pragma unroll
    for (int s = 0; s < KS; ++s)
#pragma unroll
      for (int jv = 0; jv < 8; ++jv) {
        const float v = head_ok ? qv[s][jv] * p.inv_sqrt_d : 0.0f;
        qv[s][jv] = v;
        qmax = fmaxf(qmax, fabsf(v));
      }
    qmax = col_max(qmax);
    const int eq = qmax > 0.0f ? 14 - (int)ceilf(__builtin_log2f(qmax)) : 0;
    const float qsc = __builtin_ldexpf(1.0f, eq);
#pragma unroll
    for (int s = 0; s < KS; ++s)
#pragma unroll
      for (int jv = 0; jv < 8; ++jv) {
        const float x = qv[s][jv] * qsc;
        qhi[s][jv] = (_Float16)x;
        qlo[s][jv] = (_Float16)(x - (float)qhi[s][jv]);
      }
    kq = __builtin_ldexpf(kLog2e, -(eq + ec));
  }
  // The q staging (a ring slot's, whose chunk comes later) is dead; row-wise
  // prefill's own staging area is never written again, so it needs no
  // barrier, and its second ring slot's chunk goes out now (issued with the
  // first, in the prologue, it measured slower: more loads in flight while
  // the queries and tables are awaited).
  if (rotate && !PF) lds_barrier();
  static_assert(!PF || (Sl::RING == 2 && AHEAD == 1), "row-wise pairs fill both ring slots");
  if constexpr (PF != 0) {
    if (!app_wg) issue(1);
  }

  // KF 2: a K-step spans up to kSlots adjacent groups glo[s] .. glo[s] +
  // nsl[s] - 1. Each group's part of the K-step runs MFMAs against the query
  // with the other groups' positions masked to zero (the record's per-slot
  // masks), and the token's scale of that group weights the result. A lane's 8 codes of
  // a K-step are nibbles, then bytes (the head-perm order puts every nibble
  // position first): they lie in the 8 row bytes from koff, read as two
  // words; codes 0..3 come from the first word, codes 4..7 from the word
  // starting at byte hib[s]. ext[s][k]: the code's bit offset in its word;
  // tbo[s][k]: its book's LDS table offset plus the field width (4 or 8),
  // whose low 5 bits are the width operand of the bit-field extract.
  //
  // Group packing: with at most 8 (4) query heads, one MFMA's 16 columns hold
  // the query operands of two (four) groups side by side. Column c carries
  // head hc = c % HW masked to group slot m * GP + c / HW of MFMA m, so a
  // K-step of nsl groups takes ceil(nsl / GP) MFMA triples instead of nsl.
  // Each lane weights its partial logits with its own group's scales, and
  // row rotations by 8 (and 4) lanes then sum the slots of each head: every
  // lane c ends with head hc's logit, and the real heads (c < G <= HW) are
  // where the softmax expects them.
  constexpr int kSlots = 4;
  int glo[KS2], nsl[KS2], koff[KS2], hib[KS2], nmf[KS2];
  uint32_t ext[KS2][8], tbo[KS2][8];
  half8 qbh[KS2][kSlots], qbl[KS2][kSlots];  // masked (packed) query operands of MFMA m
  const int GP = KF == 2 ? (ncol <= 4 ? 4 : ncol <= 8 ? 2 : 1) : 1;  // group slots per MFMA
  const int HW = 16 / GP, cg = col / HW;
  constexpr int NSV = KF == 2 ? 2 * Sl::NSC : 1;  // scale entries a lane moves
  int sc_src[NSV], sc_dst[NSV];
  const bool rows_aligned = KF == 2 && fl.galign[kv] != 0;  // every lane's 8 bytes start on a word
  if (KF == 2) {
#pragma unroll
    for (int s = 0; s < KS2; ++s) {
      koff[s] = (int)grec[s][0][0];
      hib[s] = (int)grec[s][0][1];
      glo[s] = (int)__builtin_amdgcn_readfirstlane(grec[s][0][2]);
      nsl[s] = (int)__builtin_amdgcn_readfirstlane(grec[s][0][3]);
      // A pair K-step keeps its pair table offsets in tbo (ext unused).
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        ext[s][k] = s < PK ? (k < 4 ? grec[s][10][k] : 0u) : grec[s][1 + (k >> 2)][k & 3];
        tbo[s][k] = s < PK ? (k < 4 ? grec[s][9][k] : 0u) : grec[s][3 + (k >> 2)][k & 3];
      }
      nmf[s] = (nsl[s] + GP - 1) / GP;
      // Head hc's operands come from lane (gq, hc); slot cg + m * GP's mask
      // keeps that group's positions (slots past the K-step's groups: none).
      const u32x4 h = __builtin_bit_cast(u32x4, qhi[s]), l = __builtin_bit_cast(u32x4, qlo[s]);
      const int src = 16 * gq + (col & (HW - 1));
      u32x4 hs, ls;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        hs[k] = (uint32_t)__shfl((int)h[k], src, 64);
        ls[k] = (uint32_t)__shfl((int)l[k], src, 64);
      }
#pragma unroll
      for (int m = 0; m < kSlots; ++m) {
        const int slot = m * GP + cg;
        u32x4 mk{0u, 0u, 0u, 0u};
#pragma unroll
        for (int i = 0; i < kSlots; ++i)
          if (slot == i) mk = grec[s][5 + i];
        qbh[s][m] = __builtin_bit_cast(half8, hs & mk);
        qbl[s][m] = __builtin_bit_cast(half8, ls & mk);
      }
    }
    // The chunk's scale rows [token][ns] become [group][32 tokens] in place
    // (lane moves entries lane + 64 k), so a lane's four tokens of one group
    // are one 8-byte read.
#pragma unroll
    for (int k = 0; k < NSV; ++k) {
      const int e = lane + 64 * k, t = e / ns;
      sc_src[k] = e < 32 * ns ? 2 * e : -1;
      sc_dst[k] = 2 * ((e - t * ns) * 32 + t);
    }
  }

  float new_x = -INFINITY;  // encoder: the new token's logit for head col (log2 domain; -inf: not attended)
  if (owner) {  // the new token's V (and FP16 K) row: convert, store to the caches
    if (lane < PR) {
      v_new16 = half_piece(p.v_new_f32, v_raw[0]);
      *reinterpret_cast<u32x4 *>(const_cast<_Float16 *>(v_base) + (int64_t)t_new * D + 8 * lane) = v_new16;
    }
    if (KF == 0 && lane < PR) {
      k_new16 = half_piece(p.k_new_f32, k_raw);
      *reinterpret_cast<u32x4 *>(reinterpret_cast<_Float16 *>(const_cast<uint8_t *>(k_base)) + (int64_t)t_new * D +
                                 8 * lane) = k_new16;
    }
  }
  if (!rowwise && encoder) {  // the encoded row to the caches; the new token's logit from it
    uint8_t *prow = const_cast<uint8_t *>(k_base) + (int64_t)t_new * rb;
#pragma unroll
    for (int jl = 0; jl < JL; ++jl)
      if (lane + 64 * jl < rb) prow[lane + 64 * jl] = (uint8_t)pk_new[0][jl];
    if (lane < ns) const_cast<uint16_t *>(n_base)[(int64_t)t_new * ns + lane] = h_new[0];
    const row_enc::Scratch<D> scr = enc_scratch(0);
    // Logit of head col: sum over this lane's positions 32 s + 8 gq + k of
    // k_j (qhi + qlo)[s][k], then over the column's four lanes; the query
    // operands carry 2^eq, kq * 2^ec takes it off (the centroids here are
    // not scaled by 2^ec).
    float part = 0.0f;
#pragma unroll
    for (int s2 = 0; s2 < KS; ++s2)
#pragma unroll
      for (int k = 0; k < 8; ++k)
        part = __builtin_fmaf(scr.xn[32 * s2 + 8 * gq + k], (float)qhi[s2][k] + (float)qlo[s2][k], part);
    const float xt = col_sum(part) * __builtin_ldexpf(kq, ec);
    new_x = head_ok && t_new < lim ? xt : -INFINITY;
    if (lg && head_ok) p.logits[((int64_t)qrow * Hq + hq0 + col) * p.logit_stride + t_new] = new_x * kLn2;
  }
  if (rowwise && app_wg) {
    // The part's rows (encoded before the rotation) laid out as one chunk in
    // wave 0's ring slot 0 the way a chunk's DMA leaves it (V rows with
    // swizzled pieces, K rows of rb bytes, scale rows of ns): wave 0 clears
    // the slot (rows past the part's are attended to as zeros), then each
    // encoder writes its rows.
    lds_barrier();  // every encoder is done with its scratch
    if (wave == 0) {
      for (int o = lane * 16; o < Sl::BYTES; o += 1024) *reinterpret_cast<u32x4 *>(ring + o) = u32x4{0u, 0u, 0u, 0u};
    }
    lds_barrier();
    const int ne = min(ER, n_a - ER * wave);  // this wave's rows (encoders: 1 .. ER)
    u32x4 vrow[ER];
    if (encoder) {
#pragma unroll
      for (int e = 0; e < ER; ++e) {
        const int r = ER * wave + e;  // row in the chunk
        vrow[e] = half_piece(p.v_new_f32, v_raw[e]);
        if (e < ne) {
          uint8_t *krow = ring + Sl::KOFF + r * rb;
#pragma unroll
          for (int jl = 0; jl < JL; ++jl)
            if (lane + 64 * jl < rb) krow[lane + 64 * jl] = (uint8_t)pk_new[e][jl];
          if (lane < ns) *reinterpret_cast<uint16_t *>(ring + Sl::NOFF + 2 * (r * ns + lane)) = h_new[e];
          if (lane < PR) *reinterpret_cast<u32x4 *>(ring + r * (2 * D) + ((lane ^ swz<D>(r)) * 16)) = vrow[e];
        }
      }
    }
    lds_barrier();
    // The rows to the caches: every unit of the (sequence, KV head) encodes
    // the same bytes, its first unit stores them.
    if (encoder && qg == 0) {
#pragma unroll
      for (int e = 0; e < ER; ++e) {
        if (e >= ne) break;
        const int64_t t = t_new + e;
        uint8_t *prow = const_cast<uint8_t *>(k_base) + t * rb;
#pragma unroll
        for (int jl = 0; jl < JL; ++jl)
          if (lane + 64 * jl < rb) prow[lane + 64 * jl] = (uint8_t)pk_new[e][jl];
        if (lane < ns) const_cast<uint16_t *>(n_base)[t * ns + lane] = h_new[e];
        if (lane < PR) *reinterpret_cast<u32x4 *>(const_cast<_Float16 *>(v_base) + t * D + 8 * lane) = vrow[e];
      }
    }
  }

  const uint32_t *tn = reinterpret_cast<const uint32_t *>(tabs);
  float m_run = -INFINITY, l_run = 0.0f;
  f32x4 O[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) O[dt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  if (!rowwise && encoder) {
    // The state of the new token alone: m = its logit, l = p = 2^15 (the P
    // scale; one lane of the column holds it), O rows (heads 4 gq + r) =
    // 2^15 v, v from the scratch copy (read before the slot's first load).
    const _Float16 *vh = reinterpret_cast<const _Float16 *>(ring + ((Sl::RING - 1) * kWaves + wave) * Sl::BYTES);
    m_run = new_x;
    l_run = new_x != -INFINITY && gq == 0 ? kPScale : 0.0f;
    // The V row's values first, unconditionally: a read under the select
    // below is a branch and an LDS round trip per element.
    float vcol[DT];
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) vcol[dt] = (float)vh[16 * dt + col];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const bool vr = __shfl(new_x, 4 * gq + r, 64) != -INFINITY;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) O[dt][r] = vr ? kPScale * vcol[dt] : 0.0f;
    }
    row_enc::wave_sync();
  }
  // Lane-constant parts of the transposed V reads.
  const int trow = 4 * gq + (col >> 2);
  const int tpiece = (col & 3) >> 1, thalf = (col & 1) * 8;

  // This lane's logits of the chunk in ring slot sb (first token c0): head
  // col, tokens c0 + 16 u + 4 gq + r in x[4 u + r], log2 domain, masked past
  // the causal ends.
  auto chunk_logits = [&](const uint8_t *sb, int c0, float (&x)[8]) {
    const uint8_t *kbuf = sb + Sl::KOFF;
    // KF 2: transpose the scale rows (every read of the wave's slot precedes
    // its writes: one wave's LDS operations complete in order).
    if (KF == 2) {
      uint8_t *ns_area = const_cast<uint8_t *>(sb) + Sl::NOFF;
      uint32_t sv[NSV];
#pragma unroll
      for (int k = 0; k < NSV; ++k)
        if (sc_src[k] >= 0) sv[k] = *reinterpret_cast<const uint16_t *>(ns_area + sc_src[k]);
#pragma unroll
      for (int k = 0; k < NSV; ++k)
        if (sc_src[k] >= 0) *reinterpret_cast<uint16_t *>(ns_area + sc_dst[k]) = (uint16_t)sv[k];
    }
    // KF 2: logits x2[u][r] = sum over K-steps s and their groups of the
    // token's group scale times that group's part of the K-step.
    float x2[2][4];
    if (KF == 2) {
#pragma unroll
      for (int u = 0; u < 2; ++u)
#pragma unroll
        for (int r = 0; r < 4; ++r) x2[u][r] = 0.0f;
      // The lane's row words of every (K-step, tile) first, so the LDS reads
      // of all four are in flight together, then every code lookup.
      uint32_t w0[KS2][2], wh[KS2][2];
      {
        uint32_t dw[KS2][2][3];
#pragma unroll
        for (int s = 0; s < KS2; ++s)
#pragma unroll
          for (int u = 0; u < 2; ++u) {
            const int rofs = (16 * u + col) * rb + koff[s];
            // kbuf is 16-byte aligned: the row offset's low bits are the address's
            const uint32_t *wp = reinterpret_cast<const uint32_t *>(kbuf + (rows_aligned ? rofs : rofs & ~3));
            dw[s][u][0] = wp[0];
            if (!rows_aligned || s >= PK) dw[s][u][1] = wp[1];
            if (!rows_aligned && s >= PK) dw[s][u][2] = wp[2];
          }
#pragma unroll
        for (int s = 0; s < KS2; ++s)
#pragma unroll
          for (int u = 0; u < 2; ++u) {
            const uint32_t sh = (uint32_t)(((16 * u + col) * rb + koff[s]) & 3);
            uint32_t w1 = 0;
            if (rows_aligned) {
              w0[s][u] = dw[s][u][0];
              if (s >= PK) w1 = dw[s][u][1];
            } else {
              w0[s][u] = __builtin_amdgcn_alignbyte(dw[s][u][1], dw[s][u][0], sh);
              if (s >= PK) w1 = __builtin_amdgcn_alignbyte(dw[s][u][2], dw[s][u][1], sh);
            }
            wh[s][u] = s < PK || hib[s] == 4 ? w1 : __builtin_amdgcn_alignbyte(w1, w0[s][u], (uint32_t)hib[s]);
          }
      }
      half8 ah[KS2][2], al[KS2][2];
#pragma unroll
      for (int s = 0; s < KS2; ++s)
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          u32x4 hi, lo;
          if (s < PK) {
            // Pair K-step: the lane's 8 nibble codes are the 4 bytes of w0;
            // each byte's pair table entry is an (hi, lo) operand pair.
            const uint8_t *pt = tabs + Sl::CTABLES;
#pragma unroll
            for (int k2 = 0; k2 < 4; ++k2) {
              const uint32_t byte8 = 8 * __builtin_amdgcn_ubfe(w0[s][u], 8 * k2, 8);
              const u32x2 e2 = *reinterpret_cast<const u32x2 *>(pt + tbo[s][k2] + byte8);
              hi[k2] = e2[0];
              lo[k2] = e2[1];
            }
          } else {
#pragma unroll
            for (int k2 = 0; k2 < 4; ++k2) {
              uint32_t e[2];
#pragma unroll
              for (int h = 0; h < 2; ++h) {
                const int k = 2 * k2 + h;
                const uint32_t code = __builtin_amdgcn_ubfe(k < 4 ? w0[s][u] : wh[s][u], ext[s][k], tbo[s][k]);
                e[h] = *reinterpret_cast<const uint32_t *>(tabs + tbo[s][k] + 4 * code);
              }
              hi[k2] = __builtin_amdgcn_perm(e[1], e[0], 0x05040100u);
              lo[k2] = __builtin_amdgcn_perm(e[1], e[0], 0x07060302u);
            }
          }
          ah[s][u] = __builtin_bit_cast(half8, hi);
          al[s][u] = __builtin_bit_cast(half8, lo);
        }
#pragma unroll
      for (int s = 0; s < KS2; ++s) {
#pragma unroll
        for (int m = 0; m < kSlots; ++m) {
          if (m >= nmf[s]) continue;
          // This lane's group; a slot past the K-step's groups has a zero
          // operand, and reads the last group's (finite) scales.
          const int g = min(glo[s] + m * GP + cg, glo[s] + nsl[s] - 1);
#pragma unroll
          for (int u = 0; u < 2; ++u) {
            f32x4 a = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
            a = mfma(ah[s][u], qbh[s][m], a);
            a = mfma(al[s][u], qbh[s][m], a);
            a = mfma(ah[s][u], qbl[s][m], a);
            const u32x2 w = *reinterpret_cast<const u32x2 *>(sb + Sl::NOFF + 2 * (g * 32 + 16 * u + 4 * gq));
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              const float sc = __half2float(__ushort_as_half((uint16_t)(w[r >> 1] >> (16 * (r & 1)))));
              x2[u][r] = __builtin_fmaf(sc, a[r], x2[u][r]);
            }
          }
        }
      }
      // Sum the group slots of each head (lanes c, c + 8 (, c + 4, c + 12)).
      if (GP >= 2) {
#pragma unroll
        for (int u = 0; u < 2; ++u)
#pragma unroll
          for (int r = 0; r < 4; ++r)
            x2[u][r] += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x2[u][r]), 0x128, 0xf, 0xf, false));
      }
      if (GP == 4) {
#pragma unroll
        for (int u = 0; u < 2; ++u)
#pragma unroll
          for (int r = 0; r < 4; ++r)
            x2[u][r] += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x2[u][r]), 0x124, 0xf, 0xf, false));
      }
    }

    // QK: acc[u][g] = sum over the K-steps of group g.
    f32x4 acc[2][2];
#pragma unroll
    for (int u = 0; u < 2; ++u) acc[u][0] = acc[u][1] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    if constexpr (KF == 1) {
      // The lane's row words of both tiles and every K-step first, then every
      // code lookup, then the MFMAs (in K-step order, as the sums were): the
      // LDS reads go out in two rounds instead of a round trip per K-step.
      uint32_t wn[2][KS];
      u32x2 wb[2][KS];
#pragma unroll
      for (int u = 0; u < 2; ++u)
#pragma unroll
        for (int s = 0; s < KS; ++s) {
          const uint8_t *row = kbuf + (16 * u + col) * RB;  // A-operand row (token) of this lane
          if (s < NN) wn[u][s] = *reinterpret_cast<const uint32_t *>(row + 16 * s + 4 * gq);
          else wb[u][s] = *reinterpret_cast<const u32x2 *>(row + 16 * NN + 32 * (s - NN) + 8 * gq);
        }
      u32x4 hi[2][KS], lo[2][KS];
#pragma unroll
      for (int u = 0; u < 2; ++u)
#pragma unroll
        for (int s = 0; s < KS; ++s) {
          if (s < NN) {
            const u32x2 *t64 = reinterpret_cast<const u32x2 *>(tn + s * 512);  // [byte]: hi pair, lo pair
#pragma unroll
            for (int k = 0; k < 4; ++k) {
              const u32x2 v = t64[(wn[u][s] >> (8 * k)) & 255u];
              hi[u][s][k] = v[0];
              lo[u][s][k] = v[1];
            }
          } else {
            const uint32_t *t32 = tn + s * 512;  // [code]: hi | lo << 16
#pragma unroll
            for (int k = 0; k < 4; ++k) {
              const uint32_t c0 = t32[(wb[u][s][k >> 1] >> (16 * (k & 1))) & 255u];
              const uint32_t c1 = t32[(wb[u][s][k >> 1] >> (16 * (k & 1) + 8)) & 255u];
              hi[u][s][k] = __builtin_amdgcn_perm(c1, c0, 0x05040100u);  // c0.hi, c1.hi
              lo[u][s][k] = __builtin_amdgcn_perm(c1, c0, 0x07060302u);  // c0.lo, c1.lo
            }
          }
        }
#pragma unroll
      for (int u = 0; u < 2; ++u)
#pragma unroll
        for (int s = 0; s < KS; ++s) {
          const int g = s < SG ? 0 : 1;
          const half8 ah = __builtin_bit_cast(half8, hi[u][s]), al = __builtin_bit_cast(half8, lo[u][s]);
          acc[u][g] = mfma(ah, qhi[s], acc[u][g]);
          acc[u][g] = mfma(al, qhi[s], acc[u][g]);
          acc[u][g] = mfma(ah, qlo[s], acc[u][g]);
        }
    }
    // FP16 K rows: swizzled 16-byte pieces.
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int t = 16 * u + col;  // A-operand row (token) of this lane
#pragma unroll
      for (int s = 0; s < (KF == 0 ? KS : 0); ++s) {
        const int piece = 4 * s + gq;
        const half8 a = *reinterpret_cast<const half8 *>(kbuf + t * (2 * D) + ((piece ^ swz<D>(t)) * 16));
        acc[u][0] = mfma(a, qhi[s], acc[u][0]);
        acc[u][0] = mfma(a, qlo[s], acc[u][0]);
      }
    }
    // logits of this lane: head col, tokens c0 + 16u + 4gq + r
#pragma unroll
    for (int u = 0; u < 2 && KF == 2; ++u) {
#pragma unroll
      for (int r = 0; r < 4; ++r) x[4 * u + r] = x2[u][r] * kq;
    }
#pragma unroll
    for (int u = 0; u < (KF == 2 ? 0 : 2); ++u) {
      u32x4 nr{0u, 0u, 0u, 0u};
      if (KF == 1) nr = *reinterpret_cast<const u32x4 *>(sb + Sl::NOFF + (16 * u + 4 * gq) * 4);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        float v;
        if (KF == 1) {
          const uint32_t w = nr[r];
          const float s0 = __half2float(__ushort_as_half((uint16_t)(w & 0xffffu)));
          if (SG < KS) {
            const float s1 = __half2float(__ushort_as_half((uint16_t)(w >> 16)));
            v = __builtin_fmaf(s1, acc[u][1][r], s0 * acc[u][0][r]);
          } else {
            v = s0 * acc[u][0][r];
          }
        } else {
          v = acc[u][0][r];
        }
        x[4 * u + r] = v * kq;
      }
    }
    if (c0 + kChunk > lim_min) {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int tok = c0 + 16 * (j >> 2) + 4 * gq + (j & 3);
        x[j] = tok < lim ? x[j] : -INFINITY;
      }
    }
  };
  // PV of the chunk in ring slot sb: O += P V, P split into fp16 hi (pha) and
  // lo (pla) parts in A-operand order.
  auto chunk_pv = [&](const uint8_t *sb, const half8 pha, const half8 pla) {
    if constexpr (VF) {
      // FP32 V: lane (gq, col) reads V[16 (j >> 2) + 4 gq + (j & 3)][16 dt + col],
      // the B operand of its P slots j = 0..7 (row reads; the four lane groups
      // hit different banks through swz32), and splits each value into FP16
      // parts v = h0 + 2^-11 h1 + 2^-22 h2: each part holds the next 11 bits
      // of what the ones before left, so the parts are exact for
      // 2^-23 <= |v| < 65504 (the host keeps larger V off this path). The
      // MFMAs weight h1 and h2 with P's hi part scaled by 2^-11 and 2^-22
      // (exact powers of two; P lo times those terms is below 2^-22 of the
      // result and left out).
      const half8 ph1 = pha * (_Float16)0x1p-11f, ph2 = pha * (_Float16)0x1p-22f;
      // Row 4 gq + (j & 3) + 16 (j >> 2), its piece 4 (dt ^ gq) + col / 4.
      const uint8_t *vl = sb + 16 * gq * D + 4 * col;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        const uint8_t *vd = vl + 64 * (dt ^ gq);
        half8 h0, h1, h2;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const float v = *reinterpret_cast<const float *>(vd + (16 * (j >> 2) + (j & 3)) * (4 * D));
          const _Float16 a = (_Float16)v;
          const float r1 = v - (float)a;
          const _Float16 c = (_Float16)(r1 * 0x1p11f);
          const float r2 = __builtin_fmaf(-(float)c, 0x1p-11f, r1);
          h0[j] = a;
          h1[j] = c;
          h2[j] = (_Float16)(r2 * 0x1p22f);
        }
        O[dt] = mfma(pha, h0, O[dt]);
        O[dt] = mfma(pla, h0, O[dt]);
        O[dt] = mfma(ph1, h1, O[dt]);
        O[dt] = mfma(ph2, h2, O[dt]);
      }
    } else {
      u32x2 vt[DT][2];
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        const int piece = 2 * dt + tpiece;
        ds_read_tr16_pair(sb + trow * (2 * D) + ((piece ^ swz<D>(trow)) * 16) + thalf,
                          sb + (16 + trow) * (2 * D) + ((piece ^ swz<D>(16 + trow)) * 16) + thalf, vt[dt][0],
                          vt[dt][1]);
      }
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        wait_dt<DT>(dt, vt[dt][0], vt[dt][1]);
        const half8 vb = __builtin_bit_cast(half8, u32x4{vt[dt][0][0], vt[dt][0][1], vt[dt][1][0], vt[dt][1][1]});
        O[dt] = mfma(pha, vb, O[dt]);
        O[dt] = mfma(pla, vb, O[dt]);
      }
    }
  };

  if constexpr (PF != 0) {
    // Row-wise prefill: a wave takes its chunks two at a time, one per ring
    // slot, as one 64-token step. The two chunks' lookups and QK products are
    // independent chains the scheduler interleaves, and one softmax update
    // (maximum, rescale) covers both. A chunk past the history (the second of
    // an odd count) arrived as zeros and is masked whole.
    for (int i = 0; i < n_chunks; i += 2) {
      if (i > 0) {  // the previous pair's reads of both slots have completed
        wait_lds();
        issue(i);
        issue(i + 1);
      }
      float x[2][8];
      // (an append workgroup's chunk comes from its own LDS writes)
      if (!app_wg) wait_vm<L>();  // chunk i has landed; chunk i + 1 may still be in flight
      chunk_logits(slot_base(0), first + i * stride, x[0]);
      if (app_wg) {  // an append workgroup's rows fill one chunk: no second one
#pragma unroll
        for (int j = 0; j < 8; ++j) x[1][j] = -INFINITY;
      } else {
        wait_vm<0>();
        chunk_logits(slot_base(1), first + (i + 1) * stride, x[1]);
      }
      float mloc = -INFINITY;
#pragma unroll
      for (int c = 0; c < 2; ++c)
        mloc = fmaxf(mloc, fmaxf(fmaxf(fmaxf(x[c][0], x[c][1]), fmaxf(x[c][2], x[c][3])),
                                 fmaxf(fmaxf(x[c][4], x[c][5]), fmaxf(x[c][6], x[c][7]))));
      const float m_new = fmaxf(m_run, col_max(mloc));
      const float alpha = m_new == -INFINITY ? 1.0f : __builtin_amdgcn_exp2f(m_run - m_new);
      const float mb = (m_new == -INFINITY ? 0.0f : m_new) - 15.0f;
      float pr[2][8], psum = 0.0f;
#pragma unroll
      for (int c = 0; c < 2; ++c)
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          pr[c][j] = __builtin_amdgcn_exp2f(x[c][j] - mb);
          psum += pr[c][j];
        }
      l_run = __builtin_fmaf(l_run, alpha, psum);
      m_run = m_new;
      u32x4 ph[2], pl[2];
#pragma unroll
      for (int c = 0; c < 2; ++c)
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          uint32_t h, l;
          split2(pr[c][2 * k], pr[c][2 * k + 1], h, l);
          ph[c][k] = h;
          pl[c][k] = l;
        }
      if (__builtin_amdgcn_ballot_w64(alpha != 1.0f)) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float ar = __shfl(alpha, 4 * gq + r, 64);
#pragma unroll
          for (int dt = 0; dt < DT; ++dt) O[dt][r] *= ar;
        }
      }
      chunk_pv(slot_base(0), __builtin_bit_cast(half8, ph[0]), __builtin_bit_cast(half8, pl[0]));
      if (!app_wg) chunk_pv(slot_base(1), __builtin_bit_cast(half8, ph[1]), __builtin_bit_cast(half8, pl[1]));
    }
  } else {
    for (int i = 0; i < n_chunks; ++i) {
      const int c0 = first + i * stride;
      // Refill the buffer computed on last iteration with chunk i + AHEAD, then
      // wait for chunk i: its DMA is older than the (up to AHEAD) chunks issued
      // after it. With materialised logits the loop also stores, so wait for all.
      if (i + AHEAD < n_chunks) {
        wait_lds();
        issue(i + AHEAD);
      }
      const int newer = lg ? 0 : min(n_chunks - 1 - i, AHEAD);
      if (newer == AHEAD) wait_vm<AHEAD * L>();
      else if (AHEAD > 2 && newer == 2) wait_vm<2 * L>();
      else if (newer >= 1) wait_vm<L>();
      else wait_vm<0>();
      const uint8_t *sb = slot_base(i % Sl::RING);
      if (i == i_new) {  // the appended row over the chunk's LDS copy (wave-uniform)
        // Packed K: the new token's logit is masked here (the encoder counts
        // it), so only its V row has to be finite.
        const int r = t_new % kChunk;
        uint8_t *wsb = const_cast<uint8_t *>(sb);
        if (lane < PR) *reinterpret_cast<u32x4 *>(wsb + r * (2 * D) + ((lane ^ swz<D>(r)) * 16)) = v_new16;
        if (KF == 0 && lane < PR)
          *reinterpret_cast<u32x4 *>(wsb + Sl::KOFF + r * (2 * D) + ((lane ^ swz<D>(r)) * 16)) = k_new16;
      }

      float x[8];
      chunk_logits(sb, c0, x);
      if (lg) {  // materialised logits for inspect() (natural units)
  #pragma unroll
        for (int j = 0; j < 8; ++j) {
          const int tok = c0 + 16 * (j >> 2) + 4 * gq + (j & 3);
          if (head_ok && tok < t_logit) p.logits[((int64_t)qrow * Hq + hq0 + col) * p.logit_stride + tok] = x[j] * kLn2;
        }
      }
      // online softmax (log2 domain) for head col
      float mloc = fmaxf(fmaxf(fmaxf(x[0], x[1]), fmaxf(x[2], x[3])), fmaxf(fmaxf(x[4], x[5]), fmaxf(x[6], x[7])));
      const float m_new = fmaxf(m_run, col_max(mloc));
      const float alpha = m_new == -INFINITY ? 1.0f : __builtin_amdgcn_exp2f(m_run - m_new);
      const float mb = (m_new == -INFINITY ? 0.0f : m_new) - 15.0f;
      float pr[8], psum = 0.0f;
  #pragma unroll
      for (int j = 0; j < 8; ++j) {
        pr[j] = __builtin_amdgcn_exp2f(x[j] - mb);
        psum += pr[j];
      }
      l_run = __builtin_fmaf(l_run, alpha, psum);
      m_run = m_new;
      u32x4 ph, pl;
  #pragma unroll
      for (int k = 0; k < 4; ++k) {
        uint32_t h, l;
        split2(pr[2 * k], pr[2 * k + 1], h, l);
        ph[k] = h;
        pl[k] = l;
      }
      if (__builtin_amdgcn_ballot_w64(alpha != 1.0f)) {
  #pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float ar = __shfl(alpha, 4 * gq + r, 64);
  #pragma unroll
          for (int dt = 0; dt < DT; ++dt) O[dt][r] *= ar;
        }
      }
      // PV: B operand = V[tokens of this lane's P slots][16 dt + col], read
      // transposed (inline asm with explicit LDS waits; the appended row's LDS
      // stores above are ordered before the reads by the memory clobber).
      // Before them the wave waits for the chunk issued at the top of this
      // iteration, so each wave has loads in flight only during the first half
      // of an iteration. Measured at 64 x 32768 tokens (layout B), this is
      // faster than keeping a ring full across iterations: 6264 GB/s against
      // 5826 for these two slots waited for at the next iteration's top, 5780
      // for three slots (two chunks ahead), 6170 for three slots waited for
      // here. PF: the history is in L2 and the ring deeper, so only the chunk
      // computed is waited for (at the top of the iteration).
      if (!PF) wait_vm<0>();
      const half8 pha = __builtin_bit_cast(half8, ph), pla = __builtin_bit_cast(half8, pl);
      chunk_pv(sb, pha, pla);
    }
  }

  // ---------------- epilogue ----------------
  const float l_tot = col_sum(l_run) * (1.0f / kPScale);
  wait_vm<0>();     // a wave without chunks still has its prologue's zero-sized chunk loads to retire
  __syncthreads();  // every wave is done with the ring
  float *comb = reinterpret_cast<float *>(smem);  // [wave][16 heads][2 + D]
  if (gq == 0) {
    comb[(wave * 16 + col) * (D + 2)] = m_run;
    comb[(wave * 16 + col) * (D + 2) + 1] = l_tot;
  }
#pragma unroll
  for (int dt = 0; dt < DT; ++dt)
#pragma unroll
    for (int r = 0; r < 4; ++r)
      comb[(wave * 16 + 4 * gq + r) * (D + 2) + 2 + 16 * dt + col] = O[dt][r] * (1.0f / kPScale);
  __syncthreads();
  if constexpr (!PF) {
    // Decode: the waves' states of each of the G heads merged by log-sum-exp,
    // a thread per element (head g, dimension dm) in rounds of kThreads. A
    // round's LDS reads of every wave's (m, l, o) are issued before any is
    // used (threads past G D read head G - 1's and store nothing), and the
    // waves without tokens (m = -inf) drop out through selects: a read under
    // a per-wave test would be an LDS round trip of its own.
    constexpr int EPR = (16 * D + kThreads - 1) / kThreads;  // rounds for up to 16 heads
#pragma unroll
    for (int k = 0; k < EPR; ++k) {
      if (k * kThreads >= G * D) break;  // wave-uniform
      const int e = tid + k * kThreads;
      const int g = e / D, dm = e - g * D;
      const int gr = g < G ? g : G - 1;
      float mw[kWaves], lw[kWaves], ow[kWaves];
#pragma unroll
      for (int w = 0; w < kWaves; ++w) {
        const float *c = comb + (w * 16 + gr) * (D + 2);
        mw[w] = c[0];
        lw[w] = c[1];
        ow[w] = c[2 + dm];
      }
      float M = -INFINITY;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) M = fmaxf(M, mw[w]);
      float Lsum = 0.0f, Ov = 0.0f;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) {
        const bool live = mw[w] != -INFINITY;
        const float wt = __builtin_amdgcn_exp2f(mw[w] - M);
        Lsum = live ? __builtin_fmaf(lw[w], wt, Lsum) : Lsum;
        Ov = live ? __builtin_fmaf(ow[w], wt, Ov) : Ov;
      }
      if (g >= G) continue;
      const int64_t head = (int64_t)qrow * Hq + hq0 + g;
      if (S == 1) {
        p.out[head * D + dm] = Ov / Lsum;
        if (dm == 0 && p.stats) {
          p.stats[head * 2] = M * kLn2;
          p.stats[head * 2 + 1] = Lsum;
        }
      } else {
        // Device-coherent (write-through) stores: the merging workgroup may run
        // on another XCD, whose L2 does not see this one's.
        float *pp = p.part + (head * S + pslot) * (D + 2);
        coherent_store(pp + 2 + dm, Ov);
        if (dm == 0) {
          coherent_store(pp, M);
          coherent_store(pp + 1, Lsum);
        }
      }
    }
  } else {
    // Row-wise prefill: the four waves' states of each column merged by
    // log-sum-exp. Every LDS
    // read of a thread's elements (column g, dimension dm) is issued before
    // any of them is used (columns past ncol read column 0's and store
    // nothing), and the waves without tokens (m = -inf) drop out through
    // selects: reads under a per-wave test would each be an LDS round trip of
    // their own.
    constexpr int EPT = UC * D / kThreads;  // elements per thread
    float mw[EPT][kWaves], lw[EPT][kWaves], ow[EPT][kWaves];
#pragma unroll
    for (int k = 0; k < EPT; ++k) {
      const int e = tid + k * kThreads;
      const int g = e / D, dm = e - g * D;
      const int gr = g < ncol ? g : 0;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) {
        const float *c = comb + (w * 16 + gr) * (D + 2);
        mw[k][w] = c[0];
        lw[k][w] = c[1];
        ow[k][w] = c[2 + dm];
      }
    }
    // Partial rows: o[D], then m, l (16-byte aligned rows of D + 4 floats).
    constexpr int PROW = D + 4;
    float Mk[EPT], Lk[EPT], Ok[EPT];
#pragma unroll
    for (int k = 0; k < EPT; ++k) {
      float M = -INFINITY;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) M = fmaxf(M, mw[k][w]);
      float Lsum = 0.0f, Ov = 0.0f;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) {
        const bool live = mw[k][w] != -INFINITY;
        const float wt = __builtin_amdgcn_exp2f(mw[k][w] - M);
        Lsum = live ? __builtin_fmaf(lw[k][w], wt, Lsum) : Lsum;
        Ov = live ? __builtin_fmaf(ow[k][w], wt, Ov) : Ov;
      }
      Mk[k] = M;
      Lk[k] = Lsum;
      Ok[k] = Ov;
    }
#pragma unroll
    for (int k = 0; k < EPT; ++k) {
      const int e = tid + k * kThreads;
      const int g = e / D, dm = e - g * D;
      const float M = Mk[k], Lsum = Lk[k], Ov = Ok[k];
      if (g >= ncol) continue;
      const int64_t head = out_row(g);
      if (S == 1) {
        p.out[head * D + dm] = Ov / Lsum;
      } else {
        // Device-coherent (write-through) stores, as above.
        float *pp = p.part + ((pbase + g) * SP + pslot) * PROW;
        coherent_store(pp + dm, Ov);
        if (dm == 0) {
          coherent_store(pp + D, M);
          coherent_store(pp + D + 1, Lsum);
        }
      }
    }
  }
  if (S == 1) return;
  // Last workgroup of this (sequence, KV head) to finish merges the splits.
  // Every thread waits for its partial stores to complete before the arrival
  // is counted, so no cache write-back is needed.
  // The flag lives in the lookup tables' LDS (dead since the loop): a
  // separate variable would add 16 bytes, and the two-scale-DMA d=64 layout
  // uses exactly half of the CU's LDS.
  int *last = reinterpret_cast<int *>(tabs);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (tid == 0)
    *last = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
            (unsigned)(S - 1);
  __syncthreads();
  if (!*last) return;
  if (PF) {
    const MergeRows mr{pbase, (int64_t)b * rows * Hq + hq0, UC * qg, G, Hq, ncol, SP};
    static_assert(kPrefillMaxSplits == 16, "merge_rows instances");
    static_assert(UC % NW == 0, "merge_rows: whole columns per wave");
    if (S <= 8) merge_rows<D, 8, UC / NW, NW>(p.part, p.out, mr, S, wave, lane);
    else merge_rows<D, 16, UC / NW, NW>(p.part, p.out, mr, S, wave, lane);
    if (tid == 0) __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return;
  }
  if (S <= kMergeOneRound) {
    if (S <= 8) merge_one_round<D, 8, NW>(p.part, p.out, p.stats, (int64_t)qrow * Hq + hq0, G, S, wave, lane);
    else if (S <= 16) merge_one_round<D, 16, NW>(p.part, p.out, p.stats, (int64_t)qrow * Hq + hq0, G, S, wave, lane);
    else if (S <= 24) merge_one_round<D, 24, NW>(p.part, p.out, p.stats, (int64_t)qrow * Hq + hq0, G, S, wave, lane);
    else merge_one_round<D, kMergeOneRound, NW>(p.part, p.out, p.stats, (int64_t)qrow * Hq + hq0, G, S, wave, lane);
    if (tid == 0) __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return;
  }
  // More splits: every load of a stage in flight at once: (m, l) of all
  // heads and splits, then per-head normalised weights, then the o rows in
  // groups of eight splits.
  float *wgt = reinterpret_cast<float *>(smem);  // [16 heads][S] (reuses the ring)
  float *mrow = wgt + 16 * S;                     // [16 heads][S] split maxima
  for (int e = tid; e < ncol * S; e += kThreads) {
    const int g = e / S, s = e - g * S;
    float *pp = p.part + ((pbase + g) * S + s) * (D + 2);
    mrow[g * S + s] = coherent_load(pp);
    wgt[g * S + s] = coherent_load(pp + 1);
  }
  __syncthreads();
  if (tid < ncol) {
    float M = -INFINITY;
    for (int s = 0; s < S; ++s) M = fmaxf(M, mrow[tid * S + s]);
    float Lsum = 0.0f;
    for (int s = 0; s < S; ++s) {
      const float m = mrow[tid * S + s];
      const float w = m == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m - M);
      Lsum = __builtin_fmaf(wgt[tid * S + s], w, Lsum);
      mrow[tid * S + s] = w;
    }
    for (int s = 0; s < S; ++s) wgt[tid * S + s] = mrow[tid * S + s] / Lsum;
    if (p.stats) {
      const int64_t head = out_row(tid);
      p.stats[head * 2] = M * kLn2;
      p.stats[head * 2 + 1] = Lsum;
    }
  }
  __syncthreads();
  for (int e = tid; e < ncol * D; e += kThreads) {
    const int g = e / D, dm = e - g * D;
    const int64_t head = out_row(g);
    float *pp = p.part + (pbase + g) * S * (D + 2) + 2 + dm;
    float Ov = 0.0f;
    for (int s0 = 0; s0 < S; s0 += 8) {
      // Unconditional loads (past S: split S - 1, weighted zero), all eight in
      // flight together; loads under a branch would go one after another.
      float o[8], w8[8];
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const int sk = min(s0 + k, S - 1);
        o[k] = coherent_load(pp + sk * (D + 2));
        w8[k] = wgt[g * S + sk];
      }
#pragma unroll
      for (int k = 0; k < 8; ++k) Ov = __builtin_fmaf(o[k], s0 + k < S ? w8[k] : 0.0f, Ov);
    }
    p.out[head * D + dm] = Ov;
  }
  if (tid == 0) __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <int D, int KF, int NN, int SG, int PK = 0, int PF = 0, int VF = 0, int NW = kWaves, int AP = 1>
__global__ __launch_bounds__(64 * NW) void decode_fast_kernel(DecodeParams p, FastLayout fl) {
  using Sl = Slot<D, KF, NN, VF, NW>;
  __shared__ __align__(16) uint8_t tabs[KF >= 1 ? Sl::TABLES : 16];
  if constexpr (AP == 1 && KF >= 1) {
    // With appended rows (every launch of this instance has them) the
    // append workgroups come after the splits; each role gets code of its
    // own, so a history split carries none of the encoder's.
    using Gm = Geo<D>;
    const int split = PF ? blockIdx.z : blockIdx.x, kv = PF ? blockIdx.x : blockIdx.y;
    BGTQ_LOAD_ARGS  // here, so the branch on p.splits waits for no load of its own
    if (split >= p.splits) decode_fast_body<D, KF, NN, SG, PK, PF, VF, NW, AP, 2>(p, fl, tabs);
    else decode_fast_body<D, KF, NN, SG, PK, PF, VF, NW, AP, 1>(p, fl, tabs);
  } else {
    decode_fast_body<D, KF, NN, SG, PK, PF, VF, NW, AP, 0>(p, fl, tabs);
  }
}
#undef BGTQ_LOAD_ARGS
#undef BGTQ_ARGS

template <int D, int KF, int NN, int SG, int PK, int PF, int VF = 0, int NW = kWaves, int AP = 1>
hipError_t launch_mode(const DecodeParams &p, const FastLayout &fl, hipStream_t stream) {
  // More than 64 KB of dynamic LDS has to be allowed per kernel (gfx950: up to 160 KB).
  static const hipError_t allowed =
      hipFuncSetAttribute((const void *)decode_fast_kernel<D, KF, NN, SG, PK, PF, VF, NW, AP>,
                          hipFuncAttributeMaxDynamicSharedMemorySize,
                          Slot<D, KF, NN, VF, NW>::DYN + (PF ? prefill_stage_bytes(D) : 0));
  if (allowed != hipSuccess) {
    (void)hipGetLastError();  // do not leave the failure behind for the caller's next HIP call
    return allowed;
  }
  constexpr int lds = Slot<D, KF, NN, VF, NW>::DYN + (PF ? prefill_stage_bytes(D) : 0);
  static_assert(lds + Slot<D, KF, NN, VF, NW>::TABLES <= kLdsLimit, "LDS of one workgroup");
  // Appended rows with packed K: app_parts more workgroups per (sequence, KV
  // head) or unit for them.
  const unsigned app = KF >= 1 && p.k_new ? (unsigned)p.app_parts : 0u;
  const dim3 grid = PF ? dim3((unsigned)p.kv_heads, (unsigned)(p.batch * p.qgroups), (unsigned)p.splits + app)
                       : dim3((unsigned)p.splits + app, (unsigned)p.kv_heads, (unsigned)p.batch);
  hipLaunchKernelGGL((decode_fast_kernel<D, KF, NN, SG, PK, PF, VF, NW, AP>), grid, dim3(64 * NW), lds, stream, p, fl);
  return hipGetLastError();
}

// Row-wise prefill (p.starts set) runs the PF variant of its unit width;
// FP32 V (decode without an appended token) the VF variant. KINDS: the kinds
// of launch whose instances this translation unit holds (the others return
// hipErrorInvalidValue; the dispatch routes each kind to its unit).
template <int KINDS, int D, int KF, int NN, int SG, int PK = 0>
hipError_t launch_one(const DecodeParams &p, const FastLayout &fl, hipStream_t stream) {
  const int kind = decode_fast_launch_kind(p);
  if (!(kind & KINDS)) return hipErrorInvalidValue;
  if (p.v_dtype == BGTQ_DTYPE_F32) {
    if constexpr ((KINDS & kKindDecode) != 0)
      if (kind == kKindDecode)
        return p.logits ? launch_mode<D, KF, NN, SG, PK, 0, 1, kWaves, 2>(p, fl, stream)
                        : launch_mode<D, KF, NN, SG, PK, 0, 1, kWaves, 0>(p, fl, stream);
    return hipErrorInvalidValue;
  }
  if constexpr ((KINDS & kKindDecode) != 0)
    if (kind == kKindDecode) {
      // The instance with the extra outputs the launch has: materialised
      // logits (2) or none (0).
      if constexpr (D == 64)
        if (p.waves == 8)
          return p.logits ? launch_mode<D, KF, NN, SG, PK, 0, 0, 8, 2>(p, fl, stream)
                          : launch_mode<D, KF, NN, SG, PK, 0, 0, 8, 0>(p, fl, stream);
      return p.logits ? launch_mode<D, KF, NN, SG, PK, 0, 0, kWaves, 2>(p, fl, stream)
                      : launch_mode<D, KF, NN, SG, PK, 0, 0, kWaves, 0>(p, fl, stream);
    }
  if constexpr ((KINDS & kKindAppend) != 0)
    if (kind == kKindAppend) {
      if constexpr (D == 64)
        if (p.waves == 8) return launch_mode<D, KF, NN, SG, PK, 0, 0, 8, 1>(p, fl, stream);
      return launch_mode<D, KF, NN, SG, PK, 0, 0, kWaves, 1>(p, fl, stream);
    }
  if constexpr ((KINDS & kKindPrefill) != 0) {
    // Row-wise prefill without appended rows runs an instance without the
    // append code (AP 0).
    constexpr int NW = decode_fast_prefill_waves(D);
    if (!p.k_new)
      return p.unit_cols == 8 ? launch_mode<D, KF, NN, SG, PK, 8, 0, NW, 0>(p, fl, stream)
                              : launch_mode<D, KF, NN, SG, PK, 16, 0, NW, 0>(p, fl, stream);
    return p.unit_cols == 8 ? launch_mode<D, KF, NN, SG, PK, 8, 0, NW>(p, fl, stream)
                            : launch_mode<D, KF, NN, SG, PK, 16, 0, NW>(p, fl, stream);
  }
  return hipErrorInvalidValue;
}

// The instance families, each over the kinds of launch in KINDS.
// Structured layouts (NN nibble K-steps, SG K-steps in group 0) and FP16 K.
template <int KINDS>
hipError_t launch_family_d64(const DecodeParams &p, const FastLayout &fl, int nn, int sg, hipStream_t stream) {
  if (p.key_format == 0) return launch_one<KINDS, 64, 0, 0, 2>(p, fl, stream);
  if (nn == 1 && sg == 1) return launch_one<KINDS, 64, 1, 1, 1>(p, fl, stream);
  if (nn == 2 && sg == 2) return launch_one<KINDS, 64, 1, 2, 2>(p, fl, stream);
  if (nn == 0 && sg == 2) return launch_one<KINDS, 64, 1, 0, 2>(p, fl, stream);
  if (nn == 2 && sg == 1) return launch_one<KINDS, 64, 1, 2, 1>(p, fl, stream);
  if (nn == 0 && sg == 1) return launch_one<KINDS, 64, 1, 0, 1>(p, fl, stream);
  return hipErrorInvalidValue;
}

template <int KINDS>
hipError_t launch_family_d128(const DecodeParams &p, const FastLayout &fl, int nn, int sg, hipStream_t stream) {
  if (p.key_format == 0) return launch_one<KINDS, 128, 0, 0, 4>(p, fl, stream);
  if (nn == 2 && sg == 2) return launch_one<KINDS, 128, 1, 2, 2>(p, fl, stream);
  if (nn == 4 && sg == 4) return launch_one<KINDS, 128, 1, 4, 4>(p, fl, stream);
  if (nn == 0 && sg == 4) return launch_one<KINDS, 128, 1, 0, 4>(p, fl, stream);
  if (nn == 4 && sg == 2) return launch_one<KINDS, 128, 1, 4, 2>(p, fl, stream);
  if (nn == 0 && sg == 2) return launch_one<KINDS, 128, 1, 0, 2>(p, fl, stream);
  return hipErrorInvalidValue;
}

// Any packed layout: one or two scale DMAs per chunk (the largest norm stride
// of the launch's heads), pair lookups for K-step 0 when every head's K-step
// 0 is a pair K-step.
template <int KINDS, int D>
hipError_t launch_family_any(const DecodeParams &p, const FastLayout &fl, hipStream_t stream) {
  int ns = 0;
  for (int h = 0; h < p.kv_heads; ++h) ns = fl.gns[h] > ns ? fl.gns[h] : ns;
  const bool pk = fl.gpair_lead >= 1;
  if (ns <= 4) return pk ? launch_one<KINDS, D, 2, 1, 1, 1>(p, fl, stream) : launch_one<KINDS, D, 2, 1, 1>(p, fl, stream);
  return pk ? launch_one<KINDS, D, 2, 2, 1, 1>(p, fl, stream) : launch_one<KINDS, D, 2, 2, 1>(p, fl, stream);
}

}  // namespace
}  // namespace bgtq
