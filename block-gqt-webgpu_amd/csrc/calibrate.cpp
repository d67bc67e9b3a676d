// Calibration-table pipeline on the host, for callers without Python: the
// greedy bit allocation (src/reference/allocator.py:4-17), the grouping of
// RoPE pairs by width (src/reference/mixed_layout.py:5-18; upstream
// _post_allocation_setup, vendor/blockgtq/block_gtq_pipeline.py:151-246) and
// the 256-bin code LUT with its per-position offsets and inverse bin widths
// (vendor/blockgtq/quant_kernels.py:276-364; Block-GTQ,
// https://github.com/JIA-Lab-research/blockgtq commit 3fe14e7, Apache License
// 2.0, whose setup steps are restated so the tables match bit for bit),
// serialised as tables(p)
// (src/webgpu/layout.ts:24-31). The per-width codebooks and rotations are
// inputs: they come from the committed calibration blobs or from the
// caller's own generator. Same arithmetic as the reference's tables:
//  * priorities s * 4^-w in FP64 from FP32 scores, first index on ties;
//  * the pairs sorted by width in the tie order of the committed tables
//    (torch's non-stable argsort as the Windows build evaluates it, below);
//  * bin offsets and inverse widths in FP64, stored as FP32;
//  * bin centres from an FP32 linspace (halves from each end, as torch
//    evaluates it) and the code of a centre = the first boundary >= it
//    (torch.searchsorted, left side), clamped to the last centroid.
#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <map>
#include <string>
#include <vector>

#include "../../include/bgtq.h"
#include "bgtq_internal.h"

// Every FP32 operation rounds on its own, as the reference's numpy/torch code.
#pragma clang fp contract(off)

namespace {

bgtq_status err(bgtq_status code, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
bgtq_status err(bgtq_status code, const char *fmt, ...) {
  char buf[256];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  return bgtq::set_error(code, buf);
}

constexpr int kBins = 256;

// The order torch.argsort(widths) (not stable) gave the reference's
// committed tables (src/reference/mixed_layout.py:7-8; the goldens were
// written on Windows). ATen's CPU sort fills indices 0..n-1 beside the keys
// and sorts the (key, index) pairs with std::sort comparing keys only; the
// Microsoft STL's std::sort (<algorithm>, _Sort_unchecked) insertion-sorts a
// range of at most 32 elements, which keeps equal widths in pair order, and
// splits a larger one around a median guess (median of three, Tukey's
// ninther above 40 elements) with a three-way partition whose swaps decide
// the order of equal widths. Restated from that published algorithm
// (Microsoft STL, Apache License 2.0 WITH LLVM-exception); with
// 33..64 pairs the result differs from a stable sort (fixtures mixed_d128,
// low_d128). Widths take at most 8 distinct values and every partition
// removes all elements equal to its pivot, so no range is split more than 8
// times and the library's heap-sort fallback (after about 1.5 log2 n splits)
// is never reached.
class TieOrderSort {
 public:
  TieOrderSort(const int64_t *widths, size_t n) : key_(n), idx_(n) {
    for (size_t i = 0; i < n; ++i) {
      key_[i] = widths[i];
      idx_[i] = (int64_t)i;
    }
  }
  std::vector<int64_t> run() {
    const int64_t n = (int64_t)key_.size();
    sort(0, n, n);
    return idx_;
  }

 private:
  std::vector<int64_t> key_, idx_;
  static constexpr int64_t kInsertionMax = 32;

  bool lt(int64_t i, int64_t j) const { return key_[i] < key_[j]; }
  void swap(int64_t i, int64_t j) {
    std::swap(key_[i], key_[j]);
    std::swap(idx_[i], idx_[j]);
  }
  void med3(int64_t f, int64_t m, int64_t l) {
    if (lt(m, f)) swap(m, f);
    if (lt(l, m)) {
      swap(l, m);
      if (lt(m, f)) swap(m, f);
    }
  }
  // Moves a median guess of [f, l] (inclusive) to m.
  void guess_median(int64_t f, int64_t m, int64_t l) {
    const int64_t count = l - f;
    if (count > 40) {
      const int64_t step = (count + 1) >> 3, two = step << 1;
      med3(f, f + step, f + two);
      med3(m - step, m, m + step);
      med3(l - two, l - step, l);
      med3(f + step, m, l - step);
    } else {
      med3(f, m, l);
    }
  }
  // Three-way partition of [first, last): returns the range of elements equal
  // to the pivot; smaller ones lie before it, larger ones after.
  std::pair<int64_t, int64_t> partition(int64_t first, int64_t last) {
    const int64_t mid = first + ((last - first) >> 1);
    guess_median(first, mid, last - 1);
    int64_t pf = mid, pl = mid + 1;
    while (first < pf && !lt(pf - 1, pf) && !lt(pf, pf - 1)) --pf;
    while (pl < last && !lt(pl, pf) && !lt(pf, pl)) ++pl;
    int64_t gf = pl, gl = pf;
    for (;;) {
      for (; gf < last; ++gf) {
        if (lt(pf, gf)) continue;
        if (lt(gf, pf)) break;
        if (pl != gf) swap(pl, gf);
        ++pl;
      }
      for (; first < gl; --gl) {
        const int64_t gp = gl - 1;
        if (lt(gp, pf)) continue;
        if (lt(pf, gp)) break;
        if (--pf != gp) swap(pf, gp);
      }
      if (gl == first && gf == last) return {pf, pl};
      if (gl == first) {  // no room below: rotate the pivot run upward
        if (pl != gf) swap(pf, pl);
        ++pl;
        swap(pf, gf);
        ++pf;
        ++gf;
      } else if (gf == last) {  // no room above: rotate it downward
        if (--gl != --pf) swap(gl, pf);
        swap(pf, --pl);
      } else {
        swap(gf, --gl);
        ++gf;
      }
    }
  }
  void insertion(int64_t first, int64_t last) {
    for (int64_t mid = first + 1; mid < last; ++mid) {
      const int64_t k = key_[mid], ix = idx_[mid];
      int64_t hole = mid;
      if (k < key_[first]) {
        for (; hole > first; --hole) {
          key_[hole] = key_[hole - 1];
          idx_[hole] = idx_[hole - 1];
        }
      } else {
        for (; k < key_[hole - 1]; --hole) {
          key_[hole] = key_[hole - 1];
          idx_[hole] = idx_[hole - 1];
        }
      }
      key_[hole] = k;
      idx_[hole] = ix;
    }
  }
  void sort(int64_t first, int64_t last, int64_t ideal) {
    for (;;) {
      // ideal <= 0 (the library's heap-sort fallback) cannot happen for widths
      // 1..8; an insertion sort keeps the result a correct sort regardless.
      if (last - first <= kInsertionMax || ideal <= 0) {
        insertion(first, last);
        return;
      }
      const std::pair<int64_t, int64_t> m = partition(first, last);
      ideal = (ideal >> 1) + (ideal >> 2);
      if (m.first - first < last - m.second) {
        sort(first, m.first, ideal);
        first = m.second;
      } else {
        sort(m.second, last, ideal);
        last = m.first;
      }
    }
  }
};

struct Grouping {
  std::vector<int64_t> order;       // pairs sorted by width (tie order above)
  std::vector<int32_t> bits;        // width of each group, ascending
  std::vector<int32_t> offsets;     // group position ranges, size groups + 1
  std::vector<uint32_t> head_perm;  // [2L]: (p, p + L) interleaved in sorted order
  std::vector<uint32_t> group_of;   // [2L]
  int32_t nibble_dims = 0, row_bytes = 0;
};

Grouping group_pairs(const int64_t *widths, size_t L) {
  Grouping g;
  g.order = TieOrderSort(widths, L).run();
  g.head_perm.resize(2 * L);
  g.group_of.resize(2 * L);
  g.offsets.push_back(0);
  for (size_t k = 0; k < L; ++k) {
    const int64_t p = g.order[k];
    g.head_perm[2 * k] = (uint32_t)p;
    g.head_perm[2 * k + 1] = (uint32_t)(p + (int64_t)L);
    if (g.bits.empty() || g.bits.back() != (int32_t)widths[p]) {
      if (!g.bits.empty()) g.offsets.push_back((int32_t)(2 * k));
      g.bits.push_back((int32_t)widths[p]);
    }
    g.group_of[2 * k] = g.group_of[2 * k + 1] = (uint32_t)(g.bits.size() - 1);
    if (widths[p] <= 4) g.nibble_dims += 2;
  }
  g.offsets.push_back((int32_t)(2 * L));
  g.row_bytes = g.nibble_dims / 2 + (int32_t)(2 * L) - g.nibble_dims;
  return g;
}

// torch.linspace(start, end, kBins) in FP32: start + step*i for the first
// half, end - step*(kBins - 1 - i) for the second.
void linspace_f32(double start_d, double end_d, float *out) {
  const float start = (float)start_d, end = (float)end_d;
  const float step = (end - start) / (float)(kBins - 1);
  for (int i = 0; i < kBins; ++i)
    out[i] = i < kBins / 2 ? start + step * (float)i : end - step * (float)(kBins - 1 - i);
}

}  // namespace

extern "C" {

bgtq_status bgtq_allocate_bits(const float *scores, size_t n_pairs, int64_t budget, int32_t min_bits,
                               int32_t max_bits, int64_t *widths) {
  if (n_pairs && (!scores || !widths)) return err(BGTQ_ERR_RANGE, "null argument");
  if (min_bits < 0 || max_bits < min_bits) return err(BGTQ_ERR_RANGE, "invalid bit range");
  int64_t remaining = budget;
  for (size_t i = 0; i < n_pairs; ++i) {
    widths[i] = min_bits;
    remaining -= min_bits;
  }
  while (remaining > 0 && n_pairs) {
    size_t best = 0;
    double best_pri = 0.0;
    for (size_t i = 0; i < n_pairs; ++i) {
      const double pri = widths[i] >= max_bits ? -1.0 : (double)scores[i] * std::pow(4.0, -(double)widths[i]);
      if (i == 0 || pri > best_pri) {
        best = i;
        best_pri = pri;
      }
    }
    if (!(best_pri > 0.0)) break;
    widths[best] += 1;
    remaining -= 1;
  }
  return BGTQ_OK;
}

bgtq_status bgtq_layout_groups(const int64_t *widths, size_t n_pairs, int32_t *n_groups, int32_t *bits,
                               int32_t *group_dims) {
  if (!widths || !n_groups || !bits || !group_dims) return err(BGTQ_ERR_RANGE, "null argument");
  if (n_pairs < 1 || n_pairs > (size_t)bgtq::kMaxDim / 2) return err(BGTQ_ERR_RANGE, "1 to 64 pairs required");
  for (size_t i = 0; i < n_pairs; ++i)
    if (widths[i] < 1 || widths[i] > 8) return err(BGTQ_ERR_RANGE, "pair %zu: width %lld outside 1..8", i, (long long)widths[i]);
  const Grouping g = group_pairs(widths, n_pairs);
  if (g.bits.size() > (size_t)bgtq::kMaxGroups) return err(BGTQ_ERR_RANGE, "more than 8 distinct widths");
  *n_groups = (int32_t)g.bits.size();
  for (size_t k = 0; k < g.bits.size(); ++k) {
    bits[k] = g.bits[k];
    group_dims[k] = g.offsets[k + 1] - g.offsets[k];
  }
  return BGTQ_OK;
}

bgtq_status bgtq_layout_build(const int64_t *widths, size_t n_pairs, const bgtq_group_tables *groups, size_t n_groups,
                              int32_t row_bytes, int32_t norm_stride, uint32_t *integer, size_t *n_integer,
                              float *floating, size_t *n_floating) {
  if (!n_integer || !n_floating) return err(BGTQ_ERR_RANGE, "null argument");
  int32_t ng = 0, gbits[bgtq::kMaxGroups], gdims[bgtq::kMaxGroups];
  if (bgtq_status s = bgtq_layout_groups(widths, n_pairs, &ng, gbits, gdims)) return s;
  if ((size_t)ng != n_groups || !groups)
    return err(BGTQ_ERR_RANGE, "%d groups in this allocation, %zu table sets given", ng, n_groups);
  const Grouping g = group_pairs(widths, n_pairs);
  const int d = (int)(2 * n_pairs);
  int maxc = 0;
  for (int k = 0; k < ng; ++k) maxc = std::max(maxc, 1 << gbits[k]);
  if (row_bytes == 0) row_bytes = g.row_bytes;
  if (norm_stride == 0) norm_stride = ng;
  if (row_bytes < g.row_bytes || norm_stride < ng) return err(BGTQ_ERR_RANGE, "row_bytes or norm_stride too small");

  // Per-position centroids [d][maxc] (zero padded) and FP32 midpoint
  // boundaries [d][maxc - 1] (infinity padded).
  std::vector<float> cents((size_t)d * maxc, 0.0f), bounds((size_t)d * std::max(maxc - 1, 1), INFINITY);
  std::vector<float> rot((size_t)d * d, 0.0f);
  for (int k = 0; k < ng; ++k) {
    const int s = g.offsets[k], e = g.offsets[k + 1], m = e - s, nc = 1 << gbits[k];
    const float *c = groups[k].centroids;
    if (!c) return err(BGTQ_ERR_RANGE, "group %d: null centroids", k);
    for (int i = 0; i + 1 < nc; ++i)
      if (!(c[i] < c[i + 1])) return err(BGTQ_ERR_RANGE, "group %d: centroids must ascend", k);
    for (int j = s; j < e; ++j) {
      for (int i = 0; i < nc; ++i) cents[(size_t)j * maxc + i] = c[i];
      for (int i = 0; i + 1 < nc; ++i) bounds[(size_t)j * (maxc - 1) + i] = (c[i] + c[i + 1]) / 2.0f;
    }
    const float *r = groups[k].rotation;
    for (int a = 0; a < m; ++a)
      for (int b = 0; b < m; ++b) rot[(size_t)(s + a) * d + (s + b)] = r ? r[a * m + b] : (a == b ? 1.0f : 0.0f);
  }

  // Offsets / inverse bin widths per position; distinct codebooks in
  // position order and their LUTs.
  std::vector<float> offs(d), inv(d);
  std::vector<uint32_t> pos_cb(d);
  std::map<std::vector<float>, uint32_t> books;
  std::vector<uint8_t> lut;
  for (int j = 0; j < d; ++j) {
    const int k = (int)g.group_of[j], nc = 1 << gbits[k];
    const float *c = &cents[(size_t)j * maxc];
    const double lo = *std::min_element(c, c + nc), hi = *std::max_element(c, c + nc);
    const double margin = (hi - lo) / std::max(nc - 1, 1) * 0.5;
    offs[j] = (float)(lo - margin);
    inv[j] = (float)(1.0 / (((hi + margin) - (lo - margin)) / kBins));
    std::vector<float> key(c, c + nc);
    auto it = books.find(key);
    if (it == books.end()) {
      const uint32_t id = (uint32_t)books.size();
      books.emplace(key, id);
      pos_cb[j] = id;
      const double width = ((hi + margin) - (lo - margin)) / kBins;
      float centers[kBins];
      linspace_f32(lo - margin + width / 2, hi + margin - width / 2, centers);
      const float *bd = &bounds[(size_t)j * (maxc - 1)];
      for (int b = 0; b < kBins; ++b) {
        int idx = 0;
        if (nc > 1) {
          idx = (int)(std::lower_bound(bd, bd + (nc - 1), centers[b]) - bd);
          idx = std::min(idx, nc - 1);
        }
        lut.push_back((uint8_t)idx);
      }
    } else {
      pos_cb[j] = it->second;
    }
  }

  const size_t ni = 10 + 3 * (size_t)d + lut.size();
  const size_t nf = (size_t)d * d + (size_t)d * maxc + 2 * (size_t)d;
  if (!integer || !floating) {
    *n_integer = ni;
    *n_floating = nf;
    return BGTQ_OK;
  }
  if (*n_integer < ni || *n_floating < nf)
    return err(BGTQ_ERR_RANGE, "table buffers of %zu / %zu elements needed", ni, nf);
  size_t o = 0;
  const uint32_t head[10] = {(uint32_t)d, (uint32_t)ng, (uint32_t)row_bytes, (uint32_t)norm_stride,
                             (uint32_t)g.nibble_dims, (uint32_t)maxc, 10, 10 + (uint32_t)d, 10 + 2 * (uint32_t)d,
                             10 + 3 * (uint32_t)d};
  for (uint32_t v : head) integer[o++] = v;
  for (int j = 0; j < d; ++j) integer[o++] = g.head_perm[j];
  for (int j = 0; j < d; ++j) integer[o++] = g.group_of[j];
  for (int j = 0; j < d; ++j) integer[o++] = pos_cb[j];
  for (uint8_t v : lut) integer[o++] = v;
  size_t f = 0;
  for (float v : rot) floating[f++] = v;
  for (float v : cents) floating[f++] = v;
  for (float v : offs) floating[f++] = v;
  for (float v : inv) floating[f++] = v;
  *n_integer = ni;
  *n_floating = nf;
  return BGTQ_OK;
}

}  // extern "C"

extern "C" {

// The rotation R and head permutation of a tables(p) blob (src/webgpu/layout.ts:24-31)
// folded into query-projection rows: out[h*d + j] = sum_i R[j][i] w[h*d + perm[i]].
// Upstream's bake_permutation_into_qproj (vendor/blockgtq/quantizer.py:1190-1244)
// does the same fold for its fused kernels; this one is written so that the
// baked queries equal the in-kernel rotation of the decode and prefill
// kernels, qr = R q[perm] (k = ((c s) R)[inv_perm], src/reference/production_math.py:27-31,
// so q . k = qr . (c s)).
bgtq_status bgtq_bake_qproj(const uint32_t *integer, size_t n_integer, const float *floating, size_t n_floating,
                            int32_t heads, int64_t in_features, const float *weight, const float *bias,
                            float *weight_out, float *bias_out) {
  if (!integer || n_integer < 10) return err(BGTQ_ERR_RANGE, "Invalid Block-GTQ layout");
  const int64_t d = integer[0], mc = integer[5];
  if (d < 2 || d > 128 || d % 2 || mc < 2 || mc > 256) return err(BGTQ_ERR_RANGE, "Invalid Block-GTQ layout");
  const uint64_t o_perm = integer[6];
  if (o_perm > n_integer || (uint64_t)d > n_integer - o_perm) return err(BGTQ_ERR_RANGE, "Invalid calibration table shape");
  const uint32_t *perm = integer + o_perm;
  std::vector<int> seen(d, 0);
  for (int64_t i = 0; i < d; ++i)
    if (perm[i] >= (uint64_t)d || seen[perm[i]]++) return err(BGTQ_ERR_RANGE, "Invalid calibration table shape");
  if (!floating || n_floating != (size_t)(d * d + d * mc + 2 * d)) return err(BGTQ_ERR_RANGE, "Invalid calibration table shape");
  for (int64_t i = 0; i < d * d; ++i)
    if (!std::isfinite(floating[i])) return err(BGTQ_ERR_RANGE, "Nonfinite calibration table");
  if (heads < 1 || in_features < 1) return err(BGTQ_ERR_RANGE, "heads and in_features must be positive");
  if (!weight || !weight_out) return err(BGTQ_ERR_RANGE, "null weight");
  if ((bias == nullptr) != (bias_out == nullptr)) return err(BGTQ_ERR_RANGE, "bias and bias_out go together");
  const float *R = floating;
  const int64_t cols = in_features;
  // Each head's rows are computed into a staging copy first, so weight_out
  // (bias_out) may be weight (bias) itself: the bake in place, as upstream's.
  std::vector<double> acc(cols);
  std::vector<float> rows((size_t)(d * cols)), brow((size_t)d);
  for (int32_t h = 0; h < heads; ++h) {
    const float *w = weight + (int64_t)h * d * cols;
    for (int64_t j = 0; j < d; ++j) {
      std::fill(acc.begin(), acc.end(), 0.0);
      double accb = 0.0;
      for (int64_t i = 0; i < d; ++i) {
        const double r = R[j * d + i];
        if (r == 0.0) continue;  // off-group entries
        const float *src = w + (int64_t)perm[i] * cols;
        for (int64_t c = 0; c < cols; ++c) acc[c] += r * (double)src[c];
        if (bias) accb += r * (double)bias[(int64_t)h * d + perm[i]];
      }
      for (int64_t c = 0; c < cols; ++c) rows[j * cols + c] = (float)acc[c];
      brow[j] = (float)accb;
    }
    std::copy(rows.begin(), rows.end(), weight_out + (int64_t)h * d * cols);
    if (bias) std::copy(brow.begin(), brow.end(), bias_out + (int64_t)h * d);
  }
  return BGTQ_OK;
}

}  // extern "C"
