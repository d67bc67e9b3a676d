// Calibration-table pipeline on the host, for callers without Python: the
// greedy bit allocation (src/reference/allocator.py:4-17), the grouping of
// RoPE pairs by width (src/reference/mixed_layout.py:5-18; upstream
// _post_allocation_setup, vendor/blockgtq/block_gtq_pipeline.py:151-246) and
// the 256-bin code LUT with its per-position offsets and inverse bin widths
// (vendor/blockgtq/quant_kernels.py:276-364), serialised as tables(p)
// (src/webgpu/layout.ts:24-31). The per-width codebooks and rotations are
// inputs: they come from the committed calibration blobs or from the
// caller's own generator. Same arithmetic as the reference's tables:
//  * priorities s * 4^-w in FP64 from FP32 scores, first index on ties;
//  * a stable sort of the pairs by width (the committed tables' tie order);
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

struct Grouping {
  std::vector<int64_t> order;       // pairs sorted by width (stable)
  std::vector<int32_t> bits;        // width of each group, ascending
  std::vector<int32_t> offsets;     // group position ranges, size groups + 1
  std::vector<uint32_t> head_perm;  // [2L]: (p, p + L) interleaved in sorted order
  std::vector<uint32_t> group_of;   // [2L]
  int32_t nibble_dims = 0, row_bytes = 0;
};

Grouping group_pairs(const int64_t *widths, size_t L) {
  Grouping g;
  g.order.resize(L);
  for (size_t i = 0; i < L; ++i) g.order[i] = (int64_t)i;
  std::stable_sort(g.order.begin(), g.order.end(), [&](int64_t a, int64_t b) { return widths[a] < widths[b]; });
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
