"""Calibration tables for a bit allocation: the setup that produces BlockGTQParameters.

Follows the published Block-GTQ setup (upstream commit 3fe14e7, as vendored by
the reference): greedy bit allocation (src/reference/allocator.py:4-17),
grouping of RoPE pairs by width (src/reference/mixed_layout.py:5-18), one
Lloyd-Max codebook per width for N(0, 1/d_group) and one Haar rotation per
width >= rotation_threshold (vendor/blockgtq/block_gtq_pipeline.py:24-92,
151-246), and the 256-bin code LUT (vendor/blockgtq/quant_kernels.py:276-364).
Tables are inputs of the hot path; this module only builds them.

Attribution: the codebook, rotation and LUT steps (_cond_mean,
gaussian_codebook, haar_rotation, code_lut) follow Block-GTQ
(https://github.com/JIA-Lab-research/blockgtq, commit 3fe14e7), licensed under
the Apache License, Version 2.0; they are restated step for step because the
regenerated tables must equal the committed ones bit for bit. tie_order
restates the ordering of the Microsoft STL's std::sort (Apache License 2.0
WITH LLVM-exception).
"""
from __future__ import annotations

import math

import numpy as np

from .layout import BlockGTQParameters


def allocate_bits(scores, budget: int, min_bits: int = 1, max_bits: int = 8) -> np.ndarray:
    """Greedy: one more bit to argmax s*4^-b (FP32 scores, FP64 powers, first index on ties)."""
    s = np.asarray(scores, dtype=np.float32)
    w = np.full(len(s), min_bits, dtype=np.int64)
    remaining = int(budget) - int(w.sum())
    while remaining > 0:
        pri = s * np.power(4.0, -w.astype(np.float64))
        pri[w >= max_bits] = -1.0
        best = int(np.argmax(pri))
        if pri[best] <= 0:
            break
        w[best] += 1
        remaining -= 1
    return w


def tie_order(widths) -> np.ndarray:
    """torch.argsort(widths) (not stable) as it ordered the reference's committed tables.

    src/reference/mixed_layout.py:7-8 keeps torch's non-stable argsort; the
    goldens were written on Windows, where ATen sorts (key, index) pairs with
    the Microsoft STL's std::sort comparing keys only. That introsort
    insertion-sorts ranges of at most 32 elements (equal widths stay in pair
    order, as a stable sort) and splits larger ones around a median guess
    (median of three; Tukey's ninther above 40 elements) with a three-way
    partition whose swaps set the order of equal widths: at 33..64 pairs the
    order differs from a stable sort (fixtures mixed_d128, low_d128). Restated
    from that published algorithm (Microsoft STL, Apache License 2.0 WITH
    LLVM-exception); libbgtq's grouping (csrc/calibrate.cpp, TieOrderSort) is
    the same code.
    """
    key = [int(x) for x in np.asarray(widths, dtype=np.int64)]
    idx = list(range(len(key)))

    def lt(i, j):
        return key[i] < key[j]

    def swap(i, j):
        key[i], key[j] = key[j], key[i]
        idx[i], idx[j] = idx[j], idx[i]

    def med3(f, m, l):
        if lt(m, f):
            swap(m, f)
        if lt(l, m):
            swap(l, m)
            if lt(m, f):
                swap(m, f)

    def partition(first, last):
        mid = first + ((last - first) >> 1)
        f, l = first, last - 1
        if l - f > 40:  # Tukey's ninther
            step = (l - f + 1) >> 3
            two = step << 1
            med3(f, f + step, f + two)
            med3(mid - step, mid, mid + step)
            med3(l - two, l - step, l)
            med3(f + step, mid, l - step)
        else:
            med3(f, mid, l)
        pf, pl = mid, mid + 1
        while first < pf and not lt(pf - 1, pf) and not lt(pf, pf - 1):
            pf -= 1
        while pl < last and not lt(pl, pf) and not lt(pf, pl):
            pl += 1
        gf, gl = pl, pf
        while True:
            while gf < last:
                if lt(pf, gf):
                    pass
                elif lt(gf, pf):
                    break
                else:
                    if pl != gf:
                        swap(pl, gf)
                    pl += 1
                gf += 1
            while first < gl:
                gp = gl - 1
                if lt(gp, pf):
                    pass
                elif lt(pf, gp):
                    break
                else:
                    pf -= 1
                    if pf != gp:
                        swap(pf, gp)
                gl -= 1
            if gl == first and gf == last:
                return pf, pl
            if gl == first:  # no room below: rotate the pivot run upward
                if pl != gf:
                    swap(pf, pl)
                pl += 1
                swap(pf, gf)
                pf += 1
                gf += 1
            elif gf == last:  # no room above: rotate it downward
                gl -= 1
                pf -= 1
                if gl != pf:
                    swap(gl, pf)
                pl -= 1
                swap(pf, pl)
            else:
                gl -= 1
                swap(gf, gl)
                gf += 1

    def insertion(first, last):
        for mid in range(first + 1, last):
            k, ix, hole = key[mid], idx[mid], mid
            while hole > first and k < key[hole - 1]:
                key[hole], idx[hole] = key[hole - 1], idx[hole - 1]
                hole -= 1
            key[hole], idx[hole] = k, ix

    def sort(first, last, ideal):
        while True:
            # ideal <= 0 (the heap-sort fallback) cannot happen for widths 1..8:
            # each split removes every element equal to its pivot.
            if last - first <= 32 or ideal <= 0:
                insertion(first, last)
                return
            m0, m1 = partition(first, last)
            ideal = (ideal >> 1) + (ideal >> 2)
            if m0 - first < last - m1:
                sort(first, m0, ideal)
                first = m1
            else:
                sort(m1, last, ideal)
                last = m0

    sort(0, len(key), len(key))
    return np.asarray(idx, dtype=np.int64)


def grouping(widths) -> dict:
    """Pairs sorted by width in the committed tables' tie order (tie_order), (p, p + L) interleaved
    (src/reference/mixed_layout.py:5-18)."""
    order = tie_order(widths)
    L = len(order)
    head_perm = np.empty(2 * L, np.int64)
    head_perm[0::2], head_perm[1::2] = order, order + L
    sorted_w = np.asarray(widths)[order]
    bits, counts = np.unique(sorted_w, return_counts=True)
    offsets = np.concatenate([[0], np.cumsum(counts * 2)])
    group_of = np.repeat(np.arange(len(bits)), counts * 2)
    ns = int((np.asarray(widths) <= 4).sum()) * 2
    return dict(pair_order=order, head_perm=head_perm, group_bits=bits, group_offsets=offsets, group_of=group_of,
                nopack_start=ns, row_bytes=ns // 2 + 2 * L - ns)


def _cond_mean(sigma, a, b):
    """E[X | a < X < b] for X ~ N(0, sigma^2)."""
    from scipy.special import ndtr
    za = a / sigma if np.isfinite(a) else a
    zb = b / sigma if np.isfinite(b) else b
    if not np.isfinite(za):
        mass = ndtr(zb)
    elif not np.isfinite(zb):
        mass = ndtr(-za)
    else:
        mass = ndtr(zb) - ndtr(za)
    if mass < 1e-15:
        if np.isfinite(a) and not np.isfinite(b):
            return a + sigma
        if np.isfinite(b) and not np.isfinite(a):
            return b - sigma
        if np.isfinite(a) and np.isfinite(b):
            return (a + b) / 2.0
        return 0.0
    phi = lambda z: 0.0 if not np.isfinite(z) else math.exp(-0.5 * z * z) / math.sqrt(2 * math.pi)
    return sigma * (phi(za) - phi(zb)) / mass


def gaussian_codebook(bits: int, dim: int) -> np.ndarray:
    """MSE-optimal scalar codebook for one coordinate of a random unit vector in R^dim."""
    n = 1 << bits
    if bits == 1:
        c = math.sqrt(2.0 / (math.pi * dim))
        return np.array([-c, c], np.float32)
    if bits == 2:
        return (np.array([-1.51, -0.453, 0.453, 1.51]) / math.sqrt(dim)).astype(np.float32)
    from scipy.special import ndtri
    sigma = 1.0 / math.sqrt(dim)
    bounds = ndtri(np.linspace(0, 1, n + 1)[1:-1]) * sigma
    cents = np.zeros(n)

    def update(bd):
        cents[0] = _cond_mean(sigma, -np.inf, bd[0])
        for i in range(1, n - 1):
            cents[i] = _cond_mean(sigma, bd[i - 1], bd[i])
        cents[-1] = _cond_mean(sigma, bd[-1], np.inf)

    update(bounds)
    for _ in range(100):
        bounds = (cents[:-1] + cents[1:]) / 2.0
        update(bounds)
    return np.sort(cents).astype(np.float32)


def haar_rotation(dim: int, seed: int) -> np.ndarray:
    """Haar-distributed rotation: QR of a Gaussian matrix, sign-fixed, det +1."""
    g = np.random.default_rng(seed).standard_normal((dim, dim))
    q, r = np.linalg.qr(g)
    s = np.sign(np.diag(r))
    s[s == 0] = 1.0
    q = q * s[None, :]
    if np.linalg.slogdet(q)[0] < 0:
        q[:, 0] = -q[:, 0]
    return q.astype(np.float32)


def code_lut(pos_centroids, pos_boundaries, n_bins: int = 256):
    """Bin -> centroid index per distinct codebook, plus per-position bin offset and 1/width."""
    import torch
    cents = np.asarray(pos_centroids, np.float32)
    bounds = np.asarray(pos_boundaries, np.float32)
    d = cents.shape[0]
    offsets = np.zeros(d, np.float32)
    inv = np.zeros(d, np.float32)
    nvalid = []
    for j in range(d):
        nc = max(int((bounds[j] < 1e30).sum()) + 1, 2)
        nvalid.append(nc)
        lo, hi = float(cents[j, :nc].min()), float(cents[j, :nc].max())
        margin = (hi - lo) / max(nc - 1, 1) * 0.5
        offsets[j] = lo - margin
        inv[j] = 1.0 / (((hi + margin) - (lo - margin)) / n_bins)
    books, pos_cb = {}, np.zeros(d, np.int64)
    reps = []
    for j in range(d):
        key = (nvalid[j], tuple(cents[j, :nvalid[j]].tolist()))
        if key not in books:
            books[key] = len(reps)
            reps.append(j)
        pos_cb[j] = books[key]
    lut = np.zeros((len(reps), n_bins), np.uint8)
    for b, j in enumerate(reps):
        nc = nvalid[j]
        c = torch.from_numpy(cents[j, :nc].copy())
        lo, hi = c.min().item(), c.max().item()
        margin = (hi - lo) / max(nc - 1, 1) * 0.5
        width = ((hi + margin) - (lo - margin)) / n_bins
        centers = torch.linspace(lo - margin + width / 2, hi + margin - width / 2, n_bins, dtype=torch.float32)
        nb = int((bounds[j] < 1e30).sum())
        if nb > 0:
            idx = torch.searchsorted(torch.from_numpy(bounds[j, :nb].copy()), centers).clamp(max=nc - 1)
        else:
            idx = (centers > (c[0] + c[1]) / 2.0).long()
        lut[b] = idx.numpy().astype(np.uint8)
    return lut, pos_cb, offsets, inv


def make_parameters(widths, rotation_threshold: int = 2, row_bytes: int | None = None,
                    norm_stride: int | None = None) -> BlockGTQParameters:
    """Full table set for a per-pair width allocation (2*len(widths) dims)."""
    import torch
    widths = np.asarray(widths, np.int64)
    grp = grouping(widths)
    d = 2 * len(widths)
    bits = [int(b) for b in grp["group_bits"]]
    offs = grp["group_offsets"]
    rot = np.zeros((d, d), np.float32)
    maxc = max(1 << b for b in bits)
    cents = np.zeros((d, maxc), np.float32)
    bnds = np.full((d, maxc - 1), np.inf, np.float32)
    for g, bw in enumerate(bits):
        s, e = int(offs[g]), int(offs[g + 1])
        rot[s:e, s:e] = np.eye(e - s, dtype=np.float32) if bw < rotation_threshold else haar_rotation(e - s, 42 + bw)
        c = gaussian_codebook(bw, e - s)
        tc = torch.from_numpy(c)
        b = ((tc[:-1] + tc[1:]) / 2.0).numpy()  # FP32 midpoints
        cents[s:e, :len(c)] = c
        bnds[s:e, :len(b)] = b
    lut, pos_cb, off, inv = code_lut(cents, bnds)
    ng = len(bits)
    return BlockGTQParameters(
        dim=d, groups=ng, rowBytes=int(row_bytes or grp["row_bytes"]), normStride=int(norm_stride or ng),
        nibbleDims=grp["nopack_start"], maxCentroids=maxc, permutation=grp["head_perm"].astype(np.uint32),
        groupOf=grp["group_of"].astype(np.uint32), positionToCodebook=pos_cb.astype(np.uint32),
        codeLut=lut.reshape(-1), rotation=rot.reshape(-1), centroids=cents.reshape(-1), offsets=off,
        inverseScales=inv)


def geometric_scores(n_pairs: int, ratio: float = 0.9) -> np.ndarray:
    """Per-pair energy decaying geometrically (ratio**i)."""
    return (ratio ** np.arange(n_pairs)).astype(np.float32)


def layout_b(dim: int) -> BlockGTQParameters:
    """Widths in {4, 8}, half each (6.0 bits average): 4 x allocate_bits(0.9**i, 1.5*pairs, 1, 2)."""
    n = dim // 2
    return make_parameters(4 * allocate_bits(geometric_scores(n), (3 * n) // 2, 1, 2))


def layout_a(dim: int) -> BlockGTQParameters:
    """allocate_bits(0.9**i, 6*pairs, 4, 8): widths 4..8 at a 6.0 average."""
    n = dim // 2
    return make_parameters(allocate_bits(geometric_scores(n), 6 * n, 4, 8))


# ---- the library's table pipeline (bgtq_allocate_bits / bgtq_layout_build) ----

def native_allocate_bits(scores, budget: int, min_bits: int = 1, max_bits: int = 8) -> np.ndarray:
    """allocate_bits in libbgtq (same results as allocate_bits above)."""
    from ._lib import check, lib, ptr
    s = np.ascontiguousarray(scores, dtype=np.float32)
    w = np.zeros(len(s), np.int64)
    check(lib().bgtq_allocate_bits(ptr(s) if len(s) else None, len(s), int(budget), int(min_bits), int(max_bits),
                                   ptr(w) if len(s) else None))
    return w


def native_layout_groups(widths) -> list[tuple[int, int]]:
    """(bits, dims) of each group of a width allocation, ascending widths."""
    import ctypes
    from ._lib import check, lib, ptr
    w = np.ascontiguousarray(widths, dtype=np.int64)
    n = ctypes.c_int32(0)
    bits = np.zeros(8, np.int32)
    dims = np.zeros(8, np.int32)
    check(lib().bgtq_layout_groups(ptr(w), len(w), ctypes.byref(n), ptr(bits), ptr(dims)))
    return [(int(bits[k]), int(dims[k])) for k in range(n.value)]


def native_tables(widths, groups, row_bytes: int = 0, norm_stride: int = 0):
    """tables(p) blobs (integer u32, floating f32) built by libbgtq from a width
    allocation and, per group in ascending width, (centroids, rotation or None)."""
    import ctypes
    from . import _lib
    from ._lib import check, lib, ptr
    w = np.ascontiguousarray(widths, dtype=np.int64)
    keep = []
    arr = (_lib.GroupTables * max(1, len(groups)))()
    for k, (c, r) in enumerate(groups):
        c = np.ascontiguousarray(c, dtype=np.float32)
        r = None if r is None else np.ascontiguousarray(r, dtype=np.float32)
        keep += [c, r]
        arr[k] = _lib.GroupTables(c.ctypes.data, None if r is None else r.ctypes.data)
    ni, nf = ctypes.c_size_t(0), ctypes.c_size_t(0)
    check(lib().bgtq_layout_build(ptr(w), len(w), arr, len(groups), row_bytes, norm_stride, None, ctypes.byref(ni),
                                  None, ctypes.byref(nf)))
    integer = np.zeros(ni.value, np.uint32)
    floating = np.zeros(nf.value, np.float32)
    check(lib().bgtq_layout_build(ptr(w), len(w), arr, len(groups), row_bytes, norm_stride, ptr(integer),
                                  ctypes.byref(ni), ptr(floating), ctypes.byref(nf)))
    return integer, floating


def bake_qproj(params: BlockGTQParameters, weight, bias=None):
    """The query-projection rows of the query heads that use one KV head, with that head's
    permutation and rotation folded in (bgtq_bake_qproj; the optimisation of
    vendor/blockgtq/quantizer.py:1190-1244): weight [heads * dim, in_features], bias [heads * dim]
    or None, FP32. Returns (weight', bias'); queries from them go to the kernels with q_rotated."""
    from . import layout
    from ._lib import RangeError, check, lib, ptr
    ints, fl = layout.tables(params)
    w = np.ascontiguousarray(weight, dtype=np.float32)
    d = int(params.dim)
    if w.ndim != 2 or w.shape[0] % d:
        raise RangeError(f"weight rows must be a multiple of dim={d}")
    heads = w.shape[0] // d
    out_w = np.empty_like(w)
    b = out_b = None
    if bias is not None:
        b = np.ascontiguousarray(bias, dtype=np.float32).reshape(-1)
        if b.shape[0] != w.shape[0]:
            raise RangeError("bias length must equal the weight rows")
        out_b = np.empty_like(b)
    check(lib().bgtq_bake_qproj(ptr(ints), len(ints), ptr(fl), len(fl), heads, w.shape[1], ptr(w), ptr(b),
                                ptr(out_w), ptr(out_b)))
    return out_w, out_b
