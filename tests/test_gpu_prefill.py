"""Chunked prefill (model forward over a chunk of prompt rows) against the oracle.

A chunk of `rows` query rows at positions start .. start+rows-1 attends
causally to the sequence's history (src/model/decoder.ts:46-56 per chunk,
src/model/compressed-dot.wgsl:28). Outputs must match the oracle's causal
attention on the same effective K within |gpu - oracle| <= 1e-5 + 1e-4 |oracle|.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

ATOL, RTOL = 1e-5, 1e-4


def _olayout(oracle, p):
    return oracle.Layout(dim=p.dim, groups=p.groups, row_bytes=p.rowBytes, norm_stride=p.normStride,
                         nibble_dims=p.nibbleDims, max_centroids=p.maxCentroids, perm=p.permutation,
                         group_of=p.groupOf, pos_to_cb=p.positionToCodebook, code_lut=p.codeLut,
                         rotation=p.rotation, centroids=p.centroids, offsets=p.offsets, inv_scales=p.inverseScales)


def _check(out, ref, what):
    err = np.abs(out.astype(np.float64) - ref)
    lim = ATOL + RTOL * np.abs(ref)
    assert np.all(err <= lim), f"{what}: max err {err.max():.3e}, worst ratio {(err / lim).max():.2f}"


class Cache:
    """K (packed or FP16) and FP16 V for batch x KV heads x cap tokens on the device."""

    def __init__(self, device, *, params, batch, hkv, dim, cap, key_format="packed", seed=0, zero_k=False,
                 pad16=False):
        import torch
        import bgtq
        from bgtq import batched
        batched.bind_torch_stream(device)
        g = torch.Generator().manual_seed(seed)
        self.k = (torch.randn((batch, hkv, cap, dim), generator=g) * 0.8).half()
        if zero_k:
            self.k.zero_()
        self.v = torch.randn((batch, hkv, cap, dim), generator=g).half()
        self.params, self.dim, self.key_format = params, dim, key_format
        self.tabs = []
        kd = self.k.cuda()
        if key_format == "packed":
            self.tabs = [bgtq.Tables(device, p) for p in params]
            rb, ns = params[0].rowBytes, params[0].normStride
            pk_len, nm_len = cap * rb, cap * ns
            if pad16:  # 16-byte aligned head and sequence strides
                pk_len, nm_len = (pk_len + 15) // 16 * 16, (nm_len + 7) // 8 * 8
            self.packed = torch.zeros((batch, hkv, pk_len), dtype=torch.uint8, device="cuda")
            self.norms = torch.zeros((batch, hkv, nm_len), dtype=torch.int16, device="cuda")
            jobs = [dict(tables=self.tabs[h], src=kd[b, h], src_row_stride=dim, rows=cap, packed=self.packed[b, h],
                         norms=self.norms[b, h]) for b in range(batch) for h in range(hkv)]
            batched.encode(device, jobs, "f16")
            self.kw = dict(tables=self.tabs, packed=self.packed, packed_seq_stride=self.packed.stride(0),
                           packed_head_stride=self.packed.stride(1), norms=self.norms,
                           norms_seq_stride=self.norms.stride(0), norms_head_stride=self.norms.stride(1))
        else:
            self.kd = kd
            self.kw = dict(k_f16=kd, k_seq_stride=kd.stride(0), k_head_stride=kd.stride(1))
        self.vd = self.v.cuda()

    def keff(self, oracle, b, h, T):
        if self.key_format != "packed":
            return self.k[b, h, :T].float().numpy()
        p = self.params[h]
        pk = self.packed[b, h, :T * p.rowBytes].cpu().numpy().reshape(T, p.rowBytes)
        nm = self.norms[b, h, :T * p.normStride].cpu().numpy().view(np.float16).reshape(T, p.normStride)
        return oracle.reconstruct(_olayout(oracle, p), oracle.unpack(pk, self.dim, p.nibbleDims), nm.astype(np.float32))

    def prefill(self, device, q, starts, max_length, split_tokens=0):
        """q: torch [B, rows, Hq, dim] on the host; returns the output as numpy."""
        import torch
        from bgtq import batched
        B, rows, hq, dim = q.shape
        qd = q.cuda()
        out = torch.full((B, rows, hq, dim), float("nan"), dtype=torch.float32, device="cuda")
        sd = torch.tensor(starts, dtype=torch.int32).cuda()
        kw = dict(batch=B, rows=rows, q_heads=hq, kv_heads=self.vd.shape[1], dim=dim, q=qd, out=out, starts=sd,
                  max_length=max_length, v=self.vd, v_seq_stride=self.vd.stride(0),
                  v_head_stride=self.vd.stride(1), split_tokens=split_tokens, **self.kw)
        ws = torch.zeros(batched.prefill_workspace_bytes(batched.prefill_desc(**kw)), dtype=torch.uint8,
                         device="cuda")
        batched.prefill(device, batched.prefill_desc(workspace=ws, **kw))
        torch.cuda.synchronize()
        return out.cpu().numpy()

    def destroy(self):
        for t in self.tabs:
            t.destroy()


def _reference(oracle, cache, q, starts, b, h, G, rows_sel=None):
    rows = q.shape[1]
    rows_sel = np.arange(rows) if rows_sel is None else np.asarray(rows_sel)
    T = starts[b] + rows
    keff = cache.keff(oracle, b, h, T)
    qq = q[b, rows_sel, h * G:(h + 1) * G].reshape(-1, q.shape[-1]).numpy()
    pos = np.repeat(starts[b] + rows_sel, G).astype(np.uint32)
    _, _, ref = oracle.attention(qq, keff, cache.v[b, h, :T].float().numpy(), pos, True)
    return ref.reshape(len(rows_sel), G, -1)


def _run(device, oracle, *, params, batch, rows, hq, hkv, dim, starts, cap, key_format="packed", split_tokens=0,
         seed=0, pad16=False):
    import torch
    cache = Cache(device, params=params, batch=batch, hkv=hkv, dim=dim, cap=cap, key_format=key_format, seed=seed,
                  pad16=pad16)
    try:
        g = torch.Generator().manual_seed(seed + 1)
        q = torch.randn((batch, rows, hq, dim), generator=g)
        got = cache.prefill(device, q, starts, cap, split_tokens)
        G = hq // hkv
        for b in range(batch):
            for h in range(hkv):
                ref = _reference(oracle, cache, q, starts, b, h, G)
                _check(got[b, :, h * G:(h + 1) * G], ref.astype(np.float64), f"b{b} kv{h} start={starts[b]}")
        return got
    finally:
        cache.destroy()


@pytest.mark.parametrize("dim", [64, 128])
def test_layout_b_ragged_starts(device, oracle, dim):
    from bgtq import calibrate
    p = calibrate.layout_b(dim)
    print("prefill layout B", dim, flush=True)
    _run(device, oracle, params=[p, p], batch=3, rows=37, hq=14, hkv=2, dim=dim, starts=[0, 5, 463], cap=500)


@pytest.mark.parametrize("dim,split_tokens", [(64, 0), (128, 0), (64, 96)])
def test_layout_a_any_layout_build(device, oracle, dim, split_tokens):
    """Layout A (groups straddling the 32-dim K-steps, norm stride 3 or 5) with 16-byte aligned
    caches: the prefill kernel's per-position K build."""
    from bgtq import calibrate
    p = calibrate.layout_a(dim)
    print("prefill layout A", dim, split_tokens, flush=True)
    _run(device, oracle, params=[p, p], batch=3, rows=37, hq=14, hkv=2, dim=dim, starts=[0, 5, 463], cap=500,
         split_tokens=split_tokens, pad16=True)


def test_smollm2_heads_any_layout_build(device, oracle):
    """The reference's SmolLM2 calibration heads (odd 37-byte rows, nibble and byte codes mixed,
    up to six groups and books): the prefill kernel's per-position K build, 32-row chunk."""
    from bgtq import BlockGTQParameters
    from conftest import REF
    m, a = oracle.read_fixture(REF / "model" / "calibration.json")
    heads = [BlockGTQParameters.from_serialized(a[f"{n}_config"], a[f"{n}_table"]) for n in ("h0", "h56", "h22")]
    rb, ns = max(h.rowBytes for h in heads), max(h.normStride for h in heads)
    for h in heads:
        h.rowBytes, h.normStride = rb, ns
    print("prefill smollm2 heads", flush=True)
    _run(device, oracle, params=heads, batch=2, rows=32, hq=9, hkv=3, dim=64, starts=[0, 700], cap=732, pad16=True)


@pytest.mark.parametrize("heads,split_tokens", [(("h0", "h2", "h7"), 0), (("h3", "h6", "h3"), 0),
                                                (("h0", "h2", "h7"), 96)])
def test_scales_past_the_history_are_ignored(device, oracle, heads, split_tokens):
    """Heads of odd norm stride (3, 5) with chunks ending at an odd token count of their last block:
    the scale DMA of that block is rounded up to 4 bytes and also brings in the first scale of the
    token after the history. Filling every scale slot past the history with 65504 (0x7bff) and
    with +inf (0x7c00) must leave the output bit-identical and finite."""
    import torch
    from bgtq import BlockGTQParameters
    from conftest import REF
    m, a = oracle.read_fixture(REF / "model" / "calibration.json")
    params = [BlockGTQParameters.from_serialized(a[f"{n}_config"], a[f"{n}_table"]) for n in heads]
    rb, ns = max(h.rowBytes for h in params), max(h.normStride for h in params)
    assert ns % 2 == 1
    for h in params:
        h.rowBytes, h.normStride = rb, ns
    starts, rows, cap = [0, 700], 33, 800  # histories of 33 and 733 tokens: 1 and 29 in the last block
    print("prefill scales past the history", heads, split_tokens, flush=True)
    cache = Cache(device, params=params, batch=2, hkv=3, dim=64, cap=cap, seed=4, pad16=True)
    try:
        q = torch.randn((2, rows, 9, 64), generator=torch.Generator().manual_seed(12))
        clean = cache.prefill(device, q, starts, cap, split_tokens)
        G = 3
        for b in range(2):
            for h in range(3):
                ref = _reference(oracle, cache, q, starts, b, h, G)
                _check(clean[b, :, h * G:(h + 1) * G], ref.astype(np.float64), f"b{b} kv{h}")
        for fill in (0x7bff, 0x7c00):
            for b in range(2):
                cache.norms[b, :, (starts[b] + rows) * ns:] = fill
            got = cache.prefill(device, q, starts, cap, split_tokens)
            assert np.isfinite(got).all(), f"non-finite output with scales {fill:#x} past the history"
            assert np.array_equal(got, clean), f"output changed with scales {fill:#x} past the history"
    finally:
        cache.destroy()


def test_widths_1_to_6_d128_any_layout_build(device, oracle):
    """d=128, widths 1..6: 79-byte rows, 98 nibble positions, norm stride 6."""
    from bgtq import calibrate
    p = calibrate.make_parameters(calibrate.allocate_bits(calibrate.geometric_scores(64), 206, 1, 8))
    print("prefill widths 1..6 d=128", flush=True)
    _run(device, oracle, params=[p, p], batch=2, rows=37, hq=14, hkv=2, dim=128, starts=[0, 463], cap=500,
         pad16=True)


def test_fp16_keys(device, oracle):
    print("prefill fp16 K", flush=True)
    _run(device, oracle, params=None, batch=2, rows=45, hq=14, hkv=2, dim=64, starts=[100, 0], cap=300,
         key_format="fp16")
    _run(device, oracle, params=None, batch=1, rows=20, hq=6, hkv=2, dim=128, starts=[77], cap=100,
         key_format="fp16")


@pytest.mark.parametrize("split_tokens", [32, 96, 256])
def test_forced_splits_merge(device, oracle, split_tokens):
    """Many token splits per tile: the last workgroup of each tile merges up to 64 partials."""
    from bgtq import calibrate
    p = calibrate.layout_b(64)
    print("prefill split_tokens", split_tokens, flush=True)
    _run(device, oracle, params=[p], batch=2, rows=70, hq=7, hkv=1, dim=64, starts=[1900, 0], cap=2000,
         split_tokens=split_tokens)


@pytest.mark.parametrize("starts,split_tokens", [([1000, 300], 96), ([1900, 0], 0), ([1900, 0, 700], 256)])
def test_rowwise_units_of_different_split_counts(device, oracle, starts, split_tokens):
    """A row-wise chunk (32 rows) of a batch whose later sequences have shorter histories: the units
    of one launch use different split counts, and each keeps its partials apart from the others'."""
    from bgtq import calibrate
    p = calibrate.layout_b(64)
    print("prefill row-wise split counts", starts, split_tokens, flush=True)
    _run(device, oracle, params=[p], batch=len(starts), rows=32, hq=7, hkv=1, dim=64, starts=starts, cap=2000,
         split_tokens=split_tokens)


def test_single_chunk_prompt(device, oracle):
    """A 1024-row prompt in one chunk: 28 query tiles per KV head, causal from token 0."""
    from bgtq import calibrate
    p = calibrate.layout_b(64)
    print("prefill 1024-row chunk", flush=True)
    _run(device, oracle, params=[p, p], batch=1, rows=1024, hq=14, hkv=2, dim=64, starts=[0], cap=1024)


def test_chunks_equal_one_chunk(device, oracle):
    """Chunks of 32 rows (the reference's chunk cap) give the one-chunk result, query for query."""
    import torch
    from bgtq import calibrate
    p = calibrate.layout_b(64)
    cache = Cache(device, params=[p, p], batch=1, hkv=2, dim=64, cap=256, seed=3)
    try:
        q = torch.randn((1, 256, 14, 64), generator=torch.Generator().manual_seed(9))
        whole = cache.prefill(device, q, [0], 256)
        parts = np.concatenate([cache.prefill(device, q[:, r:r + 32].contiguous(), [r], 256)
                                for r in range(0, 256, 32)], axis=1)
        ref = np.concatenate([_reference(oracle, cache, q, [0], 0, h, 7) for h in range(2)], axis=1)
        _check(whole[0], ref.astype(np.float64), "one chunk")
        _check(parts[0], ref.astype(np.float64), "chunks of 32")
    finally:
        cache.destroy()


def test_full_prompt_4096_sampled_rows(device, oracle):
    """The 4096-token prompt of a Qwen2.5-0.5B layer (14 q / 2 KV heads, d=64) in one chunk, checked on
    sampled rows against the oracle and on every row for finiteness."""
    import torch
    from bgtq import calibrate
    p = calibrate.layout_b(64)
    print("prefill 4096 rows", flush=True)
    cache = Cache(device, params=[p, p], batch=1, hkv=2, dim=64, cap=4096, seed=5)
    try:
        q = torch.randn((1, 4096, 14, 64), generator=torch.Generator().manual_seed(11))
        got = cache.prefill(device, q, [0], 4096)
        assert np.isfinite(got).all()
        sel = [0, 1, 31, 32, 255, 256, 1000, 2047, 2048, 3333, 4094, 4095]
        for h in range(2):
            ref = _reference(oracle, cache, q, [0], 0, h, 7, sel)
            _check(got[0, sel, h * 7:(h + 1) * 7], ref.astype(np.float64), f"kv{h} sampled rows")
    finally:
        cache.destroy()


def test_zero_queries_give_prefix_means(device, oracle):
    """Zero queries make every softmax uniform: row r returns the mean of V[0 .. start + r]."""
    import torch
    from bgtq import calibrate
    p = calibrate.layout_b(64)
    cache = Cache(device, params=[p], batch=1, hkv=1, dim=64, cap=700, seed=2)
    try:
        q = torch.zeros((1, 100, 3, 64))
        got = cache.prefill(device, q, [600], 700, split_tokens=128)
        v = cache.v[0, 0].double().numpy()
        means = np.cumsum(v, axis=0) / np.arange(1, 701)[:, None]
        ref = np.repeat(means[600:700][:, None, :], 3, axis=1)
        _check(got[0], ref, "prefix means")
    finally:
        cache.destroy()


def test_rejections(device):
    import torch
    import bgtq
    from bgtq import batched, calibrate
    # norm stride 9: beyond what the prefill kernel holds (8)
    p = calibrate.make_parameters(calibrate.allocate_bits(calibrate.geometric_scores(32), 6 * 32, 4, 8), norm_stride=9)
    t = bgtq.Tables(device, p)
    try:
        z = torch.zeros(16, device="cuda")
        kw = dict(batch=1, rows=4, q_heads=2, kv_heads=1, dim=64, q=z, out=z, starts=z, max_length=64, v=z,
                  v_seq_stride=0, v_head_stride=0, tables=[t], packed=z, norms=z)
        with pytest.raises(bgtq.RangeError):
            batched.prefill_workspace_bytes(batched.prefill_desc(**{**kw, "rows": 65}))
        with pytest.raises(bgtq.UnsupportedError):
            batched.prefill_workspace_bytes(batched.prefill_desc(**{**kw, "dim": 96}))
        ws = torch.zeros(1 << 20, dtype=torch.uint8, device="cuda")
        with pytest.raises(bgtq.UnsupportedError):
            batched.prefill(device, batched.prefill_desc(workspace=ws, **kw))
    finally:
        t.destroy()


def test_workspace_shared_across_paths(device, oracle):
    """One workspace for a tiled chunk (64 rows), then row-wise chunks (32, 7 rows) of other geometry:
    the split counters at the workspace's start stay zero after every call and each output matches
    the oracle. Starts past max_length - rows clamp to it on both paths (the chunk then ends at
    max_length)."""
    import torch
    from bgtq import batched, calibrate
    p = calibrate.layout_b(64)
    cache = Cache(device, params=[p, p], batch=2, hkv=2, dim=64, cap=700)
    try:
        ws = torch.zeros(32 << 20, dtype=torch.uint8, device="cuda")
        counter_words = 65536  # BGTQ_PREFILL_COUNTER_BYTES / 4
        for rows, hq, starts in ((64, 14, [300, 611]), (32, 14, [0, 668]), (7, 6, [693, 250]),
                                 (64, 14, [690, 5]), (32, 14, [699, 40]), (5, 6, [1000, 695])):
            g = torch.Generator().manual_seed(rows)
            q = torch.randn((2, rows, hq, 64), generator=g)
            out = torch.full((2, rows, hq, 64), float("nan"), device="cuda")
            kw = dict(batch=2, rows=rows, q_heads=hq, kv_heads=2, dim=64, q=q.cuda(), out=out,
                      starts=torch.tensor(starts, dtype=torch.int32).cuda(), max_length=700, v=cache.vd,
                      v_seq_stride=cache.vd.stride(0), v_head_stride=cache.vd.stride(1), **cache.kw)
            assert batched.prefill_workspace_bytes(batched.prefill_desc(**kw)) <= ws.numel()
            print("shared workspace", rows, hq, starts, flush=True)
            batched.prefill(device, batched.prefill_desc(workspace=ws, **kw))
            torch.cuda.synchronize()
            assert not ws[:4 * counter_words].any(), "split counters left nonzero"
            got = out.cpu().numpy()
            G = hq // 2
            eff = [min(s, 700 - rows) for s in starts]
            for b in range(2):
                for h in range(2):
                    ref = _reference(oracle, cache, q, eff, b, h, G)
                    _check(got[b, :, h * G:(h + 1) * G], ref.astype(np.float64), f"rows {rows} b{b} kv{h}")
    finally:
        cache.destroy()
