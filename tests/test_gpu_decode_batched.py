"""Batched decode (model geometry) against the oracle: GQA, ragged lengths, splits, both key formats.

The batched entry point serves the model dispatch sites (src/model/decoder.ts:46-56:
encode_k, compressed_dot, softmax, weighted) for B sequences x KV heads.
Outputs must match the oracle's attention on the same effective K within
|gpu - oracle| <= 1e-5 + 1e-4 |oracle|.
"""
import numpy as np
import pytest

from conftest import REF

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


def _run(device, oracle, *, params, batch, hq, hkv, dim, lengths, cap, key_format="packed", splits=0, seed=0,
         zero_q=False, pad16=False):
    import torch
    import bgtq
    from bgtq import batched
    batched.bind_torch_stream(device)
    g = torch.Generator().manual_seed(seed)
    k = (torch.randn((batch, hkv, cap, dim), generator=g) * 0.8).half()
    v = torch.randn((batch, hkv, cap, dim), generator=g).half()
    q = torch.randn((batch, hq, dim), generator=g)
    if zero_q:
        q.zero_()
    lengths_t = torch.tensor(lengths, dtype=torch.int32)
    out = torch.empty((batch, hq, dim), dtype=torch.float32, device="cuda")
    kw = {}
    tabs = []
    if key_format == "packed":
        tabs = [bgtq.Tables(device, p) for p in params]
        rb, ns = params[0].rowBytes, params[0].normStride
        pk_len, nm_len = cap * rb + 64, cap * ns + 32
        if pad16:  # 16-byte aligned head and sequence strides
            pk_len, nm_len = (pk_len + 15) // 16 * 16, (nm_len + 7) // 8 * 8
        packed = torch.zeros((batch, hkv, pk_len), dtype=torch.uint8, device="cuda")
        norms = torch.zeros((batch, hkv, nm_len), dtype=torch.int16, device="cuda")
        kd = k.cuda()
        jobs = [dict(tables=tabs[h], src=kd[b, h], src_row_stride=dim, rows=cap, packed=packed[b, h],
                     norms=norms[b, h]) for b in range(batch) for h in range(hkv)]
        batched.encode(device, jobs, "f16")
        kw = dict(tables=tabs, packed=packed, packed_seq_stride=packed.stride(0), packed_head_stride=packed.stride(1),
                  norms=norms, norms_seq_stride=norms.stride(0), norms_head_stride=norms.stride(1))
    else:
        kd = k.cuda()
        kw = dict(k_f16=kd, k_seq_stride=kd.stride(0), k_head_stride=kd.stride(1))
    vd, qd, ld = v.cuda(), q.cuda(), lengths_t.cuda()
    desc = batched.decode_desc(batch=batch, q_heads=hq, kv_heads=hkv, dim=dim, q=qd, out=out, lengths=ld,
                               max_length=max(lengths), v=vd, v_seq_stride=vd.stride(0), v_head_stride=vd.stride(1),
                               splits=splits, **kw)
    ws = torch.zeros(batched.workspace_bytes(desc), dtype=torch.uint8, device="cuda")
    desc = batched.decode_desc(batch=batch, q_heads=hq, kv_heads=hkv, dim=dim, q=qd, out=out, lengths=ld,
                               max_length=max(lengths), v=vd, v_seq_stride=vd.stride(0), v_head_stride=vd.stride(1),
                               splits=splits, workspace=ws, **kw)
    batched.decode(device, desc)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    G = hq // hkv
    refs = {}
    for b in range(batch):
        T = lengths[b]
        for h in range(hkv):
            if key_format == "packed":
                p = params[h]
                pk = packed[b, h, :T * p.rowBytes].cpu().numpy().reshape(T, p.rowBytes)
                nm = norms[b, h, :T * p.normStride].cpu().numpy().view(np.float16).reshape(T, p.normStride)
                keff = oracle.reconstruct(_olayout(oracle, p), oracle.unpack(pk, dim, p.nibbleDims),
                                          nm.astype(np.float32))
            else:
                keff = k[b, h, :T].float().numpy()
            qq = q[b, h * G:(h + 1) * G].numpy()
            _, _, ref = oracle.attention(qq, keff, v[b, h, :T].float().numpy(), np.full(G, T - 1), False)
            refs[(b, h)] = ref
            _check(got[b, h * G:(h + 1) * G], ref.astype(np.float64), f"b{b} kv{h} T={T}")
    for t in tabs:
        t.destroy()
    return got, v, lengths


@pytest.mark.parametrize("dim", [64, 128])
def test_layout_b_gqa_ragged(device, oracle, dim):
    from bgtq import calibrate
    p = calibrate.layout_b(dim)
    print("layout B", dim, flush=True)
    _run(device, oracle, params=[p, p], batch=3, hq=14, hkv=2, dim=dim, lengths=[1, 77, 1000], cap=1000)


@pytest.mark.parametrize("dim", [64, 128])
def test_fp16_keys_baseline(device, oracle, dim):
    print("fp16 K", dim, flush=True)
    _run(device, oracle, params=None, batch=2, hq=14, hkv=2, dim=dim, lengths=[513, 130], cap=600,
         key_format="fp16")


@pytest.mark.parametrize("splits", [1, 3, 7, 12])
def test_forced_splits(device, oracle, splits):
    from bgtq import calibrate
    p = calibrate.layout_b(64)
    print("splits", splits, flush=True)
    _run(device, oracle, params=[p], batch=2, hq=3, hkv=1, dim=64, lengths=[2000, 1500], cap=2000, splits=splits)


@pytest.mark.parametrize("splits", [30, 47])
def test_forced_splits_long(device, oracle, splits):
    """Split merges of every size class: one load round up to 40 splits, two phases beyond."""
    from bgtq import calibrate
    p = calibrate.layout_b(64)
    print("splits", splits, flush=True)
    _run(device, oracle, params=[p], batch=2, hq=7, hkv=1, dim=64, lengths=[6000, 5100], cap=6000, splits=splits)


def test_non_fast_layouts_use_general_kernel(device, oracle):
    """Layouts whose K-steps mix groups (a real SmolLM2 head; layout A) run the general kernel."""
    from bgtq import BlockGTQParameters, calibrate
    m, a = oracle.read_fixture(REF / "model" / "calibration.json")
    heads = [BlockGTQParameters.from_serialized(a[f"h{i}_config"], a[f"h{i}_table"]) for i in (3, 4, 5)]
    rb = max(h.rowBytes for h in heads)
    ns = max(h.normStride for h in heads)
    for h in heads:  # one cache stride for all heads of the layer (src/model/decoder.ts:21 keeps one per head)
        h.rowBytes, h.normStride = rb, ns
    print("smollm2 heads", flush=True)
    _run(device, oracle, params=heads, batch=2, hq=9, hkv=3, dim=64, lengths=[300, 41], cap=300)
    pa = calibrate.layout_a(64)
    print("layout A", flush=True)
    _run(device, oracle, params=[pa, pa], batch=1, hq=14, hkv=2, dim=64, lengths=[700], cap=700)


@pytest.mark.parametrize("dim,splits", [(64, 0), (128, 0), (64, 5), (128, 3)])
def test_layout_a_fused(device, oracle, dim, splits):
    """Layout A (widths 4..8: K-steps spanning two groups; at d=128 nibble and byte codes in one
    K-step and a norm stride of 5) with 16-byte aligned caches: the fused kernel's per-position
    code lookup, ragged GQA batch."""
    from bgtq import calibrate
    p = calibrate.layout_a(dim)
    print("layout A fused", dim, splits, flush=True)
    _run(device, oracle, params=[p, p], batch=3, hq=14, hkv=2, dim=dim, lengths=[1, 77, 2049], cap=2049,
         splits=splits, pad16=True)


@pytest.mark.parametrize("dim,G", [(64, 1), (64, 4), (64, 5), (64, 8), (64, 9), (64, 16), (128, 3), (128, 8),
                                   (128, 12)])
def test_any_layout_group_packing(device, oracle, dim, G):
    """The fused per-position kernel packs four (G <= 4) or two (G <= 8) group slots into one
    matrix-core product and sums them across lanes; G > 8 runs one slot per product. Every
    packing width against the oracle, on layout A (two groups per K-step) and the real heads."""
    from bgtq import calibrate
    p = calibrate.layout_a(dim)
    print("group packing", dim, G, flush=True)
    _run(device, oracle, params=[p, p], batch=2, hq=2 * G, hkv=2, dim=dim, lengths=[300, 1031], cap=1031,
         pad16=True, seed=G)
    if dim == 64:
        heads = _smollm2_heads(oracle, ["h0", "h1", "h22"])
        _run(device, oracle, params=heads, batch=1, hq=3 * G, hkv=3, dim=dim, lengths=[517], cap=517, pad16=True,
             seed=G + 1)


def _smollm2_heads(oracle, names):
    """Reference calibration heads of one layer: one cache row stride and norm stride for all
    (src/model/decoder.ts:21 keeps one per head)."""
    from bgtq import BlockGTQParameters
    m, a = oracle.read_fixture(REF / "model" / "calibration.json")
    heads = [BlockGTQParameters.from_serialized(a[f"{n}_config"], a[f"{n}_table"]) for n in names]
    rb = max(h.rowBytes for h in heads)
    ns = max(h.normStride for h in heads)
    for h in heads:
        h.rowBytes, h.normStride = rb, ns
    return heads


@pytest.mark.parametrize("names,splits", [(("h3", "h56", "h26"), 0), (("h0", "h1", "h22"), 0),
                                          (("h0", "h1", "h22"), 4)])
def test_smollm2_heads_fused(device, oracle, names, splits):
    """Real SmolLM2 calibration heads (K-steps spanning up to four groups, nibble and byte codes in
    one lane's eight positions, 3-6 books, rows of 44 or of an odd 37 bytes, norm strides 4 and 6)
    with 16-byte aligned caches: the fused kernel's per-position code lookup."""
    heads = _smollm2_heads(oracle, names)
    print("smollm2 heads fused", names, splits, flush=True)
    _run(device, oracle, params=heads, batch=2, hq=9, hkv=3, dim=64, lengths=[1000, 77], cap=1000, splits=splits,
         pad16=True)


def test_smollm2_every_layer_fused(device, oracle):
    """All 90 SmolLM2 calibration heads (30 layers x 3 KV heads) through the fused decode."""
    for layer in range(30):
        heads = _smollm2_heads(oracle, [f"h{3 * layer + h}" for h in range(3)])
        print("smollm2 layer", layer, flush=True)
        _run(device, oracle, params=heads, batch=1, hq=9, hkv=3, dim=64, lengths=[150], cap=150, pad16=True,
             seed=layer)


def _widths_1_to_6_d128():
    """d=128, widths 1..6 in six groups: 98 nibble positions (a lane's 8 codes mix nibbles and
    bytes), 79-byte rows (not word aligned), norm stride 6, up to three groups per 32 positions."""
    from bgtq import calibrate
    return calibrate.make_parameters(calibrate.allocate_bits(calibrate.geometric_scores(64), 206, 1, 8))


def test_widths_1_to_6_d128_fused(device, oracle):
    p = _widths_1_to_6_d128()
    assert (p.dim, p.nibbleDims, p.rowBytes, p.normStride) == (128, 98, 79, 6)
    print("widths 1..6 d=128", flush=True)
    _run(device, oracle, params=[p, p], batch=2, hq=14, hkv=2, dim=128, lengths=[77, 1000], cap=1000, pad16=True)


def test_full_context_closed_form(device, oracle):
    """32768-token context: zero q gives the mean of V exactly enough (uniform softmax)."""
    from bgtq import calibrate
    p = calibrate.layout_b(64)
    print("32k zero-q", flush=True)
    got, v, lengths = _run(device, oracle, params=[p, p], batch=2, hq=14, hkv=2, dim=64, lengths=[32768, 32768],
                           cap=32768, zero_q=True)
    for b in range(2):
        for h in range(2):
            mean = v[b, h].float().numpy().astype(np.float64).mean(0)
            _check(got[b, h * 7:(h + 1) * 7], np.broadcast_to(mean, (7, 64)), "mean of V")


def test_full_context_vs_oracle(device, oracle):
    from bgtq import calibrate
    p = calibrate.layout_b(64)
    print("32k random", flush=True)
    _run(device, oracle, params=[p, p], batch=1, hq=14, hkv=2, dim=64, lengths=[32768], cap=32768, seed=5)


def test_optimized_attention_fp16_values_mfma(device, oracle):
    """OptimizedAttention over layout-B packed K and FP16 V (the matrix-core path), inspect() included."""
    import bgtq
    from bgtq import calibrate
    p = calibrate.layout_b(128)
    rng = np.random.default_rng(9)
    T = 4096
    k = rng.standard_normal((T, 128)).astype(np.float16)
    v = rng.standard_normal((T, 128)).astype(np.float16).astype(np.float32)
    q = rng.standard_normal((3, 128)).astype(np.float32)
    keys = bgtq.PackedKeys.create(device, p, T)
    values = bgtq.Values(device, 128, T, dtype="f16")
    att = bgtq.OptimizedAttention.create(device, keys, values, 3)
    try:
        keys.append(k.view(np.uint16))
        values.append(v)
        packed, norms = keys.read()
        keff = oracle.reconstruct(_olayout(oracle, p), oracle.unpack(packed.reshape(T, -1), 128, p.nibbleDims),
                                  norms.view(np.float16).reshape(T, -1).astype(np.float32))
        for causal in (False, True):
            pos = np.array([0, 2047, 4095])
            out = att.attend(q, pos, causal)
            ins = att.inspect()
            rl, rp, ro = oracle.attention(q, keff, v, pos, causal)
            _check(out, ro.astype(np.float64), f"output causal={causal}")
            fin = np.isfinite(rl)
            assert np.array_equal(np.isneginf(ins["logits"]), np.isneginf(rl))
            np.testing.assert_allclose(ins["logits"][fin], rl[fin], atol=1e-4, rtol=2e-5)
            np.testing.assert_allclose(ins["probabilities"], rp, atol=1e-5, rtol=1e-4)
            if causal:
                np.testing.assert_array_equal(out[0], v[0])
    finally:
        att.destroy()
        values.destroy()
        keys.destroy()


def test_graph_replays_match_eager(device, oracle):
    """The decode captured in a HIP graph: every replay, with eager work between
    replays, equals the eager result (the split counters reset in-kernel, no
    memset nodes)."""
    import torch
    import bgtq
    from bgtq import batched, calibrate
    p = calibrate.layout_b(64)
    batch, hq, hkv, dim, T = 2, 14, 2, 64, 3000
    g = torch.Generator().manual_seed(21)
    k = torch.randn((batch, hkv, T, dim), generator=g).half().cuda()
    v = torch.randn((batch, hkv, T, dim), generator=g).half().cuda()
    q = torch.randn((batch, hq, dim), generator=g).cuda()
    tabs = [bgtq.Tables(device, p) for _ in range(hkv)]
    packed = torch.zeros((batch, hkv, T * p.rowBytes + 64), dtype=torch.uint8, device="cuda")
    norms = torch.zeros((batch, hkv, T * p.normStride + 32), dtype=torch.int16, device="cuda")
    batched.bind_torch_stream(device)
    batched.encode(device, [dict(tables=tabs[h], src=k[b, h], src_row_stride=dim, rows=T, packed=packed[b, h],
                                 norms=norms[b, h]) for b in range(batch) for h in range(hkv)], "f16")
    out = torch.empty((batch, hq, dim), device="cuda")
    lengths = torch.tensor([T, T - 123], dtype=torch.int32, device="cuda")
    args = dict(batch=batch, q_heads=hq, kv_heads=hkv, dim=dim, q=q, out=out, lengths=lengths, max_length=T, v=v,
                v_seq_stride=v.stride(0), v_head_stride=v.stride(1), tables=tabs, packed=packed,
                packed_seq_stride=packed.stride(0), packed_head_stride=packed.stride(1), norms=norms,
                norms_seq_stride=norms.stride(0), norms_head_stride=norms.stride(1), splits=5)
    ws = torch.zeros(batched.workspace_bytes(batched.decode_desc(**args)), dtype=torch.uint8, device="cuda")
    desc = batched.decode_desc(workspace=ws, **args)
    batched.decode(device, desc)
    torch.cuda.synchronize()
    eager = out.clone()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        batched.bind_torch_stream(device)
        batched.decode(device, desc)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        batched.bind_torch_stream(device)
        batched.decode(device, desc)
    batched.bind_torch_stream(device)
    for rep in range(4):
        out.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {rep} differs from the eager result"
        batched.decode(device, desc)  # eager work between replays
        torch.cuda.synchronize()
        assert torch.equal(out, eager)
    for t in tabs:
        t.destroy()


def test_batch_beyond_grid_refused(device):
    """The fused kernel's grid carries the sequence in its third dimension (at most 65535): a larger batch
    is refused before any launch."""
    import torch
    import bgtq
    from bgtq import batched
    z = torch.zeros(16, device="cuda")
    args = dict(batch=65536, q_heads=2, kv_heads=1, dim=64, q=z, out=z, lengths=z, max_length=32, v=z, v_dtype="f16",
                v_seq_stride=0, v_head_stride=0, k_f16=z, k_seq_stride=0, k_head_stride=0, splits=1)
    with pytest.raises(bgtq.UnsupportedError, match="65535 sequences"):
        batched.workspace_bytes(batched.decode_desc(**args))
