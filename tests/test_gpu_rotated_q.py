"""Queries from a query projection baked with bgtq_bake_qproj (vendor/blockgtq/quantizer.py:1160-1244:
the KV head's permutation and rotation folded into q_proj) passed with q_rotated = 1: the decode
(fused structured and per-position kernels, the general kernel, the decode-step append) and the
chunked prefill give the oracle's attention of the unbaked queries, within
|gpu - oracle| <= 1e-5 + 1e-4 |oracle|, as the same launches with the unbaked queries do."""
import numpy as np
import pytest

from conftest import REF

pytestmark = pytest.mark.gpu

ATOL, RTOL = 1e-5, 1e-4
F = 48  # projection input width


def _olayout(oracle, p):
    return oracle.Layout(dim=p.dim, groups=p.groups, row_bytes=p.rowBytes, norm_stride=p.normStride,
                         nibble_dims=p.nibbleDims, max_centroids=p.maxCentroids, perm=p.permutation,
                         group_of=p.groupOf, pos_to_cb=p.positionToCodebook, code_lut=p.codeLut,
                         rotation=p.rotation, centroids=p.centroids, offsets=p.offsets, inv_scales=p.inverseScales)


def _check(out, ref, what):
    err = np.abs(np.asarray(out, np.float64) - ref)
    lim = ATOL + RTOL * np.abs(ref)
    assert np.all(err <= lim), f"{what}: max err {err.max():.3e}, worst ratio {(err / lim).max():.2f}"


def _smollm2(oracle, names):
    from bgtq import BlockGTQParameters
    m, a = oracle.read_fixture(REF / "model" / "calibration.json")
    heads = [BlockGTQParameters.from_serialized(a[f"{n}_config"], a[f"{n}_table"]) for n in names]
    rb, ns = max(h.rowBytes for h in heads), max(h.normStride for h in heads)
    for h in heads:
        h.rowBytes, h.normStride = rb, ns
    return heads


def _params(oracle, kind):
    from bgtq import calibrate
    if kind == "B64":
        return [calibrate.layout_b(64)] * 2, 7
    if kind == "B128":
        return [calibrate.layout_b(128)] * 2, 7
    return _smollm2(oracle, ("h3", "h56", "h26")), 3


def _queries(params, lead, G, seed):
    """q = W x + b per KV head's G query heads and the same from the baked W', b': [*lead, Hq, d]."""
    from bgtq import calibrate
    rng = np.random.default_rng(seed)
    d = params[0].dim
    x = rng.standard_normal((*lead, F))
    q, qb = [], []
    for p in params:
        W = (rng.standard_normal((G * d, F)) / np.sqrt(F)).astype(np.float32)
        b = (rng.standard_normal(G * d) * 0.1).astype(np.float32)
        Wb, bb = calibrate.bake_qproj(p, W, b)
        q.append((x @ W.T.astype(np.float64) + b).reshape(*lead, G, d))
        qb.append((x @ Wb.T.astype(np.float64) + bb).reshape(*lead, G, d))
    return np.concatenate(q, axis=-2).astype(np.float32), np.concatenate(qb, axis=-2).astype(np.float32)


class Cache:
    def __init__(self, device, params, B, T, seed=0):
        import torch
        import bgtq
        from bgtq import batched
        batched.bind_torch_stream(device)
        g = torch.Generator().manual_seed(seed)
        hkv, d = len(params), params[0].dim
        self.params, self.T = params, T
        self.k = (torch.randn((B, hkv, T, d), generator=g) * 0.8).half()
        self.v = torch.randn((B, hkv, T, d), generator=g).half()
        self.tabs = [bgtq.Tables(device, p) for p in params]
        rb, ns = params[0].rowBytes, params[0].normStride
        self.packed = torch.zeros((B, hkv, (T * rb + 64 + 15) // 16 * 16), dtype=torch.uint8, device="cuda")
        self.norms = torch.zeros((B, hkv, (T * ns + 32 + 7) // 8 * 8), dtype=torch.int16, device="cuda")
        kd = self.k.cuda()
        batched.encode(device, [dict(tables=self.tabs[h], src=kd[b, h], src_row_stride=d, rows=T,
                                     packed=self.packed[b, h], norms=self.norms[b, h])
                                for b in range(B) for h in range(hkv)], "f16")
        self.vd = self.v.cuda()
        self.kw = dict(tables=self.tabs, packed=self.packed, packed_seq_stride=self.packed.stride(0),
                       packed_head_stride=self.packed.stride(1), norms=self.norms,
                       norms_seq_stride=self.norms.stride(0), norms_head_stride=self.norms.stride(1))

    def keff(self, oracle, b, h, T):
        p = self.params[h]
        pk = self.packed[b, h, :T * p.rowBytes].cpu().numpy().reshape(T, p.rowBytes)
        nm = self.norms[b, h, :T * p.normStride].cpu().numpy().view(np.float16).reshape(T, p.normStride)
        return oracle.reconstruct(_olayout(oracle, p), oracle.unpack(pk, p.dim, p.nibbleDims), nm.astype(np.float32))

    def destroy(self):
        for t in self.tabs:
            t.destroy()


@pytest.mark.parametrize("kind,v_dtype", [("B64", "f16"), ("B128", "f16"), ("S", "f16"), ("B64", "f32")])
def test_decode_with_baked_queries(device, oracle, kind, v_dtype):
    """Fused structured (layout B) and per-position (SmolLM2 heads) kernels, and the general
    kernel (FP32 V), with forced splits on the ragged batch."""
    import torch
    from bgtq import batched
    params, G = _params(oracle, kind)
    B, T, hkv, d = 3, 1500, len(params), params[0].dim
    print("decode baked q", kind, v_dtype, flush=True)
    c = Cache(device, params, B, T, seed=1)
    try:
        q, qb = _queries(params, (B,), G, seed=2)
        lengths = [T, 700, 33]
        ld = torch.tensor(lengths, dtype=torch.int32, device="cuda")
        v = c.vd if v_dtype == "f16" else c.vd.float()
        outs = {}
        for name, qq, rot in (("natural", q, False), ("baked", qb, True)):
            out = torch.full((B, hkv * G, d), float("nan"), device="cuda")
            args = dict(batch=B, q_heads=hkv * G, kv_heads=hkv, dim=d, q=torch.from_numpy(qq).cuda(), out=out,
                        lengths=ld, max_length=T, v=v, v_dtype=v_dtype, v_seq_stride=v.stride(0),
                        v_head_stride=v.stride(1), splits=0 if kind != "B64" else 5, q_rotated=rot, **c.kw)
            ws = torch.zeros(batched.workspace_bytes(batched.decode_desc(**args)), dtype=torch.uint8, device="cuda")
            batched.decode(device, batched.decode_desc(workspace=ws, **args))
            torch.cuda.synchronize()
            outs[name] = out.cpu().numpy()
        for b in range(B):
            for h in range(hkv):
                keff = c.keff(oracle, b, h, lengths[b])
                _, _, ref = oracle.attention(q[b, h * G:(h + 1) * G], keff, c.v[b, h, :lengths[b]].float().numpy(),
                                             np.full(G, lengths[b] - 1), False)
                for name in outs:
                    _check(outs[name][b, h * G:(h + 1) * G], ref.astype(np.float64), f"{name} b{b} kv{h}")
    finally:
        c.destroy()


def test_decode_append_with_baked_queries(device, oracle):
    """The decode step with its new token (SmolLM2 heads, batch 1, 4097 tokens) and baked queries
    equals the same step with the unbaked queries, and both match the oracle."""
    import torch
    from bgtq import batched
    params, G = _params(oracle, "S")
    T, hkv, d = 4097, 3, 64
    print("decode_append baked q", flush=True)
    c = Cache(device, params, 1, T, seed=3)
    try:
        q, qb = _queries(params, (1,), G, seed=4)
        rng = np.random.default_rng(5)
        knew = torch.from_numpy(rng.standard_normal((1, hkv, d)).astype(np.float32)).cuda()
        vnew = torch.from_numpy(rng.standard_normal((1, hkv, d)).astype(np.float32)).cuda()
        ld = torch.tensor([T], dtype=torch.int32, device="cuda")
        outs, snaps = {}, {}
        for name, qq, rot in (("natural", q, False), ("baked", qb, True)):
            out = torch.full((1, hkv * G, d), float("nan"), device="cuda")
            args = dict(batch=1, q_heads=hkv * G, kv_heads=hkv, dim=d, q=torch.from_numpy(qq).cuda(), out=out,
                        lengths=ld, max_length=T, v=c.vd, v_seq_stride=c.vd.stride(0), v_head_stride=c.vd.stride(1),
                        q_rotated=rot, **c.kw)
            ws = torch.zeros(batched.workspace_bytes(batched.decode_desc(**args)), dtype=torch.uint8, device="cuda")
            batched.decode_append(device, batched.decode_desc(workspace=ws, **args),
                                  batched.append_desc(k_new=knew, v_new=vnew))
            torch.cuda.synchronize()
            outs[name] = out.cpu().numpy()
            snaps[name] = (c.packed.cpu(), c.norms.cpu(), c.vd.cpu())
        for x, y in zip(snaps["natural"], snaps["baked"]):
            assert torch.equal(x, y), "the appended rows depend on the query form"
        for h in range(hkv):
            keff = c.keff(oracle, 0, h, T)
            _, _, ref = oracle.attention(q[0, h * G:(h + 1) * G], keff, c.vd[0, h].float().cpu().numpy(),
                                         np.full(G, T - 1), False)
            for name in outs:
                _check(outs[name][0, h * G:(h + 1) * G], ref.astype(np.float64), f"{name} kv{h}")
    finally:
        c.destroy()


@pytest.mark.parametrize("kind,rows", [("B64", 300), ("B64", 32), ("S", 32), ("B128", 40)])
def test_prefill_with_baked_queries(device, oracle, kind, rows):
    """Chunked prefill: long chunks (four 16-query column blocks per wave), 32-row chunks, the
    per-position K build (SmolLM2 heads) and d=128."""
    import torch
    from bgtq import batched
    params, G = _params(oracle, kind)
    B, hkv, d = 2, len(params), params[0].dim
    starts = [0, 420]
    cap = max(starts) + rows
    print("prefill baked q", kind, rows, flush=True)
    c = Cache(device, params, B, cap, seed=6)
    try:
        q, qb = _queries(params, (B, rows), G, seed=7)
        sd = torch.tensor(starts, dtype=torch.int32, device="cuda")
        outs = {}
        for name, qq, rot in (("natural", q, False), ("baked", qb, True)):
            out = torch.full((B, rows, hkv * G, d), float("nan"), device="cuda")
            kw = dict(batch=B, rows=rows, q_heads=hkv * G, kv_heads=hkv, dim=d, q=torch.from_numpy(qq).cuda(),
                      out=out, starts=sd, max_length=cap, v=c.vd, v_seq_stride=c.vd.stride(0),
                      v_head_stride=c.vd.stride(1), q_rotated=rot, **c.kw)
            ws = torch.zeros(max(16, batched.prefill_workspace_bytes(batched.prefill_desc(**kw))), dtype=torch.uint8,
                             device="cuda")
            batched.prefill(device, batched.prefill_desc(workspace=ws, **kw))
            torch.cuda.synchronize()
            outs[name] = out.cpu().numpy()
        for b in range(B):
            T = starts[b] + rows
            for h in range(hkv):
                keff = c.keff(oracle, b, h, T)
                qq = q[b, :, h * G:(h + 1) * G].reshape(-1, d)
                pos = np.repeat(starts[b] + np.arange(rows), G).astype(np.uint32)
                _, _, ref = oracle.attention(qq, keff, c.v[b, h, :T].float().numpy(), pos, True)
                for name in outs:
                    _check(outs[name][b, :, h * G:(h + 1) * G].reshape(-1, d), ref.astype(np.float64),
                           f"{name} b{b} kv{h}")
    finally:
        c.destroy()


def test_rotated_queries_need_packed_keys(device):
    import torch
    import bgtq
    from bgtq import batched
    z = torch.zeros(64, device="cuda")
    args = dict(batch=1, q_heads=2, kv_heads=1, dim=64, q=z, out=z, lengths=z, max_length=64, v=z, v_seq_stride=0,
                v_head_stride=0, k_f16=z, k_seq_stride=0, k_head_stride=0, q_rotated=True)
    with pytest.raises(bgtq.RangeError, match="q_rotated needs packed K"):
        batched.workspace_bytes(batched.decode_desc(**args))
    kw = dict(batch=1, rows=4, q_heads=2, kv_heads=1, dim=64, q=z, out=z, starts=z, max_length=64, v=z,
              v_seq_stride=0, v_head_stride=0, k_f16=z, q_rotated=True)
    with pytest.raises(bgtq.RangeError, match="q_rotated needs packed K"):
        batched.prefill_workspace_bytes(batched.prefill_desc(**kw))
