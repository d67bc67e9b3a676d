"""The launches bench.py times, built by bench.py's own workload classes at their full sizes,
checked against the oracle.

- Qwen2.5-0.5B decode: batch 64 x 32768-token context, 14 q / 2 KV heads, d=64, layout B, FP16 V,
  the library's split choice (one layer of the headline step). Zero queries give the mean of V on
  all 128 (sequence, KV head) units; random queries match the oracle on sampled units.
- Qwen2.5-0.5B 4096-token prompt in 32-row chunks (the reference's chunk cap,
  src/model/decoder.ts:15,82), encode + prefill per chunk, one layer: every row against a float64
  evaluation of src/reference/attention.py:5-22 on the oracle's effective K, sampled rows against
  the oracle itself, and the one-chunk launch on the same inputs.
- SmolLM2 decode step at batch 1 (30 layers x bgtq_decode_append over 4096 + 1 tokens, 3 KV / 9 q
  heads; src/model/decoder.ts:46-56 at rows = 1): the new rows bit-exact against the oracle's
  encoder, the V rows FP16 round-to-nearest-even, the outputs against the oracle.

Outputs must match within |gpu - ref| <= 1e-5 + 1e-4 |ref|.
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
    err = np.abs(np.asarray(out, np.float64) - ref)
    lim = ATOL + RTOL * np.abs(ref)
    assert np.all(err <= lim), f"{what}: max err {err.max():.3e}, worst ratio {(err / lim).max():.2f}"


def _keff(oracle, p, packed_row, norms_row, T):
    pk = packed_row[:T * p.rowBytes].cpu().numpy().reshape(T, p.rowBytes)
    nm = norms_row[:T * p.normStride].cpu().numpy().view(np.float16).reshape(T, p.normStride)
    return oracle.reconstruct(_olayout(oracle, p), oracle.unpack(pk, p.dim, p.nibbleDims), nm.astype(np.float32))


def test_qwen_decode_b64_t32k_library_splits(device, oracle):
    import torch
    import bench
    from bgtq import batched
    print("decode B=64 T=32768 library splits", flush=True)
    w = bench.DecodeWorkload(device, "B", layers=1)
    try:
        d = w.descs[0]
        assert d.splits == 0, "the bench launches with the library's split choice"
        # The library's choice: about two resident workgroups per CU over the 128 units.
        cus = torch.cuda.get_device_properties(0).multi_processor_count
        expect = max(1, -(-2 * cus // (w.batch * w.hkv)))
        probe = type(d).from_buffer_copy(d)
        probe.splits = expect
        assert batched.workspace_bytes(probe) == batched.workspace_bytes(d), "split count differs from the plan"
        probe.splits = expect + 1
        assert batched.workspace_bytes(probe) != batched.workspace_bytes(d)
        t = w.layer_tensors[0]
        q, v = t["q"], t["v"]
        q_rand = q.clone()
        # zero queries: uniform softmax, every (sequence, KV head) returns the mean of its V
        q.zero_()
        w.out.fill_(float("nan"))
        w.step()
        torch.cuda.synchronize()
        got = w.out.cpu().numpy()
        means = v.double().mean(dim=2).cpu().numpy()  # [B, Hkv, d]
        G = w.hq // w.hkv
        for h in range(w.hkv):
            _check(got[:, h * G:(h + 1) * G], np.repeat(means[:, h:h + 1], G, axis=1), f"mean of V, kv{h}")
        # random queries: sampled units against the oracle
        q.copy_(q_rand)
        w.out.fill_(float("nan"))
        w.step()
        torch.cuda.synchronize()
        got = w.out.cpu().numpy()
        assert np.isfinite(got).all()
        T = w.ctx
        for b, h in [(0, 0), (17, 1), (42, 0), (63, 1), (31, 1)]:
            p = t["params"][h]
            keff = _keff(oracle, p, t["packed"][b, h], t["norms"][b, h], T)
            _, _, ref = oracle.attention(q_rand[b, h * G:(h + 1) * G].cpu().numpy(), keff,
                                         v[b, h].float().cpu().numpy(), np.full(G, T - 1), False)
            _check(got[b, h * G:(h + 1) * G], ref.astype(np.float64), f"b{b} kv{h}")
    finally:
        for tab in w.tables:
            tab.destroy()


def _causal_f64(torch, q, keff, v, inv_sqrt_d):
    """float64 causal attention of every prompt row: q [rows, G, d], keff/v [rows, d] (row r sees 0..r)."""
    rows, G, d = q.shape
    qq = q.reshape(rows * G, d).double()
    logits = (qq @ keff.double().t()) * inv_sqrt_d
    r = torch.arange(rows, device=q.device).repeat_interleave(G)
    mask = torch.arange(rows, device=q.device)[None, :] > r[:, None]
    logits.masked_fill_(mask, float("-inf"))
    return (torch.softmax(logits, dim=1) @ v.double()).reshape(rows, G, d)


def test_qwen_prefill_4096_chunks_of_32(device, oracle):
    import torch
    import bench
    print("prefill 4096-token prompt, chunks of 32", flush=True)
    w32 = bench.PrefillWorkload(device, "B", chunk=32, layers=1)
    w1 = bench.PrefillWorkload(device, "B", chunk=0, layers=1)  # the same seed: the same q, K and V
    try:
        assert len(w32.descs) == 4096 // 32
        for w in (w32, w1):
            w.out.fill_(float("nan"))
            w.step()
        torch.cuda.synchronize()
        assert torch.equal(w32.packed, w1.packed) and torch.equal(w32.norms, w1.norms), \
            "chunk-by-chunk encode differs from the one-chunk encode"
        g32, g1 = w32.out[0].cpu().numpy(), w1.out[0].cpu().numpy()
        assert np.isfinite(g32).all() and np.isfinite(g1).all()
        G, d, rows = bench.HQ // bench.HKV, bench.DIM, 4096
        p = w32.params
        sel = [0, 1, 31, 32, 33, 1000, 2047, 2048, 4063, 4064, 4095]
        for h in range(bench.HKV):
            keff = _keff(oracle, p, w32.packed[0, 0, h], w32.norms[0, 0, h], rows)
            vh = w32.v[0, 0, h]
            ref = _causal_f64(torch, w32.q[0, :, h * G:(h + 1) * G], torch.from_numpy(keff).cuda(), vh,
                              1.0 / np.sqrt(d)).cpu().numpy()
            _check(g32[:, h * G:(h + 1) * G], ref, f"chunks of 32, kv{h}, every row")
            _check(g1[:, h * G:(h + 1) * G], ref, f"one chunk, kv{h}, every row")
            qq = w32.q[0, sel, h * G:(h + 1) * G].reshape(-1, d).cpu().numpy()
            pos = np.repeat(np.asarray(sel), G).astype(np.uint32)
            _, _, ro = oracle.attention(qq, keff, vh.float().cpu().numpy(), pos, True)
            _check(g32[sel, h * G:(h + 1) * G].reshape(-1, d), ro.astype(np.float64), f"kv{h} sampled rows vs oracle")
    finally:
        w32.destroy()
        w1.destroy()


@pytest.mark.parametrize("layout", ["B", "S"])
def test_smollm2_decode_step_b1(device, oracle, layout):
    import torch
    import bench
    print("SmolLM2 decode step, layout", layout, flush=True)
    w = bench.SmolLM2Step(device, layout)
    try:
        w.out.fill_(float("nan"))
        w.step()
        torch.cuda.synchronize()
        T = w.T
        out = w.out.cpu().numpy()
        G = w.HQ // w.HKV
        for l in range(w.L):
            for h in range(w.HKV):
                p = w.heads[l][h]
                L = _olayout(oracle, p)
                kbits = w.knew[l, 0, h].cpu().half().numpy().view(np.uint16)[None]  # x.half() before encode
                rp, rn = oracle.encode_pack(L, kbits)
                pk = w.packed[l, 0, h, T * p.rowBytes:(T + 1) * p.rowBytes].cpu().numpy()
                nm = w.norms[l, 0, h, T * p.normStride:(T + 1) * p.normStride].cpu().numpy().view(np.uint16)
                assert np.array_equal(pk, rp[0]), f"layer {l} kv{h}: new packed row differs from the oracle"
                assert np.array_equal(nm, rn[0]), f"layer {l} kv{h}: new scales differ from the oracle"
                vrow = w.v[l, 0, h, T].cpu()
                assert torch.equal(vrow, w.vnew[l, 0, h].cpu().half()), f"layer {l} kv{h}: V row"
                keff = _keff(oracle, p, w.packed[l, 0, h], w.norms[l, 0, h], T + 1)
                _, _, ref = oracle.attention(w.q[l, 0, h * G:(h + 1) * G].cpu().numpy(), keff,
                                             w.v[l, 0, h, :T + 1].float().cpu().numpy(), np.full(G, T), False)
                _check(out[l, 0, h * G:(h + 1) * G], ref.astype(np.float64), f"layer {l} kv{h}")
    finally:
        w.destroy()


def test_smollm2_prefill_encode_one_call(device, oracle):
    """The bulk K encode bench.py times: 30 layers x 3 KV heads x 4096 rows (FP16, pair energies
    decaying by 0.9), 90 table sets, one bgtq_encode_batched call; every packed row and scale
    bit-exact against the oracle's encoder (src/reference/production_math.py:4-24 and the
    packing of src/reference/mixed_layout.py:21-27)."""
    import torch
    import bench
    w = bench.EncodeWorkload(device, "B")
    try:
        w.call()
        torch.cuda.synchronize()
        p = w.p
        ol = _olayout(oracle, p)
        k = w.k.cpu().numpy().view(np.uint16)  # [30, 4096, 3, 64]
        packed = w.packed.cpu().numpy()
        norms = w.norms.cpu().numpy().view(np.uint16)
        for j in range(90):
            l, h = divmod(j, 3)
            ref_p, ref_n = oracle.encode_pack(ol, np.ascontiguousarray(k[l, :, h]))
            got_p = packed[j, :4096 * p.rowBytes].reshape(4096, p.rowBytes)
            got_n = norms[j, :4096 * p.normStride].reshape(4096, p.normStride)
            bad = np.nonzero(np.any(got_p != ref_p, axis=1) | np.any(got_n != ref_n, axis=1))[0]
            assert bad.size == 0, f"job {j}: {bad.size} rows differ, first {bad[:5]}"
            assert not packed[j, 4096 * p.rowBytes:].any() and not norms[j, 4096 * p.normStride:].any(), \
                f"job {j}: bytes past its rows written"
    finally:
        w.destroy()
