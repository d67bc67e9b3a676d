"""The model step's kernel protocol (ModelOps / Commands, src/model/ops.ts:6-31)
through bgtq_model_submit: the reference's own model-codec check
(tests/webgpu/model-codec-test.ts:9-27) on its committed RoPE and calibration
fixtures, and the decoder's attention dispatches (src/model/decoder.ts:46-56)
against the oracle's FP32 attention over the reconstructed keys, within the
decode tolerance (1e-4 relative, 1e-5 absolute)."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

RTOL, ATOL = 1e-4, 1e-5


def _halves(t):
    return t.cpu().numpy().view(np.uint16)


def test_model_codec_every_calibration_head(device, oracle):
    """append rounds the post-RoPE rows (rope fixture, 3 rows x 3 KV heads at
    positions 4095..4097) to FP16 in the [head][capacity][64] cache; encode_k of
    every one of the 90 calibration heads then writes the bytes and FP16
    scales PackedKeys.append writes for those FP16 rows, which are also the
    oracle's."""
    import torch
    import bgtq
    from conftest import REF
    _, rope = oracle.read_fixture(REF / "model" / "rope.json")
    y = np.asarray(rope["h3_p4095_y"], np.float32).reshape(3, 3, 64)  # [row][head][dim]
    cal = bgtq.Calibration.load(device, REF / "model")
    ops = bgtq.ModelOps.create(device)
    try:
        x = torch.from_numpy(y.reshape(-1).copy()).cuda()
        halves = torch.zeros(3 * 3 * 64, dtype=torch.int16, device="cuda")
        cmd = ops.commands()
        cmd.dispatch("append", [3, 0, 3, 3], [x, halves], 3)
        cmd.submit()
        half = _halves(halves).reshape(3, 3, 64)  # [head][row][dim]
        assert np.array_equal(half, oracle.f32_to_f16_bits(y.transpose(1, 0, 2)).reshape(3, 3, 64))
        _, blobs = oracle.read_fixture(REF / "model" / "calibration.json")
        for h in range(90):
            head, c = h % 3, cal.heads[h]
            packed = torch.zeros(3 * c.row_bytes, dtype=torch.uint8, device="cuda")
            norms = torch.zeros(3 * c.norm_stride, dtype=torch.int16, device="cuda")
            e = ops.commands()
            e.dispatch("encode_k", [3, 0, head, 3], [c.config, c.table, x, packed, norms], 3)
            e.submit()
            p = bgtq.BlockGTQParameters.from_serialized(blobs[f"h{h}_config"], blobs[f"h{h}_table"])
            ref = bgtq.PackedKeys.create(device, p, 3)
            try:
                ref.append(half[head].reshape(-1))
                rp, rn = ref.read()
            finally:
                ref.destroy()
            assert np.array_equal(packed.cpu().numpy(), rp), f"head {h}: code bytes"
            assert np.array_equal(_halves(norms), rn), f"head {h}: FP16 scale bits"
            layout = oracle.Layout.from_model_config(blobs[f"h{h}_config"], blobs[f"h{h}_table"])
            op, on = oracle.encode_pack(layout, half[head])
            assert np.array_equal(rp.reshape(3, -1), op) and np.array_equal(rn.reshape(3, -1), on), f"head {h}: oracle"
    finally:
        cal.destroy()


def _attention_case(device, oracle, key_format, heads, kvh=3, gqa=3, d=64, capacity=192, steps=((0, 150), (150, 5)),
                    seed=7):
    """Runs the decoder's per-layer dispatches for each (start, rows) step and
    checks scores, probabilities and outputs of every step against the oracle.
    heads: (device tables, oracle layout) per KV head for packed keys."""
    import torch
    import bgtq
    qh = kvh * gqa
    total = steps[-1][0] + steps[-1][1]
    g = np.random.default_rng(seed)
    kr_all = g.standard_normal((total, kvh, d)).astype(np.float32)
    v_all = g.standard_normal((total, kvh, d)).astype(np.float32)
    q_all = g.standard_normal((total, qh, d)).astype(np.float32)
    ops = bgtq.ModelOps.create(device)
    vcache = torch.zeros(kvh * capacity * d, dtype=torch.int16, device="cuda")
    kcache = torch.zeros(kvh * capacity * d, dtype=torch.int16, device="cuda")
    tables = [t for t, _ in heads] if key_format == "packed" else []
    codes = [torch.zeros(capacity * t.info["row_bytes"], dtype=torch.uint8, device="cuda") for t in tables]
    norms = [torch.zeros(capacity * t.info["norm_stride"], dtype=torch.int16, device="cuda") for t in tables]
    for start, rows in steps:
        tokens = start + rows
        kr = torch.from_numpy(kr_all[start:tokens].reshape(-1).copy()).cuda()
        vv = torch.from_numpy(v_all[start:tokens].reshape(-1).copy()).cuda()
        qr = torch.from_numpy(q_all[start:tokens].reshape(-1).copy()).cuda()
        scores = torch.full((rows * qh * tokens,), float("nan"), device="cuda")
        probs = torch.full((rows * qh * tokens,), float("nan"), device="cuda")
        attn = torch.full((rows * qh * d,), float("nan"), device="cuda")
        cmd = ops.commands()
        if key_format == "packed":
            for h in range(kvh):
                cmd.dispatch("encode_k", [rows, start, h, kvh], [tables[h], tables[h], kr, codes[h], norms[h]], rows)
        else:
            cmd.dispatch("append", [rows, start, capacity, kvh], [kr, kcache], -(-rows * kvh * d // 2 // 128))
        cmd.dispatch("append", [rows, start, capacity, kvh], [vv, vcache], -(-rows * kvh * d // 2 // 128))
        p = [rows, tokens, capacity, start, qh, kvh, gqa, d]
        bufs = [qr, kcache, vcache, scores, probs, attn]
        if key_format == "packed":
            for h in range(kvh):
                cmd.dispatch("compressed_dot", [rows, start, h, tokens, qh, gqa, d],
                             [tables[h], tables[h], qr, codes[h], norms[h], None, scores], tokens,
                             -(-rows * gqa // 128))
        else:
            cmd.dispatch("dot", p, bufs, tokens, kvh * -(-rows * gqa // 128))
        cmd.dispatch("softmax", p, bufs, rows * qh)
        cmd.dispatch("weighted", p, bufs, rows * qh * d)
        cmd.submit()
        v_half = _halves(vcache).reshape(kvh, capacity, d)
        got_s = scores.cpu().numpy().reshape(rows, qh, tokens)
        got_p = probs.cpu().numpy().reshape(rows, qh, tokens)
        got_o = attn.cpu().numpy().reshape(rows, qh, d)
        for kv in range(kvh):
            if key_format == "packed":
                t = tables[kv].info
                layout = heads[kv][1]
                cb = codes[kv].cpu().numpy().reshape(capacity, t["row_bytes"])[:tokens]
                sc = _halves(norms[kv]).reshape(capacity, t["norm_stride"])[:tokens, :t["groups"]]
                k = oracle.reconstruct(layout, oracle.unpack(cb, d, t["nibble_dims"]),
                                       sc.view(np.float16).astype(np.float32))
            else:
                k = _halves(kcache).reshape(kvh, capacity, d)[kv, :tokens].view(np.float16).astype(np.float32)
            v = v_half[kv, :tokens].view(np.float16).astype(np.float32)
            for r in range(rows):
                qs = q_all[start + r, kv * gqa:(kv + 1) * gqa]
                lg, pr, out = oracle.attention(qs, k, v, np.full(gqa, start + r, np.uint32), causal=True)
                what = f"{key_format} step {start}+{rows} row {r} kv {kv}"
                s = got_s[r, kv * gqa:(kv + 1) * gqa]
                live = np.arange(tokens) <= start + r
                assert np.all(np.isneginf(s[:, ~live])), what + ": masked scores"
                np.testing.assert_allclose(s[:, live], lg[:, live], rtol=RTOL, atol=ATOL, err_msg=what + " scores")
                np.testing.assert_allclose(got_p[r, kv * gqa:(kv + 1) * gqa], pr, rtol=RTOL, atol=ATOL,
                                           err_msg=what + " probabilities")
                np.testing.assert_allclose(got_o[r, kv * gqa:(kv + 1) * gqa], out, rtol=RTOL, atol=ATOL,
                                           err_msg=what + " output")


def _tables(device, oracle, source):
    import bgtq
    from bgtq import calibrate
    from conftest import REF
    out = []
    if source == "layout B":
        p = calibrate.layout_b(64)
        blobs = [bgtq.tables(p)] * 3
    else:
        _, a = oracle.read_fixture(REF / "model" / "calibration.json")
        blobs = [(a[f"h{h}_config"], a[f"h{h}_table"]) for h in range(3)]
    for integer, floating in blobs:
        t = bgtq.Tables(device, integer=integer, floating=floating)
        out.append((t, oracle.Layout.from_model_config(integer, floating)))
    return out


@pytest.mark.parametrize("source", ["calibration layer 0", "layout B"])
def test_model_attention_dispatches_packed(device, oracle, source):
    heads = _tables(device, oracle, source)
    try:
        print("model dispatches", source, flush=True)
        _attention_case(device, oracle, "packed", heads)
    finally:
        for t, _ in heads:
            t.destroy()


def test_model_attention_dispatches_fp16(device, oracle):
    print("model dispatches fp16", flush=True)
    _attention_case(device, oracle, "fp16", None, steps=((0, 33), (33, 1), (34, 32)))


def test_model_dispatch_coverage_and_checks(device, oracle):
    """Workgroup counts bound the covered items; failed checks queue nothing."""
    import torch
    import bgtq
    heads = _tables(device, oracle, "layout B")
    try:
        ops = bgtq.ModelOps.create(device)
        kvh, gqa, d, rows, start = 1, 2, 64, 2, 40
        qh, tokens, cap = kvh * gqa, start + rows, 64
        t = heads[0][0]
        kr = torch.randn(tokens * d, device="cuda")
        codes = torch.zeros(cap * t.info["row_bytes"], dtype=torch.uint8, device="cuda")
        norms = torch.zeros(cap * t.info["norm_stride"], dtype=torch.int16, device="cuda")
        cmd = ops.commands()
        cmd.dispatch("encode_k", [tokens, 0, 0, 1], [t, t, kr, codes, norms], tokens)
        cmd.submit()
        q = torch.randn(rows * qh * d, device="cuda")
        scores = torch.full((rows * qh * tokens,), float("nan"), device="cuda")
        cmd = ops.commands()
        cmd.dispatch("compressed_dot", [rows, start, 0, tokens, qh, gqa, d], [t, t, q, codes, norms, None, scores],
                     30, 1)
        cmd.submit()
        s = scores.cpu().numpy().reshape(rows * qh, tokens)
        assert np.isfinite(s[:, :30]).all() and np.isnan(s[:, 30:]).all()
        # encode_k covers min(rows, x) rows
        c2 = torch.zeros_like(codes)
        n2 = torch.zeros_like(norms)
        cmd = ops.commands()
        cmd.dispatch("encode_k", [tokens, 0, 0, 1], [t, t, kr, c2, n2], 5)
        cmd.submit()
        rb = t.info["row_bytes"]
        assert torch.equal(c2[:5 * rb], codes[:5 * rb]) and not c2[5 * rb:].any()
        # a failing dispatch queues nothing, also not the ones before it
        v = torch.zeros(kvh * cap * d, dtype=torch.int16, device="cuda")
        small = torch.zeros(4, device="cuda")
        cmd = ops.commands()
        cmd.dispatch("append", [rows, start, cap, kvh], [q[:rows * kvh * d], v], 1)
        cmd.dispatch("softmax", [rows, tokens, cap, start, qh, kvh, gqa, d], [q, v, v, scores, small, small],
                     rows * qh)
        with pytest.raises(bgtq.RangeError, match="binding 4 holds 16 bytes"):
            cmd.submit()
        torch.cuda.synchronize()
        assert not v.any()
        with pytest.raises(bgtq.UnsupportedError, match="rope"):
            c = ops.commands()
            c.dispatch("rope", [rows, 64, 0, 0, start, qh, 100000], [q, q, q, q], 1)
            c.submit()
        with pytest.raises(bgtq.RangeError, match="unknown model kernel"):
            c = ops.commands()
            c.dispatch("gather", [], [], 1)
            c.submit()
        with pytest.raises(bgtq.RangeError, match="Model dispatch limit"):
            ops.commands().dispatch("softmax", [], [], 1 << 31)
        with pytest.raises(bgtq.RangeError, match="capacity"):
            c = ops.commands()
            c.dispatch("append", [rows, cap - 1, cap, kvh], [q, v], 1)
            c.submit()
    finally:
        for t, _ in heads:
            t.destroy()
