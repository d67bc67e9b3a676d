"""The decode step with its new token in one launch (bgtq_decode_append) against
the two-call path of the reference's model step (src/model/decoder.ts:46-56 at
rows = 1): bgtq_encode_batched of the new K rows, the V rows written, then
bgtq_decode. Packed K rows, FP16 scales, K and V rows must be bit-identical,
for new tokens at every position inside a 32-token chunk, ragged batches and
forced splits. The outputs agree within the attention tolerance
(1e-5 + 1e-4 |ref|): with packed K the launch takes the new token's logit and
its share of the output on a separate wave (it is encoded there while the
others attend to the history), an equally precise but differently rounded
sum; FP16 K rows give bit-identical outputs."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _run(device, *, dim, key_format, lengths, splits=0, k_dtype="f32", v_dtype="f32", hkv=2, hq=14, seed=0,
         layout="B", params=None):
    import torch
    import bgtq
    from bgtq import batched, calibrate
    print("append", dim, key_format, layout, lengths, splits, k_dtype, v_dtype, flush=True)
    B, cap = len(lengths), max(lengths)
    g = torch.Generator().manual_seed(seed)
    hist = torch.randn((B, hkv, cap, dim), generator=g).half().cuda()
    v0 = torch.randn((B, hkv, cap, dim), generator=g).half().cuda()
    q = torch.randn((B, hq, dim), generator=g).cuda()
    tdt = {"f32": torch.float32, "f16": torch.float16}
    k_new = torch.randn((B, hkv, dim), generator=g).to(tdt[k_dtype]).cuda()
    v_new = torch.randn((B, hkv, dim), generator=g).to(tdt[v_dtype]).cuda()
    lens = torch.tensor(lengths, dtype=torch.int32, device="cuda")
    outs, caches, tabs = [], [], []
    if key_format == "packed":
        p = calibrate.layout_b(dim) if layout == "B" else calibrate.layout_a(dim)
        if params is not None:  # one parameter set per KV head, common row and norm strides
            p = params[0]
        tabs = [bgtq.Tables(device, params[h] if params is not None else p) for h in range(hkv)]
        rb, ns = p.rowBytes, p.normStride
        packed0 = torch.zeros((B, hkv, (cap * rb + 64 + 15) // 16 * 16), dtype=torch.uint8, device="cuda")
        # scale rows padded to 16 bytes: the fused kernel loads four tokens' scales at once
        norms0 = torch.zeros((B, hkv, (cap * ns + 32 + 7) // 8 * 8), dtype=torch.int16, device="cuda")
        batched.encode(device, [dict(tables=tabs[h], src=hist[b, h], src_row_stride=dim, rows=lengths[b] - 1,
                                     packed=packed0[b, h], norms=norms0[b, h]) for b in range(B) for h in range(hkv)],
                       "f16")
    for mode in ("two calls", "fused"):
        out = torch.full((B, hq, dim), float("nan"), device="cuda")
        v = v0.clone()
        if key_format == "packed":
            packed, norms = packed0.clone(), norms0.clone()
            kw = dict(tables=tabs, packed=packed, packed_seq_stride=packed.stride(0),
                      packed_head_stride=packed.stride(1), norms=norms, norms_seq_stride=norms.stride(0),
                      norms_head_stride=norms.stride(1))
            cache = (packed, norms, v)
        else:
            k = hist.clone()
            kw = dict(k_f16=k, k_seq_stride=k.stride(0), k_head_stride=k.stride(1))
            cache = (k, v)
        args = dict(batch=B, q_heads=hq, kv_heads=hkv, dim=dim, q=q, out=out, lengths=lens, max_length=cap, v=v,
                    v_seq_stride=v.stride(0), v_head_stride=v.stride(1), splits=splits, **kw)
        ws = torch.zeros(batched.workspace_bytes(batched.decode_desc(**args)), dtype=torch.uint8, device="cuda")
        desc = batched.decode_desc(workspace=ws, **args)
        if mode == "two calls":
            if key_format == "packed":
                batched.encode(device, [dict(tables=tabs[h], src=k_new[b, h], src_row_stride=dim, rows=1,
                                             packed=packed[b, h], norms=norms[b, h], dst_row0=lengths[b] - 1)
                                        for b in range(B) for h in range(hkv)], k_dtype)
            else:
                for b in range(B):
                    k[b, :, lengths[b] - 1] = k_new[b].half()
            for b in range(B):
                v[b, :, lengths[b] - 1] = v_new[b].half()
            batched.decode(device, desc)
        else:
            batched.decode_append(device, desc, batched.append_desc(k_new=k_new, v_new=v_new))
        torch.cuda.synchronize()
        assert not ws[:64 * B * hkv].any(), "split counters (one per 64-byte line) left nonzero"
        outs.append(out.cpu())
        caches.append([c.cpu() for c in cache])
    for a, b in zip(caches[0], caches[1]):
        assert torch.equal(a, b), "caches differ"
    assert not torch.isnan(outs[1]).any()
    if key_format == "packed":
        err = (outs[1] - outs[0]).abs()
        lim = 1e-5 + 1e-4 * outs[0].abs()
        assert bool((err <= lim).all()), float((err / lim).max())
    else:
        assert torch.equal(outs[0], outs[1]), float((outs[0] - outs[1]).abs().max())
    for t in tabs:
        t.destroy()


@pytest.mark.parametrize("dim", [64, 128])
def test_append_packed_every_chunk_position(device, dim):
    _run(device, dim=dim, key_format="packed", lengths=[1, 32, 33, 64, 97, 1000, 4096])


@pytest.mark.parametrize("splits", [1, 3, 16, 32])
def test_append_packed_forced_splits(device, splits):
    _run(device, dim=64, key_format="packed", lengths=[2000, 31, 4095], splits=splits, hkv=3, hq=9)


@pytest.mark.parametrize("dim", [64, 128])
def test_append_smollm2_step_shape(device, dim):
    """Batch 1 at 4096 + 1 tokens: the library's own split choice (one 32-token chunk per wave, the
    new token alone in the last split) and the one-round merge."""
    _run(device, dim=dim, key_format="packed", lengths=[4097], hkv=3, hq=9)


@pytest.mark.parametrize("lengths,splits", [([1, 32, 33, 97, 1000, 4096], 0), ([2000, 31, 4095], 3)])
def test_append_layout_a(device, lengths, splits):
    """Layout A at d=64 (groups straddling K-steps, norm stride 3) through the fused kernel's
    per-position code lookup: decode_append accepts only fused layouts."""
    _run(device, dim=64, key_format="packed", layout="A", lengths=lengths, splits=splits, hkv=3, hq=9)


def test_append_smollm2_heads(device, oracle):
    """Real SmolLM2 calibration heads (odd 37-byte rows, mixed nibble/byte lanes, K-steps spanning
    three groups) with 16-byte aligned caches through the fused kernel's per-position lookup."""
    from bgtq import BlockGTQParameters
    from conftest import REF
    m, a = oracle.read_fixture(REF / "model" / "calibration.json")
    heads = [BlockGTQParameters.from_serialized(a[f"{n}_config"], a[f"{n}_table"]) for n in ("h0", "h1", "h22")]
    rb, ns = max(h.rowBytes for h in heads), max(h.normStride for h in heads)
    for h in heads:
        h.rowBytes, h.normStride = rb, ns
    _run(device, dim=64, key_format="packed", layout="smollm2", lengths=[1, 33, 97, 4096], hkv=3, hq=9,
         params=heads)


def test_append_smollm2_every_layer(device, oracle):
    """decode_append accepts all 90 SmolLM2 calibration heads (it refuses layouts outside the fused
    kernel) and matches the two-call path on each layer's three heads."""
    from bgtq import BlockGTQParameters
    from conftest import REF
    m, a = oracle.read_fixture(REF / "model" / "calibration.json")
    for layer in range(30):
        heads = [BlockGTQParameters.from_serialized(a[f"h{3 * layer + h}_config"], a[f"h{3 * layer + h}_table"])
                 for h in range(3)]
        rb, ns = max(h.rowBytes for h in heads), max(h.normStride for h in heads)
        for h in heads:
            h.rowBytes, h.normStride = rb, ns
        _run(device, dim=64, key_format="packed", layout=f"smollm2 layer {layer}", lengths=[1, 40, 130], hkv=3, hq=9,
             params=heads, seed=layer)


def test_append_widths_1_to_6_d128(device):
    """d=128, widths 1..6 (79-byte rows, mixed nibble/byte lanes, norm stride 6): the append's
    encoder reads the tables from device memory when they exceed the ring slot."""
    from bgtq import calibrate
    p = calibrate.make_parameters(calibrate.allocate_bits(calibrate.geometric_scores(64), 206, 1, 8))
    _run(device, dim=128, key_format="packed", layout="widths 1..6", lengths=[1, 33, 500], hkv=2, hq=14,
         params=[p, p])


def test_append_fp16_sources(device):
    _run(device, dim=64, key_format="packed", lengths=[513, 130], k_dtype="f16", v_dtype="f16")


@pytest.mark.parametrize("dim", [64, 128])
def test_append_fp16_keys(device, dim):
    _run(device, dim=dim, key_format="fp16", lengths=[1, 40, 3000])


def test_append_unsupported_layout_is_rejected(device, oracle):
    """Caches outside the fused kernel (a real SmolLM2 head's rows, 35 bytes, at a head stride of
    T * 35 + 64 bytes: not 16-byte aligned) are refused and nothing is written; the two-call path
    serves them."""
    import torch
    import bgtq
    from bgtq import batched
    from conftest import REF
    m, a = oracle.read_fixture(REF / "model" / "calibration.json")
    p = bgtq.BlockGTQParameters.from_serialized(a["h0_config"], a["h0_table"])
    t = bgtq.Tables(device, p)
    try:
        T, dim = 100, 64
        packed = torch.zeros((1, 1, T * p.rowBytes + 64), dtype=torch.uint8, device="cuda")
        norms = torch.zeros((1, 1, T * p.normStride + 32), dtype=torch.int16, device="cuda")
        v = torch.zeros((1, 1, T, dim), dtype=torch.float16, device="cuda")
        q = torch.zeros((1, 3, dim), device="cuda")
        out = torch.zeros((1, 3, dim), device="cuda")
        args = dict(batch=1, q_heads=3, kv_heads=1, dim=dim, q=q, out=out,
                    lengths=torch.tensor([T], dtype=torch.int32, device="cuda"), max_length=T, v=v,
                    v_seq_stride=v.stride(0), v_head_stride=v.stride(1), tables=[t], packed=packed,
                    packed_seq_stride=packed.stride(0), packed_head_stride=packed.stride(1), norms=norms,
                    norms_seq_stride=norms.stride(0), norms_head_stride=norms.stride(1))
        ws = torch.zeros(batched.workspace_bytes(batched.decode_desc(**args)), dtype=torch.uint8, device="cuda")
        desc = batched.decode_desc(workspace=ws, **args)
        kn = torch.ones((1, 1, dim), device="cuda")
        with pytest.raises(bgtq.UnsupportedError, match="decode_append"):
            batched.decode_append(device, desc, batched.append_desc(k_new=kn, v_new=kn))
        torch.cuda.synchronize()
        assert not packed.any() and not v.any()
    finally:
        t.destroy()
