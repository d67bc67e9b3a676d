"""Chunked prefill with the chunk's own rows appended in the same launch (bgtq_prefill_append).

The reference decoder encodes a chunk's K rows, appends its V rows and then runs the attention
passes over the history and the chunk (src/model/decoder.ts:46-56, per chunk of up to 32 rows,
src/model/decoder.ts:15,82). bgtq_prefill_append does all of it in one launch. Against the
two-call path (bgtq_encode_batched of the rows, the V rows written, then bgtq_prefill):
- the packed rows, FP16 scales and V rows it writes are bit-identical (the chunk's rows are
  poisoned beforehand, so a row it fails to write shows);
- its outputs agree within |a - b| <= 1e-5 + 1e-4 |b|, and both agree with the oracle's causal
  attention on the same effective K.
"""
import numpy as np
import pytest

from test_gpu_prefill import Cache, _check, _reference

pytestmark = pytest.mark.gpu


def _chunk_rows(t, starts, rows):
    """[B, rows, Hkv, dim] copy of each sequence's chunk rows of t [B, Hkv, cap, dim]."""
    import torch
    return torch.stack([t[b, :, s:s + rows].transpose(0, 1) for b, s in enumerate(starts)]).contiguous()


def _append(device, cache, q, starts, max_length, k_new, v_new, split_tokens=0):
    import torch
    from bgtq import batched
    B, rows, hq, dim = q.shape
    out = torch.full((B, rows, hq, dim), float("nan"), dtype=torch.float32, device="cuda")
    kw = dict(batch=B, rows=rows, q_heads=hq, kv_heads=cache.vd.shape[1], dim=dim, q=q.cuda(), out=out,
              starts=torch.tensor(starts, dtype=torch.int32).cuda(), max_length=max_length, v=cache.vd,
              v_seq_stride=cache.vd.stride(0), v_head_stride=cache.vd.stride(1), split_tokens=split_tokens,
              **cache.kw)
    ws = torch.zeros(batched.prefill_workspace_bytes(batched.prefill_desc(**kw)), dtype=torch.uint8, device="cuda")
    app = batched.prefill_append_desc(k_new=k_new.cuda(), v_new=v_new.cuda())
    batched.prefill_append(device, batched.prefill_desc(workspace=ws, **kw), app)
    torch.cuda.synchronize()
    return out.cpu().numpy()


def _poison(cache, starts, rows):
    """Garbage in the chunk's cache rows: the append has to write every byte of them."""
    p = cache.params[0]
    for b, s in enumerate(starts):
        cache.packed[b, :, s * p.rowBytes:(s + rows) * p.rowBytes] = 0xA5
        cache.norms[b, :, s * p.normStride:(s + rows) * p.normStride] = 0x7bff
        cache.vd[b, :, s:s + rows] = float("nan")


def _case(device, oracle, *, params, batch, rows, hq, hkv, dim, starts, cap, f32=False, split_tokens=0, seed=0,
          pad16=False):
    import torch
    ref_cache = Cache(device, params=params, batch=batch, hkv=hkv, dim=dim, cap=cap, seed=seed, pad16=pad16)
    app_cache = Cache(device, params=params, batch=batch, hkv=hkv, dim=dim, cap=cap, seed=seed, pad16=pad16)
    try:
        q = torch.randn((batch, rows, hq, dim), generator=torch.Generator().manual_seed(seed + 1))
        two_calls = ref_cache.prefill(device, q, starts, cap, split_tokens)
        k_new, v_new = _chunk_rows(app_cache.k, starts, rows), _chunk_rows(app_cache.v, starts, rows)
        if f32:  # FP32 rows carrying FP16 values: rounded to FP16 first, so the same bytes
            k_new, v_new = k_new.float(), v_new.float()
        _poison(app_cache, starts, rows)
        fused = _append(device, app_cache, q, starts, cap, k_new, v_new, split_tokens)
        assert np.array_equal(app_cache.packed.cpu().numpy(), ref_cache.packed.cpu().numpy()), "packed K differs"
        assert np.array_equal(app_cache.norms.cpu().numpy(), ref_cache.norms.cpu().numpy()), "scales differ"
        assert np.array_equal(app_cache.vd.cpu().numpy(), ref_cache.vd.cpu().numpy()), "V rows differ"
        _check(fused, two_calls.astype(np.float64), "append vs two calls")
        G = hq // hkv
        for b in range(batch):
            for h in range(hkv):
                ref = _reference(oracle, ref_cache, q, starts, b, h, G)
                _check(fused[b, :, h * G:(h + 1) * G], ref.astype(np.float64), f"b{b} kv{h} start={starts[b]}")
    finally:
        ref_cache.destroy()
        app_cache.destroy()


@pytest.mark.parametrize("dim,rows,f32", [(64, 32, False), (64, 13, True), (128, 32, False), (128, 5, True)])
def test_layout_b(device, oracle, dim, rows, f32):
    from bgtq import calibrate
    p = calibrate.layout_b(dim)
    print("prefill append layout B", dim, rows, f32, flush=True)
    _case(device, oracle, params=[p, p], batch=3, rows=rows, hq=14, hkv=2, dim=dim, starts=[0, 5, 700], cap=760,
          f32=f32)


def test_layout_a(device, oracle):
    """Layout A (groups straddling the K-steps, norm stride 3): the per-position path."""
    from bgtq import calibrate
    p = calibrate.layout_a(64)
    print("prefill append layout A", flush=True)
    _case(device, oracle, params=[p, p], batch=2, rows=32, hq=14, hkv=2, dim=64, starts=[0, 463], cap=500,
          pad16=True)


def test_smollm2_heads(device, oracle):
    """The reference's SmolLM2 calibration heads (37-byte rows, nibble and byte codes mixed)."""
    from bgtq import BlockGTQParameters
    from conftest import REF
    m, a = oracle.read_fixture(REF / "model" / "calibration.json")
    heads = [BlockGTQParameters.from_serialized(a[f"{n}_config"], a[f"{n}_table"]) for n in ("h0", "h56", "h22")]
    rb, ns = max(h.rowBytes for h in heads), max(h.normStride for h in heads)
    for h in heads:
        h.rowBytes, h.normStride = rb, ns
    print("prefill append smollm2 heads", flush=True)
    _case(device, oracle, params=heads, batch=2, rows=32, hq=9, hkv=3, dim=64, starts=[0, 700], cap=732, pad16=True)


@pytest.mark.parametrize("split_tokens", [96, 512])
def test_forced_splits(device, oracle, split_tokens):
    """Many history splits beside the appended rows' workgroups (the merge takes up to 16)."""
    from bgtq import calibrate
    p = calibrate.layout_b(64)
    print("prefill append split_tokens", split_tokens, flush=True)
    _case(device, oracle, params=[p], batch=2, rows=32, hq=7, hkv=1, dim=64, starts=[1900, 0], cap=2000,
          split_tokens=split_tokens)


def test_prompt_in_chunks_of_32(device, oracle):
    """A 1024-token prompt of a Qwen2.5-0.5B layer in 32-row chunks, each chunk's rows appended by its
    own launch into an empty (poisoned) cache: the caches end bit-identical to the two-call path's and
    every chunk's output agrees with it; sampled rows against the oracle."""
    import torch
    from bgtq import calibrate
    p = calibrate.layout_b(64)
    prompt = 1024
    ref_cache = Cache(device, params=[p, p], batch=1, hkv=2, dim=64, cap=prompt, seed=8)
    app_cache = Cache(device, params=[p, p], batch=1, hkv=2, dim=64, cap=prompt, seed=8)
    try:
        q = torch.randn((1, prompt, 14, 64), generator=torch.Generator().manual_seed(21))
        _poison(app_cache, [0], prompt)
        fused, two = [], []
        for s in range(0, prompt, 32):
            qc = q[:, s:s + 32].contiguous()
            two.append(ref_cache.prefill(device, qc, [s], prompt))
            fused.append(_append(device, app_cache, qc, [s], prompt, _chunk_rows(app_cache.k, [s], 32),
                                 _chunk_rows(app_cache.v, [s], 32)))
        assert np.array_equal(app_cache.packed.cpu().numpy(), ref_cache.packed.cpu().numpy())
        assert np.array_equal(app_cache.norms.cpu().numpy(), ref_cache.norms.cpu().numpy())
        assert np.array_equal(app_cache.vd.cpu().numpy(), ref_cache.vd.cpu().numpy())
        fused, two = np.concatenate(fused, axis=1), np.concatenate(two, axis=1)
        _check(fused, two.astype(np.float64), "chunks appended vs two calls")
        sel = [0, 31, 32, 511, 512, 1023]
        for h in range(2):
            ref = _reference(oracle, ref_cache, q, [0], 0, h, 7, rows_sel=sel)
            _check(fused[0, sel, h * 7:(h + 1) * 7], ref.astype(np.float64), f"kv{h} sampled rows")
    finally:
        ref_cache.destroy()
        app_cache.destroy()


def test_rejections(device):
    """FP16 K and chunks above 32 rows are refused before anything is queued."""
    import torch
    import bgtq
    from bgtq import calibrate
    p = calibrate.layout_b(64)
    cache = Cache(device, params=[p], batch=1, hkv=1, dim=64, cap=128, key_format="fp16")
    try:
        q = torch.randn((1, 8, 2, 64))
        kn = torch.zeros((1, 8, 1, 64))
        with pytest.raises(bgtq.UnsupportedError, match="packed K"):
            _append(device, cache, q, [0], 128, kn, kn)
    finally:
        cache.destroy()
    cache = Cache(device, params=[p], batch=1, hkv=1, dim=64, cap=128)
    try:
        q = torch.randn((1, 40, 2, 64))
        kn = torch.zeros((1, 40, 1, 64))
        with pytest.raises(bgtq.UnsupportedError, match="32 rows"):
            _append(device, cache, q, [0], 128, kn, kn)
    finally:
        cache.destroy()
