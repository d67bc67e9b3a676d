"""Decode attention on the GPU against the oracle (FP32, tolerance) and closed forms.

Mirrors tests/webgpu/optimized-test.ts:12-78, tests/webgpu/attention-test.ts:22-95
and tests/webgpu/runtime-contracts.ts:9-29 through the C ABI: the same
workloads, checks and rejections. The numerical bar is the north-star one,
|gpu - oracle| <= 1e-5 + 1e-4 |oracle| for outputs, on the same effective K
(the reference's own strict gate, tests/oracles/verify_phase4.py:21-27).
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

ATOL, RTOL = 1e-5, 1e-4          # attention outputs
LOGIT_ATOL, LOGIT_RTOL = 1e-4, 2e-5  # fixture "baseline" tolerance for logits
PROB_ATOL, PROB_RTOL = 1e-5, 1e-4    # fixture "baseline" tolerance for probabilities


def _close(actual, expected, atol, rtol, what):
    a, e = np.asarray(actual, np.float64), np.asarray(expected, np.float64)
    both_inf = np.isneginf(a) & np.isneginf(e)
    err = np.where(both_inf, 0.0, np.abs(a - e))
    lim = atol + rtol * np.where(both_inf, 0.0, np.abs(e))
    bad = ~(err <= lim)
    assert not bad.any(), f"{what}: {bad.sum()} mismatches, worst {err[bad].max()} at {np.argmax(np.where(bad, err, -1))}"


def _params(lm, la):
    import bgtq
    return bgtq.BlockGTQParameters.from_mixed_fixture(lm, la)


def test_optimized_attention_fixtures(device, attention_cases, oracle):
    """Packed K + fused decode vs the oracle on the reconstructed K, and vs the goldens."""
    import bgtq
    for name, m, a, lm, la in attention_cases:
        print("case", name, flush=True)
        T, d = m["context_length"], m["dim"]
        keys = bgtq.PackedKeys.create(device, _params(lm, la), T)
        values = bgtq.Values(device, d, T)
        att = bgtq.OptimizedAttention.create(device, keys, values, m["queries"])
        try:
            k = a["k"].view(np.uint16)
            keys.append(k[:3])
            keys.append(k[3:])
            values.append(a["v"][:3])
            values.append(a["v"][3:])
            ol = oracle.Layout.from_mixed_fixture(lm, la)
            packed, norms = keys.read()
            codes = oracle.unpack(packed.reshape(T, -1), d, lm["nopack_start"])
            scales = norms.view(np.float16).reshape(T, -1).astype(np.float32)
            k_eff = oracle.reconstruct(ol, codes, scales)
            # the effective K is the reference's reconstruct (same codes and scales)
            np.testing.assert_allclose(k_eff, a["reconstructed_k"], atol=1e-5, rtol=1e-5)
            for causal in (False, True):
                prefix = "causal_" if causal else ""
                out = att.attend(a["q"], a["positions"], causal)
                ins = att.inspect()
                ref_l, ref_p, ref_o = oracle.attention(a["q"], k_eff, a["v"], a["positions"], causal)
                _close(ins["logits"], ref_l, LOGIT_ATOL, LOGIT_RTOL, f"{name} {causal} logits")
                _close(ins["probabilities"], ref_p, PROB_ATOL, PROB_RTOL, f"{name} {causal} probabilities")
                _close(out, ref_o, ATOL, RTOL, f"{name} {causal} output")
                # and against the reference goldens computed on the same effective K
                _close(out, a[prefix + "compressed_output"], ATOL, RTOL, f"{name} {causal} golden output")
                _close(ins["logits"], a[prefix + "compressed_logits"], LOGIT_ATOL, LOGIT_RTOL, f"{name} golden logits")
                probs = ins["probabilities"]
                assert np.all(probs >= 0)
                np.testing.assert_allclose(probs.sum(1), 1.0, atol=1e-4)
                if causal:
                    for r, pos in enumerate(a["positions"]):
                        assert not probs[r, pos + 1:].any()
                    # the first causal query attends to V0 only: exactly V0
                    np.testing.assert_array_equal(out[0], a["v"][0])
                if name == "t128_d64":
                    again = att.attend(a["q"], a["positions"], causal)
                    np.testing.assert_array_equal(again, out)  # deterministic
            assert not any(x["role"] == "scratch" and x["bytes"] > 4 for x in keys.allocations)
        finally:
            att.destroy()
            values.destroy()
            keys.destroy()


def test_fp16_and_compressed_sessions(device, attention_cases, oracle):
    """Phase-3 AttentionSession over FP16Keys and CompressedKeys (materialised FP32 K)."""
    import bgtq
    engine = bgtq.AttentionEngine.create(device)
    for name, m, a, lm, la in attention_cases:
        print("case", name, flush=True)
        T, d = m["context_length"], m["dim"]
        values = bgtq.Values(device, d, T)
        values.append(a["v"])
        fp16 = bgtq.FP16Keys(device, d, T)
        comp = bgtq.CompressedKeys.create(device, _params(lm, la), T)
        try:
            k = a["k"].view(np.uint16)
            for keys in (fp16, comp):
                keys.append(k[:3])
                keys.append(k[3:])
            decoded = comp.prepare()
            np.testing.assert_allclose(decoded, a["reconstructed_k"], atol=2e-6, rtol=2e-6)
            for keys, label, k_eff in ((fp16, "baseline", a["k"].astype(np.float32)), (comp, "compressed", decoded)):
                s = engine.session(keys, values, m["queries"])
                try:
                    for causal in (False, True):
                        prefix = "causal_" if causal else ""
                        out = s.attend(a["q"], a["positions"], causal)
                        ins = s.inspect()
                        ref_l, ref_p, ref_o = oracle.attention(a["q"], k_eff, a["v"], a["positions"], causal)
                        _close(ins["logits"], ref_l, LOGIT_ATOL, LOGIT_RTOL, f"{name} {label} logits")
                        _close(ins["probabilities"], ref_p, PROB_ATOL, PROB_RTOL, f"{name} {label} probs")
                        _close(out, ref_o, ATOL, RTOL, f"{name} {label} output")
                        _close(out, a[prefix + label + "_output"], ATOL, RTOL, f"{name} {label} golden output")
                finally:
                    s.destroy()
        finally:
            fp16.destroy()
            comp.destroy()
            values.destroy()


def test_runtime_contracts(device, attention_cases):
    """tests/webgpu/runtime-contracts.ts:9-29 and optimized-test.ts:58-78."""
    import bgtq
    name, m, a, lm, la = attention_cases[0]
    d = m["dim"]
    k = a["k"].view(np.uint16)
    v = a["v"]
    q = np.zeros(d, np.float32)
    packed = bgtq.PackedKeys.create(device, _params(lm, la), 3)
    stores = [bgtq.FP16Keys(device, d, 3), packed]
    for keys in stores:
        values = bgtq.Values(device, d, 3)
        s = (bgtq.OptimizedAttention.create(device, keys, values, 1) if keys is packed
             else bgtq.AttentionEngine.create(device).session(keys, values, 1))
        try:
            keys.append(k[:1])
            values.append(v[:1])
            out = s.attend(q, [0])
            np.testing.assert_array_equal(out[0], v[0])
            keys.append(k[1:3])
            values.append(v[1:3])
            out = s.attend(q, [2], True)
            np.testing.assert_allclose(out[0], (v[0] + v[1] + v[2]) / 3, atol=1e-6, rtol=1e-6)
            assert keys.length == 3 and values.length == 3
            with pytest.raises(bgtq.RangeError, match="V capacity exceeded"):
                values.append(np.zeros(d, np.float32))
            assert values.length == 3
            with pytest.raises(bgtq.RangeError, match="K capacity exceeded"):
                keys.append(k[:1])
            with pytest.raises(bgtq.RangeError):
                s.setQueries(q, [3])
            with pytest.raises(bgtq.RangeError):
                s.setQueries(np.zeros(d - 1, np.float32), [0])
            bad = q.copy()
            bad[0] = np.nan
            with pytest.raises(bgtq.RangeError, match="finite"):
                s.setQueries(bad, [0])
        finally:
            s.destroy()
            values.destroy()
            keys.destroy()


def test_mismatched_lengths_rejected(device, attention_cases):
    import bgtq
    name, m, a, lm, la = attention_cases[0]
    d = m["dim"]
    keys = bgtq.FP16Keys(device, d, 8)
    values = bgtq.Values(device, d, 8)
    s = bgtq.AttentionEngine.create(device).session(keys, values, 3)
    try:
        keys.append(a["k"].view(np.uint16)[:3])
        with pytest.raises(bgtq.RangeError, match="K/V lengths"):
            s.setQueries(a["q"], a["positions"])
    finally:
        s.destroy()
        values.destroy()
        keys.destroy()


def _bench_workload(T, d):
    """The phase-4 benchmark workload t{T}_d{d} (tests/oracles/export_attention.py:20-26):
    q ~ N(0, 1) [3, d], K = FP16(0.7 N(0, 1)), V = 0.5 N(0, 1) FP32, positions
    (0, T / 2, T - 1), from torch's CPU generator seeded 731 + d + T."""
    import torch
    g = torch.Generator().manual_seed(731 + d + T)
    q = torch.randn(3, d, generator=g)
    k = (torch.randn(T, d, generator=g) * 0.7).half()
    v = torch.randn(T, d, generator=g) * 0.5
    return q.numpy(), k.numpy(), v.numpy(), np.array([0, T // 2, T - 1], np.uint32)


@pytest.mark.parametrize("T", (1024, 2048, 4096))
def test_fp32_values_benchmark_shapes(device, attention_cases, oracle, T):
    """OptimizedAttention over FP32 Values at the benchmark's context lengths
    (benchmarks/phase4.ts:19-47) through the fused kernel's FP32-V variant,
    against the oracle on the reconstructed K, both d, causal and not."""
    import bgtq
    layouts = {m["dim"]: (lm, la) for _, m, _, lm, la in attention_cases}
    for d in (64, 128):
        print("case", T, d, flush=True)
        q, k, v, pos = _bench_workload(T, d)
        lm, la = layouts[d]
        keys = bgtq.PackedKeys.create(device, _params(lm, la), T)
        values = bgtq.Values(device, d, T)
        att = bgtq.OptimizedAttention.create(device, keys, values, 3)
        lean = bgtq.OptimizedAttention.create(device, keys, values, 3, materialize=False)
        try:
            keys.append(k.view(np.uint16))
            values.append(v)
            ol = oracle.Layout.from_mixed_fixture(lm, la)
            packed, norms = keys.read()
            codes = oracle.unpack(packed.reshape(T, -1), d, lm["nopack_start"])
            k_eff = oracle.reconstruct(ol, codes, norms.view(np.float16).reshape(T, -1).astype(np.float32))
            for causal in (False, True):
                ref_l, ref_p, ref_o = oracle.attention(q, k_eff, v, pos, causal)
                out = att.attend(q, pos, causal)
                ins = att.inspect()
                _close(out, ref_o, ATOL, RTOL, f"T{T} d{d} {causal} output")
                _close(ins["logits"], ref_l, LOGIT_ATOL, LOGIT_RTOL, f"T{T} d{d} {causal} logits")
                _close(ins["probabilities"], ref_p, PROB_ATOL, PROB_RTOL, f"T{T} d{d} {causal} probabilities")
                # without materialised intermediates: the same output
                np.testing.assert_array_equal(lean.attend(q, pos, causal), out)
            # The first causal query attends to V0 alone: the FP16 parts of an
            # FP32 value add back to it exactly.
            np.testing.assert_array_equal(att.attend(q, pos, True)[0], v[0])
        finally:
            lean.destroy()
            att.destroy()
            values.destroy()
            keys.destroy()


def test_fp32_values_beyond_fp16_range(device, attention_cases, oracle):
    """FP32 V with a value past FP16's range (|v| >= 65504) cannot be split
    into FP16 parts: the session computes it on the general kernels, with the
    same result bar, and an FP16 K session likewise."""
    import bgtq
    name, m, a, lm, la = next(c for c in attention_cases if c[0] == "t256_d64")
    T, d = m["context_length"], m["dim"]
    v = a["v"].copy()
    v[5, 3] = 1.0e6
    v[17, 0] = -7.0e4
    keys = bgtq.PackedKeys.create(device, _params(lm, la), T)
    fp16 = bgtq.FP16Keys(device, d, T)
    values = bgtq.Values(device, d, T)
    att = bgtq.OptimizedAttention.create(device, keys, values, m["queries"])
    s16 = bgtq.AttentionEngine.create(device).session(fp16, values, m["queries"])
    try:
        keys.append(a["k"].view(np.uint16))
        fp16.append(a["k"].view(np.uint16))
        values.append(v)
        for causal in (False, True):
            _, _, ref_o = oracle.attention(a["q"], a["reconstructed_k"], v, a["positions"], causal)
            _close(att.attend(a["q"], a["positions"], causal), ref_o, ATOL, RTOL, f"large V {causal}")
            _, _, ref16 = oracle.attention(a["q"], a["k"].astype(np.float32), v, a["positions"], causal)
            _close(s16.attend(a["q"], a["positions"], causal), ref16, ATOL, RTOL, f"large V fp16 K {causal}")
    finally:
        s16.destroy()
        att.destroy()
        values.destroy()
        fp16.destroy()
        keys.destroy()


def test_record_with_timestamps(device, attention_cases):
    """record(encoder, timestamps) (src/attention/attention.ts:44-58): the
    begin and end writes bracket the attention work; bad indices are rejected
    before any work is queued."""
    import bgtq
    name, m, a, lm, la = next(c for c in attention_cases if c[0] == "t512_d128")
    T, d = m["context_length"], m["dim"]
    keys = bgtq.PackedKeys.create(device, _params(lm, la), T)
    values = bgtq.Values(device, d, T)
    att = bgtq.OptimizedAttention.create(device, keys, values, m["queries"])
    ts = bgtq.Timestamps(device, 4)
    try:
        keys.append(a["k"].view(np.uint16))
        values.append(a["v"])
        att.setQueries(a["q"], a["positions"], False)
        att.record(ts, 0, 1)
        att.record(ts, 2, 3)
        ns = ts.resolve()
        assert 0 < ns[1] - ns[0] < 10_000_000 and ns[2] >= ns[1] and ns[3] > ns[2]
        _close(att.read("output"), a["compressed_output"], ATOL, RTOL, "timed record output")
        with pytest.raises(bgtq.RangeError, match="timestamp"):
            att.record(ts, 0, 4)
    finally:
        ts.destroy()
        att.destroy()
        values.destroy()
        keys.destroy()
