"""Pins the CPU oracle before it is trusted as the checker.

Every oracle function is checked against the reference's committed goldens
(tests/golden/reference, copied data), against torch itself where the
reference's arithmetic is a torch routine, and against closed forms, so that
a plausible mistake (a reduction tree of the wrong width, a non-fused dot, a
wrong clamp or rounding rule) fails here.
"""
import json
import os
import subprocess
import sys

import numpy as np
import pytest

from conftest import REF, ROOT


def _bits(x):
    return np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)


def test_mixed_encoder_bit_exact(mixed_cases, oracle):
    """tests/test_mixed.py:51-57 restated: codes, raw and corrected norms, and the rotated y."""
    for name, m, a in mixed_cases:
        L = oracle.Layout.from_mixed_fixture(m, a)
        codes, raw, corr, y = oracle.encode(L, a["original"])
        ng = m["n_groups"]
        np.testing.assert_array_equal(codes, a["codes"], err_msg=name)
        np.testing.assert_array_equal(_bits(raw), _bits(a["raw_norms"][:, :ng]), err_msg=name)
        np.testing.assert_array_equal(_bits(corr), _bits(a["corrected_f32"][:, :ng]), err_msg=name)
        np.testing.assert_array_equal(_bits(y), _bits(a["rotated"]), err_msg=name)


def test_wrong_reduction_orders_are_caught(mixed_cases, oracle):
    """The goldens discriminate: a 16-lane sum tree or an unfused/reversed dot fails."""
    for profile in ((16, 0), (8, 1), (8, 2)):
        failures = 0
        for name, m, a in mixed_cases:
            L = oracle.Layout.from_mixed_fixture(m, a)
            codes, raw, corr, y = oracle.encode(L, a["original"], profile)
            ng = m["n_groups"]
            failures += int(not np.array_equal(_bits(y), _bits(a["rotated"]))
                            or not np.array_equal(_bits(raw), _bits(a["raw_norms"][:, :ng])))
        assert failures > 0, profile


def test_pack_unpack_and_padding(mixed_cases, oracle):
    """tests/test_mixed.py:38-49: exact bytes, round trip, zero padding, >15 byte codes."""
    for name, m, a in mixed_cases:
        packed = oracle.pack(a["codes"], m["nopack_start"], m["row_bytes"])
        np.testing.assert_array_equal(packed, a["packed"], err_msg=name)
        np.testing.assert_array_equal(oracle.unpack(packed, m["dim"], m["nopack_start"]), a["codes"])
        assert not a["packed"][:, m["logical_row_bytes"]:].any()
        if name == "awkward_all_widths":
            assert np.any(a["codes"][:, m["nopack_start"]:] > 15)


def test_encode_pack_matches_attention_fixture_rows(attention_cases, oracle):
    """1,792 reference-encoded rows: packed_k and FP16 scales (export_attention.py:27-31)."""
    for name, m, a, lm, la in attention_cases:
        L = oracle.Layout.from_mixed_fixture(lm, la)
        packed, norms = oracle.encode_pack(L, a["k"].view(np.uint16))
        np.testing.assert_array_equal(packed, a["packed_k"], err_msg=name)
        np.testing.assert_array_equal(norms, a["norms"].view(np.uint16), err_msg=name)


def test_half_conversion(mixed_cases, oracle):
    """tests/test_mixed.py:66-79: edge probes, fixture scale bits, numpy IEEE RNE."""
    probes = np.array([0, -0.0, 2 ** -24, 2 ** -25, 3 * 2 ** -25, 1 + 2 ** -11, 65504, 65520], np.float32)
    np.testing.assert_array_equal(oracle.f32_to_f16_bits(probes), [0, 32768, 1, 0, 2, 15360, 31743, 31744])
    for name, m, a in mixed_cases:
        np.testing.assert_array_equal(oracle.f32_to_f16_bits(a["corrected_f32"]).reshape(a["norm_bits"].shape),
                                      a["norm_bits"])
    rng = np.random.default_rng(0)
    # every FP16 value, and the midpoints and neighbours around it
    h = np.arange(0, 0x7C00, dtype=np.uint16).view(np.float16).astype(np.float32)
    mids = ((h[:-1].astype(np.float64) + h[1:]) / 2).astype(np.float32)
    x = np.concatenate([h, -h, mids, -mids, np.nextafter(mids, np.float32(np.inf)),
                        np.nextafter(mids, np.float32(-np.inf)), rng.standard_normal(20000).astype(np.float32) * 1e4])
    with np.errstate(over="ignore"):
        np.testing.assert_array_equal(oracle.f32_to_f16_bits(x), x.astype(np.float16).view(np.uint16))


def test_reconstruct(mixed_cases, attention_cases, oracle):
    """production_math.py:27-31 vs the goldens (fixture tolerance atol 1e-3, rtol 2e-5)."""
    for name, m, a in mixed_cases:
        L = oracle.Layout.from_mixed_fixture(m, a)
        for key, scales in (("reconstructed_f32", a["corrected_f32"]),
                            ("reconstructed_f16", a["persistent_norms"].astype(np.float32))):
            r = oracle.reconstruct(L, a["codes"], scales)
            np.testing.assert_allclose(r, a[key], atol=1e-3, rtol=2e-5, err_msg=name)
    for name, m, a, lm, la in attention_cases:
        L = oracle.Layout.from_mixed_fixture(lm, la)
        T, d = m["context_length"], m["dim"]
        codes = oracle.unpack(a["packed_k"], d, lm["nopack_start"])
        r = oracle.reconstruct(L, codes, a["norms"].astype(np.float32))
        np.testing.assert_allclose(r, a["reconstructed_k"], atol=2e-6, rtol=2e-6, err_msg=name)


@pytest.mark.parametrize("fp32", [False, True])
def test_attention_against_goldens_and_closed_forms(attention_cases, oracle, fp32):
    """tests/test_attention.py:15-46: goldens within the fixture baseline tolerances, for the
    float64-accumulating oracle and its FP32 restatement (the CPU baseline's arithmetic)."""
    for name, m, a, lm, la in attention_cases:
        tol = m["tolerances"]["baseline"]
        for causal in (False, True):
            prefix = "causal_" if causal else ""
            for label, keys in (("baseline", a["k"].astype(np.float32)), ("compressed", a["reconstructed_k"]),
                                ("fp32_source", a["k_source"])):
                res = oracle.attention(a["q"], keys, a["v"], a["positions"], causal, fp32=fp32)
                for kind, got in zip(("logits", "probabilities", "output"), res):
                    exp = a[prefix + label + "_" + kind]
                    fin = np.isfinite(exp)
                    assert np.array_equal(np.isneginf(got), np.isneginf(exp))
                    np.testing.assert_allclose(got[fin], exp[fin], atol=tol[kind][0], rtol=tol[kind][1],
                                               err_msg=f"{name} {label} {kind}")
                probs, out = res[1], res[2]
                np.testing.assert_allclose(probs.sum(1), 1.0, atol=1e-6)
                if causal:
                    np.testing.assert_array_equal(out[0], a["v"][0])
    # hand-computable cases (tests/test_attention.py:39-46)
    k = np.array([[1., 2.], [3., 4.]], np.float32)
    v = np.array([[2., 4.], [6., 8.]], np.float32)
    _, p, o = oracle.attention(np.zeros((1, 2), np.float32), k, v, [1])
    np.testing.assert_array_equal(p, [[.5, .5]])
    np.testing.assert_array_equal(o, [[4., 6.]])
    _, p, o = oracle.attention(np.full((1, 2), 100., np.float32), k, v, [1])
    assert np.isfinite(o).all() and abs(p.sum() - 1) < 1e-6
    with pytest.raises(ValueError):
        oracle.attention(np.zeros((1, 64), np.float32), np.zeros((4, 64), np.float32), np.zeros((4, 64), np.float32), [4])
    q = np.zeros((1, 64), np.float32)
    q[0, 0] = np.nan
    with pytest.raises(ValueError):
        oracle.attention(q, np.zeros((4, 64), np.float32), np.zeros((4, 64), np.float32), [0])


def test_attention_matches_float64_softmax(oracle):
    rng = np.random.default_rng(3)
    q = rng.standard_normal((4, 32)).astype(np.float32)
    k = rng.standard_normal((300, 32)).astype(np.float32)
    v = rng.standard_normal((300, 32)).astype(np.float32)
    pos = np.array([0, 7, 150, 299])
    l, p, o = oracle.attention(q, k, v, pos, causal=True)
    L = q.astype(np.float64) @ k.T.astype(np.float64) / np.sqrt(32)
    L[np.arange(300)[None, :] > pos[:, None]] = -np.inf
    P = np.exp(L - L.max(1, keepdims=True))
    P /= P.sum(1, keepdims=True)
    np.testing.assert_allclose(p, P, rtol=1e-6, atol=1e-9)
    np.testing.assert_allclose(o, P @ v.astype(np.float64), rtol=1e-6, atol=1e-7)


def test_allocator(oracle):
    """fixtures/allocator.json (13 upstream cases), the mixed layouts, and the 90 real SmolLM2 heads."""
    fx = json.loads((REF / "allocator.json").read_text())
    for c in fx["cases"]:
        got = oracle.allocate_bits(c["scores"], c["budget"], c["min_bits"], c["max_bits"])
        np.testing.assert_array_equal(got, c["expected"], err_msg=c["name"])
    for name in json.loads((REF / "mixed" / "index.json").read_text())["cases"]:
        m, a = oracle.read_fixture(REF / "mixed" / f"{name['name']}.json")
        np.testing.assert_array_equal(oracle.allocate_bits(a["scores"], m["requested_budget"]), a["allocation"])
    m, a = oracle.read_fixture(REF / "model" / "calibration.json")
    for i in range(len(m["heads"])):
        got = oracle.allocate_bits(a[f"h{i}_scores"], 128, 1, 8)  # calibrate_model.py:33
        np.testing.assert_array_equal(got, a[f"h{i}_widths"], err_msg=f"head {i}")


def test_allocator_small_grid_properties(oracle):
    """tests/test_allocator.py:24-31's grid: totals, bounds and the greedy's exchange property."""
    import itertools
    for scores in itertools.product((0, 1, 4), repeat=3):
        for budget in range(0, 14):
            w = oracle.allocate_bits(scores, budget, 1, 4)
            assert np.all((w >= 1) & (w <= 4))
            s = np.asarray(scores, np.float64)
            if any(scores):
                assert w.sum() == min(max(budget, 3), sum(4 if x > 0 else 1 for x in scores)) or w.sum() == max(budget, 3)
            else:
                assert w.sum() == 3
            # no single move of one bit between pairs would raise the greedy priority order
            pri = s * 4.0 ** -w.astype(np.float64)
            for i in range(3):
                for j in range(3):
                    if i != j and w[i] < 4 and w[j] > 1 and s[j] > 0:
                        assert s[i] * 4.0 ** -(w[i]) <= s[j] * 4.0 ** -(w[j] - 1) + 1e-12


_TORCH_PROBE = r"""
import sys, numpy as np, torch
sys.path.insert(0, sys.argv[1])
from oracle import oracle as O
torch.set_num_threads(1)
assert torch.backends.cpu.get_cpu_capability() == "AVX2", torch.backends.cpu.get_cpu_capability()
rng = np.random.default_rng(11)
bad = 0
for n in list(range(1, 260)) + [511, 512, 1000, 2048, 4100]:
    x = (rng.standard_normal(n) * np.exp(rng.standard_normal(n) * 3)).astype(np.float32)
    t = torch.from_numpy(x)[None, :].sum(1).numpy()[0]
    bad += int(np.float32(t).view(np.uint32) != np.float32(O.aten_sum(x, 8)).view(np.uint32))
gbad = 0
for d in (16, 32, 64, 128):
    for n in (5, 16, 64):
        A = rng.standard_normal((n, d)).astype(np.float32); B = rng.standard_normal((d, d)).astype(np.float32)
        y = (torch.from_numpy(A) @ torch.from_numpy(B).T.contiguous()).numpy()
        gbad += int((y.view(np.uint32) != O.gemm_abt(A, B, 0).view(np.uint32)).sum())
print(bad, gbad)
"""


def test_reduction_orders_match_torch_avx2(oracle):
    """The oracle's sum tree and dot order are torch's own on an AVX2 CPU (this image's torch, forced to AVX2)."""
    env = dict(os.environ, ATEN_CPU_CAPABILITY="avx2", MKL_CBWR="AVX2", OMP_NUM_THREADS="1")
    r = subprocess.run([sys.executable, "-c", _TORCH_PROBE, str(ROOT)], env=env, capture_output=True, text=True,
                       timeout=300)
    if r.returncode != 0 and "AVX2" in r.stderr and "assert" in r.stderr.lower():
        pytest.skip("this CPU cannot run ATen's AVX2 kernels")
    assert r.returncode == 0, r.stderr[-2000:]
    assert r.stdout.split() == ["0", "0"], r.stdout
