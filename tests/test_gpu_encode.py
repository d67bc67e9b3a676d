"""K encode on the GPU: bit-exact against the reference goldens and the oracle.

Mirrors the checks of the reference's tests/test_mixed.py:38-64 (exact
packed bytes and scale bits) and tests/webgpu/optimized-test.ts:23-27 (an odd
append boundary, packed/norm buffers read back raw), through the C ABI.
"""
import json

import numpy as np
import pytest

from conftest import REF

pytestmark = pytest.mark.gpu


def _params(m, a):
    import bgtq
    return bgtq.BlockGTQParameters.from_mixed_fixture(m, a)


def _olayout(oracle, p):
    return oracle.Layout(dim=p.dim, groups=p.groups, row_bytes=p.rowBytes, norm_stride=p.normStride,
                         nibble_dims=p.nibbleDims, max_centroids=p.maxCentroids, perm=p.permutation,
                         group_of=p.groupOf, pos_to_cb=p.positionToCodebook, code_lut=p.codeLut,
                         rotation=p.rotation, centroids=p.centroids, offsets=p.offsets, inv_scales=p.inverseScales)


def test_mixed_fixture_rows_exact(device, mixed_cases):
    import bgtq
    for name, m, a in mixed_cases:
        print("case", name, flush=True)
        keys = bgtq.PackedKeys.create(device, _params(m, a), m["capacity"])
        try:
            x = a["original"].astype(np.float16).view(np.uint16)
            assert np.array_equal(x.view(np.float16).astype(np.float32), a["original"])
            keys.append(x[:2])
            keys.append(x[2:])
            packed, norms = keys.read()
            np.testing.assert_array_equal(packed, a["cache_packed"].reshape(-1), err_msg=name)
            np.testing.assert_array_equal(norms, a["cache_norms"].view(np.uint16).reshape(-1), err_msg=name)
            assert keys.length == m["rows"]
        finally:
            keys.destroy()


def test_attention_fixture_rows_exact(device, attention_cases):
    import bgtq
    for name, m, a, lm, la in attention_cases:
        print("case", name, flush=True)
        keys = bgtq.PackedKeys.create(device, _params(lm, la), m["context_length"])
        try:
            k = a["k"].view(np.uint16)
            keys.append(k[:3])  # odd row boundary shares packed words with the next append
            keys.append(k[3:])
            packed, norms = keys.read()
            np.testing.assert_array_equal(packed.reshape(a["packed_k"].shape), a["packed_k"], err_msg=name)
            np.testing.assert_array_equal(norms.reshape(a["norms"].shape), a["norms"].view(np.uint16), err_msg=name)
        finally:
            keys.destroy()


def _random_half_rows(rng, rows, dim):
    """FP16 K rows with mixed magnitudes: normal, tiny, subnormal, large, zeros, duplicates."""
    x = rng.standard_normal((rows, dim)).astype(np.float32)
    scale = np.exp(rng.uniform(-12, 8, size=(rows, 1))).astype(np.float32)
    x = (x * scale).clip(-60000, 60000)
    x[rng.random(rows) < 0.02] = 0.0
    x[rng.random((rows, dim)) < 0.01] = 0.0
    sub = rng.random(rows) < 0.01
    x[sub] = rng.integers(-1023, 1024, size=(int(sub.sum()), dim)).astype(np.float32) * 2.0 ** -24
    h = x.astype(np.float16)
    return h.view(np.uint16)


def _layouts(oracle):
    from bgtq import BlockGTQParameters
    out = []
    for name in ("low_d16", "mixed_d32", "mixed_d64", "low_d128", "mixed_d128", "awkward_all_widths", "only_high"):
        m, a = oracle.read_fixture(REF / "mixed" / f"{name}.json")
        out.append((name, BlockGTQParameters.from_mixed_fixture(m, a)))
    m, a = oracle.read_fixture(REF / "model" / "calibration.json")
    for i in (0, 1, 17, 89):
        out.append((f"smollm2_h{i}", BlockGTQParameters.from_serialized(a[f"h{i}_config"], a[f"h{i}_table"])))
    return out


def test_random_rows_bit_exact_vs_oracle(device, oracle):
    import bgtq
    rng = np.random.default_rng(2024)
    for name, p in _layouts(oracle):
        print("layout", name, flush=True)
        rows = 6000
        k = _random_half_rows(rng, rows, p.dim)
        ol = _olayout(oracle, p)
        ref_packed, ref_norms = oracle.encode_pack(ol, k)
        keys = bgtq.PackedKeys.create(device, p, rows + 5)
        try:
            cuts = [0, 1, 130, 257, 3000, rows]  # ragged appends
            for a, b in zip(cuts[:-1], cuts[1:]):
                keys.append(k[a:b])
            packed, norms = keys.read()
            packed = packed[: rows * p.rowBytes].reshape(rows, p.rowBytes)
            norms = norms[: rows * p.normStride].reshape(rows, p.normStride)
            bad = np.nonzero(np.any(packed != ref_packed, axis=1) | np.any(norms != ref_norms, axis=1))[0]
            assert bad.size == 0, f"{name}: {bad.size} rows differ, first {bad[:5]}"
        finally:
            keys.destroy()


def test_batched_encode_fp32_source_rounds_to_half(device, oracle):
    """Model path: FP32 post-RoPE rows [rows, kv_heads, dim], rounded to FP16 first (src/model/codec.wgsl:14)."""
    import torch
    import bgtq
    from bgtq import batched
    p = _layouts(oracle)[9][1]  # a real SmolLM2 head, d = 64
    tables = bgtq.Tables(device, p)
    rng = np.random.default_rng(7)
    rows, kvh = 1000, 3
    kr = (rng.standard_normal((rows, kvh, 64)) * 1.7).astype(np.float32)
    src = torch.from_numpy(kr).cuda()
    packed = torch.zeros((kvh, rows + 4, p.rowBytes), dtype=torch.uint8, device="cuda")
    norms = torch.zeros((kvh, rows + 4, p.normStride), dtype=torch.int16, device="cuda")
    jobs = [dict(tables=tables, src=src[:, h], src_row_stride=kvh * 64, rows=rows, packed=packed[h],
                 norms=norms[h], dst_row0=2) for h in range(kvh)]
    batched.encode(device, jobs, "f32")
    device.synchronize()
    ol = _olayout(oracle, p)
    for h in range(kvh):
        ref_p, ref_n = oracle.encode_pack(ol, kr[:, h].astype(np.float16).view(np.uint16))
        got_p = packed[h].cpu().numpy()
        got_n = norms[h].cpu().numpy().view(np.uint16)
        np.testing.assert_array_equal(got_p[2:2 + rows], ref_p)
        np.testing.assert_array_equal(got_n[2:2 + rows], ref_n)
        assert not got_p[:2].any() and not got_p[2 + rows:].any()
    tables.destroy()


def test_append_contracts(device, attention_cases):
    """appendCount and PackedKeys constructor rejections; failed calls leave state unchanged."""
    import bgtq
    name, m, a, lm, la = attention_cases[0]
    p = _params(lm, la)
    keys = bgtq.PackedKeys.create(device, p, 3)
    try:
        k = a["k"].view(np.uint16)
        with pytest.raises(bgtq.RangeError, match="whole nonempty rows"):
            keys.append(k[0, :5])
        with pytest.raises(bgtq.RangeError, match="whole nonempty rows"):
            keys.append(np.zeros(0, np.uint16))
        bad = k[:1].copy()
        bad[0, 3] = 0x7C00
        with pytest.raises(bgtq.RangeError, match="Finite FP16 K required"):
            keys.append(bad)
        with pytest.raises(bgtq.StateError, match="not ready"):
            keys.ready()
        keys.append(k[:3])
        with pytest.raises(bgtq.RangeError, match="K capacity exceeded"):
            keys.append(k[3:4])
        assert keys.length == 3
        keys.ready()
    finally:
        keys.destroy()
    changed = _params(lm, la)
    changed.rotation = changed.rotation.copy()
    grp = np.asarray(changed.groupOf)
    other = int(np.nonzero(grp != grp[0])[0][0])
    changed.rotation.reshape(p.dim, p.dim)[other, 0] = 0.01
    with pytest.raises(bgtq.StateError, match="Off-group transform is nonzero"):
        bgtq.PackedKeys.create(device, changed, 3)


def test_bulk_encode_bit_exact(device, oracle):
    """A launch of at least 16384 rows takes the thread-per-row encoder (smaller
    launches the wave-per-row one); both must give the oracle's bytes."""
    import torch
    import bgtq
    from bgtq import batched
    rng = np.random.default_rng(99)
    layouts = _layouts(oracle)
    for name, p in [layouts[i] for i in (0, 3, 9)]:
        print("bulk layout", name, flush=True)
        rows = 20000
        k = _random_half_rows(rng, rows, p.dim)
        ref_p, ref_n = oracle.encode_pack(_olayout(oracle, p), k)
        tables = bgtq.Tables(device, p)
        src = torch.from_numpy(k.view(np.int16)).cuda()
        packed = torch.zeros((rows, p.rowBytes), dtype=torch.uint8, device="cuda")
        norms = torch.zeros((rows, p.normStride), dtype=torch.int16, device="cuda")
        batched.encode(device, [dict(tables=tables, src=src, src_row_stride=p.dim, rows=rows, packed=packed,
                                     norms=norms)], "f16")
        device.synchronize()
        got_p, got_n = packed.cpu().numpy(), norms.cpu().numpy().view(np.uint16)
        bad = np.nonzero(np.any(got_p != ref_p, axis=1) | np.any(got_n != ref_n, axis=1))[0]
        assert bad.size == 0, f"{name}: {bad.size} rows differ, first {bad[:5]}"
        tables.destroy()


def test_bulk_layout_b_encoder_bit_exact(device, oracle):
    """Layout B tables (two equal groups, nibbles first) take the bulk encoder with the layout's structure
    compiled in: FP16 and FP32 sources, interleaved heads (row stride above dim), an offset destination,
    a launch that also carries a job of another layout kind, and at d=64 a launch large enough for
    the wide (256-row) workgroups."""
    import torch
    import bgtq
    from bgtq import batched, calibrate
    rng = np.random.default_rng(123)
    other = _layouts(oracle)[2][1]  # mixed_d64: the generic encoder in the same call
    for dim in (64, 128):
        p = calibrate.layout_b(dim)
        print("bulk layout B", dim, flush=True)
        rows, heads, row0 = (90000 if dim == 64 else 20000), 3, 5
        k = _random_half_rows(rng, rows * heads, dim).reshape(rows, heads, dim)
        tables = bgtq.Tables(device, p)
        t_other = bgtq.Tables(device, other) if dim == 64 else None
        try:
            for src_kind in ("f16", "f32"):
                if src_kind == "f16":
                    src = torch.from_numpy(k.view(np.int16)).cuda()
                else:
                    src = torch.from_numpy(k.view(np.float16).astype(np.float32)).cuda()
                packed = torch.zeros((heads, row0 + rows, p.rowBytes), dtype=torch.uint8, device="cuda")
                norms = torch.zeros((heads, row0 + rows, p.normStride), dtype=torch.int16, device="cuda")
                jobs = [dict(tables=tables, src=src[:, h], src_row_stride=heads * dim, rows=rows, packed=packed[h],
                             norms=norms[h], dst_row0=row0) for h in range(heads)]
                if t_other is not None:
                    po = torch.zeros((rows, other.rowBytes), dtype=torch.uint8, device="cuda")
                    no = torch.zeros((rows, other.normStride), dtype=torch.int16, device="cuda")
                    jobs.append(dict(tables=t_other, src=src[:, 0], src_row_stride=heads * dim, rows=rows, packed=po,
                                     norms=no))
                batched.encode(device, jobs, src_kind)
                device.synchronize()
                for h in range(heads):
                    ref_p, ref_n = oracle.encode_pack(_olayout(oracle, p), np.ascontiguousarray(k[:, h]))
                    got_p = packed[h].cpu().numpy()
                    got_n = norms[h].cpu().numpy().view(np.uint16)
                    assert not got_p[:row0].any() and not got_n[:row0].any(), "rows before dst_row0 written"
                    bad = np.nonzero(np.any(got_p[row0:] != ref_p, axis=1) | np.any(got_n[row0:] != ref_n, axis=1))[0]
                    assert bad.size == 0, f"d={dim} {src_kind} head {h}: {bad.size} rows differ, first {bad[:5]}"
                if t_other is not None:
                    ref_p, ref_n = oracle.encode_pack(_olayout(oracle, other), np.ascontiguousarray(k[:, 0]))
                    assert np.array_equal(po.cpu().numpy(), ref_p)
                    assert np.array_equal(no.cpu().numpy().view(np.uint16), ref_n)
        finally:
            tables.destroy()
            if t_other is not None:
                t_other.destroy()


def test_bulk_encoder_unaligned_source(device, oracle):
    """The bulk encoder stages rows as 16-byte pieces when the source and its row stride allow it; a
    source starting one element past a 16-byte boundary with an odd row stride takes its element-wise
    staging, FP16 and FP32, over a partial last workgroup of rows."""
    import torch
    import bgtq
    from bgtq import batched, calibrate
    rng = np.random.default_rng(321)
    dim, rows = 64, 1000
    stride = dim + 1
    p = calibrate.layout_b(dim)
    k = _random_half_rows(rng, rows, dim)
    tables = bgtq.Tables(device, p)
    try:
        ref_p, ref_n = oracle.encode_pack(_olayout(oracle, p), np.ascontiguousarray(k))
        for src_kind in ("f16", "f32"):
            flat = np.zeros(1 + rows * stride, dtype=np.float16)
            flat[1:].reshape(rows, stride)[:, :dim] = k.view(np.float16)
            src = torch.from_numpy(flat.view(np.int16) if src_kind == "f16" else flat.astype(np.float32)).cuda()
            packed = torch.zeros((rows, p.rowBytes), dtype=torch.uint8, device="cuda")
            norms = torch.zeros((rows, p.normStride), dtype=torch.int16, device="cuda")
            batched.encode(device, [dict(tables=tables, src=src[1:], src_row_stride=stride, rows=rows, packed=packed,
                                         norms=norms, dst_row0=0)], src_kind)
            device.synchronize()
            assert np.array_equal(packed.cpu().numpy(), ref_p), src_kind
            assert np.array_equal(norms.cpu().numpy().view(np.uint16), ref_n), src_kind
    finally:
        tables.destroy()


def test_calibration_load_encodes_every_head(device, oracle):
    """Calibration.load (src/model/calibration.ts:7-21) puts the 90 SmolLM2 heads on the device;
    each head's tables then encode its KV head's post-RoPE rows bit for bit as the oracle does
    with the same blob (the reference's tests/webgpu/model-codec-test.ts:13-21 on 3 rows per
    head; here 37 rows, FP32 model-path source)."""
    import torch
    import bgtq
    from bgtq import batched
    cal = bgtq.Calibration.load(device, REF / "model")
    try:
        assert len(cal.heads) == 90 and len(cal.allocations) == 90
        assert all(x["bytes"] > 0 for x in cal.allocations)
        m, a = oracle.read_fixture(REF / "model" / "calibration.json")
        rng = np.random.default_rng(90)
        rows, kvh = 37, 3
        kr = (rng.standard_normal((rows, kvh, 64)) * 2.3).astype(np.float32)
        src = torch.from_numpy(kr).cuda()
        outs, jobs = [], []
        for h, head in enumerate(cal.heads):
            p = bgtq.BlockGTQParameters.from_serialized(a[f"h{h}_config"], a[f"h{h}_table"])
            info = head.tables.info
            assert (info["dim"], info["groups"], info["row_bytes"], info["norm_stride"]) == \
                (64, p.groups, p.rowBytes, p.normStride) == (64, p.groups, head.row_bytes, head.norm_stride)
            packed = torch.zeros((rows, p.rowBytes), dtype=torch.uint8, device="cuda")
            norms = torch.zeros((rows, p.normStride), dtype=torch.int16, device="cuda")
            outs.append((p, packed, norms))
            jobs.append(dict(tables=head.tables, src=src[:, h % kvh], src_row_stride=kvh * 64, rows=rows,
                             packed=packed, norms=norms, dst_row0=0))
        batched.encode(device, jobs, "f32")
        device.synchronize()
        for h, (p, packed, norms) in enumerate(outs):
            ref_p, ref_n = oracle.encode_pack(_olayout(oracle, p), kr[:, h % kvh].astype(np.float16).view(np.uint16))
            np.testing.assert_array_equal(packed.cpu().numpy(), ref_p, err_msg=f"head {h}")
            np.testing.assert_array_equal(norms.cpu().numpy().view(np.uint16), ref_n, err_msg=f"head {h}")
    finally:
        cal.destroy()


def test_job_table_batches_and_stream_switch(device, oracle):
    """More jobs in one call than the context's device job table holds (4100 jobs of 4 rows: two table
    batches, each uploaded in chunks of 60), then, without waiting, a second call on another stream that
    rewrites the table: both calls give the oracle's bytes."""
    import torch
    import bgtq
    from bgtq import batched, calibrate
    rng = np.random.default_rng(321)
    p = calibrate.layout_b(64)
    n_a, rows_a = 4100, 4
    n_b, rows_b = 90, 200
    ka = _random_half_rows(rng, n_a * rows_a, 64)
    kb = _random_half_rows(rng, n_b * rows_b, 64)
    tables = bgtq.Tables(device, p)
    side_a, side_b = torch.cuda.Stream(), torch.cuda.Stream()
    try:
        bufs = []
        for k in (ka, kb):
            src = torch.from_numpy(k.view(np.int16)).cuda()
            packed = torch.zeros((k.shape[0], p.rowBytes), dtype=torch.uint8, device="cuda")
            norms = torch.zeros((k.shape[0], p.normStride), dtype=torch.int16, device="cuda")
            bufs.append((src, packed, norms))
        torch.cuda.synchronize()

        def jobs(buf, n, rows):
            src, packed, norms = buf
            return [dict(tables=tables, src=src[i * rows:], src_row_stride=64, rows=rows,
                         packed=packed[i * rows:], norms=norms[i * rows:]) for i in range(n)]

        device.set_stream(side_a.cuda_stream)
        batched.encode(device, jobs(bufs[0], n_a, rows_a), "f16")
        device.set_stream(side_b.cuda_stream)
        batched.encode(device, jobs(bufs[1], n_b, rows_b), "f16")
        torch.cuda.synchronize()
        for name, k, (_, packed, norms) in (("table batches", ka, bufs[0]), ("second stream", kb, bufs[1])):
            ref_p, ref_n = oracle.encode_pack(_olayout(oracle, p), k)
            got_p, got_n = packed.cpu().numpy(), norms.cpu().numpy().view(np.uint16)
            bad = np.nonzero(np.any(got_p != ref_p, axis=1) | np.any(got_n != ref_n, axis=1))[0]
            assert bad.size == 0, f"{name}: {bad.size} rows differ, first {bad[:5]}"
    finally:
        device.set_stream(None)
        torch.cuda.synchronize()
        tables.destroy()


def test_concurrent_appends_near_capacity(device, oracle):
    """Two threads append at once near the end of a store's capacity (the Node addon runs appends off
    the JS thread). The store is claimed before the capacity check, as the reference refuses a second
    append while one is in flight (src/runtime/packed-keys.ts:40-49): each append either completes or
    is refused ("Concurrent K appends unsupported" while the other runs, "K capacity exceeded" after
    it committed), never both complete, the length counts the completed rows, and the committed rows
    are the oracle's encode of the base rows and the winning append."""
    import threading
    import bgtq
    from bgtq import calibrate
    p = calibrate.layout_b(64)
    ol = _olayout(oracle, p)
    rng = np.random.default_rng(77)
    cap, base_rows, add = 96, 80, 12
    outcomes = set()
    for trial in range(24):
        keys = bgtq.PackedKeys.create(device, p, cap)
        try:
            base = _random_half_rows(rng, base_rows, 64)
            keys.append(base)
            batches = [_random_half_rows(rng, add, 64) for _ in range(2)]
            results = [None, None]
            gate = threading.Barrier(2)

            def run(i):
                gate.wait()
                try:
                    keys.append(batches[i])
                    results[i] = "ok"
                except (bgtq.StateError, bgtq.RangeError) as e:
                    results[i] = str(e)

            threads = [threading.Thread(target=run, args=(i,)) for i in range(2)]
            for t in threads:
                t.start()
            for t in threads:
                t.join()
            assert results.count("ok") == 1, results
            for r in results:
                assert r in ("ok", "Concurrent K appends unsupported", "K capacity exceeded"), r
            outcomes.add(tuple(sorted(results)))
            winner = results.index("ok")
            assert keys.length == base_rows + add
            rows = base_rows + add
            ref_p, ref_n = oracle.encode_pack(ol, np.concatenate([base, batches[winner]]))
            packed, norms = keys.read()
            np.testing.assert_array_equal(packed[: rows * p.rowBytes].reshape(rows, -1), ref_p)
            np.testing.assert_array_equal(norms[: rows * p.normStride].reshape(rows, -1), ref_n)
            assert not packed[rows * p.rowBytes:].any(), "rows past the length were written"
            with pytest.raises(bgtq.RangeError, match="K capacity exceeded"):
                keys.append(batches[1 - winner])
        finally:
            keys.destroy()
    print("outcomes", sorted(outcomes), flush=True)
