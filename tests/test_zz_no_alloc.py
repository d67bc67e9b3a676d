"""bgtq_decode_noalloc (the decode with the library's own device scratch, no allocation) against
bgtq_decode with a caller workspace, through the C ABI: identical outputs on two calls in a row,
the second with a smaller input, on the fused kernel (packed layout B, FP16 K) and the general
kernel (FP32 V); launches whose workspace exceeds the scratch are refused before anything is
queued."""
import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _case(device, *, batch, hkv, hq, dim, T, key_format, v_dtype, seed, splits=0):
    import torch
    import bgtq
    from bgtq import batched, calibrate
    g = torch.Generator().manual_seed(seed)
    k = torch.randn((batch, hkv, T, dim), generator=g).half().cuda()
    v = torch.randn((batch, hkv, T, dim), generator=g)
    v = (v.half() if v_dtype == "f16" else v.half().float()).cuda()
    q = torch.randn((batch, hq, dim), generator=g).cuda()
    lengths = torch.randint(1, T + 1, (batch,), generator=g, dtype=torch.int32)
    lengths[0] = T
    keep, tabs = [k, v, q], []
    if key_format == "packed":
        p = calibrate.layout_b(dim)
        tabs = [bgtq.Tables(device, p) for _ in range(hkv)]
        packed = torch.zeros((batch, hkv, (T * p.rowBytes + 64 + 15) // 16 * 16), dtype=torch.uint8, device="cuda")
        norms = torch.zeros((batch, hkv, (T * p.normStride + 32 + 7) // 8 * 8), dtype=torch.int16, device="cuda")
        batched.encode(device, [dict(tables=tabs[h], src=k[b, h], src_row_stride=dim, rows=T, packed=packed[b, h],
                                     norms=norms[b, h]) for b in range(batch) for h in range(hkv)], "f16")
        kw = dict(tables=tabs, packed=packed, packed_seq_stride=packed.stride(0), packed_head_stride=packed.stride(1),
                  norms=norms, norms_seq_stride=norms.stride(0), norms_head_stride=norms.stride(1))
        keep += [packed, norms]
    else:
        kw = dict(k_f16=k, k_seq_stride=k.stride(0), k_head_stride=k.stride(1))
    ld = lengths.cuda()
    keep.append(ld)
    return dict(batch=batch, q_heads=hq, kv_heads=hkv, dim=dim, q=q, lengths=ld, max_length=T, v=v, v_dtype=v_dtype,
                v_seq_stride=v.stride(0), v_head_stride=v.stride(1), splits=splits, **kw), keep, tabs


def _both(device, args):
    """Outputs of bgtq_decode (fresh zeroed workspace) and of bgtq_decode_noalloc on the same inputs."""
    import torch
    from bgtq import _lib, batched
    outs = []
    for mode in ("workspace", "noalloc"):
        out = torch.full((args["batch"], args["q_heads"], args["dim"]), float("nan"), device="cuda")
        if mode == "workspace":
            ws = torch.zeros(batched.workspace_bytes(batched.decode_desc(out=out, **args)), dtype=torch.uint8,
                             device="cuda")
            torch.cuda.synchronize()  # torch's fills land before the library's stream reads
            batched.decode(device, batched.decode_desc(out=out, workspace=ws, **args))
        else:
            torch.cuda.synchronize()
            desc = batched.decode_desc(out=out, **args)  # no workspace in the descriptor
            assert desc.workspace is None and desc.workspace_bytes == 0
            _lib.check(_lib.lib().bgtq_decode_noalloc(device.handle, ctypes.byref(desc)))
        torch.cuda.synchronize()
        outs.append(out.cpu().numpy())
    return outs


@pytest.mark.parametrize("key_format,v_dtype,dim", [("packed", "f16", 64), ("fp16", "f16", 128),
                                                    ("packed", "f32", 64)])
def test_noalloc_matches_decode_twice_second_smaller(device, key_format, v_dtype, dim):
    first = dict(batch=4, hkv=2, hq=14, T=5000, seed=1)
    second = dict(batch=2, hkv=1, hq=7, T=900, seed=2, splits=5)
    for shape in (first, second):
        print("noalloc", key_format, v_dtype, dim, shape, flush=True)
        args, keep, tabs = _case(device, dim=dim, key_format=key_format, v_dtype=v_dtype, **shape)
        try:
            ref, got = _both(device, args)
            assert np.isfinite(ref).all()
            np.testing.assert_array_equal(got, ref)
        finally:
            for t in tabs:
                t.destroy()


def test_noalloc_refuses_beyond_its_scratch(device):
    import torch
    import bgtq
    from bgtq import _lib, batched
    # 512 sequences x 16 query heads x d=128, one split: partials beyond BGTQ_DECODE_SCRATCH_BYTES
    z = torch.zeros(16, device="cuda")
    args = dict(batch=512, q_heads=16, kv_heads=1, dim=128, q=z, out=z, lengths=z, max_length=128, v=z, v_dtype="f16",
                v_seq_stride=0, v_head_stride=0, k_f16=z, k_seq_stride=0, k_head_stride=0, splits=1)
    desc = batched.decode_desc(**args)
    assert batched.workspace_bytes(desc) > (4 << 20)
    with pytest.raises(bgtq.RangeError, match="scratch of bgtq_decode_noalloc"):
        _lib.check(_lib.lib().bgtq_decode_noalloc(device.handle, ctypes.byref(desc)))


@pytest.mark.parametrize("key_format,dim", [("packed", 64), ("fp16", 128)])
def test_noalloc_allocates_nothing_and_captures(device, key_format, dim):
    """What the entry point is for: after a first call, further calls leave the device's free
    memory and torch's allocations unchanged; captured into a HIP graph on a side stream (where an
    allocation could not be captured) and replayed three times, with eager calls in between, every
    replay matches the eager output."""
    import torch
    from bgtq import _lib, batched
    args, keep, tabs = _case(device, batch=3, hkv=2, hq=14, dim=dim, T=3000, key_format=key_format, v_dtype="f16",
                             seed=5)
    try:
        out = torch.full((3, 14, dim), float("nan"), device="cuda")
        torch.cuda.synchronize()  # the library's stream is not torch's: the fill lands first
        desc = batched.decode_desc(out=out, **args)

        def call():
            _lib.check(_lib.lib().bgtq_decode_noalloc(device.handle, ctypes.byref(desc)))

        call()
        torch.cuda.synchronize()
        eager = out.cpu().numpy().copy()
        assert np.isfinite(eager).all()
        free0, alloc0 = torch.cuda.mem_get_info()[0], torch.cuda.memory_allocated()
        for _ in range(3):
            call()
        torch.cuda.synchronize()
        assert torch.cuda.mem_get_info()[0] == free0 and torch.cuda.memory_allocated() == alloc0
        np.testing.assert_array_equal(out.cpu().numpy(), eager)
        print("noalloc capture", key_format, dim, flush=True)
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        g = torch.cuda.CUDAGraph()
        try:
            with torch.cuda.graph(g, stream=s):
                batched.bind_torch_stream(device)
                call()
        finally:
            device.set_stream(None)
        torch.cuda.synchronize()
        for _ in range(3):
            out.fill_(float("nan"))
            torch.cuda.synchronize()
            g.replay()
            torch.cuda.synchronize()
            np.testing.assert_array_equal(out.cpu().numpy(), eager)
            out.fill_(float("nan"))
            torch.cuda.synchronize()
            call()
            torch.cuda.synchronize()
            np.testing.assert_array_equal(out.cpu().numpy(), eager)
        del g
    finally:
        for t in tabs:
            t.destroy()


def test_decode_workspace_shared_across_geometries(device):
    """One workspace, zeroed once, shared by bgtq_decode calls of changing geometries (a small
    batch on the general kernels, larger ones on the fused kernel, twice round), and the library
    scratch of bgtq_decode_noalloc likewise: every output equals that of a fresh workspace."""
    import torch
    from bgtq import batched
    shapes = [dict(batch=2, hkv=1, hq=7, T=900, seed=2, splits=5, key_format="packed", v_dtype="f32", dim=64),
              dict(batch=3, hkv=2, hq=14, T=3000, seed=5, key_format="packed", v_dtype="f16", dim=64),
              dict(batch=1, hkv=1, hq=7, T=500, seed=7, key_format="fp16", v_dtype="f16", dim=128),
              dict(batch=6, hkv=2, hq=14, T=2000, seed=9, key_format="packed", v_dtype="f16", dim=64)]
    cases = [_case(device, **s) for s in shapes]
    try:
        size = 0
        for args, _, _ in cases:
            out = torch.empty((args["batch"], args["q_heads"], args["dim"]), device="cuda")
            size = max(size, batched.workspace_bytes(batched.decode_desc(out=out, **args)))
        shared = torch.zeros(size, dtype=torch.uint8, device="cuda")
        for rnd in range(2):
            for i, (args, _, _) in enumerate(cases):
                print("shared workspace", rnd, shapes[i], flush=True)
                ref, got = _both(device, args)
                np.testing.assert_array_equal(got, ref)
                out = torch.full((args["batch"], args["q_heads"], args["dim"]), float("nan"), device="cuda")
                torch.cuda.synchronize()
                batched.decode(device, batched.decode_desc(out=out, workspace=shared, **args))
                torch.cuda.synchronize()
                np.testing.assert_array_equal(out.cpu().numpy(), ref)
    finally:
        for _, _, tabs in cases:
            for t in tabs:
                t.destroy()
