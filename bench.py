"""Benchmark: compressed-K decode attention at Qwen2.5-0.5B geometry on one MI355X.

Headline workload (one step): decode attention for all 24 layers of 64
independent sequences x 32768 context tokens, 14 query heads over 2 KV heads
(GQA 7:1), head_dim 64. K is Block-GTQ packed with layout B (widths 4/8 half
each, 6.0 bits average: 48 code bytes + 2 FP16 scales per token-head), V is
FP16. Inputs are synthetic N(0,1), encoded by the library's own encoder and
resident in HBM before timing. Algorithmic bytes per layer and (sequence, KV
head): T * (48 + 4 + 128). One step = 24 per-layer launches, issued as one
HIP graph (the way a serving loop replays a decode step).

Side measurements in the same JSON line: SmolLM2 K-encode throughput (4096 x 3
x 30 rows), a SmolLM2-geometry decode step at batch 1 (30 layers x encode one
token + attend over 4096), the single-head T=4096 d=128 attention, an
FP16-K kernel at the headline shape, and the Qwen2.5-0.5B 4096-token prompt
prefill (24 layers x encode + causal attention on the matrix cores, as one
chunk and in chunks of 32 rows).

    python bench.py [--steps K] [--warmup W] [--layout B|A|S] [--no-cpu] [--no-extra] [--prefill-only]

--layout A: widths 4..8 at a 6.0 average (groups straddling the 32-dim
K-steps); --layout S: the reference's SmolLM2 calibration heads (first two KV
heads of each layer, rows of 34-44 bytes, 3-6 groups), for the decode step.

Prints one JSON line (value = algorithmic HBM GB/s of the decode step).
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import re
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(ROOT / "block-gqt-webgpu_amd"))

METRIC = "compressed-attn decode HBM GB/s & µs/step; K-encode tokens/s (1 GPU)"
HBM_PEAK_GBS = 8000.0
LAYERS, BATCH, CTX, HQ, HKV, DIM = 24, 64, 32768, 14, 2, 64


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def rope(torch, x, positions, base):
    """Split-half RoPE as the reference's model applies it (pairs (i, i + d/2), angle
    pos * base^(-2i/d); vendor/blockgtq-calibration/rope_utils.py:10-20): x [..., T, d] FP32,
    positions [T]; angles in FP64, rotation in FP32."""
    d = x.shape[-1]
    half = d // 2
    inv = 1.0 / (base ** (torch.arange(0, d, 2, device=x.device, dtype=torch.float64) / d))
    ang = positions.to(device=x.device, dtype=torch.float64)[:, None] * inv[None, :]
    c, sn = torch.cos(ang).float(), torch.sin(ang).float()
    x1, x2 = x[..., :half], x[..., half:]
    return torch.cat([x1 * c - x2 * sn, x2 * c + x1 * sn], dim=-1)


def pair_energy(torch, dim, ratio=0.9, device="cuda"):
    """Per-dimension scale sqrt(ratio^i) of frequency pair i (dims i and i + d/2): post-RoPE K
    whose pair energies decay geometrically."""
    i = torch.arange(dim, device=device) % (dim // 2)
    return (ratio ** i.double()).sqrt().float()


def layout_params(name, dim):
    from bgtq import calibrate
    if name == "S":
        return smollm2_heads(0, 1)[0]
    return calibrate.layout_b(dim) if name == "B" else calibrate.layout_a(dim)


_SMOLLM2 = []


def smollm2_heads(layer, kv_heads):
    """Layout S: the reference's SmolLM2 calibration (30 layers x 3 KV heads, d=64), the first
    kv_heads heads of layer `layer` mod 30, with one row and norm stride for the layer's heads."""
    from bgtq import BlockGTQParameters, calibration
    if not _SMOLLM2:
        _SMOLLM2.extend(calibration.read(ROOT / "tests" / "golden" / "reference" / "model")[2])
    blobs = [_SMOLLM2[(layer % 30) * 3 + h] for h in range(kv_heads)]
    heads = [BlockGTQParameters.from_serialized(b.config, b.table) for b in blobs]
    rb, ns = max(h.rowBytes for h in heads), max(h.normStride for h in heads)
    for h in heads:
        h.rowBytes, h.normStride = rb, ns
    return heads


class DecodeWorkload:
    """All layers' caches for one decode shape, plus per-layer descriptors."""

    def __init__(self, dev, layout="B", layers=LAYERS, batch=BATCH, ctx=CTX, hq=HQ, hkv=HKV, dim=DIM, seed=0,
                 key_format="packed", splits=0, rope_base=None):
        import torch
        import bgtq
        from bgtq import batched
        self.torch, self.dev = torch, dev
        self.layers, self.batch, self.ctx, self.hq, self.hkv, self.dim = layers, batch, ctx, hq, hkv, dim
        g = torch.Generator(device="cuda")
        g.manual_seed(seed)
        self.tables, self.descs, self.keep, self.layer_tensors = [], [], [], []
        p = layout_params(layout, dim) if key_format == "packed" else None
        self.row_bytes = p.rowBytes if p else 2 * dim
        self.norm_stride = p.normStride if p else 0
        per_token = []  # K row, scales and V row bytes of each layer
        self.lengths = torch.full((batch,), ctx, dtype=torch.int32, device="cuda")
        self.out = torch.empty((batch, hq, dim), dtype=torch.float32, device="cuda")
        ws = None
        pos = torch.arange(ctx, device="cuda")
        for layer in range(layers):
            q = torch.randn((batch, hq, dim), generator=g, device="cuda", dtype=torch.float32)
            v = torch.randn((batch, hkv, ctx, dim), generator=g, device="cuda", dtype=torch.float32).half()
            k = torch.randn((batch, hkv, ctx, dim), generator=g, device="cuda", dtype=torch.float32)
            if rope_base:  # keys at positions 0..ctx-1, the query at the last one
                k = rope(torch, k, pos, rope_base)
                q = rope(torch, q.unsqueeze(-2), pos[-1:], rope_base).squeeze(-2).contiguous()
            k = k.half()
            if key_format == "packed":
                hp = smollm2_heads(layer, hkv) if layout == "S" else [p] * hkv
                tabs = [bgtq.Tables(dev, x) for x in hp]  # one table set per (layer, KV head)
                self.tables += tabs
                rb, ns = hp[0].rowBytes, hp[0].normStride
                per_token.append(rb + 2 * ns + 2 * dim)
                # head strides rounded to 16 bytes (the fused kernel's loads)
                packed = torch.empty((batch, hkv, (ctx * rb + 64 + 15) // 16 * 16), dtype=torch.uint8, device="cuda")
                norms = torch.empty((batch, hkv, (ctx * ns + 32 + 7) // 8 * 8), dtype=torch.int16, device="cuda")
                jobs = [dict(tables=tabs[h], src=k[b, h], src_row_stride=dim, rows=ctx, packed=packed[b, h],
                             norms=norms[b, h], dst_row0=0) for b in range(batch) for h in range(hkv)]
                batched.encode(dev, jobs, "f16")
                del k
                kw = dict(tables=tabs, packed=packed, packed_seq_stride=packed.stride(0),
                          packed_head_stride=packed.stride(1), norms=norms, norms_seq_stride=norms.stride(0),
                          norms_head_stride=norms.stride(1))
                self.keep += [packed, norms, v, q]
                self.layer_tensors.append(dict(packed=packed, norms=norms, v=v, q=q, params=hp))
            else:
                per_token.append(4 * dim)
                kw = dict(k_f16=k, k_seq_stride=k.stride(0), k_head_stride=k.stride(1))
                self.keep += [k, v, q]
                self.layer_tensors.append(dict(k=k, v=v, q=q))
            args = dict(batch=batch, q_heads=hq, kv_heads=hkv, dim=dim, q=q, out=self.out, lengths=self.lengths,
                        max_length=ctx, v=v, v_dtype="f16", v_seq_stride=v.stride(0), v_head_stride=v.stride(1),
                        splits=splits, **kw)
            if ws is None:
                ws = torch.zeros(batched.workspace_bytes(batched.decode_desc(**args)), dtype=torch.uint8,
                                 device="cuda")
            self.descs.append(batched.decode_desc(workspace=ws, **args))
        self.ws = ws
        self.per_token = per_token
        torch.cuda.synchronize()

    def bytes_per_layer(self):
        """Algorithmic bytes of one layer (the mean over layers where row strides differ)."""
        return self.batch * self.hkv * self.ctx * sum(self.per_token) / len(self.per_token)

    def set_q_rotated(self, flag):
        """Queries given in the code domain (a projection baked with bgtq_bake_qproj): the kernels
        skip their rotation. The synthetic queries are N(0, 1) either way."""
        for d in self.descs:
            d.q_rotated = int(bool(flag))

    def set_splits(self, splits):
        from bgtq import batched
        for d in self.descs:
            d.splits = splits
        self.ws = self.torch.zeros(batched.workspace_bytes(self.descs[0]), dtype=self.torch.uint8, device="cuda")
        for d in self.descs:
            d.workspace, d.workspace_bytes = ctypes.c_void_p(self.ws.data_ptr()), self.ws.numel()

    def step(self):
        from bgtq import batched
        for d in self.descs:
            batched.decode(self.dev, d)


def graph_of(torch, dev, fn, warmup=2):
    """Capture fn() (stream-ordered library calls) as a HIP graph on a side stream."""
    from bgtq import batched
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        batched.bind_torch_stream(dev)
        for _ in range(warmup):
            fn()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        batched.bind_torch_stream(dev)
        fn()
    batched.bind_torch_stream(dev)
    torch.cuda.synchronize()
    return g


def time_graph(torch, g, steps, warmup):
    for _ in range(warmup):
        g.replay()
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(steps):
        g.replay()
    b.record()
    torch.cuda.synchronize()
    return a.elapsed_time(b) / steps


def time_eager(torch, fn, steps, warmup):
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(steps):
        fn()
    b.record()
    torch.cuda.synchronize()
    return a.elapsed_time(b) / steps


class EncodeWorkload:
    """Prefill K encode at SmolLM2 geometry: 4096 tokens x 3 KV heads x 30 layers, d=64, one table set
    per (layer, KV head), all 90 jobs in one bgtq_encode_batched call."""

    def __init__(self, dev, layout="B", seed=3):
        import torch
        import bgtq
        self.dev, self.p = dev, layout_params(layout, 64)
        p = self.p
        self.tabs = [bgtq.Tables(dev, p) for _ in range(90)]
        g = torch.Generator(device="cuda")
        g.manual_seed(seed)
        # post-RoPE K whose per-pair energy decays geometrically (ratio 0.9)
        self.k = (torch.randn((30, 4096, 3, 64), generator=g, device="cuda") * pair_energy(torch, 64)).half()
        self.packed = torch.zeros((90, 4096 * p.rowBytes + 64), dtype=torch.uint8, device="cuda")
        self.norms = torch.zeros((90, 4096 * p.normStride + 32), dtype=torch.int16, device="cuda")
        self.jobs = [dict(tables=self.tabs[l * 3 + h], src=self.k[l, :, h], src_row_stride=3 * 64, rows=4096,
                          packed=self.packed[l * 3 + h], norms=self.norms[l * 3 + h], dst_row0=0)
                     for l in range(30) for h in range(3)]
        self.rows = 30 * 3 * 4096

    def call(self):
        from bgtq import batched
        batched.encode(self.dev, self.jobs, "f16")

    def destroy(self):
        for t in self.tabs:
            t.destroy()


def encode_throughput(dev, layout="B", reps=10):
    """The SmolLM2 prefill K encode (EncodeWorkload) as one call replayed in a HIP graph."""
    import torch
    w = EncodeWorkload(dev, layout)
    p = w.p
    ms = time_graph(torch, graph_of(torch, dev, w.call), reps, 5)
    ms_eager = time_eager(torch, w.call, reps, 2)
    rows = w.rows
    w.destroy()
    nbytes = rows * (128 + p.rowBytes + 2 * p.normStride)
    return {"rows_per_s": round(rows / (ms / 1e3)), "tokens_per_s": round(4096 / (ms / 1e3)), "ms": round(ms, 4),
            "gbs_algorithmic": round(nbytes / (ms / 1e3) / 1e9, 1),
            "eager_ms": round(ms_eager, 4),
            "timing": "one encode call (90 tables) replayed as a HIP graph; eager_ms: issued directly each time",
            "data": "FP16 N(0,1) K rows, frequency pair i scaled by sqrt(0.9^i)",
            "working_set_bytes": nbytes,
            "residency": "the working set fits the 256 MB Infinity Cache: replays read it from there, not HBM; "
                         "the line is VALU-bound, not an HBM rate"}


class SmolLM2Step:
    """SmolLM2-135M geometry decode step at batch 1: per layer, encode the new token's K for
    3 KV heads, then attend 9 query heads over the 4096 + 1 cached tokens. Layout S gives each
    layer its own three calibration heads (the reference model's decode step)."""

    L, HKV, HQ, T = 30, 3, 9, 4096

    def __init__(self, dev, layout="B", splits=0, seed=0, q_rotated=False):
        import torch
        import bgtq
        from bgtq import batched
        L, HKV2, HQ2, T = self.L, self.HKV, self.HQ, self.T
        self.dev, self.layout = dev, layout
        g = torch.Generator(device="cuda")
        g.manual_seed(seed)
        self.heads = [smollm2_heads(l, HKV2) if layout == "S" else [layout_params(layout, 64)] * HKV2
                      for l in range(L)]
        self.tabs = [bgtq.Tables(dev, self.heads[l][h]) for l in range(L) for h in range(HKV2)]
        rb_max = max(h[0].rowBytes for h in self.heads)
        ns_max = max(h[0].normStride for h in self.heads)
        # per-head strides rounded to 16 bytes (the fused kernel's loads)
        self.packed = torch.empty((L, 1, HKV2, ((T + 1) * rb_max + 64 + 15) // 16 * 16), dtype=torch.uint8,
                                  device="cuda")
        self.norms = torch.empty((L, 1, HKV2, ((T + 1) * ns_max + 32 + 7) // 8 * 8), dtype=torch.int16,
                                 device="cuda")
        hist = torch.randn((L, HKV2, T, 64), generator=g, device="cuda").half()
        for l in range(L):
            batched.encode(dev, [dict(tables=self.tabs[l * HKV2 + h], src=hist[l, h], src_row_stride=64, rows=T,
                                      packed=self.packed[l, 0, h], norms=self.norms[l, 0, h], dst_row0=0)
                                 for h in range(HKV2)], "f16")
        del hist
        self.knew = torch.randn((L, 1, HKV2, 64), generator=g, device="cuda")  # post-RoPE FP32 K of the new token
        self.vnew = torch.randn((L, 1, HKV2, 64), generator=g, device="cuda")  # its FP32 V
        self.v = torch.randn((L, 1, HKV2, T + 1, 64), generator=g, device="cuda").half()
        self.q = torch.randn((L, 1, HQ2, 64), generator=g, device="cuda")
        self.out = torch.empty((L, 1, HQ2, 64), device="cuda")
        self.lengths = torch.full((1,), T + 1, dtype=torch.int32, device="cuda")
        self.jobs, self.descs, ws = [], [], None
        for l in range(L):
            self.jobs.append([dict(tables=self.tabs[l * HKV2 + h], src=self.knew[l, 0, h], src_row_stride=64, rows=1,
                                   packed=self.packed[l, 0, h], norms=self.norms[l, 0, h], dst_row0=T)
                              for h in range(HKV2)])
            args = dict(batch=1, q_heads=HQ2, kv_heads=HKV2, dim=64, q=self.q[l], out=self.out[l],
                        lengths=self.lengths, max_length=T + 1, v=self.v[l], v_seq_stride=self.v.stride(1),
                        v_head_stride=self.v.stride(2), tables=self.tabs[l * HKV2:(l + 1) * HKV2],
                        packed=self.packed[l], packed_seq_stride=self.packed.stride(1),
                        packed_head_stride=self.packed.stride(2), norms=self.norms[l],
                        norms_seq_stride=self.norms.stride(1), norms_head_stride=self.norms.stride(2), splits=splits,
                        q_rotated=q_rotated)
            if ws is None:
                ws = torch.zeros(batched.workspace_bytes(batched.decode_desc(**args)), dtype=torch.uint8,
                                 device="cuda")
            self.descs.append(batched.decode_desc(workspace=ws, **args))
        self.ws = ws
        self.appends = [batched.append_desc(k_new=self.knew[l], v_new=self.vnew[l]) for l in range(L)]

    def step(self):
        """One launch per layer: the new K's encode and its V append inside the attention launch."""
        from bgtq import batched
        for l in range(self.L):
            batched.decode_append(self.dev, self.descs[l], self.appends[l])

    def step_two_calls(self):
        """The same step as two launches per layer (the V row is not written here)."""
        from bgtq import batched
        for l in range(self.L):
            batched.encode(self.dev, self.jobs[l], "f32")
            batched.decode(self.dev, self.descs[l])

    def bytes_per_step(self):
        return sum(self.HKV * (self.T + 1) * (h[0].rowBytes + 2 * h[0].normStride + 128) for h in self.heads)

    def destroy(self):
        for t in self.tabs:
            t.destroy()


def smollm2_decode_step(dev, steps, layout="B", splits=0):
    import torch
    w = SmolLM2Step(dev, layout, splits)
    ms = time_graph(torch, graph_of(torch, dev, w.step), steps, 3)
    ms2 = time_graph(torch, graph_of(torch, dev, w.step_two_calls), steps, 3)
    bytes_step = w.bytes_per_step()
    w.destroy()
    wr = SmolLM2Step(dev, layout, splits, q_rotated=True)
    ms_rot = time_graph(torch, graph_of(torch, dev, wr.step), steps, 3)
    wr.destroy()
    return {"us_per_step": round(ms * 1e3, 2), "gbs_algorithmic": round(bytes_step / (ms / 1e3) / 1e9, 1),
            "two_launches_per_layer_us_per_step": round(ms2 * 1e3, 2),
            "q_rotated_us_per_step": round(ms_rot * 1e3, 2),
            "workload": "30 layers x (encode 1 token x 3 KV heads, append its V, attend 9 q heads over 4097 "
                        f"tokens), d=64, batch 1, layout {layout}, FP16 V; one bgtq_decode_append launch per layer"}


class SmolLM2DispatchStep:
    """The same SmolLM2 decode step (30 layers, 3 KV heads, 9 query heads, 4096 cached tokens + 1,
    layout B) through the reference decoder's per-layer dispatches (src/model/decoder.ts:46-56 with
    rows = 1): encode_k per KV head, append of the V row, compressed_dot per KV head, softmax and
    weighted, each its own pass with the scores and probabilities in device memory
    (bgtq_model_submit). The dispatch arrays are built once; the timed call queues them."""

    L, HKV, HQ, T, D = 30, 3, 9, 4096, 64

    def __init__(self, dev, seed=0):
        import torch
        import bgtq
        from bgtq import _lib, batched
        from bgtq.model_ops import _binding
        L, HKV2, HQ2, T, D = self.L, self.HKV, self.HQ, self.T, self.D
        cap, gqa = T + 1, HQ2 // HKV2
        self.dev, self._lib = dev, _lib
        p = layout_params("B", D)
        g = torch.Generator(device="cuda")
        g.manual_seed(seed)
        self.tabs = [bgtq.Tables(dev, p) for _ in range(L * HKV2)]
        self.keep, self.arrays = [], []
        for l in range(L):
            codes = [torch.zeros(cap * p.rowBytes, dtype=torch.uint8, device="cuda") for _ in range(HKV2)]
            norms = [torch.zeros(cap * p.normStride, dtype=torch.int16, device="cuda") for _ in range(HKV2)]
            hist = torch.randn((HKV2, T, D), generator=g, device="cuda").half()
            batched.encode(dev, [dict(tables=self.tabs[l * HKV2 + h], src=hist[h], src_row_stride=D, rows=T,
                                      packed=codes[h], norms=norms[h], dst_row0=0) for h in range(HKV2)], "f16")
            vcache = torch.randn((HKV2 * cap * D,), generator=g, device="cuda").half().view(torch.int16)
            kr = torch.randn((HKV2 * D,), generator=g, device="cuda")
            vv = torch.randn((HKV2 * D,), generator=g, device="cuda")
            qr = torch.randn((HQ2 * D,), generator=g, device="cuda")
            scores = torch.empty((HQ2 * cap,), device="cuda")
            probs = torch.empty((HQ2 * cap,), device="cuda")
            attn = torch.empty((HQ2 * D,), device="cuda")
            tabs = self.tabs[l * HKV2:(l + 1) * HKV2]
            prm = [1, cap, cap, T, HQ2, HKV2, gqa, D]
            bufs = [qr, None, vcache, scores, probs, attn]
            disp = [("encode_k", [1, T, h, HKV2], [tabs[h], tabs[h], kr, codes[h], norms[h]], 1, 1) for h in range(HKV2)]
            disp.append(("append", [1, T, cap, HKV2], [vv, vcache], -(-HKV2 * D // 2 // 128), 1))
            disp += [("compressed_dot", [1, T, h, cap, HQ2, gqa, D],
                      [tabs[h], tabs[h], qr, codes[h], norms[h], None, scores], cap, 1) for h in range(HKV2)]
            disp.append(("softmax", prm, bufs, HQ2, 1))
            disp.append(("weighted", prm, bufs, HQ2 * D, 1))
            arr = (_lib.ModelDispatch * len(disp))()
            for i, (name, params, buffers, x, y) in enumerate(disp):
                binds = (_lib.Binding * len(buffers))(*[_binding(b) for b in buffers])
                nm = name.encode()
                self.keep += [binds, nm]
                arr[i] = _lib.ModelDispatch(nm, (ctypes.c_uint32 * 8)(*(params + [0] * (8 - len(params)))),
                                            ctypes.cast(binds, ctypes.POINTER(_lib.Binding)), len(buffers), x, y)
            self.arrays.append((arr, len(disp)))
            self.keep += [codes, norms, vcache, kr, vv, qr, scores, probs, attn]
        self.bytes = L * HKV2 * cap * (p.rowBytes + 2 * p.normStride + 2 * D)
        torch.cuda.synchronize()

    def step(self):
        for arr, n in self.arrays:
            self._lib.check(self._lib.lib().bgtq_model_submit(self.dev.handle, arr, n))

    def destroy(self):
        for t in self.tabs:
            t.destroy()


def smollm2_dispatch_step(dev, steps):
    import torch
    w = SmolLM2DispatchStep(dev)
    try:
        ms = time_graph(torch, graph_of(torch, dev, w.step), steps, 3)
        timing = "HIP graph of the 30 layers' dispatches"
    except Exception as e:  # a pass the capture refuses: time it issued directly
        ms = time_eager(torch, w.step, steps, 2)
        timing = f"issued directly ({type(e).__name__} under graph capture)"
    out = {"us_per_step": round(ms * 1e3, 2), "gbs_algorithmic": round(w.bytes / (ms / 1e3) / 1e9, 1),
           "timing": timing,
           "workload": "the SmolLM2 decode step at batch 1 (layout B) through bgtq_model_submit: per layer "
                       "3 x encode_k, append, 3 x compressed_dot, softmax, weighted (src/model/decoder.ts:46-56), "
                       "scores and probabilities materialised [9 x 4097] as the reference's passes keep them"}
    w.destroy()
    return out


def prefill_flops(prompt, hq, dim, layers):
    """Algorithmic causal attention FLOPs of a prompt: QK and PV, 2 * dim each per (query, visible token)."""
    return layers * hq * (prompt * (prompt + 1) // 2) * dim * 4


def device_ceilings():
    """Achievable ceilings of this GPU, measured now: a streaming non-temporal read of the decode step's
    byte count (one layer, 754,974,720 B) and a dense fp16 16x16x32 matrix-core loop on every CU."""
    import torch
    lib = ctypes.CDLL(str(ROOT / "block-gqt-webgpu_amd" / "lib" / "libbgtq_probes.so"))
    lib.bgtq_probe_read.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int, ctypes.POINTER(ctypes.c_double)]
    lib.bgtq_probe_mfma.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.POINTER(ctypes.c_double),
                                    ctypes.POINTER(ctypes.c_double)]
    nbytes = BATCH * HKV * CTX * 180
    buf = torch.ones(nbytes // 4, dtype=torch.int32, device="cuda")
    torch.cuda.synchronize()
    us = ctypes.c_double()
    if lib.bgtq_probe_read(buf.data_ptr(), nbytes, 20, ctypes.byref(us)) != 0:
        raise RuntimeError("read probe failed")
    del buf
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    flops, us2 = ctypes.c_double(), ctypes.c_double()
    if lib.bgtq_probe_mfma(cus, 4096, 5, ctypes.byref(flops), ctypes.byref(us2)) != 0:
        raise RuntimeError("matrix-core probe failed")
    return {"hbm_read_gbs": round(nbytes / us.value / 1e3, 1), "hbm_read_us": round(us.value, 2),
            "hbm_read_bytes": nbytes, "mfma_f16_tflops": round(flops.value / us2.value / 1e6, 1),
            "probes": "libbgtq_probes.so: grid-stride 16-byte non-temporal loads (4096 x 256 threads); "
                      "8 chains of v_mfma_f32_16x16x32_f16 per wave, 8 waves per CU"}


class PrefillWorkload:
    """Qwen2.5-0.5B-geometry prompt prefill: per layer, encode the chunk's post-RoPE K for 2 KV heads,
    then causal attention of its rows x 14 query heads over the history so far (d=64, FP16 V).
    chunk=0: the whole prompt as one chunk; else chunks of that many rows, chunk by chunk through all
    layers."""

    def __init__(self, dev, layout="B", chunk=0, prompt=4096, layers=LAYERS, seed=7):
        import torch
        import bgtq
        from bgtq import batched
        self.dev, self.layout, self.prompt, self.layers = dev, layout, prompt, layers
        p = self.params = layout_params(layout, DIM)
        self.chunk = chunk = chunk or prompt
        starts = list(range(0, prompt, chunk))
        self.tabs = [bgtq.Tables(dev, p) for _ in range(layers * HKV)]
        g = torch.Generator(device="cuda")
        g.manual_seed(seed)
        # Q/K/V FP16 N(0,1), RoPE base 1e6 on Q and K (Qwen2.5)
        pos = torch.arange(prompt, device="cuda")
        self.k = rope(torch, torch.randn((layers, HKV, prompt, DIM), generator=g, device="cuda").half().float(),
                      pos, 1e6).half()
        self.v = torch.randn((layers, 1, HKV, prompt, DIM), generator=g, device="cuda").half()
        q = torch.randn((layers, prompt, HQ, DIM), generator=g, device="cuda").half().float()
        self.q = rope(torch, q.transpose(1, 2), pos, 1e6).transpose(1, 2).contiguous()
        self.out = torch.empty((layers, prompt, HQ, DIM), device="cuda")
        self.packed = torch.empty((layers, 1, HKV, prompt * p.rowBytes), dtype=torch.uint8, device="cuda")
        self.norms = torch.empty((layers, 1, HKV, prompt * p.normStride), dtype=torch.int16, device="cuda")
        self.start_t = [torch.tensor([s], dtype=torch.int32, device="cuda") for s in starts]
        self.enc, args_list = [], []
        for c, s in enumerate(starts):
            rows = min(chunk, prompt - s)
            for l in range(layers):
                self.enc.append([dict(tables=self.tabs[l * HKV + h], src=self.k[l, h, s:s + rows], src_row_stride=DIM,
                                      rows=rows, packed=self.packed[l, 0, h], norms=self.norms[l, 0, h], dst_row0=s)
                                 for h in range(HKV)])
                args_list.append(dict(batch=1, rows=rows, q_heads=HQ, kv_heads=HKV, dim=DIM, q=self.q[l, s:s + rows],
                                      out=self.out[l, s:s + rows], starts=self.start_t[c], max_length=prompt,
                                      v=self.v[l], v_seq_stride=self.v.stride(1), v_head_stride=self.v.stride(2),
                                      tables=self.tabs[l * HKV:(l + 1) * HKV], packed=self.packed[l],
                                      packed_seq_stride=self.packed.stride(1),
                                      packed_head_stride=self.packed.stride(2), norms=self.norms[l],
                                      norms_seq_stride=self.norms.stride(1), norms_head_stride=self.norms.stride(2)))
        # one workspace for every call: they are ordered on one stream
        need = max(batched.prefill_workspace_bytes(batched.prefill_desc(**a)) for a in args_list)
        self.ws = torch.zeros(need, dtype=torch.uint8, device="cuda")
        self.descs = [batched.prefill_desc(workspace=self.ws, **a) for a in args_list]
        # the chunk's own K and V rows, [B=1, rows, Hkv, dim], for the one-launch form (bgtq_prefill_append)
        self.apps = []
        if chunk <= 32:
            for c, s in enumerate(starts):
                rows = min(chunk, prompt - s)
                for l in range(layers):
                    self.apps.append(batched.prefill_append_desc(k_new=self.k[l, :, s:s + rows].transpose(0, 1)[None],
                                                                 v_new=self.v[l, 0, :, s:s + rows].transpose(0, 1)[None]))

    def attend_only(self):
        from bgtq import batched
        for d in self.descs:
            batched.prefill(self.dev, d)

    def step(self):
        from bgtq import batched
        for e, d in zip(self.enc, self.descs):
            batched.encode(self.dev, e, "f16")
            batched.prefill(self.dev, d)

    def step_fused(self):
        """The same prompt with each chunk's K encode and V append inside its attention launch."""
        from bgtq import batched
        for d, a in zip(self.descs, self.apps):
            batched.prefill_append(self.dev, d, a)

    def flops(self):
        return prefill_flops(self.prompt, HQ, DIM, self.layers)

    def destroy(self):
        for t in self.tabs:
            t.destroy()


def qwen_prefill(dev, steps, layout="B", chunk=0, prompt=4096, layers=LAYERS):
    import torch
    w = PrefillWorkload(dev, layout, chunk, prompt, layers)
    flops = w.flops()
    ms = time_graph(torch, graph_of(torch, dev, w.step), steps, 2)
    ms_att = time_graph(torch, graph_of(torch, dev, w.attend_only), steps, 2)
    fused = {}
    if w.apps:
        ms_f = time_graph(torch, graph_of(torch, dev, w.step_fused), steps, 2)
        fused = {"one_launch_ms_per_prompt": round(ms_f, 4), "one_launch_tokens_per_s": round(prompt / (ms_f / 1e3)),
                 "one_launch": "each chunk's K encode, V append and attention in one bgtq_prefill_append launch "
                               "per layer (the K rows' bytes equal the two-launch form's)"}
    w.destroy()
    return {"ms_per_prompt": round(ms, 4), "tokens_per_s": round(prompt / (ms / 1e3)), **fused,
            "attention_only_ms": round(ms_att, 4),
            "attention_tflops_algorithmic": round(flops / (ms_att / 1e3) / 1e12, 1),
            "mfma_frac_of_fp16_dense_peak": round(flops / (ms_att / 1e3) / 2.5e15, 4),
            "algorithmic_gflop": round(flops / 1e9, 1),
            "workload": f"{prompt}-token prompt, {layers} layers x (encode K of {HKV} KV heads + causal attention of "
                        f"{HQ} q heads), d={DIM}, layout {layout}, FP16 V, "
                        + ("one chunk" if w.chunk == prompt else f"chunks of {w.chunk} rows")}


def single_head(dev, steps, layout="B", calls=32):
    """One query over T=4096, d=128, one head (the reference's CPU-runnable shape: Q/K/V N(0,1), RoPE
    base 1e4 on Q and K), timed as a HIP graph of `calls` launches, each over caches, tables and a
    query of its own, so the per-call figure is the GPU's and not the rate at which the host replays
    a one-launch graph. kernel_us: the kernel's own duration from the committed rocprofv3 trace."""
    import torch
    w = DecodeWorkload(dev, layout, layers=calls, batch=1, ctx=4096, hq=1, hkv=1, dim=128, rope_base=1e4)
    ms = time_graph(torch, graph_of(torch, dev, w.step), steps * 2, 3) / calls
    w.set_q_rotated(True)
    ms_rot = time_graph(torch, graph_of(torch, dev, w.step), steps * 2, 3) / calls
    nbytes = w.bytes_per_layer()
    return {"us_per_step": round(ms * 1e3, 2), "gbs_algorithmic": round(nbytes / (ms / 1e3) / 1e9, 1),
            "q_rotated_us_per_step": round(ms_rot * 1e3, 2), "launches_per_graph": calls,
            "kernel_us": read_profile_value("decode_fast_single_head_t4096_d128_trace.txt", "kernel_avg_us"),
            "kernel_us_source": "profiles/decode_fast_single_head_t4096_d128_trace.txt (rocprofv3 --kernel-trace "
                                "of bench.py --single-head-only; committed, not measured in this run)",
            "working_set_bytes": calls * nbytes,
            "residency": f"{calls} distinct caches of {nbytes} B: beyond the L2s, inside the 256 MB Infinity Cache",
            "workload": "1 query, T=4096, d=128, one head, layout B, FP16 V, RoPE base 1e4 on Q and K"}


# The reference's published phase-4 times (benchmarks/raw/2026-09-15T09-27-00-112Z-phase4-phase4-bench.json,
# an Intel Gen12LP integrated GPU under WebGPU), microseconds, by (T, d).
PHASE4_REFERENCE_US = {(512, 64): 196.6, (1024, 64): 262.1, (2048, 64): 524.3, (4096, 64): 917.5,
                       (512, 128): 327.7, (1024, 128): 720.9, (2048, 128): 1048.6, (4096, 128): 2162.7}


def phase4_attention(dev, samples=20, warmup=5):
    """OptimizedAttention over FP32 Values at the reference's benchmark shapes (benchmarks/phase4.ts:19-47):
    T in {512, 1024, 2048, 4096} x d in {64, 128}, the mixed_d{d} calibration, 3 queries at (0, T/2, T-1),
    non-causal, its workload generator (tests/oracles/export_attention.py:20-26). Timed as
    benchmarks/timing.ts:7-31 times it: GPU timestamps around the attention work of record() (after the
    queries' upload), 5 warmups, the median of 20 samples."""
    import numpy as np
    import torch
    import bgtq
    out = {}
    for d in (64, 128):
        params = bgtq.BlockGTQParameters.load_mixed_fixture(
            ROOT / "tests" / "golden" / "reference" / "mixed" / f"mixed_d{d}.json")
        for T in (512, 1024, 2048, 4096):
            g = torch.Generator().manual_seed(731 + d + T)
            q = torch.randn(3, d, generator=g).numpy()
            k = (torch.randn(T, d, generator=g) * 0.7).half().numpy()
            v = (torch.randn(T, d, generator=g) * 0.5).numpy()
            pos = np.array([0, T // 2, T - 1], np.uint32)
            keys = bgtq.PackedKeys.create(dev, params, T)
            values = bgtq.Values(dev, d, T)
            sessions = {"us": bgtq.OptimizedAttention.create(dev, keys, values, 3),
                        "us_no_intermediates": bgtq.OptimizedAttention.create(dev, keys, values, 3,
                                                                              materialize=False)}
            ts = bgtq.Timestamps(dev, 2 * (samples + warmup))
            try:
                keys.append(k.view(np.uint16))
                values.append(v)
                rec = {}
                for key, s in sessions.items():
                    s.setQueries(q, pos, False)
                    for i in range(samples + warmup):
                        s.record(ts, 2 * i, 2 * i + 1)
                    ns = ts.resolve().astype(np.int64)
                    rec[key] = round(float(np.median((ns[1::2] - ns[0::2])[warmup:])) / 1e3, 2)
                nbytes = T * (params.rowBytes + 2 * params.normStride + 4 * d)
                rec["bytes_k_scales_v"] = nbytes
                rec["gbs_algorithmic"] = round(nbytes / (rec["us"] * 1e3), 2)
                rec["kernel_us"] = read_profile_value("decode_fast_fp32v_phase4_trace.txt", f"t{T}_d{d}_kernel_us")
                rec["reference_us_gen12lp"] = PHASE4_REFERENCE_US[(T, d)]
                out[f"t{T}_d{d}"] = rec
            finally:
                ts.destroy()
                for s in sessions.values():
                    s.destroy()
                values.destroy()
                keys.destroy()
    out["protocol"] = ("record() with timestamps at begin and end of the attention work (the fused kernel, plus "
                       "the probabilities pass when intermediates are materialised), 5 warmups, median of 20; "
                       "FP32 V read by the kernel's FP32-V variant; kernel_us: the fused kernel plus the probabilities "
                       "kernel per record() in profiles/decode_fast_fp32v_phase4_trace.txt (rocprofv3 --kernel-trace of "
                       "bench.py --attention-only; committed, not measured in this run); reference_us_gen12lp: the reference's "
                       "published phase-4 time on its own hardware, for context only")
    return out


def cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(layout="B", budget_s=10.0, threads=None):
    """The oracle's CPU path built for this host (-O3 -march=native, no fast-math, no contraction):
    unpack + reconstruct + FP32 attention on whole (sequence, KV head) units of the headline workload,
    one thread for budget_s, then `threads` threads (the box's CPU share, at most 16; each on its own
    buffers, the ctypes calls release the GIL) for budget_s. The all-threads rate is the value. Also
    the single-head shape (T=4096, d=128, one query) on one thread, timed as the reference's
    benchmarks time (5 warm-up and 20 timed calls, the median; benchmarks/timing.ts:7-31)."""
    import os
    import statistics
    import tempfile
    import threading
    import numpy as np
    from oracle import oracle as O
    build_dir = tempfile.mkdtemp(prefix="bgtq_oracle_native_")
    O.use_native_build(build_dir)

    def olayout(p):
        return O.Layout(dim=p.dim, groups=p.groups, row_bytes=p.rowBytes, norm_stride=p.normStride,
                        nibble_dims=p.nibbleDims, max_centroids=p.maxCentroids, perm=p.permutation,
                        group_of=p.groupOf, pos_to_cb=p.positionToCodebook, code_lut=p.codeLut,
                        rotation=p.rotation, centroids=p.centroids, offsets=p.offsets, inv_scales=p.inverseScales)

    def unit(p, T, dim, nq, causal, seed):
        L = olayout(p)
        rng = np.random.default_rng(seed)
        k = rng.standard_normal((T, dim)).astype(np.float16).view(np.uint16)
        packed, norms = O.encode_pack(L, k)
        v = rng.standard_normal((T, dim)).astype(np.float16).astype(np.float32)
        q = rng.standard_normal((nq, dim)).astype(np.float32)
        pos = np.full(nq, T - 1, np.uint32)
        scales = norms.view(np.float16).astype(np.float32)

        def run():
            codes = O.unpack(packed, dim, p.nibbleDims)
            keff = O.reconstruct(L, codes, scales)
            return O.attention(q, keff, v, pos, causal, fp32=True)
        return run

    p = layout_params(layout, DIM)
    unit_bytes = CTX * (p.rowBytes + 2 * p.normStride + 2 * DIM)

    def run_for(deadline, counts, slot):
        fn = unit(p, CTX, DIM, HQ // HKV, False, slot)
        n = 0
        while time.perf_counter() < deadline or n == 0:
            fn()
            n += 1
        counts[slot] = n

    def timed(nthreads):
        counts = [0] * nthreads
        t0 = time.perf_counter()
        ts = [threading.Thread(target=run_for, args=(t0 + budget_s, counts, i)) for i in range(nthreads)]
        for t in ts:
            t.start()
        for t in ts:
            t.join()
        return sum(counts), time.perf_counter() - t0

    n1, dt1 = timed(1)
    nproc = os.cpu_count() or 1
    threads = threads or min(16, nproc)
    nn, dtn = timed(threads)

    def rate(make, budget, nthreads):
        """Calls of make(slot)() completed in about `budget` seconds on nthreads threads (each its own
        inputs); returns (calls, seconds)."""
        counts = [0] * nthreads
        fns = [make(i) for i in range(nthreads)]
        t0 = time.perf_counter()

        def go(i):
            n = 0
            while time.perf_counter() < t0 + budget or n == 0:
                fns[i]()
                n += 1
            counts[i] = n
        ts = [threading.Thread(target=go, args=(i,)) for i in range(nthreads)]
        for t in ts:
            t.start()
        for t in ts:
            t.join()
        return sum(counts), time.perf_counter() - t0

    legs = {}
    leg_s = budget_s / 3
    # C3: bulk K encode (SmolLM2 rows: FP16 N(0,1), pair i scaled by sqrt(0.9^i)), 4096 rows per call
    pe = np.sqrt(0.9 ** (np.arange(64) % 32))

    def make_encode(slot):
        L = olayout(layout_params(layout, 64))
        k = (np.random.default_rng(500 + slot).standard_normal((4096, 64)) * pe).astype(np.float16).view(np.uint16)
        return lambda: O.encode_pack(L, k)
    c3 = {}
    for nt in (1, threads):
        calls, dt = rate(make_encode, leg_s, nt)
        c3["rows_per_s" if nt > 1 else "one_thread_rows_per_s"] = round(calls * 4096 / dt)
    c3.update({"threads": threads, "ms_per_call_extrapolated": round(368640 / c3["rows_per_s"] * 1e3, 1),
               "sample": "calls of oracle encode + pack on 4096 rows (d=64, layout " + layout + "), each thread its "
                         "own rows; ms_per_call: the 368,640-row call at the all-threads rate"})
    legs["encode_smollm2_prefill"] = c3
    # C2: one decode step at SmolLM2 geometry (per layer: encode the new token's K for 3 KV heads,
    # reconstruct each head's 4097 rows, FP32 attention of its 3 query heads); layers spread over threads
    p64 = layout_params(layout, 64)

    def make_layer(slot):
        L = olayout(p64)
        rng = np.random.default_rng(700 + slot)
        hist = [O.encode_pack(L, rng.standard_normal((4096, 64)).astype(np.float16).view(np.uint16)) for _ in range(3)]
        knew = [rng.standard_normal((1, 64)).astype(np.float16).view(np.uint16) for _ in range(3)]
        v = [rng.standard_normal((4097, 64)).astype(np.float16).astype(np.float32) for _ in range(3)]
        q = [rng.standard_normal((3, 64)).astype(np.float32) for _ in range(3)]
        pos = np.full(3, 4096, np.uint32)

        def run():
            for h in range(3):
                pk, nm = O.encode_pack(L, knew[h])
                packed = np.concatenate([hist[h][0], pk])
                scales = np.concatenate([hist[h][1], nm]).view(np.float16).astype(np.float32)
                keff = O.reconstruct(L, O.unpack(packed, 64, p64.nibbleDims), scales)
                O.attention(q[h], keff, v[h], pos, False, fp32=True)
        return run
    c2 = {}
    for nt in (1, threads):
        calls, dt = rate(make_layer, leg_s, nt)
        c2["us_per_step" if nt > 1 else "one_thread_us_per_step"] = round(30 * dt / calls * 1e6, 1)
    c2.update({"threads": threads, "sample": "SmolLM2 decode-step layers (encode 1 token x 3 KV heads, reconstruct "
                                              "4097 rows per head, FP32 attention of 3 query heads each); "
                                              "us_per_step: 30 layers at the measured layer rate"})
    legs["smollm2_decode_step_b1"] = c2
    # C4: the Qwen prompt's causal attention on sampled query rows (7 heads of one KV head over the
    # row's prefix of a reconstructed 4096-token history, RoPE base 1e6 keys), as FLOP/s
    pq = layout_params(layout, DIM)

    def make_rows(slot):
        L = olayout(pq)
        rng = np.random.default_rng(900 + slot)
        ang = np.arange(4096)[:, None] * (1.0 / (1e6 ** (np.arange(0, DIM, 2) / DIM)))[None, :]
        x = rng.standard_normal((4096, DIM)).astype(np.float16).astype(np.float32)
        x1, x2 = x[:, :DIM // 2], x[:, DIM // 2:]
        kr = np.concatenate([x1 * np.cos(ang) - x2 * np.sin(ang), x2 * np.cos(ang) + x1 * np.sin(ang)], 1)
        packed, norms = O.encode_pack(L, kr.astype(np.float16).view(np.uint16))
        keff = O.reconstruct(L, O.unpack(packed, DIM, pq.nibbleDims), norms.view(np.float16).astype(np.float32))
        v = rng.standard_normal((4096, DIM)).astype(np.float16).astype(np.float32)
        rows = rng.integers(0, 4096, size=64)
        qs = [rng.standard_normal((HQ // HKV, DIM)).astype(np.float32) for _ in rows]
        state = {"i": 0, "flops": 0}

        def run():
            r = int(rows[state["i"] % len(rows)])
            O.attention(qs[state["i"] % len(rows)], keff[:r + 1], v[:r + 1], np.full(HQ // HKV, r, np.uint32),
                        True, fp32=True)
            state["i"] += 1
            state["flops"] += (HQ // HKV) * (r + 1) * DIM * 4
        run.state = state
        return run
    c4 = {}
    for nt in (1, threads):
        fns = []

        def mk(slot):
            f = make_rows(slot)
            fns.append(f)
            return f
        calls, dt = rate(mk, leg_s, nt)
        gflops = sum(f.state["flops"] for f in fns) / dt / 1e9
        c4["gflop_per_s" if nt > 1 else "one_thread_gflop_per_s"] = round(gflops, 2)
    c4.update({"threads": threads,
               "ms_per_prompt_extrapolated": round(prefill_flops(4096, HQ, DIM, LAYERS) / (c4["gflop_per_s"] * 1e9) * 1e3, 1),
               "sample": "causal FP32 attention rows (7 query heads of one KV head over a random row's prefix of a "
                         "reconstructed 4096-token layout-B history); the prompt's 721.7 GFLOP at that rate"})
    legs["qwen_prefill_4096"] = c4
    # the single-head shape, one thread
    ph = calibrate_layout_b(128) if layout != "S" else None
    c1 = None
    if ph is not None:
        fn = unit(ph, 4096, 128, 1, True, 99)
        samples = []
        for r in range(-5, 20):
            t0 = time.perf_counter()
            fn()
            if r >= 0:
                samples.append((time.perf_counter() - t0) * 1e6)
        c1 = {"us_median": round(statistics.median(samples), 1), "threads": 1,
              "workload": "1 query, T=4096, d=128, one head, layout B: unpack + reconstruct + FP32 attention; "
                          "5 warm-up and 20 timed calls, the median"}
    return {"value": round(nn * unit_bytes / dtn / 1e9, 4), "unit": "GB/s", "cores": threads, "kind": "port",
            "one_thread_value": round(n1 * unit_bytes / dt1 / 1e9, 4), "nproc": nproc, "cpu_model": cpu_model(),
            "build": "oracle/bgtq_oracle.c, gcc -O3 -march=native -ffp-contract=off -fno-fast-math, built on this host",
            "arithmetic": "fp32 (attention), fp32 FMA chains (reconstruct)",
            "single_head_t4096_d128": c1, "legs": legs,
            "sample": f"(sequence, KV head) units of {CTX} tokens x {HQ // HKV} query heads, d={DIM}: oracle "
                      f"unpack + reconstruct + FP32 attention; {nn} units on {threads} threads in {dtn:.1f} s "
                      f"({n1} units on one thread in {dt1:.1f} s)"}


def calibrate_layout_b(dim):
    from bgtq import calibrate
    return calibrate.layout_b(dim)


def read_profile_value(name, key):
    """A number recorded in a committed profile summary under profiles/, if present."""
    f = ROOT / "profiles" / name
    if f.exists():
        m = re.search(re.escape(key) + r":\s*([0-9.]+)", f.read_text())
        if m:
            return float(m.group(1))
    return None


def read_traffic():
    """HBM bytes per decode launch from the committed rocprofv3 --pmc summary, if present."""
    f = ROOT / "profiles" / "decode_fast_qwen_b64_t32k_layoutB_pmc.txt"
    if f.exists():
        m = re.search(r"traffic_bytes_per_launch:\s*(\d+)", f.read_text())
        if m:
            return int(m.group(1))
    return None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    # 30 untimed steps (about 0.1 s of back-to-back decode): the GPU's clocks
    # take that long to reach their sustained state; with 3 the timed steps
    # run about 5% slower.
    ap.add_argument("--warmup", type=int, default=30)
    ap.add_argument("--layout", default="B", choices=["A", "B", "S"])
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-extra", action="store_true", help="skip the side measurements")
    ap.add_argument("--eager", action="store_true", help="issue the per-layer launches directly, no HIP graph")
    ap.add_argument("--splits", type=int, default=0, help="token splits per (sequence, KV head); 0 = library choice")
    ap.add_argument("--sweep-splits", default="", help="comma list: time the decode at each split count and exit")
    ap.add_argument("--prefill-only", action="store_true", help="only the Qwen prompt-prefill measurements")
    ap.add_argument("--encode-only", action="store_true", help="only the SmolLM2 bulk K-encode measurement")
    ap.add_argument("--smollm2-step-only", action="store_true", help="only the SmolLM2 batch-1 decode step")
    ap.add_argument("--single-head-only", action="store_true", help="only the single-head T=4096 d=128 line")
    ap.add_argument("--attention-only", action="store_true",
                    help="only the FP32-V attention sessions at the reference's phase-4 benchmark shapes")
    ap.add_argument("--dispatch-step-only", action="store_true",
                    help="only the SmolLM2 decode step through the model dispatch protocol")
    ap.add_argument("--prefill-chunks", default="0,32", help="with --prefill-only: chunk sizes (0 = whole prompt)")
    ap.add_argument("--prefill-layers", type=int, default=LAYERS,
                    help="with --prefill-only: layers of the prompt (fewer for counter passes of a profiler)")
    ap.add_argument("--copy-probe", type=int, default=0, metavar="MIB",
                    help="only run a plain device-to-device copy of MIB MiB three times (HBM counter calibration)")
    a = ap.parse_args()
    if a.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: the decode path shards by (sequence, KV head) with no exchange, "
              "and this build runs on a single MI355X; use --gpus 1", file=sys.stderr)
        sys.exit(2)
    import torch
    if a.copy_probe:
        src = torch.ones(a.copy_probe << 18, dtype=torch.float32, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_probe_bytes": src.numel() * 4}))
        return
    import bgtq
    from bgtq import batched
    dev = bgtq.Device(0)
    batched.bind_torch_stream(dev)
    if a.encode_only:
        print(json.dumps({"encode_smollm2_prefill": encode_throughput(dev, a.layout, max(a.steps, 5))}))
        return
    if a.smollm2_step_only:
        for sp in [int(x) for x in (a.sweep_splits or str(a.splits)).split(",")]:
            print(json.dumps({"splits": sp, "smollm2_decode_step_b1": smollm2_decode_step(dev, a.steps, a.layout, sp)}),
                  flush=True)
        return
    if a.dispatch_step_only:
        print(json.dumps({"smollm2_decode_step_b1_dispatch_path": smollm2_dispatch_step(dev, a.steps)}))
        return
    if a.attention_only:
        print(json.dumps({"phase4_attention_fp32v": phase4_attention(dev)}))
        return
    if a.single_head_only:
        print(json.dumps({"single_head_t4096_d128": single_head(dev, a.steps, a.layout)}))
        return
    if a.prefill_only:
        out = {}
        for c in [int(x) for x in a.prefill_chunks.split(",")]:
            out["qwen_prefill_4096" + (f"_chunk{c}" if c else "")] = qwen_prefill(
                dev, a.steps if not c else 2, a.layout, chunk=c, layers=a.prefill_layers)
        print(json.dumps(out))
        return
    log("building workload ...")
    w = DecodeWorkload(dev, a.layout, splits=a.splits)
    if a.sweep_splits:
        for sp in [int(x) for x in a.sweep_splits.split(",")]:
            w.set_splits(sp)
            ms = time_eager(torch, w.step, a.steps, a.warmup) if a.eager else \
                time_graph(torch, graph_of(torch, dev, w.step), a.steps, a.warmup)
            print(json.dumps({"splits": sp, "ms_per_step": ms, "us_per_launch": ms * 1e3 / LAYERS,
                              "gbs": w.bytes_per_layer() * LAYERS / (ms / 1e3) / 1e9}), flush=True)
        return
    log("timing ...")
    if a.eager:
        ms_step = time_eager(torch, w.step, a.steps, a.warmup)
    else:
        ms_step = time_graph(torch, graph_of(torch, dev, w.step), a.steps, a.warmup)
    ms_eager = time_eager(torch, w.step, max(2, a.steps // 2), 1)
    w.set_q_rotated(True)  # the same step with queries from a baked projection
    ms_rot = time_graph(torch, graph_of(torch, dev, w.step), a.steps, 5)
    w.set_q_rotated(False)
    bytes_layer = w.bytes_per_layer()
    gbs = LAYERS * bytes_layer / (ms_step / 1e3) / 1e9
    ms_launch = ms_step / LAYERS  # one decode launch per layer, back to back in the graph
    achieved = bytes_layer / (ms_launch / 1e3) / 1e9
    extra = {"eager_ms_per_step": round(ms_eager, 4), "q_rotated_ms_per_step": round(ms_rot, 4)}
    log("device ceilings ...")
    ceil = device_ceilings()
    extra["ceilings"] = ceil
    if not a.no_extra:
        del w
        torch.cuda.empty_cache()
        log("FP16-K kernel at the same shape ...")
        wf = DecodeWorkload(dev, key_format="fp16")
        ms_f = time_graph(torch, graph_of(torch, dev, wf.step), max(2, a.steps // 2), 1)
        extra["fp16_k_same_shape"] = {"ms_per_step": round(ms_f, 4), "bytes_per_step": LAYERS * wf.bytes_per_layer(),
                                      "gbs_algorithmic": round(LAYERS * wf.bytes_per_layer() / (ms_f / 1e3) / 1e9, 1)}
        del wf
        torch.cuda.empty_cache()
        log("encode throughput ...")
        extra["encode_smollm2_prefill"] = encode_throughput(dev, a.layout)
        log("SmolLM2 decode step ...")
        extra["smollm2_decode_step_b1"] = smollm2_decode_step(dev, a.steps, a.layout)
        extra["smollm2_decode_step_b1"]["working_set_bytes"] = SmolLM2Step.L * SmolLM2Step.HKV * (
            SmolLM2Step.T + 1) * (layout_params(a.layout, 64).rowBytes + 2 * layout_params(a.layout, 64).normStride + 128)
        extra["smollm2_decode_step_b1"]["residency"] = ("the step's caches fit the 256 MB Infinity Cache: replays read "
                                                        "them from there; the step is a chain of 30 latency-bound "
                                                        "launches, not an HBM rate")
        if a.layout == "B":
            log("SmolLM2 decode step through the model dispatch protocol ...")
            extra["smollm2_decode_step_b1_dispatch_path"] = smollm2_dispatch_step(dev, a.steps)
        log("single head ...")
        # layout S exists at d=64 only (the SmolLM2 calibration)
        extra["single_head_t4096_d128"] = single_head(dev, a.steps, a.layout) if a.layout != "S" else None
        log("FP32-V attention sessions at the phase-4 shapes ...")
        extra["phase4_attention_fp32v"] = phase4_attention(dev)
        log("Qwen prefill, one chunk ...")
        extra["qwen_prefill_4096"] = qwen_prefill(dev, max(2, a.steps // 2), a.layout)
        log("Qwen prefill, chunks of 32 ...")
        extra["qwen_prefill_4096_chunk32"] = qwen_prefill(dev, 2, a.layout, chunk=32)
        for k in ("qwen_prefill_4096", "qwen_prefill_4096_chunk32"):
            extra[k]["mfma_frac_of_measured_ceiling"] = round(
                extra[k]["attention_tflops_algorithmic"] / ceil["mfma_f16_tflops"], 4)
    cpu = None if a.no_cpu else cpu_baseline(a.layout)
    rec = {
        "metric": METRIC, "value": round(gbs, 1), "unit": "GB/s", "n_gpus": 1, "steps": a.steps, "warmup": a.warmup,
        "ms_per_step": round(ms_step, 4), "us_per_layer": round(ms_step * 1e3 / LAYERS, 2),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "fp32 (u8 codes, fp16 scales and V; fp16 hi/lo split MFMA, fp32 accumulate)",
        "data": "synthetic N(0,1) K/V/Q, K encoded by the library",
        "config": {"workload": f"Qwen2.5-0.5B-geometry decode attention: batch {BATCH} x {CTX} ctx, {LAYERS} layers, "
                               f"{HQ} q / {HKV} kv heads, d={DIM}, layout {a.layout} (u8 codes, f16 scales), "
                               f"FP16 V, f32 accumulate",
                   "global_batch": BATCH, "seq_len": CTX, "parallelism": "single GPU",
                   "launch": "eager" if a.eager else "hip graph of 24 per-layer launches"},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": read_traffic(),
                     "traffic_source": "profiles/decode_fast_qwen_b64_t32k_layoutB_pmc.txt (rocprofv3 --pmc "
                                       "FETCH_SIZE / WRITE_SIZE of this launch, calibrated on a copy; committed, "
                                       "not measured in this run)",
                     "frac_of_measured_read_ceiling": round(achieved / ceil["hbm_read_gbs"], 4),
                     "kernel": "decode_fast_kernel<64,1,1,1,0,0,0,4,0> (one launch per layer)",
                     "bytes_per_launch": bytes_layer},
        "cpu_baseline": cpu,
        **extra,
    }
    print(json.dumps(rec))
    dev.destroy()


if __name__ == "__main__":
    main()
