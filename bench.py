"""Benchmark: compressed-K decode attention at Qwen2.5-0.5B geometry on one MI355X.

Workload (one step): decode attention for all 24 layers of 64 independent
sequences x 32768 context tokens, 14 query heads over 2 KV heads (GQA 7:1),
head_dim 64. K is Block-GTQ packed with layout B (widths 4/8 half each, 6.0
bits average: 48 code bytes + 2 FP16 scales per token-head), V is FP16. Inputs
are synthetic N(0,1), encoded by the library's own encoder, resident in HBM
before timing. Per layer and (sequence, KV head): T*(48 + 4 + 128) bytes.

    python bench.py [--steps K] [--warmup W] [--layout B|A] [--no-cpu]

Prints one JSON line (value = algorithmic HBM GB/s of the decode step).
"""
from __future__ import annotations

import argparse
import json
import os
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


def layout_params(name, dim):
    from bgtq import calibrate
    return calibrate.layout_b(dim) if name == "B" else calibrate.layout_a(dim)


class DecodeWorkload:
    """All layers' caches for the C5 shape, plus per-layer descriptors."""

    def __init__(self, dev, layout="B", layers=LAYERS, batch=BATCH, ctx=CTX, hq=HQ, hkv=HKV, dim=DIM, seed=0,
                 key_format="packed"):
        import torch
        import bgtq
        from bgtq import batched
        self.torch, self.dev = torch, dev
        self.layers, self.batch, self.ctx, self.hq, self.hkv, self.dim = layers, batch, ctx, hq, hkv, dim
        g = torch.Generator(device="cuda")
        g.manual_seed(seed)
        self.tables, self.descs, self.keep = [], [], []
        p = layout_params(layout, dim) if key_format == "packed" else None
        self.row_bytes = p.rowBytes if p else 2 * dim
        self.norm_stride = p.normStride if p else 0
        self.lengths = torch.full((batch,), ctx, dtype=torch.int32, device="cuda")
        self.out = torch.empty((batch, hq, dim), dtype=torch.float32, device="cuda")
        ws = None
        for layer in range(layers):
            q = torch.randn((batch, hq, dim), generator=g, device="cuda", dtype=torch.float32)
            v = torch.randn((batch, hkv, ctx, dim), generator=g, device="cuda", dtype=torch.float32).half()
            k = torch.randn((batch, hkv, ctx, dim), generator=g, device="cuda", dtype=torch.float32).half()
            if key_format == "packed":
                tabs = [bgtq.Tables(dev, p) for _ in range(hkv)]  # one table set per (layer, KV head)
                self.tables += tabs
                packed = torch.empty((batch, hkv, ctx * p.rowBytes + 64), dtype=torch.uint8, device="cuda")
                norms = torch.empty((batch, hkv, ctx * p.normStride + 32), dtype=torch.int16, device="cuda")
                jobs = [dict(tables=tabs[h], src=k[b, h], src_row_stride=dim, rows=ctx, packed=packed[b, h],
                             norms=norms[b, h], dst_row0=0) for b in range(batch) for h in range(hkv)]
                batched.encode(dev, jobs, "f16")
                del k
                kw = dict(tables=tabs, packed=packed, packed_seq_stride=packed.stride(0),
                          packed_head_stride=packed.stride(1), norms=norms, norms_seq_stride=norms.stride(0),
                          norms_head_stride=norms.stride(1))
                self.keep += [packed, norms, v, q]
            else:
                kw = dict(k_f16=k, k_seq_stride=k.stride(0), k_head_stride=k.stride(1))
                self.keep += [k, v, q]
            desc = batched.decode_desc(batch=batch, q_heads=hq, kv_heads=hkv, dim=dim, q=q, out=self.out,
                                       lengths=self.lengths, max_length=ctx, v=v, v_dtype="f16",
                                       v_seq_stride=v.stride(0), v_head_stride=v.stride(1), **kw)
            if ws is None:
                ws = torch.empty(batched.workspace_bytes(desc), dtype=torch.uint8, device="cuda")
            desc = batched.decode_desc(batch=batch, q_heads=hq, kv_heads=hkv, dim=dim, q=q, out=self.out,
                                       lengths=self.lengths, max_length=ctx, v=v, v_dtype="f16",
                                       v_seq_stride=v.stride(0), v_head_stride=v.stride(1), workspace=ws, **kw)
            self.descs.append(desc)
        self.ws = ws
        torch.cuda.synchronize()

    def bytes_per_layer(self):
        per_token = self.row_bytes + 2 * self.norm_stride + 2 * self.dim
        return self.batch * self.hkv * self.ctx * per_token

    def step(self, events=None):
        from bgtq import batched
        for i, d in enumerate(self.descs):
            if events is not None:
                events[i][0].record()
            batched.decode(self.dev, d)
            if events is not None:
                events[i][1].record()


def time_decode(w, steps, warmup):
    torch = w.torch
    for _ in range(warmup):
        w.step()
    torch.cuda.synchronize()
    ev = [[(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in w.descs]
          for _ in range(steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for s in range(steps):
        w.step(ev[s])
    stop.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    total_ms = start.elapsed_time(stop)
    per_launch = [a.elapsed_time(b) for row in ev for a, b in row]
    return total_ms / steps, sum(per_launch) / len(per_launch), wall


def encode_throughput(dev, layout="B", reps=5):
    """Prefill K encode at SmolLM2 geometry: 4096 tokens x 3 KV heads x 30 layers, d=64."""
    import torch
    import bgtq
    from bgtq import batched
    p = layout_params(layout, 64)
    tabs = [bgtq.Tables(dev, p) for _ in range(90)]
    k = torch.randn((30, 4096, 3, 64), device="cuda").half()
    packed = torch.empty((90, 4096 * p.rowBytes + 64), dtype=torch.uint8, device="cuda")
    norms = torch.empty((90, 4096 * p.normStride + 32), dtype=torch.int16, device="cuda")
    jobs = [dict(tables=tabs[l * 3 + h], src=k[l, :, h], src_row_stride=3 * 64, rows=4096, packed=packed[l * 3 + h],
                 norms=norms[l * 3 + h], dst_row0=0) for l in range(30) for h in range(3)]
    batched.encode(dev, jobs, "f16")
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(reps):
        batched.encode(dev, jobs, "f16")
    b.record()
    torch.cuda.synchronize()
    ms = a.elapsed_time(b) / reps
    rows = 30 * 3 * 4096
    for t in tabs:
        t.destroy()
    return {"rows_per_s": rows / (ms / 1e3), "tokens_per_s": 4096 / (ms / 1e3), "ms": ms,
            "gbs_algorithmic": rows * (128 + p.rowBytes + 2 * p.normStride) / (ms / 1e3) / 1e9}


def cpu_baseline(layout="B", budget_s=12.0):
    """The oracle (scalar C, 1 thread) on whole (sequence, KV head) units of the same workload."""
    import numpy as np
    from oracle import oracle as O
    p = layout_params(layout, DIM)
    L = O.Layout(dim=p.dim, groups=p.groups, row_bytes=p.rowBytes, norm_stride=p.normStride, nibble_dims=p.nibbleDims,
                 max_centroids=p.maxCentroids, perm=p.permutation, group_of=p.groupOf, pos_to_cb=p.positionToCodebook,
                 code_lut=p.codeLut, rotation=p.rotation, centroids=p.centroids, offsets=p.offsets,
                 inv_scales=p.inverseScales)
    rng = np.random.default_rng(0)
    k = rng.standard_normal((CTX, DIM)).astype(np.float16).view(np.uint16)
    packed, norms = O.encode_pack(L, k)
    v = rng.standard_normal((CTX, DIM)).astype(np.float16).astype(np.float32)
    q = rng.standard_normal((HQ // HKV, DIM)).astype(np.float32)
    pos = np.full(HQ // HKV, CTX - 1, np.uint32)
    units, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < budget_s or units == 0:
        codes = O.unpack(packed, DIM, p.nibbleDims)
        keff = O.reconstruct(L, codes, norms.view(np.float16).astype(np.float32))
        O.attention(q, keff, v, pos, False)
        units += 1
    dt = time.perf_counter() - t0
    unit_bytes = CTX * (p.rowBytes + 2 * p.normStride + 2 * DIM)
    return {"value": units * unit_bytes / dt / 1e9, "unit": "GB/s", "cores": 1, "kind": "port",
            "sample": f"{units} (sequence, KV head) units of {CTX} tokens x {HQ // HKV} query heads, d={DIM}, "
                      f"oracle unpack+reconstruct+attention, {dt:.1f} s"}


def read_traffic():
    """HBM bytes per decode launch from the committed rocprofv3 --pmc summary, if present."""
    f = ROOT / "profiles" / "decode_c5_layoutB_pmc.json"
    if f.exists():
        return json.loads(f.read_text()).get("traffic_bytes_per_launch")
    return None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--layout", default="B", choices=["A", "B"])
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-extra", action="store_true", help="skip the encode and FP16-K side measurements")
    a = ap.parse_args()
    if a.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: the decode path shards by (sequence, KV head) with no exchange, "
              "and this build runs on a single MI355X; use --gpus 1", file=sys.stderr)
        sys.exit(2)
    import torch
    import bgtq
    from bgtq import batched
    dev = bgtq.Device(0)
    batched.bind_torch_stream(dev)
    log("building workload ...")
    w = DecodeWorkload(dev, a.layout)
    log("timing ...")
    ms_step, ms_launch, wall = time_decode(w, a.steps, a.warmup)
    bytes_layer = w.bytes_per_layer()
    gbs = LAYERS * bytes_layer / (ms_step / 1e3) / 1e9
    achieved = bytes_layer / (ms_launch / 1e3) / 1e9
    extra = {}
    if not a.no_extra:
        del w
        torch.cuda.empty_cache()
        log("encode throughput ...")
        extra["encode_smollm2_prefill"] = encode_throughput(dev, a.layout)
        log("FP16-K baseline kernel ...")
        wf = DecodeWorkload(dev, key_format="fp16")
        ms_f, _, _ = time_decode(wf, max(2, a.steps // 2), 1)
        extra["fp16_k_baseline"] = {"ms_per_step": ms_f,
                                    "gbs_algorithmic": LAYERS * wf.bytes_per_layer() / (ms_f / 1e3) / 1e9}
        del wf
    cpu = None if a.no_cpu else cpu_baseline(a.layout)
    rec = {
        "metric": METRIC, "value": round(gbs, 1), "unit": "GB/s", "n_gpus": 1, "steps": a.steps, "warmup": a.warmup,
        "ms_per_step": round(ms_step, 4), "us_per_layer": round(ms_step * 1e3 / LAYERS, 2),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "u8 codes + f16 scales/V, f32 accumulate",
        "data": "synthetic N(0,1) K/V/Q, K encoded by the library",
        "config": {"workload": f"Qwen2.5-0.5B-geometry decode attention: batch {BATCH} x {CTX} ctx, {LAYERS} layers, "
                               f"{HQ} q / {HKV} kv heads, d={DIM}, layout {a.layout}, FP16 V",
                   "global_batch": BATCH, "seq_len": CTX, "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": read_traffic(),
                     "kernel": "bgtq decode (per-layer launch)", "bytes_per_launch": bytes_layer},
        "cpu_baseline": cpu,
        **extra,
    }
    print(json.dumps(rec))
    dev.destroy()


if __name__ == "__main__":
    main()
