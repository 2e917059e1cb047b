"""Benchmark: batched bf16 Newton–Schulz (NS5) on one MI355X.

Workload (one "step"): NS5, 5 quintic iterations, on 32 bf16 matrices
4096x4096 plus 32 bf16 matrices 4096x11008 (Llama-7B-like projection
shapes), inputs = Nesterov momentum (β=0.95) of three seeded N(0, 1e-3)
gradients, resident in HBM before timing. Two batched calls of
pytorch_opt.ops.newton_schulz_orthogonalize through the HIP library.

Prints one JSON line: the metric (algorithmic TFLOP/s, LAWN-41 counting),
the roofline of the dominant kernel (timed live with HIP events on its own
stream), the CPU oracle's rate on a bounded sample of the same workload,
and the single-matrix 4096² figure.
"""

from __future__ import annotations

import argparse
import json
import os
import subprocess
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "pytorch-opt_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

BF16_PEAK_TFLOPS = 2516.6  # MI355X dense bf16 MFMA (256 CU x 2.4 GHz x 4096 flop/clk)
SHAPES = [(32, 4096, 4096, 1000), (32, 4096, 11008, 2000)]  # (batch, rows, cols, seed base)


def ns5_flops(m, n, steps=5):
    m, n = min(m, n), max(m, n)
    return steps * (m * (m + 1) * n + m * m * (m + 1) + 2 * m * m * n)


def kernel_flops(kind, m, n):
    """Algorithmic flops of one NS5 iteration's launch of `kind`, per matrix."""
    m, n = min(m, n), max(m, n)
    return {"ns5_gram": m * (m + 1) * n, "ns5_square": m * m * (m + 1), "ns5_update": 2 * m * m * n}[kind]


def make_inputs(torch, batch, rows, cols, seed0, dev):
    out = torch.empty(batch, rows, cols, dtype=torch.bfloat16, device=dev)
    for i in range(batch):
        g = torch.Generator(device=dev).manual_seed(seed0 + i)
        buf = torch.zeros(rows, cols, device=dev)
        gt = None
        for _ in range(3):
            gt = 1e-3 * torch.randn(rows, cols, generator=g, device=dev)
            buf.mul_(0.95).add_(gt)
        out[i] = (gt + 0.95 * buf).bfloat16()
    return out


def cpu_baseline(inputs):
    """The numpy oracle (fp32, OpenBLAS) on one matrix of each shape, scaled
    linearly to the 32 + 32 batch."""
    import numpy as np
    from threadpoolctl import threadpool_info

    from oracle import ops_oracle as oo

    threads = max([d.get("num_threads", 1) for d in threadpool_info() if d.get("user_api") == "blas"] or [1])
    total_s = 0.0
    for (batch, rows, cols, _), G in zip(SHAPES, inputs):
        x = G[0].float().cpu().numpy()
        oo.ns5(x[:256, :512])  # warm the BLAS threads
        t0 = time.perf_counter()
        oo.ns5(x)
        total_s += (time.perf_counter() - t0) * batch
    flops = sum(b * ns5_flops(r, c) for b, r, c, _ in SHAPES)
    try:
        model = subprocess.run(["bash", "-c", "lscpu | grep 'Model name' | head -1"], capture_output=True,
                               text=True).stdout.split(":", 1)[-1].strip()
    except Exception:
        model = ""
    return {"value": flops / total_s / 1e12, "unit": "TFLOP/s", "cores": int(threads), "kind": "port",
            "sample": "oracle NS5 (numpy fp32) on 1 matrix 4096x4096 + 1 matrix 4096x11008 of the same inputs, "
                      f"time scaled x32 each; est. full workload {total_s:.1f} s; host {model}, nproc "
                      f"{os.cpu_count()}"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=5)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only; --gpus {args.gpus} is not supported "
              "(matrices shard by whole matrices across GPUs; see the design notes).", file=sys.stderr)
        sys.exit(2)

    import torch

    from pytorch_opt import ops

    if not ops.load_native():
        raise RuntimeError("libpytorch_opt_hip.so did not load; run __graft_entry__.build()")
    ops.set_backend("native")
    hip = ops._NATIVE
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    inputs = [make_inputs(torch, b, r, c, s, dev) for b, r, c, s in SHAPES]
    torch.cuda.synchronize()

    def step():
        return [ops.newton_schulz_orthogonalize(G) for G in inputs]

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()

    hip.prof_reset()
    hip.prof_enable(True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        outs = step()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    hip.prof_enable(False)
    del outs

    ms_per_step = wall * 1e3 / args.steps
    flops_step = sum(b * ns5_flops(r, c) for b, r, c, _ in SHAPES)
    value = flops_step / (ms_per_step / 1e3) / 1e12

    kinds = {}
    for kind in ("ns5_gram", "ns5_square", "ns5_update"):
        ms, launches = hip.prof_query(kind)
        fl = args.steps * 5 * sum(b * kernel_flops(kind, r, c) for b, r, c, _ in SHAPES)
        kinds[kind] = {"ms_total": ms, "launches": launches, "avg_ms": ms / max(launches, 1),
                       "tflops": fl / (ms / 1e3) / 1e12 if ms > 0 else None}
    dom = max(kinds, key=lambda k: kinds[k]["ms_total"])
    achieved = kinds[dom]["tflops"]

    # single 4096x4096 matrix (the headline shape, unbatched)
    single = inputs[0][:1].contiguous()
    for _ in range(3):
        ops.newton_schulz_orthogonalize(single)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    reps = 10
    e0.record()
    for _ in range(reps):
        ops.newton_schulz_orthogonalize(single)
    e1.record()
    torch.cuda.synchronize()
    single_ms = e0.elapsed_time(e1) / reps
    single_tflops = ns5_flops(4096, 4096) / (single_ms / 1e3) / 1e12

    cpu = None if args.no_cpu_baseline else cpu_baseline(inputs)

    line = {
        "metric": "NS5 TFLOP/s (algorithmic, LAWN-41) on 32x4096^2 + 32x4096x11008 bf16, 5 iterations",
        "value": round(value, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic: seeded N(0,1e-3) gradients folded into Nesterov momentum (beta 0.95, 3 steps)",
        "config": {"workload": "batched NS5 bf16: 32 x 4096x4096 + 32 x 4096x11008, 5 quintic iterations",
                   "alg_flops_per_step": flops_step, "pct_bf16_mfma_peak": round(100 * value / BF16_PEAK_TFLOPS, 2),
                   "peak_tflops": BF16_PEAK_TFLOPS},
        "roofline": {"bound": "mfma", "kernel": dom, "achieved": round(achieved, 2), "peak": BF16_PEAK_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(achieved / BF16_PEAK_TFLOPS, 4), "traffic": None},
        "kernels": {k: {kk: (round(vv, 4) if isinstance(vv, float) else vv) for kk, vv in v.items()}
                    for k, v in kinds.items()},
        "single_4096": {"ms": round(single_ms, 3), "tflops": round(single_tflops, 2),
                        "pct_bf16_mfma_peak": round(100 * single_tflops / BF16_PEAK_TFLOPS, 2)},
        "cpu_baseline": cpu,
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
