#!/usr/bin/env python3
"""Decode-layer benchmark on one MI355X — BASELINE.json's metric on configs[1]: the 27B-class NVFP4 gated MLP
(gate|up 2×[17408×5120] with the silu·mul epilogue, then down [5120×17408] with the residual add) at M = 1 decode,
with the M = 8 verify step measured beside it.

One step = one MLP forward over one token batch. Inputs and weights are resident in HBM before the timed region;
the weights rotate through ≥ 2 GB of distinct copies so the 256 MB MALL cannot serve them. Synthetic data:
weights N(0, 0.02) quantized with the reference NVFP4 rule, activations N(0, 1) in BF16.

Prints ONE JSON line. ``value`` is the MLP's algorithmic HBM GB/s at M = 1; ``roofline`` is for the dominant kernel
(the gate|up GEMV); ``cpu_baseline`` times the C/OpenMP restatement of the reference's CPU oracle GEMV on the host.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "lithos-metal_amd"))

HIDDEN, INTER = 5120, 17408
HBM_PEAK_GBS = 8000.0


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=200)
    p.add_argument("--warmup", type=int, default=20)
    p.add_argument("--copies-gb", type=float, default=2.2)
    p.add_argument("--cpu-seconds", type=float, default=12.0)
    p.add_argument("--no-cpu", action="store_true")
    return p.parse_args()


def mlp_bytes(m: int) -> int:
    w = 3 * INTER * HIDDEN * 9 // 16                   # three NVFP4 matrices: 0.5 B codes + 1/16 B scales per weight
    act = m * HIDDEN * 2 + m * INTER * 2                 # gate|up: x in, act out
    act += m * INTER * 2 + m * HIDDEN * 2 * 2            # down: act in, residual in, y out
    return w + act


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU (each box here has one MI355X); --gpus {args.gpus} is not "
              f"supported — the multi-GPU sharding is described in DESIGN.md", file=sys.stderr)
        sys.exit(2)
    import torch
    from monolith_mi355 import kernels
    from monolith_mi355.formats import device as DV
    from monolith_mi355.runtime import hip

    hip.load()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    g = torch.Generator(device=dev)
    g.manual_seed(1)

    # ---- weights: quantize once, replicate into distinct HBM copies --------------------------------------------
    def quant(n, k):
        w = torch.randn(n, k, generator=g, device=dev) * 0.02
        return DV.nvfp4_quantize(w)
    gc, gs, g2 = quant(INTER, HIDDEN)
    uc, us, u2 = quant(INTER, HIDDEN)
    dc, ds, d2 = quant(HIDDEN, INTER)
    gu_codes = DV.interleave_rows(gc, uc)
    gu_scales = DV.interleave_rows(gs, us)
    gu_rs = DV.interleave_rows(torch.full((INTER, 1), g2, device=dev), torch.full((INTER, 1), u2, device=dev)).reshape(-1)
    gu_pack = DV.pack_nvfp4(gu_codes, gu_scales)
    dn_pack = DV.pack_nvfp4(dc, ds)
    dn_rs = torch.full((HIDDEN,), d2, device=dev)
    del gc, gs, uc, us, dc, ds, gu_codes, gu_scales
    per_copy = gu_pack.numel() + dn_pack.numel()
    copies = max(2, int(args.copies_gb * 1e9 // per_copy) + 1)
    gu_w = [kernels.PackedWeight("nvfp4", 2 * INTER, HIDDEN, 1, gu_pack.clone(), gu_rs) for _ in range(copies)]
    dn_w = [kernels.PackedWeight("nvfp4", HIDDEN, INTER, 1, dn_pack.clone(), dn_rs) for _ in range(copies)]

    def run(m, steps, warmup):
        x = torch.randn(m, HIDDEN, generator=g, device=dev).to(torch.bfloat16)
        h = torch.randn(m, HIDDEN, generator=g, device=dev).to(torch.bfloat16)
        act = torch.empty(m, INTER, dtype=torch.bfloat16, device=dev)
        y = torch.empty(m, HIDDEN, dtype=torch.bfloat16, device=dev)
        stream = torch.cuda.current_stream()

        def step(i):
            kernels.gemv(gu_w[i % copies], x, epilogue="silu_mul", out=act)
            kernels.gemv(dn_w[i % copies], act, epilogue="residual", residual=h, out=y)

        for i in range(warmup):
            step(i)
        torch.cuda.synchronize()
        # the timed steps as one HIP graph, so host launch cost is not in the number
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            for i in range(steps):
                step(i)
        graph.replay()
        torch.cuda.synchronize()
        t0 = hip.Event(); t1 = hip.Event()
        torch.cuda.synchronize()
        t0.record(stream)
        graph.replay()
        t1.record(stream)
        t1.synchronize()
        ms = t0.elapsed_ms(t1) / steps
        # the dominant kernel alone (gate|up GEMV), HIP events on the stream it is launched on
        kg = torch.cuda.CUDAGraph()
        with torch.cuda.graph(kg):
            for i in range(steps):
                kernels.gemv(gu_w[i % copies], x, epilogue="silu_mul", out=act)
        kg.replay()
        torch.cuda.synchronize()
        t0.record(stream)
        kg.replay()
        t1.record(stream)
        t1.synchronize()
        k_ms = t0.elapsed_ms(t1) / steps
        return ms, k_ms

    ms1, kms1 = run(1, args.steps, args.warmup)
    ms8, kms8 = run(8, args.steps, args.warmup)
    b1, b8 = mlp_bytes(1), mlp_bytes(8)
    gbs1 = b1 / (ms1 * 1e-3) / 1e9
    gbs8 = b8 / (ms8 * 1e-3) / 1e9
    gu_bytes = 2 * INTER * HIDDEN * 9 // 16 + HIDDEN * 2 + INTER * 2
    k_gbs = gu_bytes / (kms1 * 1e-3) / 1e9

    traffic = None
    prof = ROOT / "profiles" / "gemv_nvfp4_gateup_m1_traffic.json"
    if prof.exists():
        traffic = json.loads(prof.read_text()).get("hbm_bytes_per_launch")

    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(args.cpu_seconds)

    line = {
        "metric": "decode-layer HBM GB/s (% of peak) + tokens/s at M=1 and M=8, one MI355X",
        "value": round(gbs1, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms1, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "nvfp4 weights x bf16 activations, fp32 accumulate",
        "data": "synthetic: weights N(0,0.02) quantized to NVFP4 (reference rule), activations N(0,1) bf16",
        "config": {"workload": "27B NVFP4 gated MLP decode step: gate|up 2x[17408x5120] silu_mul + down "
                               "[5120x17408] residual (BASELINE configs[1])", "m": 1, "hidden": HIDDEN,
                   "intermediate": INTER, "weight_copies": copies, "bytes_per_step": b1},
        "pct_of_hbm_peak": round(100 * gbs1 / HBM_PEAK_GBS, 2),
        "tokens_per_s_m1": round(1e3 / ms1, 1),
        "m8": {"ms_per_step": round(ms8, 5), "GB/s": round(gbs8, 1), "pct_of_hbm_peak": round(100 * gbs8 / HBM_PEAK_GBS, 2),
               "tokens_per_s": round(8e3 / ms8, 1), "bytes_per_step": b8},
        "roofline": {"kernel": "gemv (NVFP4 gate|up 34816x5120, silu_mul, M=1)", "bound": "hbm",
                     "achieved": round(k_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(k_gbs / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "algorithmic_bytes": gu_bytes, "avg_launch_us": round(kms1 * 1e3, 3),
                     "m8_avg_launch_us": round(kms8 * 1e3, 3)},
        "cpu_baseline": cpu,
    }
    print(json.dumps(line))


def cpu_baseline(seconds: float):
    """The C/OpenMP restatement of the reference's oracle GEMV (dequantize to FP32, multiply) on this host's cores,
    over the down projection [5120×17408] at M = 1, repeated for about ``seconds``; reported as the same MLP GB/s
    figure (the MLP's bytes ÷ three GEMVs' time at that rate)."""
    import numpy as np
    sys.path.insert(0, str(ROOT))
    from oracle import cpu as OC
    rng = np.random.default_rng(0)
    m = {"weight": rng.integers(0, 256, size=(HIDDEN, INTER // 2), dtype=np.uint8),
         "weight_scale": rng.integers(0x20, 0x48, size=(HIDDEN, INTER // 16), dtype=np.uint8),
         "weight_scale_2": 0.02 / (6 * 448) * 64}
    x = rng.standard_normal((1, INTER)).astype(np.float32)
    nt = OC.threads()
    OC.nvfp4_gemv(m, x, nt)
    reps, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        OC.nvfp4_gemv(m, x, nt)
        reps += 1
    dt = (time.perf_counter() - t0) / reps
    w_bytes = HIDDEN * INTER * 9 // 16
    gbs = w_bytes / dt / 1e9
    return {"value": round(gbs, 2), "unit": "GB/s", "cores": nt, "kind": "port",
            "sample": f"{reps} runs of the NVFP4 down GEMV [5120x17408] at M=1 ({seconds:.0f} s), "
                      f"{dt * 1e3:.2f} ms each; MLP step at this rate = {3 * dt * 1e3:.1f} ms"}


if __name__ == "__main__":
    main()
