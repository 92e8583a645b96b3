#!/usr/bin/env python3
"""Decode-layer benchmark on one MI355X — BASELINE.json's metric: decode-layer HBM GB/s (% of the 8 TB/s peak) and
tokens/s at M = 1 and M = 8.

The workload (``config.workload``) is one 27B-class decode layer, ``h += mixer(norm1(h)); h += mlp(norm2(h))``:
a Gated DeltaNet mixer (16 key / 48 value heads of 128, conv 4; in_proj 16480×5120 and out_proj 5120×6144 NVFP4)
and the NVFP4 gated MLP of BASELINE configs[1] (gate|up 2×17408×5120 with silu·mul, down 5120×17408 with the
residual). ``value`` is that layer's algorithmic HBM bytes ÷ its step time at M = 1. Beside it: the same layer at
M = 8, the gated-GQA layer (24 q / 4 KV heads of 128, int8 KV cache at a 32K context; configs[2]) at M = 1 and 8,
and the MLP alone; the FP8 E4M3 GEMV (the 27B checkpoint's format for its mixer projections) at the
GDN in_proj shape with its fused norm, M = 1 and 8; the hybrid MoE layer's feed-forward (configs[4]: router, top-8 of
256 NVFP4 experts, shared expert, combine), M = 1 and 8; and the GPU-resident token loop (embedding, a GDN and an
attention layer, the BF16 LM head over a 248320-token vocabulary, argmax and advance, replayed as a graph by the
native pump; wall time per token), and the speculative round on the same model (eight rows verified per step).

One step = one layer forward over one token batch. Weights, states and KV caches are resident in HBM before the
timed region; the step rotates over ``--layers`` distinct layer instances (≥ 2 GB in all), so the 256 MB MALL
cannot serve them — like consecutive layers of one model. The timed steps are one HIP graph (host launch cost is
not in the number), bracketed by HIP events on the stream they run on. Synthetic data: weights N(0, 0.02) quantized
with the reference NVFP4 rule on the GPU, activations N(0, 1) BF16, GDN state N(0, 0.1), KV codes uniform int8.

Per-config lines beside the layer: configs[0] (INT4 4096², M = 1, rotated over ≥ 2 GiB of copies), each
configs[1] GEMV alone (gate|up, down; M = 1 and 8), the configs[2] attention core alone at 4K / 16K / 32K (M = 1
and 8, ≥ 2 GiB of KV caches rotated) and the configs[3] Gated DeltaNet step alone (M = 1 and 8, ≥ 2 GiB of states
rotated).

Prints ONE JSON line. ``roofline`` is for the dominant kernel (the gate|up GEMV, 34816×5120 NVFP4 at M = 1) timed
alone the same way; ``cpu_baseline`` times the reference's CPU path for the same layer on the host (numpy and the
C/OpenMP restatement of its oracle GEMV, M = 1 and 8) and configs[0] on one core.
"""

from __future__ import annotations

import argparse
import json
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "lithos-metal_amd"))

HBM_PEAK_GBS = 8000.0
CTX = 32768


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=100)
    p.add_argument("--warmup", type=int, default=10)
    p.add_argument("--layers", type=int, default=10, help="distinct layer instances the steps rotate over")
    p.add_argument("--cpu-seconds", type=float, default=20.0)
    p.add_argument("--no-cpu", action="store_true")
    p.add_argument("--only", choices=["gdn", "attn", "mlp", "gateup", "gemv", "fp8", "int4", "gqa", "gdnstep", "moe", "loop", "copy"], default=None,
                   help="time one workload only (profiling runs; copy = a 256 MiB device copy, the counter reference)")
    return p.parse_args()


def timed_graph(fn, steps, warmup, stream):
    """Run ``fn(i)`` for ``warmup`` steps eagerly, capture ``steps`` of them as one graph, replay twice and time the
    second replay with HIP events on ``stream``. Returns ms per step."""
    import torch
    from monolith_mi355.runtime import hip
    for i in range(warmup):
        fn(i)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        for i in range(steps):
            fn(i)
    graph.replay()
    torch.cuda.synchronize()
    t0, t1 = hip.Event(), hip.Event()
    t0.record(stream)
    graph.replay()
    t1.record(stream)
    t1.synchronize()
    return t0.elapsed_ms(t1) / steps


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU (each box here has one MI355X); --gpus {args.gpus} is not "
              f"supported — the multi-GPU sharding is design-only in this build", file=sys.stderr)
        sys.exit(2)
    import torch
    from monolith_mi355 import kernels
    from monolith_mi355.layers import AttnDecoderLayer, GdnDecoderLayer
    from monolith_mi355.runtime import hip

    hip.load()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    stream = torch.cuda.Stream(dev)
    gen = torch.Generator(device=dev)
    gen.manual_seed(1)
    n = args.layers
    out = {}

    def xin(m):
        return torch.randn(m, 5120, generator=gen, device=dev).to(torch.bfloat16)

    if args.only == "copy":
        # a plain device-to-device copy of known size: what HBM counters read for 256 MiB in + 256 MiB out
        with torch.cuda.stream(stream):
            srcs = [torch.empty(64 << 20, dtype=torch.float32, device=dev).fill_(1.0) for _ in range(4)]
            dst = torch.empty(64 << 20, dtype=torch.float32, device=dev)
            ms = timed_graph(lambda i: dst.copy_(srcs[i % 4]), 20, 2, stream)
        print(json.dumps({"copy": {"ms": round(ms, 5), "bytes_read": 256 << 20, "bytes_written": 256 << 20}}))
        return

    def chained(layers, x, *args):
        """One layer of a chain: at M >= 3 a layer reads its normalized input (written by the layer before) and
        writes the next one's inside its MLP's split-K reduction; at M <= 2 each layer normalizes its own input."""
        if x.shape[0] < 3:
            return lambda i: layers[i % n].step(x, *args)
        xins = [kernels.norm_apply(x, layer.norm_w, eps=layer.eps) for layer in layers]
        xn = torch.empty_like(x)
        return lambda i: layers[i % n].step(x, *args, x_in=xins[i % n],
                                            next_norm=(layers[(i + 1) % n].norm_w, xn, layers[(i + 1) % n].eps))

    with torch.cuda.stream(stream):
        gdn = [GdnDecoderLayer(seed=10 + i, device=dev) for i in range(n)] if args.only in (None, "gdn", "mlp", "gateup", "gemv") else []
        for m in (1, 8):
            if args.only not in (None, "gdn"):
                break
            x = xin(m)
            ms = timed_graph(chained(gdn, x), args.steps, args.warmup, stream)
            out[f"gdn_m{m}"] = (ms, gdn[0].bytes_per_step(m))
        for m in (1, 8):
            if args.only not in (None, "mlp"):
                break
            x = xin(m)
            ms = timed_graph(lambda i: gdn[i % n].mlp(x), args.steps, args.warmup, stream)
            out[f"mlp_m{m}"] = (ms, gdn[0].mlp.bytes_per_step(m))
        if args.only in (None, "gateup"):
            x = xin(1)
            act = torch.empty(1, 17408, dtype=torch.bfloat16, device=dev)
            ms = timed_graph(lambda i: kernels.gemv(gdn[i % n].mlp.gate_up.packed, x, epilogue="silu_mul", out=act),
                             args.steps, args.warmup, stream)
            out["gateup_m1"] = (ms, 34816 * 5120 * 9 // 16 + 5120 * 2 + 17408 * 2)
        if args.only in (None, "gemv"):
            # each MLP GEMV alone — gate|up (silu·mul) and down (+ residual) at M = 1 and 8
            for m in (1, 8):
                x, xa = xin(m), torch.randn(m, 17408, generator=gen, device=dev).to(torch.bfloat16)
                act = torch.empty(m, 17408, dtype=torch.bfloat16, device=dev)
                y = torch.empty(m, 5120, dtype=torch.bfloat16, device=dev)
                if m > 1:
                    ms = timed_graph(lambda i: kernels.gemv(gdn[i % n].mlp.gate_up.packed, x, epilogue="silu_mul",
                                                            out=act), args.steps, args.warmup, stream)
                    out[f"gateup_m{m}"] = (ms, 34816 * 5120 * 9 // 16 + m * 5120 * 2 + m * 17408 * 2)
                ms = timed_graph(lambda i: kernels.gemv(gdn[i % n].mlp.down.packed, xa, epilogue="residual", residual=x,
                                                        out=y), args.steps, args.warmup, stream)
                out[f"down_m{m}"] = (ms, 5120 * 17408 * 9 // 16 + m * 17408 * 2 + 2 * m * 5120 * 2)
        del gdn
        torch.cuda.empty_cache()
        if args.only in (None, "fp8"):
            # the 27B checkpoint's mixer projections are FP8 E4M3: the GDN in_proj shape (16480×5120) with its fused
            # norm, M = 1 and 8; random finite codes drawn straight in the packed layout, a per-row tensor scale
            n8, k8 = 16480, 5120
            nb = (n8 + 15) // 16 * 16 * k8
            mats = []
            for i in range(n):
                c = torch.randint(0, 253, (nb,), dtype=torch.int16, generator=gen, device=dev)
                c = (c + (c >= 0x7F).to(torch.int16)).to(torch.uint8)            # every code but the NaNs
                rs = torch.full(((n8 + 15) // 16 * 16,), 1e-3, dtype=torch.float32, device=dev)
                mats.append(kernels.PackedWeight("fp8_e4m3", n8, k8, 1, c, rs))
            nw = 1.0 + torch.randn(k8, generator=gen, device=dev) * 0.1
            for m in (1, 8):
                x = xin(m)
                y8 = torch.empty(m, n8, dtype=torch.bfloat16, device=dev)
                ms = timed_graph(lambda i: kernels.gemv(mats[i % n], x, norm_w=nw, out=y8), args.steps, args.warmup,
                                 stream)
                out[f"fp8_m{m}"] = (ms, nb + m * k8 * 2 + m * n8 * 2)
            del mats
        if args.only in (None, "int4"):
            # affine 4-bit (MLX rule, group 64, BF16 scale + bias), weights N(0, 0.02) quantized by the product's
            # quantizer: configs[0] (4096², M = 1) rotated over ≥ 2 GiB of distinct device copies (one per launch of
            # the timed graph, so the 256 MB MALL holds none of them), and the 27B gate|up shape with silu·mul
            # (M = 1 and 8; 512 quantized rows repeated down the matrix, ten device copies)
            from monolith_mi355.formats import DequantSpec, INT4Affine
            import numpy as np
            rng = np.random.default_rng(1)

            def int4_matrix(n4, k4, block=512):
                q = INT4Affine().quantize(rng.standard_normal((min(block, n4), k4)).astype(np.float32) * 0.02)
                reps = -(-n4 // q.tensors["weight"].shape[0])
                t = {k_: np.tile(v, (reps, 1))[:n4].copy() for k_, v in q.tensors.items()}
                return kernels.upload(DequantSpec("int4_affine", (n4, k4), t, dict(q.params)), device=dev)

            c1 = int4_matrix(4096, 4096, block=4096)
            c1_copies = -(-(2 << 30) // c1.nbytes)
            mats = [c1] + [kernels.PackedWeight("int4_affine", 4096, 4096, 1, c1.data.clone(), None)
                           for _ in range(c1_copies - 1)]
            x = torch.randn(1, 4096, generator=gen, device=dev).to(torch.bfloat16)
            y4 = torch.empty(1, 4096, dtype=torch.bfloat16, device=dev)
            ms = timed_graph(lambda i: kernels.gemv(mats[i % len(mats)], x, out=y4), max(args.steps, len(mats)),
                             args.warmup, stream)
            out["int4_4096_m1"] = (ms, 4096 * 4096 * 9 // 16 + 4096 * 2 + 4096 * 2)
            c1_info = {"copies_rotated": len(mats), "bytes_rotated": len(mats) * c1.nbytes}
            del mats, c1
            gu = int4_matrix(34816, 5120)
            mats = [gu] + [kernels.PackedWeight("int4_affine", 34816, 5120, 1, gu.data.clone(), None)
                           for _ in range(n - 1)]
            for m in (1, 8):
                x = torch.randn(m, 5120, generator=gen, device=dev).to(torch.bfloat16)
                y4 = torch.empty(m, 17408, dtype=torch.bfloat16, device=dev)
                ms = timed_graph(lambda i: kernels.gemv(mats[i % len(mats)], x, epilogue="silu_mul", out=y4),
                                 args.steps, args.warmup, stream)
                out[f"int4_gateup_m{m}"] = (ms, 34816 * 5120 * 9 // 16 + m * 5120 * 2 + m * 17408 * 2)
            del mats, gu
        if args.only in (None, "gqa"):
            # the attention core alone (q/k norm, RoPE, int8 append, attention, gate) at 4K / 16K / 32K,
            # M = 1 and 8, rotated over ≥ 2 GiB of distinct KV caches (one per launch of the timed graph)
            from monolith_mi355.kernels import KVCache
            cos, sin = kernels.rope_tables(1e6, 64, CTX, device=dev)
            qn = 1.0 + torch.randn(128, generator=gen, device=dev) * 0.1
            kn = 1.0 + torch.randn(128, generator=gen, device=dev) * 0.1
            for ctx in (4096, 16384, 32768):
                per = ctx * 4 * (2 * 128 + 4)
                caches = [KVCache(4, ctx, 128, device=dev) for _ in range(-(-(2 << 30) // per))]
                for c in caches:
                    c.k_codes.random_(-127, 128, generator=gen)
                    c.v_codes.random_(-127, 128, generator=gen)
                    c.k_scales.fill_(3.0 / 127)
                    c.v_scales.fill_(3.0 / 127)
                for m in (1, 8):
                    pos = ctx - 16
                    proj = torch.randn(m, 7168, generator=gen, device=dev).to(torch.bfloat16)
                    o = torch.empty(m, 3072, dtype=torch.bfloat16, device=dev)
                    ms = timed_graph(lambda i: kernels.gqa_decode(proj, caches[i % len(caches)], pos, heads=24,
                                                                  rope_cos=cos, rope_sin=sin, q_norm=qn, k_norm=kn,
                                                                  out=o), len(caches), args.warmup, stream)
                    nkv = pos + m
                    out[f"gqa_{ctx // 1024}k_m{m}"] = (ms, nkv * 4 * (2 * 128 + 4) + m * 7168 * 2 + m * 3072 * 2
                                                       + m * 4 * (2 * 128 + 4))
                del caches
                torch.cuda.empty_cache()
            # the reference's own attention geometry (24 / 4 heads of 256, BF16 cache: nn/attention.py:87-89) at 32K
            cos2, sin2 = kernels.rope_tables(1e6, 64, CTX, device=dev)
            qn2 = 1.0 + torch.randn(256, generator=gen, device=dev) * 0.1
            kn2 = 1.0 + torch.randn(256, generator=gen, device=dev) * 0.1
            per = CTX * 4 * 4 * 256
            caches = [KVCache(4, CTX, 256, device=dev, dtype="bf16") for _ in range(-(-(2 << 30) // per))]
            for c in caches:
                c.k_codes.normal_(generator=gen)
                c.v_codes.normal_(generator=gen)
            for m in (1, 8):
                pos = CTX - 16
                proj = torch.randn(m, 24 * 512 + 8 * 256, generator=gen, device=dev).to(torch.bfloat16)
                o = torch.empty(m, 24 * 256, dtype=torch.bfloat16, device=dev)
                ms = timed_graph(lambda i: kernels.gqa_decode(proj, caches[i % len(caches)], pos, heads=24,
                                                              rope_cos=cos2, rope_sin=sin2, q_norm=qn2, k_norm=kn2,
                                                              out=o), len(caches), args.warmup, stream)
                out[f"gqa_ref_m{m}"] = (ms, (pos + m) * 4 * 4 * 256 + m * proj.shape[1] * 2 + m * 6144 * 2
                                        + m * 4 * 4 * 256)
            del caches
            torch.cuda.empty_cache()
        if args.only in (None, "gdnstep"):
            # the Gated DeltaNet step alone (conv, gates, delta rule, gated norm; output bf16) at M = 1
            # and 8, rotated over ≥ 2 GiB of distinct recurrent states (one per launch of the timed graph)
            hk, hv, d = 16, 48, 128
            conv_dim, n1 = 2 * hk * d + hv * d, hv * d + 2 * hk * d + hv * d + 2 * hv
            per = hv * d * d * 4
            count = -(-(2 << 30) // per)
            recs = torch.randn(count, hv, d, d, generator=gen, device=dev) * 0.1
            convs = (torch.randn(count, 2, conv_dim, 3, generator=gen, device=dev) * 0.5).to(torch.bfloat16)
            prm = dict(conv_w=(torch.randn(conv_dim, 4, generator=gen, device=dev) * 0.3).to(torch.bfloat16),
                       neg_exp_a=-torch.ones(hv, device=dev), dt_bias=torch.zeros(hv, device=dev),
                       norm_w=1.0 + torch.randn(d, generator=gen, device=dev) * 0.2)
            for m in (1, 8):
                proj = torch.randn(m, n1, generator=gen, device=dev).to(torch.bfloat16)
                y = torch.empty(m, hv * d, dtype=torch.bfloat16, device=dev)
                ms = timed_graph(lambda i: kernels.gdn_step(proj, convs[i % count, 0], convs[i % count, 1],
                                                            recs[i % count], recs[i % count], k_heads=hk, v_heads=hv,
                                                            out=y, **prm), count, args.warmup, stream)
                out[f"gdnstep_m{m}"] = (ms, 2 * per + 2 * conv_dim * 3 * 2 + conv_dim * 4 * 2 + 3 * hv * 4 + d * 4
                                        + m * n1 * 2 + m * hv * d * 2)
            # the step as the M = 1 layer runs it: the conv done by the input projection's epilogue, the step reading
            # the convolved q|k|v (pre) and the gates, the read-out left to the output projection (defer_norm)
            pre = torch.randn(1, conv_dim, generator=gen, device=dev).to(torch.bfloat16)
            proj = torch.randn(1, n1, generator=gen, device=dev).to(torch.bfloat16)
            y = torch.empty(1, hv * d, dtype=torch.bfloat16, device=dev)
            ms = timed_graph(lambda i: kernels.gdn_step(proj, None, None, recs[i % count], recs[i % count], k_heads=hk,
                                                        v_heads=hv, out=y, pre=pre, defer_norm=True, **prm),
                             count, args.warmup, stream)
            out["gdnstep_pre_m1"] = (ms, 2 * per + conv_dim * 2 + 2 * hv * 2 + 3 * hv * 4 + hv * d * 2)
            del recs, convs
            torch.cuda.empty_cache()
        if args.only in (None, "attn"):
            attn = [AttnDecoderLayer(seed=40 + i, ctx=CTX, device=dev) for i in range(n)]
            for layer in attn:
                layer.fill_cache(CTX, gen)
            pos = CTX - 16
            for m in (1, 8):
                x = xin(m)
                ms = timed_graph(chained(attn, x, pos), args.steps, args.warmup, stream)
                out[f"attn_m{m}"] = (ms, attn[0].bytes_per_step(m, pos))
            del attn

        if args.only in (None, "moe"):
            # the hybrid MoE layer's feed-forward: hidden 2048, 256 NVFP4 experts of 512, top-8 +
            # shared expert; two instances rotate (each ≈ 0.45 GB of experts); bytes count the experts chosen
            from monolith_mi355.layers import MoeBlock
            blocks = [MoeBlock(seed=80 + i, device=dev) for i in range(2)]
            for m in (1, 8):
                x = torch.randn(m, 2048, generator=gen, device=dev).to(torch.bfloat16)
                if m >= 3:      # one block of a chain, the input norm handed over as for the M = 8 layers
                    xins = [kernels.norm_apply(x, b.norm_w, eps=b.eps) for b in blocks]
                    xn = torch.empty_like(x)
                    fn = lambda i: blocks[i % 2](x, x_in=xins[i % 2], next_norm=(blocks[(i + 1) % 2].norm_w, xn,
                                                                                 blocks[(i + 1) % 2].eps))
                else:
                    fn = lambda i: blocks[i % 2](x)
                ms = timed_graph(fn, args.steps, args.warmup, stream)
                distinct = [len(set(b.buffers(m)[1][0][:, :b.top_k].flatten().tolist())) for b in blocks]
                nbytes = sum(b.bytes_per_step(m, d) for b, d in zip(blocks, distinct)) // len(blocks)
                out[f"moe_m{m}"] = (ms, nbytes)
                moe_experts = distinct
            del blocks
        if args.only in (None, "loop"):
            # the GPU-resident token loop: embed → GDN layer → attention layer (32K context) → final norm + BF16
            # lm_head (248320×5120) → argmax → advance, replayed as a graph of 2 steps by the native pump
            from monolith_mi355.layers import DecoderModel
            from monolith_mi355.runtime.step import StepProgram, StepState
            layers = [GdnDecoderLayer(seed=70, device=dev), AttnDecoderLayer(seed=71, ctx=CTX, device=dev)]
            layers[1].fill_cache(CTX - 512, gen)
            model = DecoderModel(layers, vocab=248320, hidden=5120, device=dev)
            st = StepState(ring_capacity=4096, device=dev)
            prog = StepProgram(model, st, ctx_cap=CTX, steps_per_graph=2)
            start = CTX - 512
            st.start(position=start, token=11)
            prog.step_eager(2)
            st.start(position=start, token=11)
            prog.run(32, launches_per_batch=8, in_flight=2)                    # warm
            st.start(position=start, token=11)
            rep = prog.run(256, launches_per_batch=8, in_flight=2)
            loop_ms = rep.wall_ms / rep.steps_submitted
            out["loop"] = (loop_ms, model.step_bytes(start + 128))
            loop_info = {"tokens": len(rep.tokens), "gpu_ms_per_token": round(rep.gpu_ms / rep.steps_submitted, 5),
                         "host_busy_fraction": round(rep.host_busy_ms / rep.wall_ms, 4)}
            del prog, model, layers
            # the speculative round (gamma = 7: eight rows verified per step) on the same two layers + LM head,
            # drafts from a table the accept scan rejects (random ids): the round's time; every row is computed
            # whatever is accepted, so tokens per second scale with the accepted drafts per step
            from monolith_mi355.runtime.step import SpecProgram
            layers = [GdnDecoderLayer(seed=72, device=dev), AttnDecoderLayer(seed=73, ctx=CTX, device=dev)]
            layers[1].fill_cache(CTX - 1024, gen)
            model = DecoderModel(layers, vocab=248320, hidden=5120, device=dev)
            st = StepState(ring_capacity=8192, device=dev)
            table = torch.randint(0, 248320, (CTX, 7), generator=gen, device=dev, dtype=torch.int32)
            prog = SpecProgram(model, st, gamma=7, draft_table=table, ctx_cap=CTX - 16, steps_per_graph=2)
            start = CTX - 1024
            st.start(position=start, token=11)
            prog.step_eager(2)
            st.start(position=start, token=11)
            prog.run(16, launches_per_batch=8, in_flight=2)
            st.start(position=start, token=11)
            rep = prog.run(128, launches_per_batch=8, in_flight=2)
            spec_ms = rep.wall_ms / rep.steps_submitted
            spec_info = {"ms_per_round": round(spec_ms, 5), "rows_per_round": 8,
                         "tokens_per_s_at_0_accepted": round(1e3 / spec_ms, 1),
                         "tokens_per_s_if_all_7_accepted": round(8e3 / spec_ms, 1),
                         "workload": "embed + GDN layer + attention layer (32K) + BF16 lm_head 248320 at M = 8 + "
                                     "argmax + accept_scan + gdn_commit + draft table + verify_select, graph replay"}
            del prog, model, layers

    def rate(key):
        ms, b = out[key]
        gbs = b / (ms * 1e-3) / 1e9
        return ms, b, gbs

    if args.only:
        print(json.dumps({k: {"ms": round(v[0], 5), "bytes": v[1], "GB/s": round(rate(k)[2], 1)} for k, v in out.items()}))
        return

    traffic = None
    prof = ROOT / "profiles" / "gemv_nvfp4_gateup_m1_traffic.json"
    if prof.exists():
        traffic = json.loads(prof.read_text()).get("hbm_bytes_per_launch")
    counters = None                                    # per-kernel HBM traffic ratios and MFMA busy fractions
    cprof = ROOT / "profiles" / "kernel_counters.json"
    if cprof.exists():
        counters = json.loads(cprof.read_text())
    cpu = None if args.no_cpu else cpu_baseline(args.cpu_seconds, b1_bytes=out["gdn_m1"][1],
                                                  b8_bytes=out["gdn_m8"][1])

    def entry(key, m):
        ms, b, gbs = rate(key)
        return {"ms_per_step": round(ms, 5), "GB/s": round(gbs, 1), "pct_of_hbm_peak": round(100 * gbs / HBM_PEAK_GBS, 2),
                "tokens_per_s": round(m * 1e3 / ms, 1), "bytes_per_step": b}

    ms1, b1, gbs1 = rate("gdn_m1")
    k_ms, k_bytes, k_gbs = rate("gateup_m1")
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
        "dtype": "nvfp4 weights x bf16 activations, fp32 accumulate; fp32 GDN state; int8 KV cache",
        "data": "synthetic: weights N(0,0.02) quantized to NVFP4 (reference rule), activations N(0,1) bf16, "
                "GDN state N(0,0.1), KV int8",
        "config": {"workload": "27B decode layer, M=1: GDN mixer (hk16/hv48 x128, in_proj 16480x5120, out_proj "
                               "5120x6144) + NVFP4 gated MLP (gate|up 2x17408x5120, down 5120x17408), fused norms "
                               "and residuals", "m": 1, "hidden": 5120, "layers_rotated": args.layers,
                   "bytes_per_step": b1},
        "pct_of_hbm_peak": round(100 * gbs1 / HBM_PEAK_GBS, 2),
        "tokens_per_s_m1": round(1e3 / ms1, 1),
        "gdn_layer_m8": dict(entry("gdn_m8", 8), workload="one layer of a chain: its normalized input from the layer "
                             "before, the next layer's written by its MLP's split-K reduction"),
        "attn_layer_ctx32k_m1": entry("attn_m1", 1),
        "attn_layer_ctx32k_m8": dict(entry("attn_m8", 8), workload="one layer of a chain, the input norm handed over "
                                     "as for gdn_layer_m8"),
        "mlp_m1": entry("mlp_m1", 1),
        "mlp_m8": entry("mlp_m8", 8),
        "fp8_in_proj_m1": entry("fp8_m1", 1),
        "fp8_in_proj_m8": entry("fp8_m8", 8),
        "int4_gemv_4096_m1": dict(entry("int4_4096_m1", 1), **c1_info,
                                  workload="configs[0]: affine 4-bit GEMV 4096x4096, M=1, N(0,0.02) weights quantized "
                                           "(MLX rule), rotated over distinct device copies"),
        "gemv_gateup_m1": dict(entry("gateup_m1", 1), workload="configs[1]: NVFP4 gate|up 34816x5120 + silu_mul"),
        "gemv_gateup_m8": entry("gateup_m8", 8),
        "gemv_down_m1": dict(entry("down_m1", 1), workload="configs[1]: NVFP4 down 5120x17408 + residual"),
        "gemv_down_m8": entry("down_m8", 8),
        "gqa_core": {f"ctx{c}k_m{m}": entry(f"gqa_{c}k_m{m}", m) for c in (4, 16, 32) for m in (1, 8)},
        "gqa_core_workload": "configs[2]: the attention core alone (query and key preparation, cache append, attention, merge, gate) (24 q / 4 KV heads x 128, int8 KV, "
                             "q/k norm, RoPE 64 of 128, gate), position ctx-16, rotated over >= 2 GiB of KV caches",
        "gqa_core_reference_geometry": {f"ctx32k_m{m}": entry(f"gqa_ref_m{m}", m) for m in (1, 8)},
        "gqa_core_reference_geometry_workload": "the reference's attention (24 q / 4 KV heads x 256, BF16 KV cache, "
                                                "q/k norm, RoPE 64, gate) at 32K, rotated over >= 2 GiB of caches",
        "gdn_step_m1": dict(entry("gdnstep_m1", 1), workload="configs[3]: Gated DeltaNet step alone (hk16/hv48 x128, "
                            "conv 4, gated norm, bf16 out), rotated over >= 2 GiB of recurrent states"),
        "gdn_step_m8": entry("gdnstep_m8", 8),
        "gdn_step_m1_conv_in_projection": dict(entry("gdnstep_pre_m1", 1), workload="the same step as the M = 1 layer "
                                               "runs it: q|k|v already convolved by the input projection's epilogue, "
                                               "read-out left to the output projection"),
        "int4_gateup_m1": dict(entry("int4_gateup_m1", 1), workload="affine 4-bit gate|up 34816x5120 + silu_mul"),
        "int4_gateup_m8": entry("int4_gateup_m8", 8),
        "moe_block_m1": dict(entry("moe_m1", 1), workload="MoE feed-forward: router + top-8 of 256 NVFP4 experts "
                             "(hidden 2048, intermediate 512) + shared expert + combine"),
        "moe_block_m8": dict(entry("moe_m8", 8), workload="one block of a chain: its normalized input from the layer "
                             "before, the next one's written by its combine"),
        "spec_round_2layers_ctx32k": spec_info,
        "token_loop_2layers_ctx32k": dict(entry("loop", 1), **loop_info,
                                          workload="embed + GDN layer + attention layer (32K) + BF16 lm_head 248320 "
                                                   "+ argmax + advance, graph replay through the native pump"),
        "roofline": {"kernel": "gemv_rowp (NVFP4 gate|up 34816x5120, silu_mul, M=1: 768 workgroups over 2-3 tiles each)", "bound": "hbm",
                     "achieved": round(k_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(k_gbs / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "algorithmic_bytes": k_bytes, "avg_launch_us": round(k_ms * 1e3, 3)},
        "cpu_baseline": cpu,
        "counters": counters,
    }
    print(json.dumps(line))


def cpu_baseline(seconds: float, b1_bytes: int, b8_bytes: int):
    """The reference's CPU path for the same decode layer on this host (``oracle/baseline.py``): numpy (dequantize to
    float32 + BLAS matmul, the oracle's mixer) and the C/OpenMP restatement of the oracle GEMV (packed weights
    streamed once, rows over all cores) with the same mixer, the 27B GDN layer at M = 1 and 8; and configs[0] (INT4
    4096², M = 1) on one core. ``value``: the C/OpenMP layer at M = 1, in the GPU line's unit (the layer's
    algorithmic bytes ÷ its step time)."""
    sys.path.insert(0, str(ROOT))
    from oracle import baseline as OB
    r = OB.run(seconds)

    def gbs(key, nbytes):
        return round(nbytes / r[key]["s_per_step"] / 1e9, 3)
    legs = {k: dict(v, s_per_step=round(v["s_per_step"], 5)) for k, v in r.items()}
    for m, b in ((1, b1_bytes), (8, b8_bytes)):
        legs[f"numpy_m{m}"]["GB/s"] = gbs(f"numpy_m{m}", b)
        legs[f"c_openmp_m{m}"]["GB/s"] = gbs(f"c_openmp_m{m}", b)
        for leg in ("numpy", "c_openmp"):
            legs[f"{leg}_m{m}"]["tokens_per_s"] = round(m / r[f"{leg}_m{m}"]["s_per_step"], 3)
    legs["c1_int4_4096_m1_1thread"]["GB/s"] = gbs("c1_int4_4096_m1_1thread", 4096 * 4096 * 9 // 16 + 4 * 4096)
    return {"value": legs["c_openmp_m1"]["GB/s"], "unit": "GB/s", "cores": r["c_openmp_m1"]["threads"],
            "kind": "port",
            "sample": f"one 27B GDN decode layer (weights N(0,0.02) NVFP4-quantized), about {seconds:.0f} s of CPU "
                      f"time in all: C/OpenMP GEMVs + numpy mixer at M=1 and 8 ({r['c_openmp_m1']['reps']} and "
                      f"{r['c_openmp_m8']['reps']} steps), the numpy oracle path (dequantize + matmul) one step each, "
                      f"INT4 4096x4096 M=1 on 1 core",
            "legs": legs}


if __name__ == "__main__":
    main()
