"""The reference's CPU path for the decode layer, timed as the benchmark's CPU baseline (TEST INFRASTRUCTURE: only
``bench.py``'s ``cpu_baseline`` leg calls this; nothing in the product does).

The reference computes a layer on the CPU as its oracle does: dequantize each weight to float32
(``monolith/formats/nvfp4.py:139-144``, ``int4_affine.py:85-91``) and multiply in float32
(``monolith/nn/oracle.py:20-22``), the mixer in numpy / torch float32 (``nn/oracle.py:76-134``). Two legs:

* ``numpy``: exactly that — ``nvfp4_dequantize`` then a BLAS float32 ``x @ Wᵀ`` per projection, the norms, and the
  oracle's Gated DeltaNet step (``oracle.nn.gdn_mix``);
* ``c_openmp``: the projections through the C/OpenMP restatement (``oracle/c/gemv_cpu.c``: the packed weights
  streamed once, float64 accumulation, rows over threads), the mixer and norms as in ``numpy``.

Weights are the config's: N(0, 0.02) quantized by the reference's NVFP4 rule. Quantizing the 27B layer's 382 M
weights in numpy would take minutes, so one quantized block of rows per K is repeated down each matrix (the values
are quantized N(0, 0.02) weights; the CPU's work does not depend on which)."""

from __future__ import annotations

import os
import time
from typing import Callable, Dict

import numpy as np

from . import cpu as OC
from . import formats as OF
from . import nn as ON
from .fp import rbf

EPS = 1e-6


def _tiled_nvfp4(n: int, k: int, rng: np.random.Generator, block_rows: int = 128) -> dict:
    blk = OF.nvfp4_quantize(rng.standard_normal((block_rows, k)).astype(np.float32) * np.float32(0.02))
    reps = -(-n // block_rows)
    return {"format": "nvfp4", "weight": np.tile(blk["weight"], (reps, 1))[:n].copy(),
            "weight_scale": np.tile(blk["weight_scale"], (reps, 1))[:n].copy(),
            "weight_scale_2": blk["weight_scale_2"]}


def gdn_layer(rng: np.random.Generator, *, hidden=5120, k_heads=16, v_heads=48, d=128, conv=4, inter=17408) -> dict:
    """The 27B Gated DeltaNet decode layer's weights (NVFP4) and state."""
    conv_dim = 2 * k_heads * d + v_heads * d
    n_proj = v_heads * d + conv_dim + 2 * v_heads
    return {"w_in": _tiled_nvfp4(n_proj, hidden, rng), "w_out": _tiled_nvfp4(hidden, v_heads * d, rng),
            "gate": _tiled_nvfp4(inter, hidden, rng), "up": _tiled_nvfp4(inter, hidden, rng),
            "down": _tiled_nvfp4(hidden, inter, rng),
            "norm1": rbf(rng.standard_normal(hidden) * 0.1), "norm2": rbf(rng.standard_normal(hidden) * 0.1),
            "gdn": dict(conv_w=rbf(rng.standard_normal((conv_dim, conv)) * 0.3), a_log=np.zeros(v_heads, np.float32),
                        dt_bias=np.zeros(v_heads, np.float32), norm_w=rbf(1 + rng.standard_normal(d) * 0.2),
                        k_heads=k_heads, v_heads=v_heads, dk=d, dv=d, eps=EPS),
            "conv": rbf(rng.standard_normal((conv_dim, conv - 1)) * 0.5),
            "rec": (rng.standard_normal((v_heads, d, d)) * 0.1).astype(np.float32)}


def _numpy_linear(q: dict, x: np.ndarray) -> np.ndarray:
    return x.astype(np.float32) @ OF.nvfp4_dequantize(q).T


def _port_linear(threads: int) -> Callable[[dict, np.ndarray], np.ndarray]:
    return lambda q, x: OC.nvfp4_gemv(q, x, threads)


def layer_step(L: dict, h: np.ndarray, linear) -> np.ndarray:
    """One step of the layer (``nn/decoder.py:20-22``): ``h += out_proj(gdn(in_proj(norm1 h))); h += mlp(norm2 h)``,
    with BF16 roundings where the reference's torch layer rounds. The recurrent / conv state is not carried over
    (each timed step starts from the same state)."""
    xn = ON.rms_norm(h, L["norm1"], EPS)
    proj = rbf(linear(L["w_in"], xn))
    o, _, _ = ON.gdn_mix(proj, L["conv"], L["rec"], **L["gdn"])
    h1 = rbf(linear(L["w_out"], o) + h)
    x2 = ON.rms_norm(h1, L["norm2"], EPS)
    act = rbf(ON.silu(linear(L["gate"], x2)) * linear(L["up"], x2))
    return rbf(linear(L["down"], act) + h1)


def _time(fn: Callable[[], object], seconds: float, min_reps: int = 1, warm: bool = True):
    if warm:
        fn()                                        # warm (page the weights in, build LUTs, spin up threads)
    reps, t0 = 0, time.perf_counter()
    while reps < min_reps or time.perf_counter() - t0 < seconds:
        fn()
        reps += 1
    return (time.perf_counter() - t0) / reps, reps


def threads() -> int:
    return OC.threads()


def run(seconds: float = 20.0) -> Dict[str, dict]:
    """Time the layer at M = 1 and 8 on both legs and C1 single-threaded, within about ``seconds`` of CPU time in
    all. Returns seconds per step per case with what it ran."""
    rng = np.random.default_rng(0)
    L = gdn_layer(rng)
    nt = threads()
    share = seconds / 6
    out: Dict[str, dict] = {}
    for m in (1, 8):
        h = rbf(rng.standard_normal((m, 5120)))
        dt, reps = _time(lambda: layer_step(L, h, _numpy_linear), share, 1, warm=False)   # seconds per step
        out[f"numpy_m{m}"] = {"s_per_step": dt, "reps": reps, "threads": int(os.environ.get("OMP_NUM_THREADS", nt))}
        dt, reps = _time(lambda: layer_step(L, h, _port_linear(nt)), share, 3)
        out[f"c_openmp_m{m}"] = {"s_per_step": dt, "reps": reps, "threads": nt}
    # the affine 4-bit 4096² GEMV at M = 1, one thread
    c1 = OF.int4_quantize(rng.standard_normal((4096, 4096)).astype(np.float32) * np.float32(0.02))
    x = rbf(rng.standard_normal((1, 4096)))
    dt, reps = _time(lambda: OC.int4_gemv(c1, x, 1), share, 3)
    out["c1_int4_4096_m1_1thread"] = {"s_per_step": dt, "reps": reps, "threads": 1}
    return out
