"""The C/OpenMP restatement of the oracle GEMV (``oracle/c/gemv_cpu.c``, the timed CPU baseline) pinned to the
numpy oracle: NVFP4 and affine-INT4, M = 1 / 3 / 8, random codes over the whole code space (every E2M1 nibble, E4M3
block scales across their range, BF16 scale / bias pairs) and quantized N(0, 0.02) weights, 1 and 4 threads.

Both dequantize the same way (``(e2m1 · e4m3) · s2``, one rounding; ``code · scale + bias``) and accumulate in
float64, so they may differ only by the order of the float64 sum: within 1e-6 relative of the row's Σ|x·w| (a
plausible slip — a swapped nibble, a scale from the wrong block, a dropped bias — moves results by far more)."""

import numpy as np
import pytest

from oracle import cpu as OC
from oracle import formats as OF
from oracle.nn import matmul_acc


def _close(got, w, x):
    ref = matmul_acc(x, w)
    bound = 1e-6 * (np.abs(x).astype(np.float64) @ np.abs(w).astype(np.float64).T) + 1e-30
    assert np.all(np.abs(got.astype(np.float64) - ref) <= bound), float(np.max(np.abs(got - ref) / bound))


@pytest.mark.parametrize("m", [1, 3, 8])
@pytest.mark.parametrize("threads", [1, 4])
def test_nvfp4_port_matches_oracle(m, threads):
    rng = np.random.default_rng(10 * m + threads)
    for q in (OF.nvfp4_random(96, 512, rng), OF.nvfp4_quantize(rng.standard_normal((80, 256)) * 0.02)):
        x = rng.standard_normal((m, q["weight"].shape[1] * 2)).astype(np.float32)
        _close(OC.nvfp4_gemv(q, x, threads), OF.nvfp4_dequantize(q), x)


@pytest.mark.parametrize("m", [1, 3, 8])
@pytest.mark.parametrize("threads", [1, 4])
def test_int4_port_matches_oracle(m, threads):
    rng = np.random.default_rng(20 * m + threads)
    for q in (OF.int4_random(96, 512, rng), OF.int4_quantize(rng.standard_normal((64, 256)) * 0.02)):
        x = rng.standard_normal((m, q["weight"].shape[1] * 2)).astype(np.float32)
        _close(OC.int4_gemv(q, x, threads), OF.int4_dequantize(q), x)


def test_port_detects_a_wrong_scale():
    """The bar is tight enough to see one block scale off by one code."""
    rng = np.random.default_rng(3)
    q = OF.nvfp4_random(16, 256, rng)
    x = rng.standard_normal((1, 256)).astype(np.float32)
    bad = dict(q, weight_scale=q["weight_scale"].copy())
    bad["weight_scale"][5, 3] += 1
    with pytest.raises(AssertionError):
        _close(OC.nvfp4_gemv(bad, x, 1), OF.nvfp4_dequantize(q), x)
