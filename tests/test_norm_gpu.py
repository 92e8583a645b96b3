"""The standalone RMSNorm ops (``rmsnorm_stat`` and ``norm_apply``, ``ops/norm.py:11-12``) against the oracle's
``rms_norm`` (``nn/oracle.py:25-32``): the statistic within 1e-5 relative of numpy's float64 Σh² (the sum order
differs), the normalized row within one BF16 ULP element-wise and ≥ 99 % bit-identical (a rounding boundary can flip
when the two sums differ in their last bit), the statistic path equal to the fused path bit for bit, a strided input
and output, and the partial-sum form (``stat [t, parts]``) equal to the one-part form."""

import numpy as np
import pytest

from helpers import from_dev_bf16, to_dev_bf16
from oracle import nn as ON
from oracle.fp import rbf

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("t,k", [(1, 5120), (8, 5120), (3, 2048), (1, 8), (5, 17408)])
def test_norm_matches_oracle(torch_gpu, t, k):
    torch = torch_gpu
    from monolith_mi355 import kernels
    rng = np.random.default_rng(t * 7 + k)
    h = rbf(rng.standard_normal((t, k)) * 3.0)
    w = rbf(rng.standard_normal(k) * 0.1)
    hd = to_dev_bf16(torch, h)
    wd = torch.tensor(1.0 + w.astype(np.float32), device="cuda")
    stat = kernels.rmsnorm_stat(hd)
    ref_stat = (h.astype(np.float64) ** 2).sum(axis=1)
    np.testing.assert_allclose(stat.cpu().numpy(), ref_stat, rtol=1e-5)
    fused = from_dev_bf16(kernels.norm_apply(hd, wd, eps=1e-6))
    split = from_dev_bf16(kernels.norm_apply(hd, wd, stat=stat, eps=1e-6))
    assert np.array_equal(fused, split)
    ref = ON.rms_norm(h, w, 1e-6)
    diff = np.abs(fused.astype(np.float64) - ref)
    ulp = np.maximum(np.abs(ref), 1e-30) * 2.0 ** -7
    assert (diff <= ulp).all(), float((diff / ulp).max())
    assert (diff == 0).mean() >= 0.99


def test_norm_strided_and_partials(torch_gpu):
    torch = torch_gpu
    from monolith_mi355 import kernels
    rng = np.random.default_rng(5)
    t, k = 4, 1024
    big = to_dev_bf16(torch, rbf(rng.standard_normal((t, 3 * k))))
    h = big[:, k:2 * k]                                  # a strided view
    wd = torch.tensor(1.0 + rbf(rng.standard_normal(k) * 0.1).astype(np.float32), device="cuda")
    out_big = torch.zeros(t, 2 * k, dtype=torch.bfloat16, device="cuda")
    out = out_big[:, :k]
    kernels.norm_apply(h, wd, eps=1e-5, out=out)
    dense = kernels.norm_apply(h.contiguous(), wd, eps=1e-5)
    assert torch.equal(out, dense) and bool((out_big[:, k:] == 0).all())
    stat = kernels.rmsnorm_stat(h)
    parts = torch.stack([stat * 0.5, stat * 0.5, stat * 0], dim=1).contiguous()   # sums exactly to stat
    assert torch.equal(kernels.norm_apply(h, wd, stat=parts, eps=1e-5), dense)


def test_norm_rejects_bad_shapes(torch_gpu):
    torch = torch_gpu
    from monolith_mi355 import kernels
    h = torch.zeros(2, 12, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(Exception, match="multiple of 8"):
        kernels.rmsnorm_stat(h)
