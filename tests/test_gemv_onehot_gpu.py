"""The decode inside each hot GEMV kernel is exact: with a one-hot activation row e_j the FP32 output (``out_f32``,
no BF16 rounding) is column j of the weight matrix, so every output must equal the oracle's ``dequantize`` bit for
bit — a single product 1·w and additions of zeros round nothing. This pins the decode each kernel actually runs
(``gemv_row``'s BF16 pairs with the block scale's mantissa applied once per block, ``gemv_rowp``, the split-K fold, ``gemv_row`` over several token passes,
``gemv_rowm``'s and ``gemv_tk``'s exact F16 operands on the matrix cores), not only ``mi_dequant``'s, for every
weight format (a weight of −0, an E2M1 code, comes out as +0, the sign a sum of zeros has). Ragged N (a partial last tile) and K long enough for three K splits are covered."""

import numpy as np
import pytest

from helpers import spec_of
from oracle import formats as OF

pytestmark = pytest.mark.gpu

# plan name → (tokens per call, environment that pins the kernel)
PLANS = {
    "row": (1, {}),
    "row_m2": (2, {}),
    "rowp": (1, {"MI_GEMV_ROW": "0,1,2"}),
    "row_split3": (1, {"MI_GEMV_ROW": "0,3,0"}),
    "row_passes": (8, {}),                          # two tokens per workgroup along grid z (small BF16)
    "rowm": (16, {"MI_GEMV_PASSES": "0"}),
    "rowm_split3": (8, {"MI_GEMV_ROWM": "3,0", "MI_GEMV_PASSES": "0"}),
    "tk": (16, {"MI_GEMV_KERNEL": "tk"}),
    "tk_m1": (1, {"MI_GEMV_KERNEL": "tk"}),
}
KERNEL = {1: "gemv_row", 2: "gemv_tk", 3: "gemv_rowm"}


def _matrix(fmt, n, k, rng):
    if fmt == "nvfp4":
        m = OF.nvfp4_random(n, k, rng)
        m["weight_scale"] = rng.integers(0, 0x7F, m["weight_scale"].shape).astype(np.uint8)   # every finite scale
        m["weight"] = rng.integers(0, 256, m["weight"].shape).astype(np.uint8)                # every code pair
        return m
    if fmt == "fp8_e4m3":
        return OF.fp8_random(n, k, rng)
    if fmt == "int4_affine":
        return OF.int4_random(n, k, rng)
    from oracle.fp import f32_to_bf16
    return {"format": "bf16", "weight": f32_to_bf16((rng.standard_normal((n, k)) * 0.02).astype(np.float32))}


def _dequant(m):
    if m["format"] == "bf16":
        from oracle.fp import bf16_to_f32
        return bf16_to_f32(m["weight"])
    return OF.dequantize(m)


@pytest.mark.parametrize("fmt", ["nvfp4", "int4_affine", "fp8_e4m3", "bf16"])
@pytest.mark.parametrize("plan", list(PLANS))
def test_one_hot_columns_are_the_dequantized_weights(torch_gpu, fmt, plan, monkeypatch):
    torch = torch_gpu
    import ctypes as C
    from monolith_mi355 import kernels
    from monolith_mi355.runtime import hip
    mtok, env = PLANS[plan]
    if fmt == "fp8_e4m3" and plan.startswith("tk"):
        pytest.skip("gemv_tk has no FP8 path: FP8 runs on gemv_row / gemv_rowm")
    if fmt != "bf16" and plan == "row_passes":
        pytest.skip("the token passes plan takes small BF16 matrices (and grouped NVFP4, tested with the MoE)")
    if fmt == "bf16" and plan.startswith("rowm"):
        pytest.skip("gemv_rowm takes NVFP4, FP8 and INT4; BF16 at M >= 3 runs on gemv_tk")
    for key, val in env.items():
        monkeypatch.setenv(key, val)
    if fmt == "int4_affine" and plan.startswith("rowm"):      # INT4 takes gemv_rowm only when it is pinned
        monkeypatch.setenv("MI_GEMV_KERNEL", "rowm")
    n = 40
    k = 3072 if "split" in plan else 1024
    rng = np.random.default_rng(abs(hash((fmt, plan))) % 2 ** 32)
    m = _matrix(fmt, n, k, rng)
    w = kernels.upload(spec_of(m))
    ref = _dequant(m).T                                            # [k, n]: row j = column j of W
    # the plan this shape and environment give (the test is about that kernel)
    probe = torch.zeros(mtok, k, dtype=torch.bfloat16, device="cuda")
    d = hip.MiGemvDesc(format=hip.MI_FMT[fmt], n=n, k=k, m=mtok, w=hip.ptr(w.data), row_scale=hip.ptr(w.row_scale),
                       x=hip.ptr(probe), ldx=k, y=16, ldy=n, out_f32=1)
    p = (C.c_int32 * 7)()
    hip.call("mi_gemv_plan", C.byref(d), p)
    want = {"row": 1, "row_m2": 1, "rowp": 1, "row_split3": 1, "row_passes": 1, "rowm": 3, "rowm_split3": 3, "tk": 2,
            "tk_m1": 2}[plan]
    assert p[0] == want, (plan, list(p))
    if "split" in plan:
        assert p[4] == 3, list(p)
    if plan == "rowp":
        assert p[3] > 1, list(p)
    print(f"one-hot {fmt} {plan}: {KERNEL[p[0]]} plan {list(p)}", flush=True)
    # token r of call c is e_{c·mtok + r}: the k columns in k / mtok calls, all launched before one synchronize
    calls = k // mtok
    x = torch.zeros(calls, mtok, k, dtype=torch.bfloat16, device="cuda")
    cols = torch.arange(k, device="cuda").view(calls, mtok)
    x.view(-1, k)[torch.arange(k, device="cuda"), cols.view(-1)] = 1.0
    out = torch.empty(k, n, dtype=torch.float32, device="cuda")
    for c in range(calls):
        kernels.gemv(w, x[c], out=out[c * mtok:(c + 1) * mtok], out_f32=True)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    # bit for bit, except that a zero weight of either sign gives +0: the output is a sum (0 + (−0)·1 = +0), and
    # the oracle's own matmul gives +0 there too
    same = (got.view(np.uint32) == ref.view(np.uint32)) | ((got == 0) & (ref == 0))
    bad = np.argwhere(~same)
    assert bad.size == 0, (f"{len(bad)} of {got.size} weights differ; first (column, row):", bad[:4].tolist(),
                           got[tuple(bad[0])], ref[tuple(bad[0])])
