"""The HIP GEMV / skinny GEMM against the oracle (the reference's ``tests/kernels/test_gemv_T.py`` strategy):

* dequantized weights decoded by the kernels' own decode path are bit-identical to the oracle's ``dequantize``
  (all four formats, including every E4M3 block-scale code and every finite FP8 code, signed zero included);
* ``y = x·Wᵀ`` within the reference's leaf gate (``OracleCheck.ok``: ≤ 2 BF16 ULP at the output RMS, relative error
  < 1e-4) against a float64 matmul of the exact dequantized matrix, for M = 1, 2, 8, 16, ragged N, the residual and
  silu·mul epilogues (rounded chains gated by ``ok_rounded``) and the fused input RMSNorm;
* the BASELINE shapes (INT4 4096×4096, NVFP4 17408×5120 and 5120×17408 at M = 1 and 8).
"""

import numpy as np
import pytest

from helpers import from_dev_bf16, spec_of, to_dev_bf16
from oracle import formats as OF
from oracle import nn as ON
from oracle.fp import rbf
from oracle.gates import check_against_oracle

pytestmark = pytest.mark.gpu


def _matrix(fmt, n, k, rng):
    if fmt == "nvfp4":
        return OF.nvfp4_random(n, k, rng)
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


def _upload(torch, m):
    from monolith_mi355 import kernels
    return kernels.upload(spec_of(m))


@pytest.mark.parametrize("fmt", ["nvfp4", "int4_affine", "bf16", "fp8_e4m3"])
@pytest.mark.parametrize("n,k", [(16, 128), (37, 512), (300, 1024)])
def test_dequant_bit_exact(torch_gpu, fmt, n, k, rng):
    from monolith_mi355 import kernels
    if fmt == "bf16" and k % 32:
        pytest.skip()
    m = _matrix(fmt, n, k, rng)
    w = _upload(torch_gpu, m)
    got = kernels.dequant(w).cpu().numpy()
    ref = _dequant(m)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


def test_dequant_every_scale_code(torch_gpu, rng):
    """All 126 finite non-negative E4M3 block-scale codes and all 16 E2M1 codes, bit for bit
    (the reference's tests/kernels/test_nvfp4_scale_decode.py:11-27)."""
    from monolith_mi355 import kernels
    n, k = 128, 256
    m = OF.nvfp4_random(n, k, rng)
    codes = np.arange(n * k // 16) % 0x7F                      # 0x00..0x7E cycling
    m["weight_scale"] = codes.astype(np.uint8).reshape(n, k // 16)
    m["weight"] = (np.arange(n * k // 2) % 256).astype(np.uint8).reshape(n, k // 2)
    got = kernels.dequant(_upload(torch_gpu, m)).cpu().numpy()
    assert np.array_equal(got.view(np.uint32), OF.nvfp4_dequantize(m).view(np.uint32))


def _run(torch, m, x, **kw):
    """FP32 output, as the reference's gemv_T test reads it (tests/kernels/test_gemv_T.py:21-46)."""
    from monolith_mi355 import kernels
    w = _upload(torch, m)
    y = kernels.gemv(w, to_dev_bf16(torch, x), out_f32=True, **kw)
    torch.cuda.synchronize()
    return y.cpu().numpy()


@pytest.mark.parametrize("fmt", ["nvfp4", "int4_affine", "bf16", "fp8_e4m3"])
@pytest.mark.parametrize("mtok", [1, 2, 3, 8, 16])
@pytest.mark.parametrize("n,k", [(48, 256), (77, 1024), (1040, 2048)])
def test_gemv_matches_oracle(torch_gpu, fmt, mtok, n, k, rng):
    m = _matrix(fmt, n, k, rng)
    x = rbf(rng.standard_normal((mtok, k)).astype(np.float32))
    got = _run(torch_gpu, m, x)
    ref = ON.matmul_acc(x, _dequant(m))
    chk = check_against_oracle(got, ref)
    assert chk.ok() and chk.within, (fmt, mtok, n, k, chk)
    from monolith_mi355 import kernels                      # the BF16 output is the same number rounded once
    yb = from_dev_bf16(kernels.gemv(_upload(torch_gpu, m), to_dev_bf16(torch_gpu, x)))
    assert np.array_equal(yb, rbf(got))


@pytest.mark.parametrize("fmt", ["nvfp4", "int4_affine", "fp8_e4m3"])
@pytest.mark.parametrize("mtok", [1, 8])
def test_gemv_residual(torch_gpu, fmt, mtok, rng):
    n, k = 160, 1024
    m = _matrix(fmt, n, k, rng)
    x = rbf(rng.standard_normal((mtok, k)))
    res = rbf(rng.standard_normal((mtok, n)))
    from monolith_mi355 import kernels
    w = _upload(torch_gpu, m)
    y = kernels.gemv(w, to_dev_bf16(torch_gpu, x), epilogue="residual", residual=to_dev_bf16(torch_gpu, res))
    got = from_dev_bf16(y)
    ref = ON.linear(x, _dequant(m), epilogue="residual", residual=res)
    chk = check_against_oracle(got, ref)
    assert chk.ok_rounded() and chk.within and chk.max_ulp_elementwise <= 1, chk


@pytest.mark.parametrize("fmt", ["nvfp4", "int4_affine", "fp8_e4m3"])
@pytest.mark.parametrize("rounded", [False, True])
@pytest.mark.parametrize("mtok", [1, 8])
def test_gemv_silu_mul(torch_gpu, fmt, rounded, mtok, rng):
    inter, k = 96, 512
    gate, up = _matrix(fmt, inter, k, rng), _matrix(fmt, inter, k, rng)
    if fmt == "nvfp4":
        up["weight_scale_2"] = gate["weight_scale_2"] * 1.5              # distinct tensor scales per part
    if fmt == "fp8_e4m3":
        up["weight_scale"] = gate["weight_scale"] * 1.5
    slab = OF.stack_rows([gate, up])
    perm = ON.interleave_chunks(inter, inter, 8)
    slab = OF.permute_rows(slab, perm)
    from monolith_mi355 import kernels
    from monolith_mi355.formats import DequantSpec
    spec = spec_of(dict(slab, weight_scale=1.0) if fmt == "fp8_e4m3" else dict(slab, weight_scale_2=1.0))
    w = kernels.upload(spec, row_scales=[slab["row_scale"]] if fmt in ("nvfp4", "fp8_e4m3") else None)
    x = rbf(rng.standard_normal((mtok, k)))
    epi = "silu_mul_rounded" if rounded else "silu_mul"
    got = from_dev_bf16(kernels.gemv(w, to_dev_bf16(torch_gpu, x), epilogue=epi))
    wg, wu = OF.dequantize(gate), OF.dequantize(up)
    ref = ON.linear(x, np.concatenate([wg, wu]), epilogue="silu_mul", round_silu=rounded)
    chk = check_against_oracle(got, ref)
    assert got.shape == (mtok, inter)
    assert chk.ok_rounded() and chk.within, chk


@pytest.mark.parametrize("fmt", ["nvfp4", "int4_affine", "bf16", "fp8_e4m3"])
@pytest.mark.parametrize("mtok", [1, 8])
def test_gemv_fused_norm(torch_gpu, fmt, mtok, rng):
    n, k = 200, 2048
    m = _matrix(fmt, n, k, rng)
    h = rbf(rng.standard_normal((mtok, k)) * 3)
    wn = rbf(rng.standard_normal(k) * 0.2)
    nw = (1.0 + wn).astype(np.float32)
    from monolith_mi355 import kernels
    w = _upload(torch_gpu, m)
    got = kernels.gemv(w, to_dev_bf16(torch_gpu, h), norm_w=torch_gpu.from_numpy(nw).cuda(), eps=1e-6,
                       out_f32=True).cpu().numpy()
    xn = ON.rms_norm(h, wn, 1e-6)
    ref = ON.matmul_acc(xn, _dequant(m))
    chk = check_against_oracle(got, ref)
    assert chk.ok_rounded() and chk.within, chk


@pytest.mark.parametrize("fmt,n,k,mtok", [("int4_affine", 4096, 4096, 1), ("nvfp4", 17408, 5120, 1),
                                          ("nvfp4", 17408, 5120, 8), ("nvfp4", 5120, 17408, 1),
                                          ("nvfp4", 5120, 17408, 8)])
def test_gemv_baseline_shapes(torch_gpu, fmt, n, k, mtok):
    rng = np.random.default_rng(n + k + mtok)
    m = _matrix(fmt, n, k, rng)
    x = rbf(rng.standard_normal((mtok, k)))
    got = _run(torch_gpu, m, x)
    w = _dequant(m)
    ref = ON.matmul_acc(x, w)
    chk = check_against_oracle(got, ref)
    assert chk.ok() and chk.within, chk


def test_gemv_repeat_is_bit_identical(torch_gpu, rng):
    """Split-K partials are combined in a fixed order: two runs give the same bits."""
    from monolith_mi355 import kernels
    m = _matrix("nvfp4", 5120, 17408, rng)
    w = _upload(torch_gpu, m)
    x = to_dev_bf16(torch_gpu, rbf(rng.standard_normal((8, 17408))))
    a = kernels.gemv(w, x).clone()
    b = kernels.gemv(w, x)
    assert torch_gpu.equal(a, b)


@pytest.mark.parametrize("fmt", ["nvfp4", "int4_affine", "bf16", "fp8_e4m3"])
@pytest.mark.parametrize("n,k", [(1040, 2048), (336, 1664)])
@pytest.mark.parametrize("epi", [None, "residual", "silu_mul"])
def test_gemv_tiles_per_workgroup(torch_gpu, fmt, n, k, epi, rng, monkeypatch):
    """M = 1 with a workgroup streaming 1..5 tiles (the fused-norm plan): every tile's K slices are added in the
    same order, so the output is bit-identical to one tile per workgroup, and within the oracle bar."""
    from monolith_mi355 import kernels
    if epi == "silu_mul":
        n = n // 16 * 16
    m = _matrix(fmt, n, k, rng)
    w = _upload(torch_gpu, m)
    h = rbf(rng.standard_normal((1, k)) * 3)
    wn = rbf(rng.standard_normal(k) * 0.2)
    nw = torch_gpu.from_numpy((1.0 + wn).astype(np.float32)).cuda()
    res = rbf(rng.standard_normal((1, n)))
    kw = dict(norm_w=nw, eps=1e-6, epilogue=epi)
    if epi == "residual":
        kw["residual"] = to_dev_bf16(torch_gpu, res)
    outs = {}
    for rt in (1, 2, 3, 5):
        monkeypatch.setenv("MI_GEMV_ROW", f"4,1,{rt}")
        outs[rt] = from_dev_bf16(kernels.gemv(w, to_dev_bf16(torch_gpu, h), **kw))
    monkeypatch.delenv("MI_GEMV_ROW")
    for rt in (2, 3, 5):
        assert np.array_equal(outs[rt].view(np.uint16), outs[1].view(np.uint16)), rt
    xn = ON.rms_norm(h, wn, 1e-6)
    wd = _dequant(m)
    if epi == "silu_mul":
        ref = ON.linear(xn, wd[np.argsort(ON.interleave_chunks(n // 2, n // 2, 8))], epilogue="silu_mul")
    else:
        ref = ON.linear(xn, wd, epilogue=epi, residual=res if epi else None)
    chk = check_against_oracle(outs[1], ref)
    assert chk.ok_rounded() and chk.within, chk


@pytest.mark.parametrize("fmt", ["nvfp4", "int4_affine"])
@pytest.mark.parametrize("mtok", [1, 2, 3, 8, 16])
@pytest.mark.parametrize("plan", [None, "4,3", "tk", "rowm2"])
def test_gemv_gated_head_norm(torch_gpu, fmt, mtok, plan, rng, monkeypatch):
    """The Gated DeltaNet output norm fused into the output projection's input staging: per 128-column head,
    bf16(bf16(bf16(w)·bf16(o·r))·silu(z)), then the GEMV — against the oracle's gated_rms_norm and matmul (M ≥ 3:
    gemv_tk, whatever gemv_rowm split is asked for)."""
    from monolith_mi355 import kernels
    if plan == "tk":
        monkeypatch.setenv("MI_GEMV_KERNEL", "tk")
    elif plan == "rowm2":
        monkeypatch.setenv("MI_GEMV_ROWM", "2,0")
    elif plan:
        monkeypatch.setenv("MI_GEMV_ROW", plan)
    heads, n = 12, 320
    k = heads * 128
    m = _matrix(fmt, n, k, rng)
    o = rbf(rng.standard_normal((mtok, k)) * 0.3)
    zfull = rbf(rng.standard_normal((mtok, k + 64)) * 2)       # z as a view with its own row stride
    wn = rbf(1 + rng.standard_normal(128) * 0.2).astype(np.float32)
    zd = to_dev_bf16(torch_gpu, zfull)[:, 32: 32 + k]
    got = kernels.gemv(_upload(torch_gpu, m), to_dev_bf16(torch_gpu, o), out_f32=True,
                       gated_norm=(torch_gpu.from_numpy(wn).cuda(), zd, 1e-6)).cpu().numpy()
    xn = ON.gated_rms_norm(o.reshape(mtok, heads, 128), zfull[:, 32: 32 + k].reshape(mtok, heads, 128), wn, 1e-6)
    ref = ON.matmul_acc(xn.reshape(mtok, k), _dequant(m))
    chk = check_against_oracle(got, ref)
    assert chk.ok_rounded() and chk.within, (fmt, mtok, plan, chk)


@pytest.mark.parametrize("fmt", ["nvfp4", "fp8_e4m3", "int4_affine"])
@pytest.mark.parametrize("mtok", [3, 8, 16])
@pytest.mark.parametrize("n,k,plan", [(1040, 2048, None), (1040, 2048, "1,3"), (336, 6144, "2,1"),
                                      (336, 6144, "3,2"), (5120, 17408, None)])
@pytest.mark.parametrize("epi", [None, "residual", "silu_mul"])
def test_gemv_rowm_plans(torch_gpu, fmt, mtok, n, k, plan, epi, rng, monkeypatch):
    """The M >= 3 kernel (K slices per wave on the matrix cores, several tiles per workgroup; NVFP4, FP8, INT4) over
    forced K splits and tiles per workgroup, against the oracle."""
    from monolith_mi355 import kernels
    if plan:
        monkeypatch.setenv("MI_GEMV_ROWM", plan)
    if fmt == "int4_affine":                       # INT4 takes gemv_rowm only when it is pinned
        monkeypatch.setenv("MI_GEMV_KERNEL", "rowm")
    m = _matrix(fmt, n, k, rng)
    x = rbf(rng.standard_normal((mtok, k)))
    res = rbf(rng.standard_normal((mtok, n)))
    kw = dict(epilogue=epi)
    if epi == "residual":
        kw["residual"] = to_dev_bf16(torch_gpu, res)
    got = from_dev_bf16(kernels.gemv(_upload(torch_gpu, m), to_dev_bf16(torch_gpu, x), **kw))
    wd = _dequant(m)
    if epi == "silu_mul":
        ref = ON.linear(x, wd[np.argsort(ON.interleave_chunks(n // 2, n // 2, 8))], epilogue="silu_mul")
    else:
        ref = ON.linear(x, wd, epilogue=epi, residual=res if epi else None)
    chk = check_against_oracle(got, ref)
    assert chk.ok_rounded() and chk.within, (mtok, n, k, plan, epi, chk)


def test_fp8_dequant_every_code(torch_gpu):
    """Every finite E4M3 code (signed zero, subnormals, ±448) decodes bit-exactly; the tensor scale multiplies once."""
    from monolith_mi355 import kernels
    from oracle.fp import e4m3_to_f32
    codes = np.array([c for c in range(256) if c & 0x7F != 0x7F], np.uint8)
    w = np.resize(codes, (32, 256)).astype(np.uint8)
    for s in (1.0, 0.0123):
        m = {"format": "fp8_e4m3", "weight": w, "weight_scale": float(np.float32(s))}
        got = kernels.dequant(_upload(torch_gpu, m)).cpu().numpy()
        ref = (e4m3_to_f32(w) * np.float32(s)).astype(np.float32)
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), s


def test_gemv_split_k_fold_in_kernel(torch_gpu):
    """Split-K plans of gemv_row (M ≤ 2) fold their splits inside the kernel (gemv_rowm, M ≥ 3, in the reduction
    launch, which measured faster there) (arrival counters in the workspace): shapes with
    different tile counts interleaved, each repeated — the counters re-arm, the partials of one shape never disturb
    another's, the results repeat bit for bit, match the oracle, and a caller's zeroed workspace gives the same bits."""
    torch = torch_gpu
    import ctypes as C
    from monolith_mi355 import kernels
    from monolith_mi355.runtime import hip
    rng = np.random.default_rng(77)
    cases = []
    for n, k, mtok in [(4096, 12288, 1), (5120, 17408, 1), (1040, 17408, 2), (5120, 12288, 2), (5120, 17408, 8),
                       (2048, 17408, 5)]:
        m = _matrix("nvfp4", n, k, rng)
        w = _upload(torch, m)
        x = rbf(rng.standard_normal((mtok, k)))
        xd = to_dev_bf16(torch, x)
        yd = torch.empty(mtok, n, dtype=torch.float32, device="cuda")
        d = hip.MiGemvDesc(format=1, n=n, k=k, m=mtok, w=hip.ptr(w.data), row_scale=hip.ptr(w.row_scale),
                           x=hip.ptr(xd), ldx=k, y=hip.ptr(yd), ldy=n, out_f32=1)
        plan = (C.c_int32 * 7)()
        hip.call("mi_gemv_plan", C.byref(d), plan)
        assert plan[0] in (1, 3) and plan[4] > 1, (n, k, list(plan))     # gemv_row / gemv_rowm with K splits
        cases.append((m, w, x, xd, d))
    first = []
    for rep in range(3):
        for i, (m, w, x, xd, d) in enumerate(cases):
            y = kernels.gemv(w, xd, out_f32=True)
            torch.cuda.synchronize()
            y = y.cpu().numpy()
            if rep == 0:
                chk = check_against_oracle(y, ON.matmul_acc(x, _dequant(m)))
                assert chk.ok() and chk.within, (i, chk)
                first.append(y)
            else:
                assert np.array_equal(y, first[i]), (rep, i)
    ws_bytes = max(hip.load().mi_gemv_workspace_bytes(C.byref(d)) for *_, d in cases)
    ws = torch.zeros(ws_bytes, dtype=torch.uint8, device="cuda")
    for i, (m, w, x, xd, d) in enumerate(cases * 2):
        y = kernels.gemv(w, xd, out_f32=True, workspace=ws)
        torch.cuda.synchronize()
        assert np.array_equal(y.cpu().numpy(), first[i % len(cases)]), i


@pytest.mark.parametrize("fmt,n,k,mtok,epi,env", [
    ("nvfp4", 5120, 17408, 8, "residual", {}),              # gemv_rowm, K splits: the reduction writes x_next
    ("nvfp4", 5120, 17408, 3, "residual", {}),
    ("int4_affine", 2048, 8192, 8, "residual", {}),         # gemv_tk splits
    ("nvfp4", 1040, 17408, 1, "residual", {"MI_GEMV_FOLD": "0"}),   # gemv_row splits through the reduction launch
    ("nvfp4", 5120, 17408, 1, "residual", {}),              # splits folded in the kernel: a norm launch follows
    ("nvfp4", 2048, 5120, 8, None, {}),                     # one split: a norm launch follows
    ("nvfp4", 3000, 12288, 8, None, {}),                    # ragged N (whole 8-column vectors)
    ("nvfp4", 8192, 12288, 4, "residual", {}),              # the widest row one reduction workgroup takes
    ("nvfp4", 8200, 12288, 4, "residual", {}),              # wider: the reduction, then a norm launch
    ("nvfp4", 1032, 12288, 16, "residual", {}),             # N not a multiple of 16, sixteen tokens
    ("fp8_e4m3", 5120, 17408, 8, "residual", {}),           # per-row scales applied in the reduction
    ("bf16", 2048, 8192, 8, None, {}),                      # BF16 weights (gemv_tk)
])
def test_gemv_next_norm(torch_gpu, fmt, n, k, mtok, epi, env, rng, monkeypatch):
    """``next_norm``: y is bit-identical to the same GEMV without it, and x_next bit-identical to ``norm_apply`` of
    that y (the next GEMV's M ≥ 3 input norm), whichever launch computes it."""
    torch = torch_gpu
    from monolith_mi355 import kernels
    for kk, v in env.items():
        monkeypatch.setenv(kk, v)
    m = _matrix(fmt, n, k, rng)
    w = _upload(torch, m)
    xd = to_dev_bf16(torch, rbf(rng.standard_normal((mtok, k))))
    res = to_dev_bf16(torch, rbf(rng.standard_normal((mtok, n + 24))))[:, :n] if epi else None   # row stride > n
    nw = torch.from_numpy((1.0 + rng.standard_normal(n) * 0.1).astype(np.float32)).cuda()
    y0 = kernels.gemv(w, xd, epilogue=epi, residual=res)
    x0 = kernels.norm_apply(y0, nw, eps=1e-6)
    xn = torch.full((mtok, n), 7.0, dtype=torch.bfloat16, device="cuda")
    for rep in range(2):
        y1 = kernels.gemv(w, xd, epilogue=epi, residual=res, next_norm=(nw, xn, 1e-6))
        torch.cuda.synchronize()
        assert torch.equal(y1.view(torch.int16), y0.view(torch.int16)), rep
        assert torch.equal(xn.view(torch.int16), x0.view(torch.int16)), rep
        xn.fill_(7.0)
