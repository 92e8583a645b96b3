"""The fused GEMV chain (``mi_gemv_chain``: several dependent one-token NVFP4 GEMVs in one persistent launch)
against the same GEMVs launched one by one (``mi_gemv``): bit for bit — each phase runs the same per-tile
arithmetic in the same order — at the 27B layer shapes (the MLP's gate|up → down; out_proj with the gated head norm
→ gate|up → down) and small ragged ones, repeated (the counters re-arm) and replayed from a graph; and the small
shapes against the oracle."""

import numpy as np
import pytest

from helpers import from_dev_bf16, to_dev_bf16
from oracle import nn as ON
from oracle.fp import rbf

pytestmark = pytest.mark.gpu


def _say(*a):
    print(*a, flush=True)


def _mlp_parts(torch, hidden, inter, seed):
    from monolith_mi355.layers import nvfp4_matrix
    gen = torch.Generator(device="cuda")
    gen.manual_seed(seed)
    gu = nvfp4_matrix(2 * inter, hidden, gen, "cuda", gate_up=True)
    dn = nvfp4_matrix(hidden, inter, gen, "cuda")
    nw = 1.0 + torch.randn(hidden, generator=gen, device="cuda") * 0.1
    h = torch.randn(1, hidden, generator=gen, device="cuda").to(torch.bfloat16)
    return gu, dn, nw, h, gen


def _unfused_mlp(kernels, gu, dn, nw, h):
    act = kernels.gemv(gu.packed, h, epilogue="silu_mul", norm_w=nw)
    return act, kernels.gemv(dn.packed, act, epilogue="residual", residual=h)


@pytest.mark.parametrize("hidden,inter", [(5120, 17408), (1024, 1536), (640, 2048)])
def test_mlp_chain_equals_separate_gemvs(torch_gpu, hidden, inter):
    torch = torch_gpu
    from monolith_mi355 import kernels
    _say(f"chain mlp {hidden}x{inter}")
    gu, dn, nw, h, _ = _mlp_parts(torch, hidden, inter, hidden + inter)
    act_ref, y_ref = _unfused_mlp(kernels, gu, dn, nw, h)
    act = torch.empty(1, inter, dtype=torch.bfloat16, device="cuda")
    y = torch.empty(1, hidden, dtype=torch.bfloat16, device="cuda")
    for rep in range(3):
        act.fill_(float("nan"))
        y.fill_(float("nan"))
        kernels.gemv_chain([(gu.packed, h, dict(epilogue="silu_mul", norm_w=nw, out=act)),
                            (dn.packed, act, dict(epilogue="residual", residual=h, out=y))])
        torch.cuda.synchronize()
        assert torch.equal(act, act_ref), rep
        assert torch.equal(y, y_ref), rep
    assert _chain_error() == 0


def _chain_error():
    import ctypes as C
    from monolith_mi355.runtime import hip
    import torch
    flag = C.c_uint32(7)
    hip.call("mi_gemv_chain_error", None, hip.stream_handle(torch.cuda.current_stream()), C.byref(flag))
    return flag.value


def test_small_mlp_chain_matches_oracle(torch_gpu):
    torch = torch_gpu
    from monolith_mi355 import kernels
    from oracle import formats as OF
    from oracle.gates import check_against_oracle
    hidden, inter = 640, 1664                                  # 13 chunks of down K, an odd scale group
    gu, dn, nw, h, _ = _mlp_parts(torch, hidden, inter, 5)
    act = kernels.gemv_chain([(gu.packed, h, dict(epilogue="silu_mul", norm_w=nw))])[0]
    y = torch.empty(1, hidden, dtype=torch.bfloat16, device="cuda")
    kernels.gemv_chain([(gu.packed, h, dict(epilogue="silu_mul", norm_w=nw, out=act)),
                        (dn.packed, act, dict(epilogue="residual", residual=h, out=y))])
    torch.cuda.synchronize()

    def deq(q):
        return OF.dequantize_rows({"format": "nvfp4", "weight": q.codes.cpu().numpy(),
                                   "weight_scale": q.scales.cpu().numpy(), "row_scale": q.row_scale.cpu().numpy(),
                                   "weight_scale_2": 1.0})
    wgu = deq(gu)
    wgu = wgu[np.argsort(ON.interleave_chunks(inter, inter, 8))]
    hh = from_dev_bf16(h)
    xn = ON.rms_norm(hh, nw.cpu().numpy() - 1.0, 1e-6)
    a_ref = ON.linear(xn, wgu, epilogue="silu_mul")
    chk = check_against_oracle(from_dev_bf16(act), a_ref)
    assert chk.ok_rounded() and chk.within, chk
    y_ref = ON.linear(from_dev_bf16(act), deq(dn), epilogue="residual", residual=hh)
    chk = check_against_oracle(from_dev_bf16(y), y_ref)
    assert chk.ok_rounded() and chk.within, chk


def test_layer_tail_chain_equals_separate_gemvs(torch_gpu):
    """out_proj (gated head norm on o with z, residual h) → gate|up (norm on h1) → down (residual h1): the GDN
    layer's tail at 27B shapes, h1 passing between phases inside the launch; then a graph replays it."""
    torch = torch_gpu
    from monolith_mi355 import kernels
    from monolith_mi355.layers import nvfp4_matrix
    from monolith_mi355.runtime import hip
    _say("chain layer tail")
    gu, dn, nw, h, gen = _mlp_parts(torch, 5120, 17408, 9)
    wo = nvfp4_matrix(5120, 6144, gen, "cuda")
    o = (torch.randn(1, 6144, generator=gen, device="cuda") * 0.3).to(torch.bfloat16)
    z = (torch.randn(1, 6144, generator=gen, device="cuda")).to(torch.bfloat16)
    gw = (1.0 + torch.randn(128, generator=gen, device="cuda") * 0.2).to(torch.bfloat16).float()
    h1_ref = kernels.gemv(wo.packed, o, epilogue="residual", residual=h, gated_norm=(gw, z, 1e-6))
    act_ref, y_ref = _unfused_mlp(kernels, gu, dn, nw, h1_ref)
    h1 = torch.empty_like(h1_ref)
    act = torch.empty_like(act_ref)
    y = torch.empty_like(y_ref)
    phases = [(wo.packed, o, dict(epilogue="residual", residual=h, gated_norm=(gw, z, 1e-6), out=h1)),
              (gu.packed, h1, dict(epilogue="silu_mul", norm_w=nw, out=act)),
              (dn.packed, act, dict(epilogue="residual", residual=h1, out=y))]
    kernels.gemv_chain(phases)
    torch.cuda.synchronize()
    assert torch.equal(h1, h1_ref) and torch.equal(act, act_ref) and torch.equal(y, y_ref)
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        kernels.gemv_chain(phases, stream=s)                   # the stream's scratch exists before the capture
    s.synchronize()
    g = hip.Graph(s)
    with g:
        kernels.gemv_chain(phases, stream=s)
    for _ in range(3):
        for t in (h1, act, y):
            t.fill_(float("nan"))
        torch.cuda.synchronize()
        g.launch()
        s.synchronize()
        assert torch.equal(h1, h1_ref) and torch.equal(act, act_ref) and torch.equal(y, y_ref)


def test_chain_rejects_bad_phases(torch_gpu):
    torch = torch_gpu
    from monolith_mi355 import kernels
    gu, dn, nw, h, _ = _mlp_parts(torch, 640, 2048, 1)
    with pytest.raises(ValueError):
        kernels.gemv_chain([])
    h2 = torch.zeros(2, 640, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(ValueError):
        kernels.gemv_chain([(gu.packed, h2, dict(epilogue="silu_mul"))])
