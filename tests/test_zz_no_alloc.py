"""mi_gemv_noalloc — mi_gemv without any allocation (its split-K scratch is a fixed device-resident array per GPU):
through the C ABI its outputs equal mi_gemv's bit for bit, on two calls in a row the second with a smaller input,
for a split-K plan folded in the kernel (arrival counters), a split-K plan with a reduction launch (partials) and a
plan with no scratch; a shape that needs more scratch than the array holds is refused before anything runs."""

import ctypes as C

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _say(*a):
    print(*a, flush=True)


def _desc(hip, w, x, y, n, k, m):
    return hip.MiGemvDesc(format=1, n=n, k=k, m=m, w=hip.ptr(w.data), row_scale=hip.ptr(w.row_scale), x=hip.ptr(x),
                          ldx=k, y=hip.ptr(y), ldy=n, out_f32=1)


@pytest.mark.parametrize("n,k,m1,m2", [(5120, 17408, 2, 1),      # gemv_row, 3 K splits folded in the kernel
                                       (5120, 17408, 16, 8),     # gemv_rowm, 3 K splits + the reduction launch
                                       (2048, 4096, 8, 3)])      # no split: no scratch at all
def test_noalloc_gemv_equals_mi_gemv(torch_gpu, n, k, m1, m2):
    torch = torch_gpu
    from monolith_mi355.layers import nvfp4_matrix
    from monolith_mi355.runtime import hip
    lib = hip.load()
    _say(f"noalloc gemv n={n} k={k} m={m1},{m2}")
    gen = torch.Generator(device="cuda")
    gen.manual_seed(n + k)
    w = nvfp4_matrix(n, k, gen, "cuda").packed
    s = torch.cuda.current_stream()
    for m in (m1, m2):                               # the second call smaller: the array keeps the first's contents
        x = torch.randn(m, k, generator=gen, device="cuda").to(torch.bfloat16)
        y_ref = torch.full((m, n), float("nan"), device="cuda")
        y = torch.full((m, n), float("nan"), device="cuda")
        d = _desc(hip, w, x, y_ref, n, k, m)
        plan = (C.c_int32 * 7)()
        hip.call("mi_gemv_plan", C.byref(d), plan)
        need = lib.mi_gemv_workspace_bytes(C.byref(d))
        assert need <= lib.mi_gemv_noalloc_scratch_bytes(), need
        _say(f"  m={m} plan {list(plan)} scratch {need} B")
        hip.call("mi_gemv", C.byref(d), hip.stream_handle(s))
        d.y = hip.ptr(y)
        hip.call("mi_gemv_noalloc", C.byref(d), hip.stream_handle(s))
        torch.cuda.synchronize()
        assert torch.isfinite(y_ref).all()
        assert torch.equal(y.view(torch.int32), y_ref.view(torch.int32)), m
        hip.call("mi_gemv_noalloc", C.byref(d), hip.stream_handle(s))   # again: counters re-armed
        torch.cuda.synchronize()
        assert torch.equal(y.view(torch.int32), y_ref.view(torch.int32)), m


def test_noalloc_gemv_refuses_shapes_beyond_its_array(torch_gpu):
    from monolith_mi355.runtime import hip
    lib = hip.load()
    n, k, m = 65536, 17408, 16                       # split-K partials of 3 × 16 × 65536 FP32 > 8 MiB
    d = hip.MiGemvDesc(format=1, n=n, k=k, m=m, w=256, row_scale=0, x=256, ldx=k, y=256, ldy=n, out_f32=1)
    assert lib.mi_gemv_workspace_bytes(C.byref(d)) > lib.mi_gemv_noalloc_scratch_bytes()
    assert lib.mi_gemv_noalloc(C.byref(d), None) == 1
    assert "more than" in hip.last_error(), hip.last_error()
    d.workspace, d.workspace_bytes = 256, 1 << 20
    assert lib.mi_gemv_noalloc(C.byref(d), None) == 1 and "workspace = NULL" in hip.last_error()
