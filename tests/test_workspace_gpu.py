"""The library's own scratch buffers (split-K partials and fold counters) stay valid for graphs captured before
they grew, and never grow inside a capture."""

import pytest

pytestmark = pytest.mark.gpu


def _say(*a):
    print(*a, flush=True)


def test_captured_gemv_survives_a_larger_eager_call(torch_gpu):
    torch = torch_gpu
    from monolith_mi355 import kernels
    from monolith_mi355.layers import nvfp4_matrix
    from monolith_mi355.runtime import hip
    _say("workspace: capture, grow, replay")
    gen = torch.Generator(device="cuda")
    gen.manual_seed(3)
    small = nvfp4_matrix(1024, 17408, gen, "cuda")          # M = 1: three K splits folded in the kernel
    big = nvfp4_matrix(5120, 17408, gen, "cuda")            # M = 8: split-K partials, a larger workspace
    s = torch.cuda.Stream()
    x = (torch.randn(1, 17408, generator=gen, device="cuda")).to(torch.bfloat16)
    x8 = (torch.randn(8, 17408, generator=gen, device="cuda")).to(torch.bfloat16)
    y = torch.empty(1, 1024, dtype=torch.bfloat16, device="cuda")
    torch.cuda.synchronize()
    with torch.cuda.stream(s):
        kernels.gemv(small.packed, x, out=y, stream=s)      # grows the stream's scratch to this shape
    s.synchronize()
    ref = y.clone()
    g = hip.Graph(s)
    with g:
        kernels.gemv(small.packed, x, out=y, stream=s)
    y.zero_()
    torch.cuda.synchronize()
    g.launch()
    s.synchronize()
    assert torch.equal(y, ref)
    with torch.cuda.stream(s):
        y8 = kernels.gemv(big.packed, x8, stream=s)         # needs more scratch: a new buffer, the old one kept
    s.synchronize()
    assert torch.isfinite(y8.float()).all()
    for _ in range(3):
        y.zero_()
        torch.cuda.synchronize()
        g.launch()
        s.synchronize()
        assert torch.equal(y, ref), "the replay after the scratch grew differs"


def test_scratch_refuses_to_grow_during_a_capture(torch_gpu):
    torch = torch_gpu
    from monolith_mi355 import kernels
    from monolith_mi355.layers import nvfp4_matrix
    from monolith_mi355.runtime import hip
    _say("workspace: no growth inside a capture")
    gen = torch.Generator(device="cuda")
    gen.manual_seed(4)
    w = nvfp4_matrix(2048, 17408, gen, "cuda")
    s = torch.cuda.Stream()                                 # a fresh stream: its scratch does not exist yet
    x = torch.randn(8, 17408, generator=gen, device="cuda").to(torch.bfloat16)
    y = torch.empty(8, 2048, dtype=torch.bfloat16, device="cuda")
    torch.cuda.synchronize()
    g = hip.Graph(s)
    with pytest.raises(hip.MiError, match="during a graph capture"):
        with g:
            kernels.gemv(w.packed, x, out=y, stream=s)
