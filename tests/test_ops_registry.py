"""The operator API (the reference's ``monolith/ops/registry.py`` and ``compiler/coverage.py`` contract): bindings
resolve per profile with the wildcard fallback, rebinding is refused, every hot-path op kind has a gfx950 binding to
an entry point the library exports, coverage fails loudly for an unbound or unknown op, and ``run`` dispatches."""

import pytest


def test_registry_semantics():
    from monolith_mi355.ops import KernelBinding, OpClass, OpDef, Registry, WILDCARD
    od = OpDef("x_test", OpClass.MAP, "rows")
    od.bind(WILDCARD, KernelBinding("k_any"))
    od.bind("gfx950", KernelBinding("k_950", {"A": 1}))
    assert od.binding_for("gfx950").kernel == "k_950" and od.binding_for("other").kernel == "k_any"
    od.bind("gfx950", KernelBinding("k_950", {"A": 1}))            # identical rebinding is fine
    with pytest.raises(ValueError):
        od.bind("gfx950", KernelBinding("k_other"))
    reg = Registry("thing")
    reg.register("a", 1)
    with pytest.raises(ValueError):
        reg.register("a", 2)
    assert reg.resolve("b") is None and "a" in reg


def test_hot_path_ops_bound_to_exported_entry_points():
    import re
    from pathlib import Path
    from monolith_mi355.ops import OPS, PROFILE, check_coverage
    from monolith_mi355.ops.defs import DECODE_LAYER_OPS, STEP_OPS
    check_coverage(DECODE_LAYER_OPS + STEP_OPS)
    header = (Path(__file__).resolve().parents[1] / "include" / "lithos_mi355.h").read_text()
    declared = set(re.findall(r"\b(mi_[a-z0-9_]+)\s*\(", header))
    for kind in DECODE_LAYER_OPS + STEP_OPS:
        assert OPS[kind].binding_for(PROFILE).kernel in declared, kind


def _unbound():
    from monolith_mi355.ops import OPS, OpClass, OpDef, register_op
    if "test_unbound" not in OPS:
        register_op(OpDef("test_unbound", OpClass.MAP, "rows"))       # an op with no gfx950 binding
    return "test_unbound"


def test_coverage_reports_missing():
    from monolith_mi355.ops import CoverageError, check_coverage
    name = _unbound()
    with pytest.raises(CoverageError) as e:
        check_coverage(["gemv", name, "no_such_op"])
    assert f"{name} (no binding)" in str(e.value) and "no_such_op (unknown op)" in str(e.value)


def test_run_refuses_fused_and_unbound_ops():
    from monolith_mi355.ops import CoverageError, run
    with pytest.raises(CoverageError):
        run("norm_apply")
    with pytest.raises(CoverageError):
        run(_unbound())


@pytest.mark.gpu
def test_run_gemv_matches_kernel_call(torch_gpu):
    import numpy as np
    from helpers import spec_of, to_dev_bf16
    from oracle import formats as OF
    from monolith_mi355 import kernels
    from monolith_mi355.ops import run
    rng = np.random.default_rng(5)
    m = OF.nvfp4_random(64, 512, rng)
    w = kernels.upload(spec_of(m))
    x = to_dev_bf16(torch_gpu, rng.standard_normal((1, 512)))
    a = run("gemv", x, w).view(torch_gpu.int16)
    b = kernels.gemv(w, x).view(torch_gpu.int16)
    assert torch_gpu.equal(a, b)


@pytest.mark.gpu
def test_run_gdn_commit_matches_kernel_call(torch_gpu):
    """``gdn_commit`` through the op registry: the same state as the kernel's commit pass."""
    import numpy as np
    import torch
    from monolith_mi355 import kernels
    from monolith_mi355.ops import run
    hk, hv = 2, 4
    conv_dim = 2 * hk * 128 + hv * 128
    g = torch.Generator(device="cuda").manual_seed(3)
    proj = (torch.randn(4, hv * 128 + conv_dim + 2 * hv, generator=g, device="cuda")).to(torch.bfloat16)
    prm = dict(conv_w=(torch.randn(conv_dim, 4, generator=g, device="cuda") * 0.3).to(torch.bfloat16),
               neg_exp_a=-torch.ones(hv, device="cuda"), dt_bias=torch.zeros(hv, device="cuda"),
               norm_w=torch.ones(128, device="cuda"), k_heads=hk, v_heads=hv)
    conv_a = (torch.randn(conv_dim, 3, generator=g, device="cuda")).to(torch.bfloat16)
    rec_a = torch.randn(hv, 128, 128, generator=g, device="cuda") * 0.1
    n = torch.tensor([2], dtype=torch.int32, device="cuda")
    outs = []
    for via_run in (False, True):
        conv_b = torch.zeros_like(conv_a)
        rec_b = torch.zeros_like(rec_a)
        if via_run:
            run("gdn_commit", proj, conv_a, conv_b, rec_a, rec_b, committed=n, **prm)
        else:
            kernels.gdn_step(proj, conv_a, conv_b, rec_a, rec_b, commit=True, t_dev=n, **prm)
        torch.cuda.synchronize()
        outs.append((conv_b.cpu(), rec_b.cpu()))
    assert torch.equal(outs[0][0], outs[1][0]) and torch.equal(outs[0][1], outs[1][1])
