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
