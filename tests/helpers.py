"""Conversions between the oracle's quantized-matrix dicts and the product's DequantSpec, and BF16 tensors."""

from __future__ import annotations

import numpy as np

from monolith_mi355.formats import DequantSpec
from oracle.fp import bf16_to_f32, f32_to_bf16


def spec_of(m: dict) -> DequantSpec:
    """The product's DequantSpec for an oracle quantized-matrix dict."""
    n = m["weight"].shape[0]
    if m["format"] == "nvfp4":
        k = m["weight"].shape[1] * 2
        return DequantSpec("nvfp4", (n, k), {"weight": m["weight"], "weight_scale": m["weight_scale"]},
                           {"weight_scale_2": m["weight_scale_2"]})
    if m["format"] == "int4_affine":
        k = m["weight"].shape[1] * 2
        return DequantSpec("int4_affine", (n, k), {"weight": m["weight"], "scales": m["scales"], "biases": m["biases"]},
                           {"group": 64})
    if m["format"] == "fp8_e4m3":
        return DequantSpec("fp8_e4m3", m["weight"].shape, {"weight": m["weight"]}, {"weight_scale": m["weight_scale"]})
    return DequantSpec("bf16", m["weight"].shape, {"weight": m["weight"]})


def to_dev_bf16(torch, a, device="cuda"):
    """float32 numpy (BF16-valued or not) → device bfloat16 tensor (RNE)."""
    u = f32_to_bf16(np.asarray(a, np.float32)).astype(np.int16)
    return torch.from_numpy(u).view(torch.bfloat16).to(device)


def from_dev_bf16(t) -> np.ndarray:
    return bf16_to_f32(t.detach().cpu().view(__import__("torch").int16).numpy().astype(np.uint16))


def graph_from_json(d):
    """A ``monolith_mi355.core.Graph`` rebuilt from a fixture written by ``golden/make_graph_golden.py`` (the graph
    the reference's own model lowered): the same values, ops, attrs and order."""
    from monolith_mi355.core import BlockDomain, DType, Graph, OpClass, Sym

    def val(x):
        if isinstance(x, dict) and set(x) == {"sym"}:
            return Sym(x["sym"])
        if isinstance(x, dict):
            return {k: val(v) for k, v in x.items()}
        if isinstance(x, list):
            return [val(v) for v in x]
        return x

    g = Graph(d["name"])
    for v in d["values"]:
        shape = tuple(val(s) for s in v["shape"])
        dt = DType.parse(v["dtype"])
        if v["is_input"]:
            g.input(v["name"], shape, dt)
        elif v["is_weight"]:
            g.weight(v["name"], shape, v["format"])
        elif v["is_state"]:
            g.state(v["name"], shape, dt)
        elif v["is_const"]:
            g.const(v["name"], shape, dt)
        elif v["view_of"] is not None:
            continue
        else:
            g.value(v["name"], shape, dt, format=v["format"], scoped=False)
    for v in d["values"]:
        if v["view_of"] is not None:
            base, row = v["view_of"]
            g.view(v["name"], g.values[base], row, int(v["shape"][0]))
    for op in d["ops"]:
        attrs = val(op["attrs"])
        g.op(op["kind"], [g.values[n] for n in op["inputs"]], [g.values[n] for n in op["outputs"]],
             domain=BlockDomain(op["domain"][0], val(op["domain"][1])), klass=OpClass(op["klass"]), **attrs)
    return g, g.values[d["token"]]
