"""Writes the step graphs the reference's own model classes lower, as JSON fixtures: the op contract the gfx950
compiler must accept (op kinds, input positions, attrs, value and slab names).

Run in a container that has the reference checkout (``/root/reference`` or ``$LITHOS_REFERENCE``):
``python tests/golden/make_graph_golden.py``. It builds the reference's ``Qwen3_5Model`` (a Gated DeltaNet layer and
a gated-attention layer with dense MLPs) and ``Qwen3_5MoeModel`` (the same mixers with sparse MoE feed-forwards) at
a small geometry, binds NVFP4 storage to every projection except the BF16 router / shared-expert gate / embedding /
LM head, calls ``model.lower(g)`` and saves every value (name, shape, dtype, format, role flags, view) and every op
(kind, input and output names, domain, class, attrs) to ``graph_<model>.json`` next to this script, and the layout
those names stand for — each stacked slab's row permutation and the pack's RoPE tables (BF16 bits) — to
``graph_layout.npz``. The fixtures are data; the reference code is not needed where the tests run.
"""

from __future__ import annotations

import json
import os
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
REF = Path(os.environ.get("LITHOS_REFERENCE", "/root/reference"))

GEOMETRY = dict(hidden_size=1024, num_hidden_layers=2, num_attention_heads=4, num_key_value_heads=1, head_dim=128,
                layer_types=["linear_attention", "full_attention"], linear_num_key_heads=2, linear_num_value_heads=4,
                linear_key_head_dim=128, linear_value_head_dim=128, linear_conv_kernel_dim=4, rms_norm_eps=1e-6,
                vocab_size=4096, max_position_embeddings=256, rope_theta=1e6, partial_rotary_factor=0.5)
MAX_CONTEXT = 256


def _attr(v):
    if isinstance(v, dict):
        return {str(k): _attr(x) for k, x in v.items()}
    if isinstance(v, (list, tuple)):
        return [_attr(x) for x in v]
    if isinstance(v, (np.integer,)):
        return int(v)
    if isinstance(v, (np.floating,)):
        return float(v)
    if hasattr(v, "name") and type(v).__name__ == "Sym":
        return {"sym": v.name}
    if isinstance(v, (str, int, float, bool)) or v is None:
        return v
    raise TypeError(f"attr value {v!r} ({type(v).__name__}) has no JSON form")


def graph_json(g) -> dict:
    values = []
    for v in g.values.values():
        values.append(dict(name=v.name, shape=[_attr(d) for d in v.shape], dtype=str(v.dtype), format=v.format,
                           is_input=v.is_input, is_weight=v.is_weight, is_state=v.is_state, is_const=v.is_const,
                           view_of=list(v.view_of) if v.view_of is not None else None))
    ops = [dict(kind=op.kind, inputs=[v.name for v in op.inputs], outputs=[v.name for v in op.outputs],
                domain=[op.domain.kind, _attr(op.domain.n_blocks)], klass=op.klass.value, attrs=_attr(op.attrs))
           for op in g.ops]
    return dict(name=g.name, values=values, ops=ops)


def bind_nvfp4(model) -> None:
    from monolith.nn.linear import Linear
    for _, mod in model.named_modules():
        if isinstance(mod, Linear) and not any(s in mod.prefix for s in ("router.", "shared_gate.")):
            for p in mod.parts:
                mod.set_format(p.local, "nvfp4")


def main():
    sys.path.insert(0, str(REF))
    from monolith.core.ir import Graph
    from monolith.models.qwen3_5.config import Qwen3_5Config
    from monolith.models.qwen3_5.model import Qwen3_5Model
    from monolith.models.qwen3_5_moe.config import Qwen3_5MoeConfig
    from monolith.models.qwen3_5_moe.model import Qwen3_5MoeModel

    dense = Qwen3_5Model(Qwen3_5Config(intermediate_size=1024, **GEOMETRY), max_context=MAX_CONTEXT)
    moe = Qwen3_5MoeModel(Qwen3_5MoeConfig(moe_intermediate_size=512, shared_expert_intermediate_size=512,
                                           num_experts=64, num_experts_per_tok=8, **GEOMETRY), max_context=MAX_CONTEXT)
    # the layout data the graph's names stand for: each slab's row permutation and the pack's RoPE tables
    perms = {}
    for _, mod in dense.named_modules():
        if hasattr(mod, "slab_groups") and hasattr(mod, "parts"):
            for grp in mod.slab_groups():
                if grp.row_perm is not None:
                    perms[grp.name] = np.asarray(grp.row_perm, np.int64)
    tables = {k: np.asarray(arr) for k, (_dtype, arr) in dense.tables().items()}
    np.savez_compressed(HERE / "graph_layout.npz", **{f"perm:{k}": v for k, v in perms.items()},
                        **{f"table:{k}": v for k, v in tables.items()})
    for tag, model in (("qwen3_5", dense), ("qwen3_5_moe", moe)):
        bind_nvfp4(model)
        g = Graph("step")
        token = model.lower(g)
        g.check()
        out = graph_json(g)
        out["token"] = token.name
        out["geometry"] = dict(GEOMETRY, max_context=MAX_CONTEXT)
        (HERE / f"graph_{tag}.json").write_text(json.dumps(out, indent=0, sort_keys=True))
        print(tag, len(g.ops), "ops", len(g.values), "values")


if __name__ == "__main__":
    main()
