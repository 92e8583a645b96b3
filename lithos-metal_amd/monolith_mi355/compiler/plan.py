"""The gfx950 lowering of a step graph in the reference's op contract: a private op list the passes rewrite (the
caller's ``Graph`` is never modified) and the passes that fold the reference's op split into this backend's
launches.

The reference splits a decode layer into many small dispatches for its GPU (a norm statistic, a core writing FP32
partials, a merge, sibling GEMVs over row ranges of one slab). On MI355X each of those is a kernel boundary of
3–5 µs, so the backend's entry points carry them fused; these passes rewrite the op list into those entry points'
terms, each pass checking the pattern it folds and leaving anything else as it is:

* ``merge_row_ranges`` — GEMVs that read the same input (and norm) over row ranges that tile one slab become one
  launch over the whole slab; each range's output is a column view of the merged output (the GDN ``z`` rows beside
  ``qkv|a|b``, attention's gate rows beside ``q|k|v``);
* ``merge_adjacent_slabs`` — GEMVs of one input and norm whose slabs lie back to back in the pack (same format and
  K, the first a whole number of tiles) become one launch over the stacked matrix (the MoE router and the shared
  expert's gate);
* ``fuse_norm_stat`` — ``rmsnorm_stat`` whose every consumer takes the norm on load (``gemv`` / ``lm_head`` with
  ``norm``, ``norm_apply``) disappears: those entry points compute the statistic themselves;
* ``fold_norm_apply`` — a ``norm_apply`` whose output feeds only GEMVs becomes their fused input norm;
* ``fuse_gdn`` — ``gdn_mixer`` + its ``gdn_norm`` become one ``mi_gdn_step``; at T ≤ 2 the norm moves onto the
  output projection's load (``defer``), as the hand-built layer does;
* ``fold_gdn_conv`` — at T ≤ 2 the GDN short conv runs in the input projection's epilogue, and the step reads the
  convolved values;
* ``fuse_gqa`` — ``gqa_decode`` + ``gqa_merge`` become one ``mi_gqa_decode`` (the merge and the gate inside);
* ``fuse_shared_expert`` — a MoE block whose shared expert has the routed experts' shape and sits right after them
  in the pack runs it as one more slot of the grouped launches and the combine (its weight bf16(σ(gate)) written by
  the route); at T = 1 the gate|up launch then routes for itself;
* ``plan_moe_groups`` — the expert-group records each route writes for the grouped GEMVs that read its ids.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import Any, Callable, Dict, List, Optional, Sequence, Tuple

from ..core.shapes import bind, step_bindings


@dataclass(eq=False)
class PVal:
    """A value the passes create (a merged output, a route's expert groups): name, bound shape, dtype name."""

    name: str
    shape: Tuple[int, ...]
    dtype: str
    is_input: bool = False
    is_weight: bool = False
    is_state: bool = False
    is_const: bool = False
    view_of: Any = None
    format: Optional[str] = None


@dataclass(eq=False)
class POp:
    kind: str
    inputs: List[Any]
    outputs: List[Any]
    attrs: Dict[str, Any]
    name: str = ""


@dataclass(frozen=True)
class Alias:
    """A value stored inside another value's buffer: ``col`` elements into each of its rows, the base's row stride."""

    base: str
    col: int


def dtype_name(v) -> str:
    return str(v.dtype).split(".")[-1].lower() if not isinstance(v.dtype, str) else v.dtype


@dataclass
class Plan:
    ops: List[POp]
    t: int
    values: Dict[str, Any]                       # the graph's values and the passes' own, by name
    alias: Dict[str, Alias] = field(default_factory=dict)
    slabs: Dict[str, dict] = field(default_factory=dict)   # pack manifest entries by slab name
    report: Dict[str, int] = field(default_factory=dict)

    @classmethod
    def from_graph(cls, g, t: int, slabs: Dict[str, dict]) -> "Plan":
        ops = [POp(op.kind, list(op.inputs), list(op.outputs), dict(op.attrs), op.kind) for op in g.ops]
        return cls(ops, t, dict(g.values), {}, slabs)

    # ---- shapes and buffers ---------------------------------------------------------------------------------
    def shape(self, v) -> Tuple[int, ...]:
        return tuple(v.shape) if isinstance(v, PVal) else bind(v.shape, step_bindings(self.t))

    def width(self, v) -> int:
        """Elements per row of a value's own shape."""
        s = self.shape(v)
        n = 1
        for d in s[1:]:
            n *= d
        return n

    def root(self, v) -> Tuple[str, int]:
        """(buffer-owning value, column offset in elements) of a value: follows aliases."""
        name, col = v.name, 0
        while name in self.alias:
            a = self.alias[name]
            name, col = a.base, col + a.col
        return name, col

    def ld(self, v) -> int:
        """Row stride in elements: the buffer owner's row width."""
        name, _ = self.root(v)
        return self.width(self.values[name])

    def new_value(self, name: str, shape: Sequence[int], dtype: str) -> PVal:
        base, i = name, 0
        while name in self.values:
            i += 1
            name = f"{base}.{i}"
        v = PVal(name, tuple(int(d) for d in shape), dtype)
        self.values[name] = v
        return v

    # ---- structure ------------------------------------------------------------------------------------------
    def consumers(self, v) -> List[POp]:
        return [op for op in self.ops if any(x is v for x in op.inputs)]

    def readers(self, name: str) -> List[POp]:
        """Ops that read the value ``name`` or any alias of it."""
        names = {name} | {a for a, al in self.alias.items() if al.base == name}
        return [op for op in self.ops if any(getattr(x, "name", None) in names for x in op.inputs)]

    def bump(self, what: str) -> None:
        self.report[what] = self.report.get(what, 0) + 1


# ---- passes ------------------------------------------------------------------------------------------------------
def _norm_key(op: POp):
    """What a GEMV reads: x and the norm it applies on load (weight value and eps), however it is expressed — the
    reference's ``norm`` inputs or a folded ``norm_apply`` (the statistic is recomputed either way)."""
    x = op.inputs[0]
    if op.attrs.get("norm"):
        return (id(x), id(op.inputs[3]), float(op.attrs.get("eps", 1e-6)))
    if op.attrs.get("fused_norm") is not None:
        nw, eps = op.attrs["fused_norm"]
        return (id(x), id(nw), float(eps))
    return (id(x), None, None)


def _plain(op: POp) -> bool:
    """A GEMV without an epilogue or other option the merge would have to reconcile."""
    a = op.attrs
    return (op.kind == "gemv" and a.get("epilogue") is None and not a.get("round_silu")
            and not a.get("round_residual") and a.get("gated_norm") is None)


def merge_row_ranges(p: Plan) -> None:
    groups: Dict[Tuple, List[POp]] = {}
    for op in p.ops:
        if _plain(op):
            groups.setdefault((id(op.inputs[1]),) + _norm_key(op), []).append(op)
    for key, ops in groups.items():
        if len(ops) < 2:
            continue
        w = ops[0].inputs[1]
        n = p.shape(w)[0]
        rng = {id(op): tuple(op.attrs.get("row_range") or (0, n)) for op in ops}
        pos, ok = 0, True
        for op in sorted(ops, key=lambda o: rng[id(o)][0]):
            start, count = rng[id(op)]
            ok &= start == pos
            pos = start + count
        if not ok or pos != n:
            continue
        order = sorted(ops, key=p.ops.index)          # the merged launch takes the earliest one's place
        _merge(p, order, [rng[id(op)][0] for op in order], n, f"{w.name}.y")
        p.bump("merge_row_ranges")


def _merge(p: Plan, ops: List[POp], cols: List[int], n: int, out_name: str, weights=None) -> POp:
    """Replace ``ops`` (same input and norm) by one GEMV of ``n`` rows; op i's output becomes the columns
    ``cols[i]..`` of its output, whose rows are padded to 8 elements (16-byte aligned rows). The merged op takes the
    place of the first; the others disappear."""
    first = ops[0]
    y0 = first.outputs[0]
    y = p.new_value(out_name, (p.shape(y0)[0], -(-n // 8) * 8), "bf16")
    attrs = dict(first.attrs)
    attrs.pop("row_range", None)
    attrs.pop("sibling", None)
    attrs["n_rows"] = n
    if weights is not None:
        attrs["stacked"] = weights
    merged = POp("gemv", list(first.inputs), [y], attrs, f"gemv:{out_name}")
    for op, c in zip(ops, cols):
        p.alias[op.outputs[0].name] = Alias(y.name, c)
    i = p.ops.index(first)
    p.ops[i] = merged
    for op in ops[1:]:
        p.ops.remove(op)
    return merged


def merge_adjacent_slabs(p: Plan) -> None:
    groups: Dict[Tuple, List[POp]] = {}
    for op in p.ops:
        if _plain(op) and op.attrs.get("row_range") is None and op.inputs[1].name in p.slabs:
            groups.setdefault(_norm_key(op), []).append(op)
    for ops in groups.values():
        if len(ops) < 2:
            continue
        ops = sorted(ops, key=lambda o: p.slabs[o.inputs[1].name]["offset"])
        run = [ops[0]]
        for op in ops[1:] + [None]:
            if op is not None and _adjacent(p.slabs[run[-1].inputs[1].name], p.slabs[op.inputs[1].name]):
                run.append(op)
                continue
            if len(run) > 1:
                slabs = [p.slabs[o.inputs[1].name] for o in run]
                cols = [0]
                for s in slabs[:-1]:
                    cols.append(cols[-1] + s["n"])
                n = cols[-1] + slabs[-1]["n"]
                order = sorted(run, key=lambda o: p.ops.index(o))
                by_op = dict(zip(run, cols))
                _merge(p, order, [by_op[o] for o in order], n, "+".join(o.inputs[1].name for o in run) + ".y",
                       weights=[o.inputs[1].name for o in run])
                p.bump("merge_adjacent_slabs")
            run = [op] if op is not None else []


def _adjacent(a: dict, b: dict) -> bool:
    """Slab ``b`` continues slab ``a`` as more rows of one matrix: same format and K, ``a`` whole tiles, codes and
    row-scale tables back to back."""
    if a["format"] != b["format"] or a["k"] != b["k"] or a["experts"] != 1 or b["experts"] != 1 or a["n"] % 16:
        return False
    if b["offset"] != a["offset"] + a["nbytes"]:
        return False
    ra, rb = a.get("row_scales_offset"), b.get("row_scales_offset")
    if (ra is None) != (rb is None):
        return False
    return ra is None or rb == ra + 4 * a["row_scales_len"]


def fuse_norm_stat(p: Plan) -> None:
    for op in list(p.ops):
        if op.kind != "rmsnorm_stat":
            continue
        if op.attrs.get("round_before_scale"):
            raise NotImplementedError("rmsnorm_stat: round_before_scale (a BF16 rounding between the normalization and "
                                      "the weight) is not built for gfx950")
        stat = op.outputs[0]
        users = p.consumers(stat)
        if all((u.kind in ("gemv", "lm_head") and u.attrs.get("norm") and u.inputs[2] is stat)
               or (u.kind == "norm_apply" and u.inputs[1] is stat) for u in users):
            p.ops.remove(op)
            for u in users:
                u.attrs["stat_computed"] = True          # the entry point computes the statistic itself
            p.bump("fuse_norm_stat")


def fold_norm_apply(p: Plan) -> None:
    for op in list(p.ops):
        if op.kind != "norm_apply":
            continue
        xn = op.outputs[0]
        users = p.readers(xn.name)
        if not users or any(u.kind not in ("gemv", "moe_gemv") or u.inputs[0] is not xn or u.attrs.get("norm")
                            or u.attrs.get("fused_norm") is not None for u in users):
            continue
        h, _, nw = op.inputs
        for u in users:
            u.inputs[0] = h
            u.attrs["fused_norm"] = (nw, float(op.attrs.get("eps", 1e-6)))
        p.ops.remove(op)
        p.bump("fold_norm_apply")


def fuse_gdn(p: Plan, defer_max_t: int = 2) -> None:
    for op in list(p.ops):
        if op.kind != "gdn_mixer":
            continue
        o_part = op.outputs[0]
        users = p.consumers(o_part)
        if len(users) != 1 or users[0].kind != "gdn_norm":
            raise NotImplementedError("gdn_mixer: the FP32 read-out must feed one gdn_norm (the backend runs the "
                                      "gated norm inside the step or on the output projection's load)")
        norm = users[0]
        _, z, nw = norm.inputs
        y = norm.outputs[0]
        op.outputs = [y]
        op.attrs.update(z=z, norm_w=nw, norm_eps=float(norm.attrs.get("eps", op.attrs.get("eps", 1e-6))))
        p.ops.remove(norm)
        for c in p.ops:                               # the commit pass of the same layer reads the same operands
            if c.kind == "gdn_commit" and c.inputs == op.inputs:
                c.attrs.update(z=z, norm_w=nw, norm_eps=op.attrs["norm_eps"])
        # at T <= 2 the output projection applies the norm while it stages its input (gemv_row's 16-lane rows
        # hold a 128-column head)
        outs = p.consumers(y)
        if (p.t <= defer_max_t and len(outs) == 1 and outs[0].kind == "gemv" and outs[0].inputs[0] is y
                and not outs[0].attrs.get("norm") and outs[0].attrs.get("fused_norm") is None
                and p.ld(z) % 8 == 0 and p.slabs.get(outs[0].inputs[1].name, {}).get("format") in ("nvfp4", "int4_affine")):
            op.attrs["defer_norm"] = True
            outs[0].attrs["gated_norm"] = (nw, z, op.attrs["norm_eps"])
        p.bump("fuse_gdn")


def fold_gdn_conv(p: Plan) -> None:
    """At T <= 2 the GDN short conv moves into the input projection's epilogue (``mi_gemv_desc.conv_*``): the GEMV
    that produces the step's q|k|v rows convolves each of them where it is computed and writes the convolved values
    to a buffer the step reads (``mi_gdn_desc.pre``); the step then skips its conv section (≈ 4 µs of dependent
    loads at one token). The commit pass of a speculative program keeps its own conv."""
    if p.t > 2:
        return
    for op in p.ops:
        if op.kind != "gdn_mixer":
            continue
        a = op.attrs
        ps = a["proj_segments"]
        qkv_val = op.inputs[ps["in_proj_qkv"][0]]
        root, col = p.root(qkv_val)
        prod = next((o for o in p.ops if o.kind == "gemv" and o.outputs[0].name == root), None)
        if prod is None or prod.attrs.get("epilogue") is not None or prod.attrs.get("row_range") is not None:
            continue
        n_main = 1 + max(idx for idx, _, _ in ps.values())
        cs = op.inputs[n_main]
        conv_w = op.inputs[n_main + 2]
        channels = 2 * a["k_heads"] * a["dk"] + a["v_heads"] * a["dv"]
        row0 = col + ps["in_proj_qkv"][1]
        if row0 % 16 or channels % 16:
            continue
        pre = p.new_value(f"{op.outputs[0].name}.pre", (p.t, channels), "bf16")
        prod.attrs["conv"] = dict(w=conv_w, state=cs, out=pre, row0=row0, channels=channels)
        a["pre"] = pre
        p.bump("fold_gdn_conv")


def fuse_gqa(p: Plan) -> None:
    for op in list(p.ops):
        if op.kind != "gqa_decode":
            continue
        users = p.consumers(op.outputs[0])
        if len(users) != 1 or users[0].kind != "gqa_merge":
            raise NotImplementedError("gqa_decode: its partials must feed one gqa_merge (fused in mi_gqa_decode)")
        merge = users[0]
        op.attrs["gate_value"] = merge.inputs[2] if len(merge.inputs) > 2 else None
        op.attrs["gate"] = bool(merge.attrs.get("gate", op.attrs["gate_value"] is not None))
        op.outputs = [merge.outputs[0]]
        p.ops.remove(merge)
        p.bump("fuse_gqa")


def fuse_shared_expert(p: Plan) -> None:
    for comb in list(p.ops):
        if comb.kind != "moe_combine" or not comb.attrs.get("has_shared"):
            continue
        hk, weights, s_out, s_gate = comb.inputs[:4]
        down = next((o for o in p.ops if hk in o.outputs and o.kind == "moe_gemv"), None)
        sdown = next((o for o in p.ops if s_out in o.outputs and o.kind == "gemv"), None)
        if down is None or sdown is None:
            continue
        act = down.inputs[0]
        gu = next((o for o in p.ops if act in o.outputs and o.kind == "moe_gemv"), None)
        s_act = sdown.inputs[0]
        sgu = next((o for o in p.ops if s_act in o.outputs and o.kind == "gemv"), None)
        route = next((o for o in p.ops if o.kind == "moe_route" and down.inputs[2] in o.outputs), None)
        if gu is None or sgu is None or route is None:
            continue
        e_slabs = [p.slabs.get(gu.inputs[1].name), p.slabs.get(down.inputs[1].name)]
        s_slabs = [p.slabs.get(sgu.inputs[1].name), p.slabs.get(sdown.inputs[1].name)]
        if None in e_slabs or None in s_slabs:
            continue
        ok = True
        for e, s, rows in zip(e_slabs, s_slabs, (gu.attrs["expert_rows"], down.attrs["expert_rows"])):
            n_exp = e["n"] * e["experts"] // rows
            ok &= (s["n"] * s["experts"] == rows and s["format"] == e["format"] and s["k"] == e["k"]
                   and rows % 16 == 0 and s["offset"] == e["offset"] + e["nbytes"]
                   and (e.get("row_scales_offset") is None or
                        s.get("row_scales_offset") == e["row_scales_offset"] + 4 * e["row_scales_len"]))
        # the shared expert's input must be the experts' (the same normalized h), its gate|up one rounding
        ok &= _norm_key(sgu) == _norm_key(gu) and sgu.attrs.get("epilogue") == "silu_mul"
        ok &= sdown.attrs.get("epilogue") is None and gu.attrs.get("x_per_slot") is False
        # the shared gate's logit sits in the router's merged output, one column after the experts
        gate_root, gate_col = p.root(s_gate)
        logit_root, logit_col = p.root(route.inputs[0])
        n_exp = int(route.attrs["n_experts"])
        ok &= gate_root == logit_root and gate_col == logit_col + n_exp
        if not ok:
            continue
        k = int(route.attrs["top_k"])
        t = p.shape(route.inputs[0])[0]
        ids, wts = route.outputs
        ids2 = p.new_value(f"{ids.name}.slots", (t, k + 1), "i32")       # the shared expert is slot k of every token
        wts2 = p.new_value(f"{wts.name}.slots", (t, k + 1), "f32")
        route.outputs = [ids2, wts2]
        act, hk2 = gu.outputs[0], None                # k + 1 slots of rows in the experts' outputs
        act2 = p.new_value(f"{act.name}.slots", (t, (k + 1) * (gu.attrs["expert_rows"] // 2)), "bf16")
        hk2 = p.new_value(f"{hk.name}.slots", (t, (k + 1) * down.attrs["expert_rows"]), "bf16")
        gu.outputs[0] = act2
        down.inputs[0] = act2
        down.outputs[0] = hk2
        route.attrs.update(shared_expert=n_exp, shared_gate_col=n_exp)
        for op in (gu, down):
            op.inputs[2] = ids2
            op.attrs["slots"] = k + 1
        gu.attrs.update(shared_expert=n_exp, shared_epilogue="silu_mul")   # its own rounding; down has no epilogue
        comb.attrs.update(has_shared=False, slots=k + 1, shared_fused=True)
        comb.inputs = [hk2, wts2] + comb.inputs[4:]
        p.ops.remove(sgu)
        p.ops.remove(sdown)
        if p.t == 1:                                  # one token: the gate|up launch routes for itself
            route.attrs["inline"] = True
            gu.attrs["route_op"] = route
        p.bump("fuse_shared_expert")


def plan_moe_groups(p: Plan) -> None:
    """Each route's expert groups (the grouped GEMV's records): a buffer of ``max_groups`` records of 18 words —
    one per (token, slot) pair in records of at most two pairs at T >= 3, else one per distinct expert."""
    for route in p.ops:
        if route.kind != "moe_route":
            continue
        t = p.shape(route.inputs[0])[0]
        e, k = int(route.attrs["n_experts"]), int(route.attrs["top_k"])
        sh = 1 if route.attrs.get("shared_expert") else 0
        ppr = 2 if t > 2 else 0
        n = t * (k + sh) if ppr else min(e, t * k) + sh
        if route.attrs.get("inline"):
            n = k + sh                                # record g = slot g
        groups = p.new_value(f"{route.outputs[0].name}.groups", (n, 18), "i32")
        route.attrs.update(groups=groups, pairs_per_record=ppr)
        for op in p.ops:
            if op.kind == "moe_gemv" and op.inputs[2] is route.outputs[0]:
                op.attrs.update(groups=groups, pairs_per_record=ppr)


def _norm_of(op: POp):
    """(weight value, eps) of the RMSNorm a GEMV applies on load, or None."""
    if op.attrs.get("norm"):
        return op.inputs[3], float(op.attrs.get("eps", 1e-6))
    if op.attrs.get("fused_norm") is not None:
        nw, eps = op.attrs["fused_norm"]
        return nw, float(eps)
    return None


def hand_over_norm(p: Plan) -> None:
    """At T >= 3 a dense residual GEMV or a MoE combine whose output feeds GEMVs that normalize it on load (the next
    layer's input projections, the LM head) writes the normalized rows itself — its split-K reduction or the combine
    computes them (``mi_gemv`` / ``mi_moe_combine`` ``next_norm``) — and those GEMVs read them as they are: the input
    norm takes no launch of its own. The same values (the norm is ``norm_apply``'s either way); at T <= 2 the GEMVs
    keep the norm fused on load."""
    if p.t < 3:
        return
    for prod in list(p.ops):
        dense_res = (prod.kind == "gemv" and prod.attrs.get("epilogue") == "residual"
                     and prod.attrs.get("gated_norm") is None and not prod.attrs.get("round_residual"))
        if not (dense_res or prod.kind == "moe_combine"):
            continue
        h = prod.outputs[0]
        users = [u for u in p.consumers(h) if u.inputs[0] is h and u.kind in ("gemv", "lm_head")
                 and _norm_of(u) is not None]
        norms = {(id(_norm_of(u)[0]), _norm_of(u)[1]) for u in users}
        if not users or len(norms) != 1 or p.width(h) % 8:
            continue
        nw, eps = _norm_of(users[0])
        xn = p.new_value(f"{h.name}.normed", (p.t, p.width(h)), "bf16")
        prod.attrs["next_norm"] = (nw, xn, eps)
        for u in users:
            if u.attrs.get("norm"):
                u.inputs = [xn, u.inputs[1]] + list(u.inputs[4:])
                u.attrs["norm"] = False
                u.attrs.pop("stat_computed", None)
            else:
                u.inputs[0] = xn
                u.attrs["fused_norm"] = None
        p.bump("hand_over_norm")


PASSES: Tuple[Callable[[Plan], None], ...] = (merge_row_ranges, merge_adjacent_slabs, fuse_norm_stat, fold_norm_apply,
                                              fuse_gdn, fold_gdn_conv, fuse_gqa, fuse_shared_expert, plan_moe_groups,
                                              hand_over_norm)


def run_passes(p: Plan, passes: Sequence[Callable[[Plan], None]] = PASSES) -> Plan:
    for fn in passes:
        fn(p)
    return p
