"""Graph builders in the reference's op contract: the ``lower`` half of ``monolith/nn`` for the decode layer, so a
step graph can be written here exactly as the reference's modules would write it (the same op kinds, input
positions, attrs, value and slab names) and fed to :func:`monolith_mi355.compiler.emit_program` — the same entry a
graph lowered by the reference itself takes. Only lowering lives here: the numerics are the oracle's, and the
kernels are the library's.

Conventions carried over because the emitter and the pack resolve by them:

* ``Linear`` (``nn/linear.py:63-191``): one ``gemv`` per format group of row-stacked parts; inputs
  ``[x, w, (stat, norm_w) if norm, residual if epilogue == "residual"]``; attrs ``norm``, ``epilogue``, ``format``,
  ``eps``, ``chunk``, ``row_range``, ``segments``, ``sibling``; the slab is named ``prefix + "+".join(parts)``;
* ``RMSNorm`` (``nn/norm.py:35-44``): a ``rmsnorm_stat`` op and the ``(1 + w)`` weight constant ``prefix + "weight"``;
* ``GatedDeltaNet`` (``nn/gdn.py:95-120``): the ``qkv|a|b`` rows, ``gdn_mixer`` into an FP32 ``o_part``, the ``z`` rows
  as a sibling, ``gdn_norm``, ``out_proj`` with the residual; states ``conv_state`` ``[2, conv_dim, W-1]`` BF16 and
  ``rec_state`` ``[2, hv, dk, dv]`` FP32 (two slots);
* ``GQAAttention`` (``nn/attention.py:133-155``): slab rows ``[q | k | v | gate]`` with the RoPE head-dim permutation
  on q and k, ``gqa_decode`` into partials, the gate rows as a sibling, ``gqa_merge``, ``o_proj`` with the residual;
  caches ``k_cache`` / ``v_cache`` ``[max_context, kv, D]`` BF16; RoPE tables ``rope_cos`` / ``rope_sin``
  ``[max_context, D]`` in the permuted layout;
* ``GatedMLP``, ``SparseMoE`` (``nn/mlp.py``, ``nn/moe.py:138-161``), ``Embedding``, ``LMHead``, ``GreedySampler``,
  ``DecoderLayer`` and the hybrid model's ``lower`` (``models/qwen3_5/model.py:103-117``).
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import Any, Dict, List, Optional, Sequence, Tuple

import numpy as np

from .core import BlockDomain, DType, Graph, OpClass, T, Value

CHUNK = 8                      # gate|up rows interleaved 8 by 8 (a 16-row tile holds 8 outputs of silu(gate)·up)


# ---- row permutations (packs/transforms.py:16-45) ----------------------------------------------------------------
def interleave_chunks(n_a: int, n_b: int, chunk: int) -> np.ndarray:
    """``perm[new] = old`` over ``[A; B]``: every ``2·chunk`` rows are ``chunk`` rows of A then the same of B."""
    if n_a != n_b or n_a % chunk:
        raise ValueError(f"interleave_chunks: need equal halves that are multiples of {chunk}")
    a = np.arange(n_a).reshape(-1, chunk)
    return np.concatenate([a, a + n_a], axis=1).reshape(-1)


def rope_head_perm(head_dim: int, rotary_dim: int) -> np.ndarray:
    """One head's dims reordered (``perm[new] = old``) so HF's partial-rotary pairs ``(i, i + rotary/2)`` sit at
    ``(i, i + head_dim/2)``: full-width pairs, the non-rotary dims in the remaining slots, in order."""
    if rotary_dim % 2 or head_dim % 2 or rotary_dim > head_dim:
        raise ValueError("rope_head_perm: rotary_dim even and <= head_dim (even)")
    r2, d2 = rotary_dim // 2, head_dim // 2
    pass_lo = np.arange(rotary_dim, rotary_dim + d2 - r2)          # the first half's non-rotary dims
    pass_hi = np.arange(rotary_dim + d2 - r2, head_dim)
    return np.concatenate([np.arange(r2), pass_lo, np.arange(r2, rotary_dim), pass_hi]).astype(np.int64)


def rope_tables_permuted(theta: float, head_dim: int, rotary_dim: int, max_pos: int) -> Tuple[np.ndarray, np.ndarray]:
    """FP32 ``[max_pos, head_dim]`` cos / sin in the permuted layout: the rotary frequencies at ``[0, rotary/2)`` and
    ``[D/2, D/2 + rotary/2)``, identity (cos 1, sin 0) elsewhere (``nn/rope.py:72-84``)."""
    inv = (1.0 / (theta ** (np.arange(0, rotary_dim, 2, dtype=np.float32) / rotary_dim))).astype(np.float32)
    ang = np.outer(np.arange(max_pos, dtype=np.float32), inv).astype(np.float32)
    full = np.zeros((max_pos, head_dim), np.float32)
    full[:, : rotary_dim // 2] = ang
    full[:, head_dim // 2: head_dim // 2 + rotary_dim // 2] = ang
    return np.cos(full).astype(np.float32), np.sin(full).astype(np.float32)


# ---- module plumbing ----------------------------------------------------------------------------------------------
@dataclass(frozen=True)
class StateEntry:
    """A per-sequence buffer the program allocates (``nn/module.py:44-62``); ``checkpoints`` slots of ``shape``."""

    name: str
    shape: Tuple[Any, ...]
    dtype: DType
    checkpoints: int = 1

    @property
    def buffer_shape(self) -> Tuple[Any, ...]:
        return ((self.checkpoints,) + tuple(self.shape)) if self.checkpoints > 1 else tuple(self.shape)


@dataclass
class LowerContext:
    states: Dict[str, Value] = field(default_factory=dict)
    consts: Dict[str, Value] = field(default_factory=dict)
    t: Any = T


@dataclass(frozen=True)
class NormInput:
    stat: Value
    weight: Value
    eps: float


@dataclass(frozen=True)
class SlabGroup:
    """A slab the pack holds and one ``gemv`` streams: ``parts`` ``(local, rows)`` stacked, then ``row_perm``."""

    name: str
    format: str
    parts: Tuple[Tuple[str, int], ...]
    row_perm: Optional[np.ndarray]
    k: int

    @property
    def rows(self) -> int:
        return sum(r for _, r in self.parts)


@dataclass
class Projection:
    values: List[Value]
    segments: Dict[str, Tuple[int, int, int]] = field(default_factory=dict)   # local -> (value, column, columns)

    @property
    def value(self) -> Value:
        if len(self.values) != 1:
            raise ValueError("projection has several outputs (mixed-format parts)")
        return self.values[0]


def _weight(g: Graph, name: str, shape, fmt: str) -> Value:
    v = g.values.get(name)
    if v is None:
        return g.weight(name, shape, fmt)
    if not v.is_weight or tuple(v.shape) != tuple(shape) or v.format != fmt:
        raise ValueError(f"slab {name!r} is already in the graph with another shape or format")
    return v


def _const(g: Graph, name: str, shape, dtype: DType) -> Value:
    v = g.values.get(name)
    if v is None:
        return g.const(name, shape, dtype)
    if not v.is_const:
        raise ValueError(f"{name!r} is not a constant of the graph")
    return v


class Linear:
    """Row-stacked checkpoint matrices ``parts`` ``[(local, rows)]`` over ``in_features``; ``formats`` maps a part to
    its storage format (default ``fmt``). Consecutive parts of one format form one slab."""

    def __init__(self, in_features: int, parts: Sequence[Tuple[str, int]], *, prefix: str, fmt: str = "nvfp4",
                 formats: Optional[Dict[str, str]] = None, row_perm=None, epilogue: Optional[str] = None,
                 chunk: Optional[int] = None):
        if epilogue not in (None, "residual", "silu_mul"):
            raise ValueError(f"Linear: unknown epilogue {epilogue!r}")
        self.k, self.parts, self.prefix = in_features, tuple(parts), prefix
        self.formats = {p: (formats or {}).get(p, fmt) for p, _ in self.parts}
        self.row_perm = None if row_perm is None else np.asarray(row_perm, np.int64)
        self.epilogue, self.chunk = epilogue, chunk
        if epilogue == "silu_mul" and (len(self.parts) != 2 or self.parts[0][1] != self.parts[1][1] or not chunk):
            raise ValueError("Linear: silu_mul needs two equal parts (gate, up) and a chunk")

    def slab_groups(self) -> List[SlabGroup]:
        groups: List[List[Tuple[str, int]]] = []
        fmts: List[str] = []
        for local, rows in self.parts:
            f = self.formats[local]
            if fmts and fmts[-1] == f:
                groups[-1].append((local, rows))
            else:
                groups.append([(local, rows)])
                fmts.append(f)
        if len(groups) > 1 and self.row_perm is not None:
            raise ValueError(f"Linear {self.prefix}: a row permutation cannot span storage formats {fmts}")
        return [SlabGroup(self.prefix + "+".join(p for p, _ in grp), f, tuple(grp),
                          self.row_perm if i == 0 else None, self.k) for i, (grp, f) in enumerate(zip(groups, fmts))]

    def lower(self, g: Graph, x: Value, *, norm: Optional[NormInput] = None, residual: Optional[Value] = None,
              name: Optional[str] = None, rows: Optional[Tuple[int, int]] = None,
              groups: Optional[Sequence[int]] = None, sibling: bool = False) -> Projection:
        if (self.epilogue == "residual") != (residual is not None):
            raise ValueError(f"Linear {self.prefix}: the residual epilogue and a residual input go together")
        if rows is not None and self.epilogue == "silu_mul":
            raise ValueError(f"Linear {self.prefix}: a row range cannot cut a silu_mul projection")
        all_groups = self.slab_groups()
        which = list(range(len(all_groups))) if groups is None else list(groups)
        proj = Projection([])
        for i, gi in enumerate(which):
            grp = all_groups[gi]
            w = _weight(g, grp.name, (grp.rows, grp.k), grp.format)
            ins = [x, w] + ([norm.stat, norm.weight] if norm is not None else []) + \
                  ([residual] if residual is not None else [])
            ranged = rows is not None and gi == 0
            start, count = (int(rows[0]), int(rows[1])) if ranged else (0, grp.rows)
            if start < 0 or count <= 0 or start + count > grp.rows:
                raise ValueError(f"Linear {self.prefix}: rows {rows} outside the slab's {grp.rows}")
            n_out = count // 2 if self.epilogue == "silu_mul" else count
            out = name if (name and len(which) == 1) else f"{grp.name}.y" + (f".r{start}" if ranged else "")
            y = g.value(out, (x.shape[0], n_out), DType.BF16)
            attrs: Dict[str, Any] = dict(norm=norm is not None, epilogue=self.epilogue, format=grp.format)
            if norm is not None:
                attrs["eps"] = norm.eps
            if self.epilogue == "silu_mul":
                attrs["chunk"] = self.chunk
            if ranged:
                attrs["row_range"] = (start, count)
            if sibling:
                attrs["sibling"] = True
            segs, col = [], 0
            for local, nrows in grp.parts:
                lo, hi = max(col, start), min(col + nrows, start + count)
                if hi > lo:
                    segs.append((local, hi - lo))
                    proj.segments[local] = (i, lo - start, hi - lo)
                col += nrows
            attrs["segments"] = segs
            g.op("gemv", ins, [y], domain=BlockDomain("rows", count), klass=OpClass.MAP, **attrs)
            proj.values.append(y)
        return proj


class RMSNorm:
    def __init__(self, dim: int, eps: float, *, prefix: str):
        self.dim, self.eps, self.prefix = dim, eps, prefix

    def lower(self, g: Graph, h: Value) -> NormInput:
        stat = g.value(f"{self.prefix}stat", (h.shape[0],), DType.F32)
        g.op("rmsnorm_stat", [h], [stat], domain=BlockDomain("span", self.dim), klass=OpClass.REDUCE, eps=self.eps,
             round_before_scale=False)
        return NormInput(stat, _const(g, f"{self.prefix}weight", (self.dim,), DType.F32), self.eps)


class GatedMLP:
    def __init__(self, hidden: int, inter: int, *, prefix: str, fmt: str = "nvfp4", chunk: int = CHUNK):
        self.hidden, self.inter, self.prefix = hidden, inter, prefix
        self.gate_up = Linear(hidden, [("gate_proj", inter), ("up_proj", inter)], prefix=f"{prefix}gate_up.", fmt=fmt,
                              row_perm=interleave_chunks(inter, inter, chunk), epilogue="silu_mul", chunk=chunk)
        self.down = Linear(inter, [("down_proj", hidden)], prefix=f"{prefix}down.", fmt=fmt, epilogue="residual")

    def linears(self) -> List[Linear]:
        return [self.gate_up, self.down]

    def lower(self, g: Graph, h: Value, norm: NormInput, ctx: LowerContext) -> Value:
        act = self.gate_up.lower(g, h, norm=norm).value
        return self.down.lower(g, act, residual=h, name=f"{self.prefix}h").value


class GatedDeltaNet:
    def __init__(self, hidden: int, k_heads: int, v_heads: int, dk: int, dv: int, conv_width: int, eps: float, *,
                 prefix: str, fmt: str = "nvfp4", formats: Optional[Dict[str, str]] = None):
        if v_heads % k_heads:
            raise ValueError("GatedDeltaNet: v_heads must be a multiple of k_heads")
        self.hidden, self.hk, self.hv, self.dk, self.dv, self.w, self.eps = hidden, k_heads, v_heads, dk, dv, conv_width, eps
        self.prefix = prefix
        self.key_dim, self.value_dim = k_heads * dk, v_heads * dv
        self.conv_dim = 2 * self.key_dim + self.value_dim
        self.in_proj = Linear(hidden, [("in_proj_z", self.value_dim), ("in_proj_qkv", self.conv_dim),
                                       ("in_proj_a", v_heads), ("in_proj_b", v_heads)],
                              prefix=f"{prefix}in_proj.", fmt=fmt, formats=formats)
        self.out_proj = Linear(self.value_dim, [("out_proj", hidden)], prefix=f"{prefix}out_proj.", fmt=fmt,
                               epilogue="residual")

    def linears(self) -> List[Linear]:
        return [self.in_proj, self.out_proj]

    def kernel_segments(self) -> List[Tuple[str, int, int]]:
        kd, vd, hv = self.key_dim, self.value_dim, self.hv
        return [("z", 0, vd), ("q", vd, kd), ("k", vd + kd, kd), ("v", vd + 2 * kd, vd),
                ("a", vd + self.conv_dim, hv), ("b", vd + self.conv_dim + hv, hv)]

    def state_entries(self) -> List[StateEntry]:
        return [StateEntry(f"{self.prefix}conv_state", (self.conv_dim, self.w - 1), DType.BF16, 2),
                StateEntry(f"{self.prefix}rec_state", (self.hv, self.dk, self.dv), DType.F32, 2)]

    def lower(self, g: Graph, h: Value, norm: NormInput, ctx: LowerContext) -> Value:
        vd = self.value_dim
        n0 = self.in_proj.slab_groups()[0].rows
        main = self.in_proj.lower(g, h, norm=norm, rows=(vd, n0 - vd))
        cs, rs = ctx.states[f"{self.prefix}conv_state"], ctx.states[f"{self.prefix}rec_state"]
        conv_w = _const(g, f"{self.prefix}conv_w", (self.conv_dim, self.w), DType.BF16)
        nea = _const(g, f"{self.prefix}a_log", (self.hv,), DType.F32)        # holds −exp(A_log)
        dtb = _const(g, f"{self.prefix}dt_bias", (self.hv,), DType.F32)
        t = h.shape[0]
        o_part = g.value(f"{self.prefix}o_part", (t, vd), DType.F32)
        g.op("gdn_mixer", [*main.values, cs, rs, conv_w, nea, dtb], [o_part], domain=BlockDomain("heads", self.hv),
             klass=OpClass.MAP, updates=[cs.name, rs.name], k_heads=self.hk, v_heads=self.hv, dk=self.dk, dv=self.dv,
             conv_width=self.w, eps=self.eps, segments=self.kernel_segments(), proj_segments=main.segments,
             commit_kind="gdn_commit")
        z = self.in_proj.lower(g, h, norm=norm, rows=(0, vd), groups=[0], sibling=True).value
        nw = _const(g, f"{self.prefix}norm_w", (self.dv,), DType.F32)
        o = g.value(f"{self.prefix}mix", (t, vd), DType.BF16)
        g.op("gdn_norm", [o_part, z, nw], [o], domain=BlockDomain("heads", self.hv), klass=OpClass.MAP,
             v_heads=self.hv, dv=self.dv, eps=self.eps)
        return self.out_proj.lower(g, o, residual=h, name=f"{self.prefix}h").value


ATTN_CHUNK = 64


class GQAAttention:
    def __init__(self, hidden: int, heads: int, kv_heads: int, head_dim: int, rotary_dim: int, rope_theta: float,
                 eps: float, *, prefix: str, max_context: int, gate: bool = True, fmt: str = "nvfp4"):
        if heads % kv_heads:
            raise ValueError("GQAAttention: heads must be a multiple of kv_heads")
        self.hidden, self.heads, self.kv, self.d = hidden, heads, kv_heads, head_dim
        self.rotary_dim, self.theta, self.eps, self.gate, self.prefix = rotary_dim, rope_theta, eps, gate, prefix
        self.max_context = max_context
        hd, kd = heads * head_dim, kv_heads * head_dim
        self.qkv = Linear(hidden, [("q_proj", heads * (2 if gate else 1) * head_dim), ("k_proj", kd), ("v_proj", kd)],
                          prefix=f"{prefix}qkv.", fmt=fmt, row_perm=self.row_perm())
        self.o_proj = Linear(hd, [("o_proj", hidden)], prefix=f"{prefix}o_proj.", fmt=fmt, epilogue="residual")

    def linears(self) -> List[Linear]:
        return [self.qkv, self.o_proj]

    def row_perm(self) -> np.ndarray:
        """Checkpoint rows ``[q_proj (q|gate per head) | k_proj | v_proj]`` → ``[q (permuted) | k (permuted) | v |
        gate]`` (``nn/attention.py:52-64``): the core's rows and the gate's are two tile-aligned ranges."""
        d, hp = self.d, rope_head_perm(self.d, self.rotary_dim)
        stride = 2 * d if self.gate else d
        q = np.concatenate([h * stride + hp for h in range(self.heads)])
        base = self.heads * stride
        k = base + np.concatenate([j * d + hp for j in range(self.kv)])
        v = base + self.kv * d + np.arange(self.kv * d)
        parts = [q, k, v]
        if self.gate:
            parts.append(np.concatenate([h * stride + d + np.arange(d) for h in range(self.heads)]))
        return np.concatenate(parts)

    @property
    def core_rows(self) -> int:
        return (self.heads + 2 * self.kv) * self.d

    def kernel_segments(self) -> List[Tuple[str, int, int]]:
        hd, kd = self.heads * self.d, self.kv * self.d
        segs = [("q", 0, hd), ("k", hd, kd), ("v", hd + kd, kd)]
        return segs + ([("gate", hd + 2 * kd, hd)] if self.gate else [])

    def state_entries(self) -> List[StateEntry]:
        shape = (self.max_context, self.kv, self.d)
        return [StateEntry(f"{self.prefix}k_cache", shape, DType.BF16), StateEntry(f"{self.prefix}v_cache", shape, DType.BF16)]

    def lower(self, g: Graph, h: Value, norm: NormInput, ctx: LowerContext) -> Value:
        hd = self.heads * self.d
        proj = self.qkv.lower(g, h, norm=norm, rows=(0, self.core_rows)).value
        kc, vc = ctx.states[f"{self.prefix}k_cache"], ctx.states[f"{self.prefix}v_cache"]
        cos, sin = ctx.consts["rope_cos"], ctx.consts["rope_sin"]
        qn = _const(g, f"{self.prefix}q_norm", (self.d,), DType.F32)
        kn = _const(g, f"{self.prefix}k_norm", (self.d,), DType.F32)
        rep = self.heads // self.kv
        # the partials' shape is the reference kernel's (chunks down to 16 keys); gfx950 folds them inside
        # mi_gqa_decode, so these values are never allocated
        n_chunks = -(-self.max_context // 16)
        t = h.shape[0]
        part_o = g.value(f"{self.prefix}part_o", (t, self.kv * n_chunks * rep * self.d), DType.F32)
        part_md = g.value(f"{self.prefix}part_md", (t, self.kv * n_chunks * rep * 2), DType.F32)
        g.op("gqa_decode", [proj, kc, vc, cos, sin, qn, kn], [part_o, part_md], domain=BlockDomain("heads", self.heads),
             klass=OpClass.MAP, updates=[kc.name, vc.name], heads=self.heads, kv_heads=self.kv, head_dim=self.d,
             rotary_dim=self.rotary_dim, eps=self.eps, scaling=self.d ** -0.5, qk_norm=True,
             segments=[s for s in self.kernel_segments() if s[0] != "gate"], rope="permuted", chunk=ATTN_CHUNK)
        ins = [part_o, part_md]
        if self.gate:
            ins.append(self.qkv.lower(g, h, norm=norm, rows=(self.core_rows, hd), sibling=True).value)
        o = g.value(f"{self.prefix}attn", (t, hd), DType.BF16)
        g.op("gqa_merge", ins, [o], domain=BlockDomain("heads", self.heads), klass=OpClass.MAP, heads=self.heads,
             kv_heads=self.kv, head_dim=self.d, gate=self.gate, qk_norm=True, chunk=ATTN_CHUNK)
        return self.o_proj.lower(g, o, residual=h, name=f"{self.prefix}h").value


class Experts:
    """``n_experts`` copies of one projection in one slab (``nn/moe.py:22-89``); gate|up chunk-interleaved per
    expert; the epilogue is the grouped GEMV's."""

    def __init__(self, in_features: int, n_experts: int, parts: Sequence[Tuple[str, int]], *, prefix: str,
                 fmt: str = "nvfp4", epilogue: Optional[str] = None, chunk: Optional[int] = None):
        self.n_experts, self.k, self.prefix, self.epilogue, self.chunk = n_experts, in_features, prefix, epilogue, chunk
        self.rows_per_expert = sum(r for _, r in parts)
        perm = None
        if epilogue == "silu_mul":
            inter = parts[0][1]
            one = interleave_chunks(inter, inter, chunk)
            perm = np.concatenate([one + e * 2 * inter for e in range(n_experts)])
        self.slab = Linear(in_features, [(f"e{e}.{local}", rows) for e in range(n_experts) for local, rows in parts],
                           prefix=prefix, fmt=fmt, row_perm=perm)

    @property
    def n_out(self) -> int:
        return self.rows_per_expert // 2 if self.epilogue == "silu_mul" else self.rows_per_expert

    def lower(self, g: Graph, x: Value, ids: Value, top_k: int, *, x_per_slot: bool, name: str) -> Value:
        grp = self.slab.slab_groups()[0]
        w = _weight(g, grp.name, (grp.rows, grp.k), grp.format)
        y = g.value(name, (ids.shape[0], top_k * self.n_out), DType.BF16)
        attrs: Dict[str, Any] = dict(top_k=top_k, expert_rows=self.rows_per_expert, epilogue=self.epilogue,
                                     format=grp.format, x_per_slot=x_per_slot)
        if self.epilogue == "silu_mul":
            attrs["chunk"] = self.chunk
        g.op("moe_gemv", [x, w, ids], [y], domain=BlockDomain("rows", ids.shape[0]), klass=OpClass.MAP, **attrs)
        return y


class SparseMoE:
    def __init__(self, hidden: int, n_experts: int, top_k: int, inter: int, *, prefix: str, fmt: str = "nvfp4",
                 renorm: bool = True, shared_inter: Optional[int] = None, chunk: int = CHUNK):
        self.hidden, self.n_experts, self.top_k, self.inter, self.renorm = hidden, n_experts, top_k, inter, renorm
        self.prefix, self.shared_inter = prefix, shared_inter
        self.router = Linear(hidden, [("gate", n_experts)], prefix=f"{prefix}router.", fmt="bf16")
        self.gate_up = Experts(hidden, n_experts, [("gate_proj", inter), ("up_proj", inter)],
                               prefix=f"{prefix}experts_gate_up.", fmt=fmt, epilogue="silu_mul", chunk=chunk)
        self.down = Experts(inter, n_experts, [("down_proj", hidden)], prefix=f"{prefix}experts_down.", fmt=fmt)
        if shared_inter:
            si = shared_inter
            self.shared_gate_up = Linear(hidden, [("gate_proj", si), ("up_proj", si)], prefix=f"{prefix}shared_gate_up.",
                                         fmt=fmt, row_perm=interleave_chunks(si, si, chunk), epilogue="silu_mul",
                                         chunk=chunk)
            self.shared_down = Linear(si, [("down_proj", hidden)], prefix=f"{prefix}shared_down.", fmt=fmt)
            self.shared_gate = Linear(hidden, [("shared_expert_gate", 1)], prefix=f"{prefix}shared_gate.", fmt="bf16")

    def linears(self) -> List[Linear]:
        out = [self.router, self.gate_up.slab, self.down.slab]
        if self.shared_inter:
            out += [self.shared_gate_up, self.shared_down, self.shared_gate]
        return out

    def lower(self, g: Graph, h: Value, norm: NormInput, ctx: LowerContext) -> Value:
        t, p = h.shape[0], self.prefix
        logits = self.router.lower(g, h, norm=norm).value
        xn = g.value(f"{p}xn", h.shape, DType.BF16)
        g.op("norm_apply", [h, norm.stat, norm.weight], [xn], domain=BlockDomain("span", self.hidden),
             klass=OpClass.MAP, eps=norm.eps)
        ids = g.value(f"{p}ids", (t, self.top_k), DType.I32)
        weights = g.value(f"{p}weights", (t, self.top_k), DType.F32)
        g.op("moe_route", [logits], [ids, weights], domain=BlockDomain("rows", t), klass=OpClass.MAP,
             n_experts=self.n_experts, top_k=self.top_k, renorm=self.renorm)
        act = self.gate_up.lower(g, xn, ids, self.top_k, x_per_slot=False, name=f"{p}act")
        hk = self.down.lower(g, act, ids, self.top_k, x_per_slot=True, name=f"{p}hk")
        ins = [hk, weights]
        attrs: Dict[str, Any] = dict(top_k=self.top_k, has_shared=False, has_residual=True)
        if self.shared_inter:
            s_act = self.shared_gate_up.lower(g, h, norm=norm).value
            s_out = self.shared_down.lower(g, s_act, name=f"{p}shared").value
            s_gate = self.shared_gate.lower(g, h, norm=norm, name=f"{p}shared_gate").value
            ins += [s_out, s_gate]
            attrs["has_shared"] = True
        ins.append(h)
        out = g.value(f"{p}h", (t, self.hidden), DType.BF16)
        g.op("moe_combine", ins, [out], domain=BlockDomain("rows", t), klass=OpClass.MAP, **attrs)
        return out


class DecoderLayer:
    def __init__(self, index: int, input_norm: RMSNorm, mixer, post_norm: RMSNorm, mlp, *, prefix: str):
        self.index, self.input_norm, self.mixer, self.post_norm, self.mlp = index, input_norm, mixer, post_norm, mlp
        self.prefix = prefix

    def lower(self, g: Graph, h: Value, ctx: LowerContext) -> Value:
        h = self.mixer.lower(g, h, self.input_norm.lower(g, h), ctx)
        return self.mlp.lower(g, h, self.post_norm.lower(g, h), ctx)


class Embedding:
    def __init__(self, vocab: int, hidden: int, *, prefix: str = "embed_tokens.", fmt: str = "bf16"):
        self.vocab, self.hidden, self.prefix, self.fmt = vocab, hidden, prefix, fmt

    @property
    def slab_name(self) -> str:
        return f"{self.prefix}weight"

    def lower(self, g: Graph, tokens: Value, ctx: LowerContext) -> Value:
        w = _weight(g, self.slab_name, (self.vocab, self.hidden), self.fmt)
        h = g.value(f"{self.prefix}h", (tokens.shape[0], self.hidden), DType.BF16)
        g.op("embed", [tokens, w], [h], domain=BlockDomain("rows", tokens.shape[0]), klass=OpClass.MAP, packed=True)
        return h


class LMHead:
    def __init__(self, hidden: int, vocab: int, *, prefix: str = "lm_head.", fmt: str = "bf16"):
        self.hidden, self.vocab, self.prefix, self.fmt = hidden, vocab, prefix, fmt

    @property
    def slab_name(self) -> str:
        return f"{self.prefix}weight"

    def lower(self, g: Graph, h: Value, norm: Optional[NormInput], ctx: LowerContext, *, name: str = "logits") -> Value:
        w = _weight(g, self.slab_name, (self.vocab, self.hidden), self.fmt)
        logits = g.value(name, (h.shape[0], self.vocab), DType.BF16)
        ins = [h, w] + ([norm.stat, norm.weight] if norm is not None else [])
        attrs: Dict[str, Any] = dict(norm=norm is not None, out="bf16", format=self.fmt)
        if norm is not None:
            attrs["eps"] = norm.eps
        g.op("lm_head", ins, [logits], domain=BlockDomain("rows", self.vocab), klass=OpClass.MAP, **attrs)
        return logits


class GreedySampler:
    def lower(self, g: Graph, logits: Value, ctx: LowerContext) -> Value:
        token = g.value("token", (logits.shape[0],), DType.I32)
        g.op("argmax", [logits], [token], domain=BlockDomain("span", logits.shape[1]), klass=OpClass.REDUCE)
        return token


class HybridDecoder:
    """The hybrid decoder's module tree (``models/qwen3_5/model.py``): embedding → layers (``"gdn"`` or
    ``"attention"`` mixers; each with a gated MLP or, given ``moe``, a sparse MoE) → final norm → LM head → greedy
    sampler. ``lower(g)`` writes the step graph and returns the sampled ``token`` value."""

    def __init__(self, *, vocab: int, hidden: int, layer_types: Sequence[str], inter: int, eps: float = 1e-6,
                 gdn: Optional[dict] = None, attention: Optional[dict] = None, moe: Optional[dict] = None,
                 moe_layers: Sequence[int] = (), max_context: int = 4096, fmt: str = "nvfp4"):
        self.vocab, self.hidden, self.eps, self.max_context = vocab, hidden, eps, max_context
        self.embed_tokens = Embedding(vocab, hidden)
        self.blocks: List[DecoderLayer] = []
        self.attention_cfg = dict(attention or {})
        for i, kind in enumerate(layer_types):
            lp = f"layers.{i}."
            if kind == "gdn":
                c = dict(gdn or {})
                mixer = GatedDeltaNet(hidden, c.get("k_heads", 16), c.get("v_heads", 48), c.get("dk", 128),
                                      c.get("dv", 128), c.get("conv_width", 4), eps, prefix=f"{lp}linear_attn.", fmt=fmt)
            elif kind == "attention":
                c = self.attention_cfg
                mixer = GQAAttention(hidden, c.get("heads", 24), c.get("kv_heads", 4), c.get("head_dim", 128),
                                     c.get("rotary_dim", 64), c.get("theta", 1e6), eps, prefix=f"{lp}self_attn.",
                                     max_context=max_context, gate=c.get("gate", True), fmt=fmt)
            else:
                raise ValueError(f"HybridDecoder: unknown layer type {kind!r}")
            if i in moe_layers:
                m = dict(moe or {})
                mlp = SparseMoE(hidden, m.get("experts", 256), m.get("top_k", 8), m.get("inter", 512),
                                prefix=f"{lp}mlp.", fmt=fmt, shared_inter=m.get("shared_inter"))
            else:
                mlp = GatedMLP(hidden, inter, prefix=f"{lp}mlp.", fmt=fmt)
            self.blocks.append(DecoderLayer(i, RMSNorm(hidden, eps, prefix=f"{lp}input_norm."), mixer,
                                            RMSNorm(hidden, eps, prefix=f"{lp}post_norm."), mlp, prefix=lp))
        self.norm = RMSNorm(hidden, eps, prefix="norm.")
        self.lm_head = LMHead(hidden, vocab)
        self.sampler = GreedySampler()

    def state_entries(self) -> List[StateEntry]:
        return [e for b in self.blocks for e in b.mixer.state_entries()]

    def tables(self) -> Dict[str, Tuple[str, np.ndarray]]:
        """Computed constants the pack stores: the permuted RoPE tables (BF16 bits) when a layer attends."""
        attn = [b.mixer for b in self.blocks if isinstance(b.mixer, GQAAttention)]
        if not attn:
            return {}
        a = attn[0]
        from .formats.fp import f32_to_bf16
        cos, sin = rope_tables_permuted(a.theta, a.d, a.rotary_dim, self.max_context)
        return {"rope_cos": ("BF16", f32_to_bf16(cos)), "rope_sin": ("BF16", f32_to_bf16(sin))}

    def lower(self, g: Graph, tokens: Optional[Value] = None) -> Value:
        tokens = tokens if tokens is not None else g.input("tokens", (T,), DType.I32)
        ctx = LowerContext(t=tokens.shape[0])
        for e in self.state_entries():
            ctx.states[e.name] = g.state(e.name, e.buffer_shape, e.dtype)
        for name, (dtype, arr) in self.tables().items():
            ctx.consts[name] = g.const(name, tuple(arr.shape), DType.parse(dtype))
        h = self.embed_tokens.lower(g, tokens, ctx)
        for blk in self.blocks:
            h = blk.lower(g, h, ctx)
        logits = self.lm_head.lower(g, h, self.norm.lower(g, h), ctx)
        return self.sampler.lower(g, logits, ctx)
