"""Backend selection and the emission context: the gfx950 side of the reference's compiler extension points.

* ``Gfx950Backend`` has the reference backend's hooks (``monolith/backends/metal/base.py:6-23``): ``emit`` and
  ``compile`` wrap the shared pipeline, ``handler(kind, shared_handlers)`` picks the emitter of an op kind.
* ``dispatch(entry)`` selects the backend named by ``profile.backend`` for the decorated entry point and stamps the
  program with the backend id and the profile's fingerprint (``backends/metal/context.py:39-53``); the active backend
  is a context variable, so nested and concurrent compiles do not see each other's (``:9-23``).
* ``EmitContext`` is the handler API (``compiler/emit.py:97-166``): ``ctx.kernel(key, source, function, macros)`` for
  a run-time compiled HIP kernel, ``ctx.library(entry)`` for a typed entry point of libmi355, ``ctx.params(name,
  bytes)``, ``ctx.buf(value)``, ``ctx.scratch(name, nbytes, shared)`` and ``ctx.add(kernel, bindings, grid, tg,
  name, writes=…, **meta)``.

An op on a library entry point is an ``OpSpec`` whose kernel is ``KernelSpec("", "lib:<entry>")``: ``meta["desc"]``
holds the descriptor's scalar fields, and each binding ``(field index, buffer, offset)`` puts a buffer address into
the descriptor's pointer field of that index (the descriptor layouts are ``include/lithos_mi355.h``). The entry point
chooses its own launch geometry, so such an op's grid and threadgroup are ``(0, 0, 0)``.
"""

from __future__ import annotations

import hashlib
import json
from contextlib import contextmanager
from contextvars import ContextVar
from dataclasses import asdict, dataclass, field
from functools import wraps
from inspect import signature
from typing import Any, Dict, List, Optional, Sequence, Tuple

from ..runtime.program import BufferSpec, KernelSpec, OpSpec, Program, StepStateLayout

STATE_LAYOUT = (16, 15)                     # mi_step_state: StepStateLayout(t_max=16, gamma_max=15)


@dataclass
class Profile:
    """What a compile targets (the reference's ``ChipConfig`` as far as emission reads it): the backend, the op
    registry's binding key, the token ring, the stop rules, and the KV cache the attention ops keep (``"bf16"``,
    the reference's, or ``"int8"`` with per-token scales in state buffers of their own)."""

    backend: str = "gfx950"
    ring_capacity: int = 4096
    ctx_cap: int = 0                        # positions a sequence may occupy (0: unbounded)
    eos: Tuple[int, ...] = ()
    kv_cache: str = "bf16"
    name: str = "MI355X"
    extra: Dict[str, Any] = field(default_factory=dict)

    @property
    def key(self) -> str:
        return "gfx950"

    @property
    def fingerprint(self) -> str:
        return hashlib.sha256(json.dumps(asdict(self), sort_keys=True, default=str).encode()).hexdigest()[:16]


class Gfx950Backend:
    """The MI355X backend: the shared emission with this backend's handlers (the library entry points)."""

    id = "gfx950"

    def emit(self, shared_emit, *args, **kwargs):
        return shared_emit(*args, **kwargs)

    def compile(self, shared_compile, *args, **kwargs):
        return shared_compile(*args, **kwargs)

    def handler(self, kind: str, shared_handlers):
        if kind not in shared_handlers:
            from ..ops.coverage import CoverageError
            from ..ops.registry import OPS, PROFILE
            raise CoverageError(PROFILE, [(kind, OPS.resolve(kind))])
        return shared_handlers[kind]

    def validate_device(self, info) -> None:
        if not str(info.arch).startswith("gfx950"):
            raise ValueError(f"backend {self.id} runs on gfx950 (MI355X); this device is {info.arch}")


_BACKENDS: Dict[str, Gfx950Backend] = {"gfx950": Gfx950Backend()}
_ACTIVE: ContextVar = ContextVar("monolith_mi355_backend", default=None)


def register_backend(backend) -> None:
    if backend.id in _BACKENDS and _BACKENDS[backend.id] is not backend:
        raise ValueError(f"backend {backend.id!r} is already registered")
    _BACKENDS[backend.id] = backend


def get_backend(name: str):
    try:
        return _BACKENDS[name]
    except KeyError:
        raise ValueError(f"unknown backend {name!r} (known: {sorted(_BACKENDS)})") from None


def current_backend():
    return _ACTIVE.get() or _BACKENDS["gfx950"]


@contextmanager
def using_backend(backend):
    b = get_backend(backend) if isinstance(backend, str) else backend
    token = _ACTIVE.set(b)
    try:
        yield b
    finally:
        _ACTIVE.reset(token)


def dispatch(entry: str):
    """Route the decorated shared implementation through the backend ``profile.backend`` names
    (``backend.<entry>(shared, *args, **kwargs)``) and stamp the program it returns."""

    def wrap(shared):
        sig = signature(shared)

        @wraps(shared)
        def run(*args, **kwargs):
            profile = sig.bind(*args, **kwargs).arguments["profile"]
            with using_backend(profile.backend) as backend:
                program = getattr(backend, entry)(shared, *args, **kwargs)
            program.backend_id = backend.id
            program.config_digest = profile.fingerprint
            return program
        return run
    return wrap


WINDOW_BYTES = 2 << 30          # a file window of the pack is at most 2 GiB (``compiler/emit.py:38``)


class EmitContext:
    """The program under construction (``compiler/emit.py:97-205``'s ``_Ctx``): where each value of the plan lives —
    pack windows for weights and constants, the step state for inputs named after its fields, program buffers for
    states (role ``state``) and activations (role ``arena``); aliases and row views as offsets into their base."""

    def __init__(self, profile: Profile, plan, packs: Sequence[Any] = (), *, layout: Optional[StepStateLayout] = None,
                 ring_capacity: Optional[int] = None, ctx_cap: Optional[int] = None) -> None:
        self.profile, self.plan, self.t = profile, plan, plan.t
        self.layout = layout or StepStateLayout(*STATE_LAYOUT)
        if (self.layout.t_max, self.layout.gamma_max) != STATE_LAYOUT:
            raise ValueError(f"the gfx950 step state is StepStateLayout{STATE_LAYOUT} (mi_step_state)")
        ring = profile.ring_capacity if ring_capacity is None else ring_capacity
        self.program = Program(kernels={}, buffers={}, ops=[], ring_capacity=ring, layout=self.layout,
                               context_capacity=profile.ctx_cap if ctx_cap is None else ctx_cap)
        self.program.buffers[self.program.step_state] = BufferSpec(self.layout.size, None, "step_state")
        self.program.buffers[self.program.ring] = BufferSpec(8 * ring, None, "ring")
        self.packs = list(packs)
        self.slabs: Dict[str, dict] = {}
        self.aux: Dict[str, dict] = {}
        self.windows: Dict[str, Tuple[str, int]] = {}       # slab / aux name -> (buffer, offset)
        self.row_scales: Dict[str, Tuple[str, int]] = {}
        self._map_packs()
        self._shared: Dict[str, str] = {}
        self.counter = 0

    def _name(self, stem: str) -> str:
        self.counter += 1
        return f"{stem}.{self.counter}"

    # ---- the pack ----------------------------------------------------------------------------------------------
    def _map_packs(self) -> None:
        """Each pack's slabs, row-scale tables and aux entries grouped into page-aligned file windows of at most
        2 GiB, in file order (``compiler/emit.py:220-256``)."""
        n_win = 0
        for pk in self.packs:
            man = pk.manifest
            path = str(pk.dir / man["pack"])
            align, file_bytes = int(man.get("alignment", 4096)), int(man["nbytes"])
            entries = []
            for s in man["slabs"]:
                if s["name"] in self.slabs:
                    raise ValueError(f"emit: two packs hold a slab named {s['name']!r}")
                self.slabs[s["name"]] = s
                entries.append((s["offset"], s["nbytes"], "slab", s["name"]))
                if s.get("row_scales_offset") is not None:
                    entries.append((s["row_scales_offset"], 4 * s["row_scales_len"], "rs", s["name"]))
            for a in man["aux"]:
                if a["name"] in self.aux:
                    raise ValueError(f"emit: two packs hold an entry named {a['name']!r}")
                self.aux[a["name"]] = a
                entries.append((a["offset"], a["nbytes"], "aux", a["name"]))
            entries.sort()
            windows, start, end, members = [], None, 0, []
            for off, nb, kind, name in entries:
                if start is None or off + nb - start > WINDOW_BYTES:
                    if start is not None:
                        windows.append((start, end, members))
                    start, end, members = off - off % align, off + nb, []
                end = max(end, off + nb)
                members.append((off, kind, name))
            if start is not None:
                windows.append((start, end, members))
            for start, end, members in windows:
                bname = f"pack.{n_win}"
                n_win += 1
                end = min(-(-end // align) * align, file_bytes)
                self.program.buffers[bname] = BufferSpec(end - start, None, "weights", path, start)
                for off, kind, name in members:
                    (self.row_scales if kind == "rs" else self.windows)[name] = (bname, off - start)

    def slab(self, name: str) -> dict:
        try:
            return self.slabs[name]
        except KeyError:
            raise KeyError(f"emit: no pack holds the slab {name!r}") from None

    # ---- where values live -------------------------------------------------------------------------------------
    def buf(self, v) -> Optional[Tuple[str, int]]:
        """``(buffer name, byte offset)`` of a plan value (or an explicit ``(buffer, offset)`` pair)."""
        if v is None or isinstance(v, tuple):
            return v
        p = self.plan
        if v.name in p.alias:
            root, col = p.root(v)
            bname, off = self.buf(p.values[root])
            return bname, off + col * _itemsize(p.values[root])
        if getattr(v, "view_of", None) is not None:
            base_name, row = v.view_of
            base = p.values[base_name]
            bname, off = self.buf(base)
            return bname, off + row * p.width(base) * _itemsize(base)
        if v.is_weight or v.is_const:
            if v.name not in self.windows:
                raise KeyError(f"emit: the pack has no entry for {v.name!r}")
            return self.windows[v.name]
        if v.is_input:
            fld = "pending_tokens" if v.name == "tokens" else v.name
            if fld in self.layout.offsets:
                return self.program.step_state, self.layout.offset(fld)
        nbytes = max(_itemsize(v) * _numel(p.shape(v)), 16)
        role = "state" if v.is_state else "arena"
        spec = self.program.buffers.get(v.name)
        if spec is None:
            self.program.buffers[v.name] = BufferSpec(nbytes, None, role)
        elif spec.nbytes < nbytes:
            spec.nbytes = nbytes
        return v.name, 0

    def ld(self, v) -> int:
        return self.plan.ld(v)

    def field(self, name: str) -> Tuple[str, int]:
        return self.program.step_state, self.layout.offset(name)

    def params(self, name: str, data: bytes) -> str:
        bname = self._name(f"params.{name}")
        self.program.buffers[bname] = BufferSpec(len(data), bytes(data), "params")
        return bname

    def scratch(self, name: str, nbytes: int, shared: bool = False) -> str:
        """A zero-initialized workspace; ``shared``: one per name for the whole program, sized to the largest
        request (ops run in order, so consecutive users never overlap)."""
        nbytes = max(int(nbytes), 16)
        if shared:
            bname = self._shared.get(name)
            if bname is None:
                bname = self._shared[name] = f"ws.{name}"
                self.program.buffers[bname] = BufferSpec(nbytes, None, "arena")
            elif self.program.buffers[bname].nbytes < nbytes:
                self.program.buffers[bname].nbytes = nbytes
            return bname
        bname = self._name(f"ws.{name}")
        self.program.buffers[bname] = BufferSpec(nbytes, None, "arena")
        return bname

    # ---- kernels and ops ---------------------------------------------------------------------------------------
    def kernel(self, key: str, source: str, function: str, macros: Dict[str, str], language_version: int = 0) -> str:
        macros = dict(macros)
        k = f"{function}|{key}|" + ",".join(f"{m}={macros[m]}" for m in sorted(macros))
        if k not in self.program.kernels:
            self.program.kernels[k] = KernelSpec(source, function, macros, language_version)
        return k

    def library(self, entry: str) -> str:
        k = f"lib:{entry}"
        self.program.kernels.setdefault(k, KernelSpec("", k))
        return k

    def add(self, kernel: str, bindings: Sequence[Tuple[int, str, int]], grid, tg, name: str, *,
            writes: Optional[Sequence[int]] = None, **meta: Any) -> OpSpec:
        if writes is not None:
            meta["writes"] = sorted(int(i) for i in writes)
        op = OpSpec(kernel, [tuple(b) for b in bindings], tuple(grid), tuple(tg), True, [], name, dict(meta))
        self.program.ops.append(op)
        return op


_ITEM = {"bf16": 2, "f16": 2, "f32": 4, "i32": 4, "u32": 4, "i64": 8, "u8": 1, "bool": 1, "i8": 1}


def _itemsize(v) -> int:
    it = getattr(v.dtype, "itemsize", None)
    return int(it) if it is not None else _ITEM[str(v.dtype)]


def _numel(shape) -> int:
    n = 1
    for d in shape:
        n *= int(d)
    return n
