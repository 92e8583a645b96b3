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
from .ir import Value

STATE_LAYOUT = (16, 15)                     # mi_step_state: StepStateLayout(t_max=16, gamma_max=15)


@dataclass
class Profile:
    """What a compile targets: the backend, the token ring, the stop rules."""

    backend: str = "gfx950"
    ring_capacity: int = 4096
    ctx_cap: int = 0                        # positions a sequence may occupy (0: unbounded)
    eos: Tuple[int, ...] = ()
    extra: Dict[str, Any] = field(default_factory=dict)

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


class EmitContext:
    """The program under construction and where each value lives in it."""

    def __init__(self, profile: Profile, t: int = 1) -> None:
        self.profile, self.t = profile, t
        self.layout = StepStateLayout(*STATE_LAYOUT)
        self.program = Program(kernels={}, buffers={}, ops=[], ring_capacity=profile.ring_capacity,
                               layout=self.layout, context_capacity=profile.ctx_cap)
        self.program.buffers[self.program.step_state] = BufferSpec(self.layout.size, None, "step_state")
        self.program.buffers[self.program.ring] = BufferSpec(8 * profile.ring_capacity, None, "ring")
        self.bound: Dict[str, Any] = {}      # buffer name -> the tensor whose storage it is (handed to Engine)
        self._by_storage: Dict[int, str] = {}
        self._by_value: Dict[int, str] = {}
        self._shared: Dict[str, str] = {}
        self.counter = 0

    def _name(self, stem: str) -> str:
        self.counter += 1
        return f"{stem}.{self.counter}"

    # ---- where values live -------------------------------------------------------------------------------------
    def buf(self, v: Optional[Value]) -> Optional[Tuple[str, int]]:
        """``(buffer name, byte offset)`` of a value: its step-state field, the storage of its bound tensor, or a
        buffer the program allocates."""
        if v is None:
            return None
        if v.base is not None:
            name, off = self.buf(v.base)
            return name, off + v.offset
        if v.role == "step_state":
            return self.program.step_state, self.layout.offset(v.field) + v.offset
        if v.tensor is not None:
            st = v.tensor.untyped_storage()
            base = st.data_ptr()
            name = self._by_storage.get(base)
            if name is None:
                name = self._name(f"{v.role}.{v.name}")
                self._by_storage[base] = name
                self.program.buffers[name] = BufferSpec(st.nbytes(), None, v.role)
                self.bound[name] = v.tensor
            return name, v.tensor.data_ptr() - base + v.offset
        name = self._by_value.get(id(v))
        if name is None:
            name = self._name(f"{v.role}.{v.name}")
            self._by_value[id(v)] = name
            self.program.buffers[name] = BufferSpec(max(v.nbytes, 16), None, v.role)
        return name, v.offset

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
