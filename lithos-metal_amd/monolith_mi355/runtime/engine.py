"""Run a :class:`Program` on the GPU: the reference's ``Engine`` interface (``monolith/runtime/engine.py:30-122``:
the constructor, ``run`` / ``profile`` / ``state`` / ``read``, ``StepReport``, ``compile_pipelines``) over this
backend's runtime.

How it maps onto gfx950:

* **Buffers.** Every buffer spec becomes device memory, zero-filled, with its ``init`` bytes written in — except the
  step state and the token ring, which live in pinned host memory so the native pump reads ``done`` / ``error`` and
  writes ``ring_tail`` in place, and file windows (``Buffer.from_file``). ``buffers`` shares memory by name across
  programs (never a params record), including memory the program does not own (``Buffer.view`` of a tensor).
* **Ops.** An op is either a run-time compiled HIP kernel (``KernelSpec.source``, hiprtc, its bindings as kernel
  parameters in index order) or a typed entry point of libmi355 (``KernelSpec.function = "lib:<entry>"``): its
  descriptor is built once from ``meta["desc"]`` with each binding's address put into the pointer field of that index.
  Both kinds launch on a stream and capture into a HIP graph.
* **Replay.** A step's ops are captured into graphs of ``steps_per_cb`` steps (the reference's ICB replayed per
  command buffer); ``mi_runner_run`` launches one graph per batch with ``in_flight`` batches queued and drains the
  ring after each. ``reencode=True`` launches op by op instead.
"""

from __future__ import annotations

import ctypes as C
import time
from dataclasses import dataclass, field
from typing import Any, Dict, List, Optional, Sequence, Tuple

import numpy as np

from . import hip
from . import native as nt
from .program import BufferSpec, Program


@dataclass
class StepReport:
    """What a run did: steps submitted, command buffers (graph launches), GPU / wall / pump-thread milliseconds,
    whether the program stopped, and the tokens the ring delivered."""

    steps: int = 0
    command_buffers: int = 0
    gpu_ms: float = 0.0
    wall_ms: float = 0.0
    host_busy_ms: float = 0.0
    done: bool = False
    tokens: List[int] = field(default_factory=list)
    encode_ms: float = 0.0
    commit_ms: float = 0.0
    wait_ms: float = 0.0

    @property
    def host_fraction(self) -> float:
        return self.host_busy_ms / self.wall_ms if self.wall_ms else 0.0

    def add_runner(self, stats: "hip.MiRunnerStats", steps_per_launch: int) -> None:
        self.steps += int(stats.launches) * steps_per_launch
        self.command_buffers += int(stats.batches)
        self.gpu_ms += float(stats.gpu_ms)
        self.wall_ms += float(stats.wall_ms)
        self.host_busy_ms += float(stats.host_busy_ms)
        self.encode_ms += float(stats.launch_ms)
        self.wait_ms += float(stats.wait_ms)
        self.done = bool(stats.done)


# the descriptor type of each library entry point a program may name
DESCRIPTORS = {"mi_gemv": hip.MiGemvDesc, "mi_gdn_step": hip.MiGdnDesc, "mi_gqa_decode": hip.MiGqaDesc,
               "mi_moe_route": hip.MiMoeRouteDesc, "mi_moe_combine": hip.MiMoeCombineDesc, "mi_embed": hip.MiEmbedDesc,
               "mi_argmax": hip.MiArgmaxDesc, "mi_advance": hip.MiAdvanceDesc, "mi_rmsnorm_stat": hip.MiNormDesc,
               "mi_norm_apply": hip.MiNormDesc, "mi_accept_scan": hip.MiAcceptScanDesc,
               "mi_verify_select": hip.MiVerifySelectDesc}
LIB_PREFIX = "lib:"


class LibraryCall:
    """One op on a typed entry point: the descriptor, built once, and the call."""

    def __init__(self, entry: str, desc: Dict[str, Any], pointers: Sequence[Tuple[int, int]]) -> None:
        if entry not in DESCRIPTORS:
            raise ValueError(f"program names library entry point {entry!r}, which this runtime does not know")
        self.entry = entry
        cls = DESCRIPTORS[entry]
        names = [f for f, _ in cls._fields_]
        self.desc = cls()
        for key, value in desc.items():
            current = getattr(self.desc, key)
            if isinstance(value, (list, tuple)):           # fixed arrays (the advance's EOS ids)
                for i, v in enumerate(value):
                    current[i] = v
            else:
                setattr(self.desc, key, value)
        for index, address in pointers:
            setattr(self.desc, names[index], address)
        self._fn = getattr(hip.load(), entry)

    def launch(self, stream=None) -> None:
        rc = self._fn(C.byref(self.desc), hip.stream_handle(stream) if stream is not None else None)
        if rc != 0:
            raise hip.MiError(f"{self.entry} failed ({rc}): {hip.last_error()}")


def compile_pipelines(program: Program, device: nt.Device, *, fast_math: bool = False, cache=None):
    """The program's run-time kernels, one hiprtc compile per distinct (source, macros, language version, fast
    math) shared by every function it provides; library entry points need none (they map to None)."""
    libraries: Dict[tuple, nt.Library] = {}
    pipelines: Dict[str, Optional[nt.Pipeline]] = {}
    for key, spec in program.kernels.items():
        if spec.function.startswith(LIB_PREFIX):
            pipelines[key] = None
            continue
        unit = (device, spec.source, tuple(sorted(spec.macros.items())), spec.language_version, fast_math)
        cached = cache.get(unit + (spec.function,)) if cache is not None else None
        if cached is not None:
            pipelines[key] = cached
            continue
        lib = libraries.get(unit)
        if lib is None:
            lib = libraries[unit] = nt.Library(device, spec.source, spec.macros, spec.language_version, fast_math)
        pipelines[key] = nt.Pipeline(lib, spec.function, True)
        if cache is not None:
            cache[unit + (spec.function,)] = pipelines[key]
    return pipelines


def bound_buffers(program: Program, device: Optional[nt.Device] = None) -> Dict[str, nt.Buffer]:
    """Views of the tensors a program emitted from live layers binds (``program.bound_tensors``), for ``buffers=``."""
    dev = device or nt.Device()
    out = {}
    for name, t in getattr(program, "bound_tensors", {}).items():
        st = t.untyped_storage()
        out[name] = nt.Buffer.view(dev, st.data_ptr(), st.nbytes(), owner=t)
    return out


_HOST_ROLES = ("step_state", "ring")


class Engine:
    def __init__(self, program: Program, device: Optional[nt.Device] = None,
                 buffers: Optional[Dict[str, nt.Buffer]] = None, fast_math: bool = False,
                 pipeline_cache: Optional[dict] = None) -> None:
        self.program = program
        self.fast_math = fast_math
        self.dev = device or nt.Device()
        self.buffers = {name: self._place(name, spec, buffers or {}) for name, spec in program.buffers.items()}
        for name in (program.step_state, program.ring):
            if not isinstance(self.buffers.get(name), nt.HostResidentBuffer):
                raise ValueError(f"buffer {name}: the step state and the ring live in pinned host memory "
                                 f"(roles 'step_state' / 'ring')")
        if self.buffers[program.ring].nbytes < 8 * program.ring_capacity:
            raise ValueError("the token ring needs 8 bytes per slot: (sequence << 32) | token")
        self.pipelines = compile_pipelines(program, self.dev, fast_math=fast_math, cache=pipeline_cache)
        self.ops = [self._op(o) for o in program.ops]
        self._q = nt.Queue(self.dev)
        self._graphs: Dict[int, hip.Graph] = {}
        self._ctl = nt.HostResidentBuffer(self.dev, 16)     # [0]: the host's ring tail
        self._graph(1)

    # ---- construction ------------------------------------------------------------------------------------------
    def _place(self, name: str, spec: BufferSpec, shared: Dict[str, nt.Buffer]) -> nt.Buffer:
        given = shared.get(name)
        if given is not None and spec.role != "params":
            if given.nbytes < spec.nbytes:
                raise ValueError(f"shared buffer {name}: {given.nbytes} bytes, the program needs {spec.nbytes}")
            return given
        if spec.file is not None:
            return nt.Buffer.from_file(self.dev, spec.file, spec.file_offset, spec.nbytes)
        if spec.init is not None and len(spec.init) > spec.nbytes:
            raise ValueError(f"buffer {name}: {len(spec.init)} init bytes for {spec.nbytes}")
        buf = nt.HostResidentBuffer(self.dev, spec.nbytes) if spec.role in _HOST_ROLES else nt.Buffer(self.dev,
                                                                                                     spec.nbytes)
        if spec.init:
            buf.write(spec.init, 0)
        return buf

    def _op(self, o):
        spec = self.program.kernels[o.kernel]
        if spec.function.startswith(LIB_PREFIX):
            pointers = [(index, self.buffers[b].gpu_address + off) for index, b, off in o.bindings]
            return LibraryCall(spec.function[len(LIB_PREFIX):], dict(o.meta.get("desc", {})), pointers)
        d = (nt.Dispatch().pipeline(self.pipelines[o.kernel]).grid(*o.grid).threadgroup(*o.threadgroup)
             .barrier(o.barrier_before))
        for index, b, off in o.bindings:
            d.buffer(index, self.buffers[b], off)
        for index, nbytes in o.threadgroup_memory:
            d.threadgroup_memory(index, nbytes)
        return d

    def _graph(self, steps: int) -> hip.Graph:
        """The graph of ``steps`` consecutive steps (captured once)."""
        g = self._graphs.get(steps)
        if g is None:
            g = hip.Graph(self._q.stream)
            with g:
                for _ in range(steps):
                    for op in self.ops:
                        op.launch(self._q.stream)
            self._graphs[steps] = g
        return g

    # ---- running -----------------------------------------------------------------------------------------------
    def _state_word(self, name: str) -> int:
        return self.buffers[self.program.step_state].word(self.program.layout.offset(name))

    def run(self, max_steps: int, *, steps_per_cb: int = 8, in_flight: int = 3, reencode: bool = False,
            max_tokens: int = 0) -> StepReport:
        """Replay up to ``max_steps`` steps; ``max_tokens`` > 0 stops submitting once that many tokens arrived (the
        batches already queued complete)."""
        if steps_per_cb < 1 or in_flight < 1:
            raise RuntimeError("steps_per_cb and in_flight must be >= 1")
        if reencode:
            return self._run_op_by_op(max_steps, steps_per_cb, in_flight, max_tokens)
        cap = max_steps * self.program.layout.t_max + 16
        tokens = np.zeros(cap, np.int32)
        d = hip.MiRunnerDesc(stream=self._q.stream, ring=self.buffers[self.program.ring].gpu_address,
                             ring_capacity=self.program.ring_capacity, host_ctl=self._ctl.gpu_address,
                             launches_per_batch=1, in_flight=in_flight, tokens=tokens.ctypes.data,
                             tokens_capacity=cap, n_tokens=0, state_ring_tail=self._state_word("ring_tail"),
                             state_done=self._state_word("done"), state_error=self._state_word("error"))
        report = StepReport()
        full, rest = divmod(max_steps, steps_per_cb)
        for per_launch, launches in ((steps_per_cb, full), (rest, 1)):
            if not per_launch or not launches or report.done or (max_tokens and d.n_tokens >= max_tokens):
                continue
            d.graph_exec, d.max_launches = self._graph(per_launch).exec, launches
            d.max_tokens = max_tokens - d.n_tokens if max_tokens else 0
            stats = hip.MiRunnerStats()
            try:
                hip.call("mi_runner_run", C.byref(d), C.byref(stats))
            except hip.MiError as e:
                raise RuntimeError(str(e)) from e
            report.add_runner(stats, per_launch)
        report.tokens = tokens[: d.n_tokens].tolist()
        return report

    def _take_ring(self, tokens: List[int]) -> None:
        cap = self.program.ring_capacity
        ring = np.frombuffer(self.buffers[self.program.ring].read(0, 8 * cap), np.uint64)
        tail = int(np.frombuffer(self._ctl.read(0, 4), np.uint32)[0])
        while int(ring[tail % cap]) >> 32 == tail + 1:
            tokens.append(int(np.uint32(int(ring[tail % cap]) & 0xFFFFFFFF).view(np.int32)))
            tail += 1
        self._ctl.write(np.uint32(tail).tobytes(), 0)

    def _run_op_by_op(self, max_steps, steps_per_cb, in_flight, max_tokens) -> StepReport:
        report = StepReport()
        t0, cpu0 = time.perf_counter(), time.thread_time()
        stream = self._q.stream
        queued: List[Tuple[hip.Event, hip.Event]] = []

        def settle():
            start, end = queued.pop(0)
            w = time.perf_counter()
            end.synchronize()
            report.wait_ms += (time.perf_counter() - w) * 1e3
            report.gpu_ms += start.elapsed_ms(end)
            report.command_buffers += 1
            self._take_ring(report.tokens)
            report.done = bool(self.state()["done"])

        while report.steps < max_steps and not report.done and not (max_tokens and len(report.tokens) >= max_tokens):
            e0 = time.perf_counter()
            C.c_uint32.from_address(self._state_word("ring_tail")).value = int(
                np.frombuffer(self._ctl.read(0, 4), np.uint32)[0])
            n = min(steps_per_cb, max_steps - report.steps)
            start, end = hip.Event(), hip.Event()
            start.record(stream)
            for _ in range(n):
                for op in self.ops:
                    op.launch(stream)
            end.record(stream)
            report.encode_ms += (time.perf_counter() - e0) * 1e3
            queued.append((start, end))
            report.steps += n
            while len(queued) >= in_flight:
                settle()
        while queued:
            settle()
        report.wall_ms = (time.perf_counter() - t0) * 1e3
        report.host_busy_ms = (time.thread_time() - cpu0) * 1e3
        return report

    # ---- inspection --------------------------------------------------------------------------------------------
    def profile(self, steps: int = 3) -> List[List[Tuple[float, float]]]:
        """Per-op GPU (start, end) milliseconds of ``steps`` steps launched op by op."""
        return [self._q.profile(self.ops) for _ in range(steps)]

    def state(self) -> Dict[str, object]:
        return self.program.layout.unpack(self.buffers[self.program.step_state].read(0, self.program.layout.size))

    def read(self, name: str, nbytes: Optional[int] = None) -> bytes:
        b = self.buffers[name]
        return b.read(0, b.nbytes if nbytes is None else nbytes)
