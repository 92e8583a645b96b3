"""Instantiate a :class:`Program` on the GPU and replay it through the native pump (``monolith/runtime/engine.py:
30-122``): the same constructor, ``run`` / ``profile`` / ``state`` / ``read`` and ``StepReport`` as the reference.

gfx950 mapping: the program's ops are captured into HIP graphs (the reference's ICB) of ``steps_per_cb`` steps, and
``mi_runner_run`` replays one graph per batch with ``in_flight`` batches queued, draining the token ring after
each (one launch per batch: a graph launch costs the host about as much as a small step costs the GPU). The step state and the ring are placed in pinned host memory (``HostResidentBuffer``), so the pump
reads ``done`` / ``error`` and writes ``ring_tail`` in place, the way the reference's runner touches them in
unified memory; every other buffer is device memory (weights from a file window through ``Buffer.from_file``).
``reencode=True`` launches the ops one by one instead of replaying the graph (the reference's re-encode fallback).
"""

from __future__ import annotations

import ctypes as C
import time
from dataclasses import dataclass
from typing import Dict, List, Optional, Tuple

import numpy as np

from . import hip
from . import native as nt
from .program import Program


@dataclass
class StepReport:
    steps: int
    command_buffers: int
    gpu_ms: float
    wall_ms: float
    host_busy_ms: float
    done: bool
    tokens: List[int]
    encode_ms: float = 0.0
    commit_ms: float = 0.0
    wait_ms: float = 0.0

    @property
    def host_fraction(self) -> float:
        """CPU time of the pump over wall time."""
        return self.host_busy_ms / self.wall_ms if self.wall_ms else 0.0


def compile_pipelines(program: Program, device: nt.Device, *, fast_math: bool = False, cache=None):
    """Kernels of the program, compiled once per (device, source, macros, language version, fast math, function)."""
    pipelines = {}
    for key, k in program.kernels.items():
        identity = (device, k.source, tuple(sorted(k.macros.items())), k.language_version, fast_math, k.function)
        pipeline = cache.get(identity) if cache is not None else None
        if pipeline is None:
            lib = nt.Library(device, k.source, k.macros, k.language_version, fast_math)
            pipeline = nt.Pipeline(lib, k.function, True)
            if cache is not None:
                cache[identity] = pipeline
        pipelines[key] = pipeline
    return pipelines


_HOST_ROLES = ("step_state", "ring")


class Engine:
    """``buffers`` lets several programs share buffers by name (weights, states, the step state and ring); a params
    record is never shared."""

    def __init__(self, program: Program, device: Optional[nt.Device] = None,
                 buffers: Optional[Dict[str, nt.Buffer]] = None, fast_math: bool = False,
                 pipeline_cache: Optional[dict] = None) -> None:
        self.program = program
        self.fast_math = fast_math
        self.dev = device or nt.Device()
        self.buffers: Dict[str, nt.Buffer] = {}
        for name, spec in program.buffers.items():
            if buffers is not None and name in buffers and spec.role != "params" and buffers[name].nbytes >= spec.nbytes:
                self.buffers[name] = buffers[name]
                continue
            if buffers is not None and name in buffers and spec.role in ("state", "step_state", "ring", "weights"):
                raise ValueError(f"shared buffer {name}: {buffers[name].nbytes} bytes, program needs {spec.nbytes}")
            if spec.file is not None:
                self.buffers[name] = nt.Buffer.from_file(self.dev, spec.file, spec.file_offset, spec.nbytes)
                continue
            if spec.init is not None and len(spec.init) > spec.nbytes:
                raise ValueError(f"buffer {name}: init larger than nbytes")
            buf = (nt.HostResidentBuffer(self.dev, spec.nbytes) if spec.role in _HOST_ROLES
                   else nt.Buffer(self.dev, spec.nbytes))
            if spec.init is not None:
                buf.write(spec.init, 0)
            self.buffers[name] = buf
        for name in (program.step_state, program.ring):
            if not isinstance(self.buffers.get(name), nt.HostResidentBuffer):
                raise ValueError(f"buffer {name}: the step state and the ring must be host-resident "
                                 f"(role 'step_state' / 'ring')")
        self.pipelines = compile_pipelines(program, self.dev, fast_math=fast_math, cache=pipeline_cache)
        self.ops: List[nt.Dispatch] = []
        for o in program.ops:
            d = (nt.Dispatch().pipeline(self.pipelines[o.kernel]).grid(*o.grid).threadgroup(*o.threadgroup)
                 .barrier(o.barrier_before))
            for index, bname, off in o.bindings:
                d.buffer(index, self.buffers[bname], off)
            for index, length in o.threadgroup_memory:
                d.threadgroup_memory(index, length)
            self.ops.append(d)
        ring = self.buffers[program.ring]
        if ring.nbytes < program.ring_capacity * 8:
            raise ValueError("the token ring needs 8 bytes per slot: (sequence << 32) | token")
        self.icb = nt.Icb(self.dev, self.ops)
        self._graphs: Dict[int, hip.Graph] = {1: self.icb.graph}   # k steps per graph: one launch per batch
        self._ctl = nt.HostResidentBuffer(self.dev, 16)        # [0]: the host's ring tail

    def _graph(self, k: int) -> hip.Graph:
        if k not in self._graphs:
            g = hip.Graph(self.icb._q.stream)
            with g:
                for _ in range(k):
                    for op in self.ops:
                        op.launch(self.icb._q.stream)
            self._graphs[k] = g
        return self._graphs[k]

    # ---- the pump ---------------------------------------------------------------------------------------------
    def _word(self, field: str) -> int:
        return self.buffers[self.program.step_state].word(self.program.layout.offset(field))

    def run(self, max_steps: int, *, steps_per_cb: int = 8, in_flight: int = 3, reencode: bool = False,
            max_tokens: int = 0) -> StepReport:
        """Replay up to ``max_steps`` steps (``max_tokens`` > 0: stop submitting once that many tokens arrived; the
        queued batches still complete, so a few more steps may run)."""
        if steps_per_cb < 1 or in_flight < 1:
            raise RuntimeError("steps_per_cb and in_flight must be >= 1")
        if reencode:
            return self._run_reencode(max_steps, steps_per_cb, in_flight, max_tokens)
        cap = max_steps * self.program.layout.t_max + 16
        tokens = np.zeros(cap, np.int32)
        d = hip.MiRunnerDesc()
        d.stream = self.icb._q.stream
        d.state, d.ring, d.ring_capacity = None, self.buffers[self.program.ring].gpu_address, self.program.ring_capacity
        d.host_ctl = self._ctl.gpu_address
        d.in_flight, d.launches_per_batch = in_flight, 1
        d.tokens, d.tokens_capacity, d.n_tokens = tokens.ctypes.data, cap, 0
        d.state_ring_tail, d.state_done, d.state_error = self._word("ring_tail"), self._word("done"), self._word("error")
        rep = StepReport(0, 0, 0.0, 0.0, 0.0, False, [])
        # a graph of steps_per_cb steps per batch, then one graph for the remainder
        for k, launches in ((steps_per_cb, max_steps // steps_per_cb), (max_steps % steps_per_cb, 1)):
            if k == 0 or launches == 0 or rep.done:
                continue
            if max_tokens and d.n_tokens >= max_tokens:
                break
            d.graph_exec, d.max_launches = self._graph(k).exec, launches
            d.max_tokens = max_tokens - d.n_tokens if max_tokens else 0
            st = hip.MiRunnerStats()
            try:
                hip.call("mi_runner_run", C.byref(d), C.byref(st))
            except hip.MiError as e:
                raise RuntimeError(str(e)) from e
            rep.steps += int(st.launches) * k
            rep.command_buffers += int(st.batches)
            rep.gpu_ms += float(st.gpu_ms)
            rep.wall_ms += float(st.wall_ms)
            rep.host_busy_ms += float(st.host_busy_ms)
            rep.encode_ms += float(st.launch_ms)
            rep.wait_ms += float(st.wait_ms)
            rep.done = bool(st.done)
        rep.tokens = tokens[:d.n_tokens].tolist()
        self._check_done(rep)
        return rep

    def _drain(self, tokens: List[int]) -> None:
        ring = np.frombuffer(self.buffers[self.program.ring].read(0, 8 * self.program.ring_capacity), np.uint64)
        tail = int(np.frombuffer(self._ctl.read(0, 4), np.uint32)[0])
        while True:
            v = int(ring[tail % self.program.ring_capacity])
            if (v >> 32) != tail + 1:
                break
            tokens.append(int(np.uint32(v & 0xFFFFFFFF).view(np.int32)))
            tail += 1
        self._ctl.write(np.uint32(tail).tobytes(), 0)

    def _run_reencode(self, max_steps, steps_per_cb, in_flight, max_tokens) -> StepReport:
        t0, c0 = time.perf_counter(), time.thread_time()
        stream = self.icb._q.stream
        tokens: List[int] = []
        pending: List[Tuple[hip.Event, hip.Event]] = []
        steps = batches = 0
        gpu = enc = wait = 0.0
        done = False

        def observe():
            nonlocal gpu, wait, batches, done
            a, b = pending.pop(0)
            w = time.perf_counter()
            b.synchronize()
            wait += (time.perf_counter() - w) * 1e3
            gpu += a.elapsed_ms(b)
            batches += 1
            self._drain(tokens)
            done = bool(self.state()["done"])

        while steps < max_steps and not done and (max_tokens == 0 or len(tokens) < max_tokens):
            e = time.perf_counter()
            C.c_uint32.from_address(self._word("ring_tail")).value = int(np.frombuffer(self._ctl.read(0, 4), np.uint32)[0])
            n = min(steps_per_cb, max_steps - steps)
            a, b = hip.Event(), hip.Event()
            a.record(stream)
            for _ in range(n):
                for op in self.ops:
                    op.launch(stream)
            b.record(stream)
            enc += (time.perf_counter() - e) * 1e3
            pending.append((a, b))
            steps += n
            while len(pending) >= in_flight:
                observe()
        while pending:
            observe()
        rep = StepReport(steps, batches, gpu, (time.perf_counter() - t0) * 1e3, (time.thread_time() - c0) * 1e3,
                         done, tokens, encode_ms=enc, commit_ms=0.0, wait_ms=wait)
        self._check_done(rep)
        return rep

    def _check_done(self, rep: StepReport) -> None:
        if rep.done and int(self.state()["error"]) == 3:
            raise RuntimeError("Megakernel: bounded worker barrier timed out")

    # ---- inspection ---------------------------------------------------------------------------------------------
    def profile(self, steps: int = 3) -> List[List[Tuple[float, float]]]:
        """Per-dispatch GPU (start, end) ms of ``steps`` steps launched op by op."""
        q = nt.Queue(self.dev)
        return [q.profile(self.ops) for _ in range(steps)]

    def state(self) -> Dict[str, object]:
        buf = self.buffers[self.program.step_state]
        return self.program.layout.unpack(buf.read(0, self.program.layout.size))

    def read(self, name: str, nbytes: Optional[int] = None) -> bytes:
        b = self.buffers[name]
        return b.read(0, nbytes if nbytes is not None else b.nbytes)
