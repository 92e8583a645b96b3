"""The reference's native runtime surface on HIP: ``Device``, ``Buffer``, ``Library``, ``Pipeline``, ``Dispatch``,
``Queue``, ``Icb`` (``runtime/src/native.mm:13-95``, ``runtime/src/metal_core.h:20-116``), over the C ABI.

Same names, argument meanings and error behaviour as the reference's classes, so code written against
``monolith.runtime._native`` runs here unchanged except for the kernel language:

* ``Library(device, source, macros)`` compiles HIP C++ for gfx950 at run time (hiprtc, which provides the HIP
  device API itself: sources include no ``hip_runtime.h``). A compile error raises
  ``MiError`` carrying the compiler log's tail (the reference raises ``RuntimeError("MSL compile failed: …")``;
  ``MiError`` is a ``RuntimeError``). ``Pipeline(lib, "name")`` raises "no kernel named name" for a missing kernel.
* Argument binding: Metal binds buffers and bytes by index; a HIP kernel takes one parameter list. ``Dispatch``
  lays its slots out in index order as that list: a buffer binds as its device address plus offset (an 8-byte
  pointer), ``bytes`` as the raw bytes at their natural alignment (the largest power of two ≤ 8 dividing the
  length, or ``align=``). ``threadgroup_memory`` lengths add up to the launch's dynamic LDS.
* ``grid`` counts workgroups (Metal's ``dispatchThreadgroups``), ``threadgroup`` threads per workgroup.
* ``Buffer.read`` / ``write`` copy between host bytes and device memory (HBM is not host-mapped); out-of-range
  windows raise ``IndexError`` (nanobind maps ``std::out_of_range`` to it).
* ``Queue.run`` executes dispatches in order on one stream (``concurrent`` is accepted; in-stream order already
  satisfies every ``barrier``) and returns ``RunResult(gpu_ms, wall_ms, error)`` — errors come back in ``error``
  as in the reference. ``Queue.profile`` gives (start_ms, end_ms) per dispatch from HIP events.
* ``Icb(device, ops)`` captures the dispatches into a HIP graph (``launch`` replays it); the token-loop runner is
  ``runtime.step.StepProgram`` over ``mi_runner_run``.
"""

from __future__ import annotations

import ctypes as C
import os
import time
from dataclasses import dataclass
from typing import Dict, List, Optional, Sequence, Tuple

from . import hip


@dataclass
class DeviceInfo:
    """``DeviceInfo`` (``metal_core.h:20-27``) with the gfx950 meanings: ``gpu_cores`` = compute units,
    ``apple_family`` → ``arch`` (the gfx target), working set = HBM size, no unified memory."""
    name: str
    gpu_cores: int
    arch: str
    max_buffer_length: int
    recommended_working_set: int
    has_unified_memory: bool = False


class Device:
    def __init__(self, index: int = 0):
        self.index = index
        hip.call("mi_set_device", index)

    def info(self) -> DeviceInfo:
        i = hip.device_info(self.index)
        return DeviceInfo(i.name.decode(), int(i.compute_units), i.arch.decode(), int(i.hbm_bytes), int(i.hbm_bytes))


class Buffer:
    """Device memory owned by this object (freed when it is collected). ``Buffer(device, nbytes)`` is zero-filled;
    ``Buffer(device, data)`` holds a copy of ``data``."""

    def __init__(self, device: Device, nbytes_or_data):
        self.device = device
        self._p = C.c_void_p()
        if isinstance(nbytes_or_data, (bytes, bytearray, memoryview)):
            data = bytes(nbytes_or_data)
            self._n = len(data)
            self._alloc()
            if self._n:
                hip.call("mi_memcpy_h2d", self._p, data, self._n, None)
        else:
            self._n = int(nbytes_or_data)
            if self._n < 0:
                raise ValueError("Buffer: negative size")
            self._alloc()
            if self._n:
                hip.call("mi_memset", self._p, 0, self._n, None)
                hip.call("mi_stream_synchronize", None)

    def _alloc(self):
        hip.call("mi_malloc", C.byref(self._p), max(self._n, 1))

    @classmethod
    def from_file(cls, device: Device, path: str, offset: int, nbytes: int) -> "Buffer":
        """A window of a file (page-aligned offset and length, as ``metal_core.mm:70-90`` requires)."""
        b = cls.__new__(cls)
        b.device, b._n, b._p = device, int(nbytes), C.c_void_p()
        hip.call("mi_buf_from_file", os.fsencode(path), int(offset), int(nbytes), C.byref(b._p))
        return b

    @classmethod
    def view(cls, device: Device, address: int, nbytes: int, owner=None) -> "Buffer":
        """Device memory this object does not own — a window of an allocation made elsewhere (a torch tensor's
        storage, another buffer); ``owner`` is kept alive as long as the view."""
        b = cls.__new__(cls)
        b.device, b._n, b._p = device, int(nbytes), C.c_void_p(int(address))
        b._owner, b._borrowed = owner, True
        return b

    @property
    def nbytes(self) -> int:
        return self._n

    @property
    def gpu_address(self) -> int:
        return int(self._p.value or 0)

    def read(self, offset: int = 0, nbytes: int = 0) -> bytes:
        if offset < 0 or nbytes < 0 or offset + nbytes > self._n:
            raise IndexError("Buffer.read out of range")
        out = C.create_string_buffer(max(nbytes, 1))
        if nbytes:
            hip.call("mi_memcpy_d2h", out, self.gpu_address + offset, nbytes, None)
        return out.raw[:nbytes]

    def write(self, data, offset: int = 0) -> None:
        data = bytes(data)
        if offset < 0 or offset + len(data) > self._n:
            raise IndexError("Buffer.write out of range")
        if data:
            hip.call("mi_memcpy_h2d", self.gpu_address + offset, data, len(data), None)

    def fill(self, value: int) -> None:
        hip.call("mi_memset", self._p, int(value) & 0xFF, self._n, None)
        hip.call("mi_stream_synchronize", None)

    def __del__(self):
        try:
            if getattr(self, "_borrowed", False):
                return
            if getattr(self, "_p", None) and self._p.value and hip._lib is not None:
                hip._lib.mi_free(self._p)
                self._p = C.c_void_p()
        except Exception:
            pass


class HostResidentBuffer(Buffer):
    """A buffer in pinned, device-accessible host memory (``mi_host_alloc``): what a program's step state and
    token ring live in when the host pump reads them without a copy. ``gpu_address`` is valid on the device."""

    def __init__(self, device: Device, nbytes: int):
        self.device, self._n = device, int(nbytes)
        addr = hip.load().mi_host_alloc(max(self._n, 1))
        if not addr:
            raise hip.MiError(f"mi_host_alloc({nbytes}) failed: {hip.last_error()}")
        self._addr = int(addr)
        C.memset(self._addr, 0, max(self._n, 1))
        self._p = C.c_void_p()            # nothing for Buffer.__del__ to free

    @property
    def gpu_address(self) -> int:
        return self._addr

    def word(self, offset: int) -> int:
        """Host address of the 4-byte word at ``offset``."""
        if offset < 0 or offset + 4 > self._n:
            raise IndexError("HostResidentBuffer.word out of range")
        return self._addr + offset

    def read(self, offset: int = 0, nbytes: int = 0) -> bytes:
        if offset < 0 or nbytes < 0 or offset + nbytes > self._n:
            raise IndexError("Buffer.read out of range")
        return C.string_at(self._addr + offset, nbytes)

    def write(self, data, offset: int = 0) -> None:
        data = bytes(data)
        if offset < 0 or offset + len(data) > self._n:
            raise IndexError("Buffer.write out of range")
        C.memmove(self._addr + offset, data, len(data))

    def fill(self, value: int) -> None:
        C.memset(self._addr, int(value) & 0xFF, self._n)

    def __del__(self):
        try:
            if getattr(self, "_addr", 0) and hip._lib is not None:
                hip._lib.mi_host_free(C.c_void_p(self._addr))
                self._addr = 0
        except Exception:
            pass


def compile_source(source: str, macros: Optional[Dict[str, str]] = None, fast_math: bool = False) -> bytes:
    """HIP C++ → a gfx950 code object (bytes). Needs no GPU."""
    macros = macros or {}
    flat = []
    for k, v in macros.items():
        flat += [str(k).encode(), str(v).encode()]
    arr = (C.c_char_p * max(len(flat), 1))(*flat)
    code, n = C.c_void_p(), C.c_size_t()
    hip.call("mi_library_compile", source.encode(), arr, len(macros), int(bool(fast_math)), C.byref(code),
             C.byref(n))
    try:
        return C.string_at(code, n.value)
    finally:
        hip.load().mi_code_free(code)


class Library:
    """Kernels compiled from source at run time (``metal_core.h:50-57``). ``language_version`` is accepted for the
    reference's signature and ignored (the kernels are C++17 HIP)."""

    def __init__(self, device: Device, source: str, macros: Optional[Dict[str, str]] = None,
                 language_version: int = 0, fast_math: bool = False):
        self.device = device
        self.code = compile_source(source, macros, fast_math)
        self._h = C.c_void_p()
        self._load()

    @classmethod
    def from_code(cls, device: Device, code: bytes) -> "Library":
        lib = cls.__new__(cls)
        lib.device, lib.code, lib._h = device, bytes(code), C.c_void_p()
        lib._load()
        return lib

    def _load(self):
        self._buf = C.create_string_buffer(self.code, len(self.code))
        hip.call("mi_library_load", self._buf, len(self.code), C.byref(self._h))

    def __del__(self):
        try:
            if getattr(self, "_h", None) and self._h.value and hip._lib is not None:
                hip._lib.mi_library_release(self._h)
                self._h = C.c_void_p()
        except Exception:
            pass


class Pipeline:
    """One kernel of a library (``metal_core.h:59-66``); keeps the library alive."""

    def __init__(self, library: Library, function: str, support_icb: bool = False):
        self.library, self.function = library, function
        self._k = C.c_void_p()
        hip.call("mi_kernel_get", library._h, function.encode(), C.byref(self._k))
        self.attrs = hip.MiKernelAttrs()
        hip.call("mi_kernel_info", self._k, C.byref(self.attrs))

    @property
    def max_threads_per_threadgroup(self) -> int:
        return int(self.attrs.max_threads_per_block)

    @property
    def thread_execution_width(self) -> int:
        return int(self.attrs.wave_size)


def _natural_align(n: int) -> int:
    a = 1
    while a < 8 and n % (2 * a) == 0:
        a *= 2
    return a


class Dispatch:
    """A launch description built by chaining (``native.mm:51-65``)."""

    def __init__(self):
        self._pipeline: Optional[Pipeline] = None
        self._slots: Dict[int, Tuple[str, object, int]] = {}
        self._lds: Dict[int, int] = {}
        self._grid = (1, 1, 1)
        self._tg = (1, 1, 1)
        self.barrier_before = False

    def pipeline(self, p: Pipeline) -> "Dispatch":
        self._pipeline = p
        return self

    def buffer(self, index: int, buffer: Buffer, offset: int = 0) -> "Dispatch":
        if offset < 0 or offset > buffer.nbytes:
            raise IndexError("Dispatch.buffer: offset outside the buffer")
        self._slots[int(index)] = ("buffer", buffer, int(offset))
        return self

    def bytes(self, index: int, data, align: Optional[int] = None) -> "Dispatch":
        data = bytes(data)
        self._slots[int(index)] = ("bytes", data, int(align) if align else _natural_align(len(data)))
        return self

    def threadgroup_memory(self, index: int, length: int) -> "Dispatch":
        self._lds[int(index)] = int(length)
        return self

    def grid(self, x: int, y: int = 1, z: int = 1) -> "Dispatch":
        self._grid = (int(x), int(y), int(z))
        return self

    def threadgroup(self, x: int, y: int = 1, z: int = 1) -> "Dispatch":
        self._tg = (int(x), int(y), int(z))
        return self

    def barrier(self, on: bool = True) -> "Dispatch":
        self.barrier_before = bool(on)
        return self

    def kernargs(self) -> bytes:
        """The packed parameter block: slots in index order, each at its alignment."""
        out = bytearray()
        for idx in sorted(self._slots):
            kind, obj, extra = self._slots[idx]
            if kind == "buffer":
                payload, align = (obj.gpu_address + extra).to_bytes(8, "little"), 8
            else:
                payload, align = obj, extra
            out += b"\0" * ((-len(out)) % align)
            out += payload
        return bytes(out)

    def launch(self, stream=None) -> None:
        if self._pipeline is None:
            raise RuntimeError("Dispatch: no pipeline")
        args = self.kernargs()
        grid = (C.c_uint32 * 3)(*self._grid)
        tg = (C.c_uint32 * 3)(*self._tg)
        hip.call("mi_launch", self._pipeline._k, args if args else None, len(args), grid, tg, sum(self._lds.values()),
                 hip.stream_handle(stream) if stream is not None else None)


@dataclass
class RunResult:
    gpu_ms: float
    wall_ms: float
    error: str = ""


class Queue:
    """An in-order HIP stream with timed runs (``metal_core.h:83-96``)."""

    def __init__(self, device: Device):
        self.device = device
        self._s = C.c_void_p()
        hip.call("mi_stream_create", C.byref(self._s))

    @property
    def stream(self) -> int:
        return int(self._s.value)

    def run(self, dispatches: Sequence[Dispatch], concurrent: bool = False) -> RunResult:
        t0 = time.perf_counter()
        a, b = hip.Event(), hip.Event()
        err = ""
        try:
            a.record(self.stream)
            for d in dispatches:
                d.launch(self.stream)
            b.record(self.stream)
            hip.call("mi_stream_synchronize", self._s)
            gpu = a.elapsed_ms(b)
        except hip.MiError as e:
            err, gpu = str(e), 0.0
            try:
                hip.call("mi_stream_synchronize", self._s)
            except hip.MiError:
                pass
        return RunResult(gpu, (time.perf_counter() - t0) * 1e3, err)

    def profile(self, dispatches: Sequence[Dispatch]) -> List[Tuple[float, float]]:
        """(start_ms, end_ms) of each dispatch from the first one's start."""
        if not dispatches:
            return []
        ev = [(hip.Event(), hip.Event()) for _ in dispatches]
        for (s, e), d in zip(ev, dispatches):
            s.record(self.stream)
            d.launch(self.stream)
            e.record(self.stream)
        hip.call("mi_stream_synchronize", self._s)
        base = ev[0][0]
        return [(base.elapsed_ms(s), base.elapsed_ms(e)) for s, e in ev]

    def supports_profiling(self) -> bool:
        return True

    def __del__(self):
        try:
            if getattr(self, "_s", None) and self._s.value and hip._lib is not None:
                hip._lib.mi_stream_destroy(self._s)
                self._s = C.c_void_p()
        except Exception:
            pass


class Icb:
    """Pre-encoded dispatches (``metal_core.h:106-116``) as a captured HIP graph."""

    def __init__(self, device: Device, ops: Sequence[Dispatch]):
        if not ops:
            raise RuntimeError("Icb: no ops")
        self.device, self.ops = device, list(ops)
        self._q = Queue(device)
        self.graph = hip.Graph(self._q.stream)
        with self.graph:
            for d in self.ops:
                d.launch(self._q.stream)

    @property
    def count(self) -> int:
        return len(self.ops)

    def launch(self, stream=None) -> None:
        self.graph.launch(stream if stream is not None else self._q.stream)

    def synchronize(self) -> None:
        hip.call("mi_stream_synchronize", self._q._s)
