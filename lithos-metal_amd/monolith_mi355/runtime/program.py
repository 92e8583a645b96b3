"""The step program format (``program.json``, version 1) and the StepState layout it carries: the contract between
a compiler that emits a program and the runtime that replays it (``monolith/runtime/program.py:16-89``,
``monolith/core/step_state.py:28-118``).

The format and the field order are kept as the reference defines them, so a program serialized there loads here
and the reverse; only the kernel language differs (``KernelSpec.source`` is HIP C++ for gfx950, compiled with
hiprtc; ``StepStateLayout.to_hip`` declares the struct for it as ``to_msl`` does for Metal). ``mi_step_state``
of the C ABI is ``StepStateLayout(t_max=16, gamma_max=15)``.
"""

from __future__ import annotations

import json
import struct
from dataclasses import dataclass, field, fields
from pathlib import Path
from typing import Dict, List, Mapping, Optional, Sequence, Tuple

# (name, dtype, count) in the binary order; count "t" = t_max, "g" = max(gamma_max, 1)
_FIELDS = [
    ("step", "u32", 1), ("position", "u32", 1), ("kv_len", "u32", 1), ("t_this_step", "u32", 1),
    ("pending_tokens", "i32", "t"), ("rng_lo", "u32", 1), ("rng_hi", "u32", 1), ("anchor", "i32", 1),
    ("gamma", "u32", 1), ("draft_tokens", "i32", "g"), ("confidence", "f32", "g"), ("verify_len", "u32", 1),
    ("accepted", "u32", 1), ("checkpoint_index", "u32", 1), ("drafter_ctx_len", "u32", 1), ("done", "u32", 1),
    ("error", "u32", 1), ("ring_head", "u32", 1), ("ring_tail", "u32", 1), ("prefill_left", "u32", 1),
    ("n_inject", "u32", 1), ("stop_at", "u32", 1), ("n_chain", "u32", 1),
]
_CODE = {"u32": "I", "i32": "i", "f32": "f"}
_CTYPE = {"u32": "unsigned int", "i32": "int", "f32": "float"}


class StepStateLayout:
    """Field offsets of the StepState for a given ``t_max`` / ``gamma_max``: 4-byte scalars or arrays of them, in
    a fixed order, the size padded to 16 bytes."""

    def __init__(self, t_max: int = 8, gamma_max: int = 7) -> None:
        if t_max < 1 or gamma_max < 0 or t_max < gamma_max + 1:
            raise ValueError(f"StepStateLayout: need t_max >= gamma_max + 1 >= 1, got t_max={t_max}, "
                             f"gamma_max={gamma_max}")
        self.t_max, self.gamma_max = t_max, gamma_max
        g = max(gamma_max, 1)
        self.fields: List[Tuple[str, str, int]] = [
            (n, d, t_max if c == "t" else g if c == "g" else c) for n, d, c in _FIELDS]
        self.offsets: Dict[str, int] = {}
        off = 0
        for n, _, c in self.fields:
            self.offsets[n] = off
            off += 4 * c
        self.size = (off + 15) // 16 * 16

    def offset(self, name: str) -> int:
        return self.offsets[name]

    def to_hip(self, struct_name: str = "StepState") -> str:
        lines = [f"struct {struct_name} {{"]
        for n, d, c in self.fields:
            lines.append(f"  {_CTYPE[d]} {n}" + (f"[{c}]" if c > 1 else "") + ";")
        pad = self.size - sum(4 * c for _, _, c in self.fields)
        if pad:
            lines.append(f"  unsigned int pad_[{pad // 4}];")
        lines.append("};")
        return "\n".join(lines)

    def pack(self, values: Mapping[str, object]) -> bytes:
        buf = bytearray(self.size)
        for n, d, c in self.fields:
            raw = values.get(n, [] if c > 1 else 0)
            seq: Sequence = list(raw) if c > 1 else [raw]
            if len(seq) > c:
                raise ValueError(f"StepState.{n}: {len(seq)} values for {c} slots")
            seq = list(seq) + [0] * (c - len(seq))
            struct.pack_into("<" + _CODE[d] * c, buf, self.offsets[n], *seq)
        return bytes(buf)

    def unpack(self, data: bytes) -> Dict[str, object]:
        if len(data) < self.size:
            raise ValueError(f"StepState.unpack: need {self.size} bytes, got {len(data)}")
        out: Dict[str, object] = {}
        for n, d, c in self.fields:
            vals = struct.unpack_from("<" + _CODE[d] * c, data, self.offsets[n])
            out[n] = list(vals) if c > 1 else vals[0]
        return out


@dataclass
class KernelSpec:
    source: str                          # HIP C++ (extern "C" __global__ kernels); "" for a library kernel
    function: str                        # kernel name, or "lib:<entry point>" — a typed entry point of libmi355
    macros: Dict[str, str] = field(default_factory=dict)
    language_version: int = 0            # carried for the format; HIP sources compile as C++17


@dataclass
class BufferSpec:
    nbytes: int
    init: Optional[bytes] = None         # initial contents (zeros if None)
    role: str = "arena"                  # "weights" | "state" | "arena" | "step_state" | "ring" | "params"
    file: Optional[str] = None           # weights: a page-aligned window of this file
    file_offset: int = 0


@dataclass
class OpSpec:
    kernel: str                          # key into Program.kernels
    bindings: List[Tuple[int, str, int]]  # (parameter index, buffer name, byte offset)
    grid: Tuple[int, int, int]           # workgroups
    threadgroup: Tuple[int, int, int]    # threads per workgroup
    barrier_before: bool = True
    threadgroup_memory: List[Tuple[int, int]] = field(default_factory=list)
    name: str = ""
    meta: Dict[str, object] = field(default_factory=dict)


# ---- program.json v1 --------------------------------------------------------------------------------------------------
# Each spec class serializes field by field; a codec entry renames a field in the file and/or converts its value
# (name in the file, to_json, from_json). Fields without an entry are written as they are. The key names and value
# forms are the v1 format's, so files written by either side load on the other.
def _hex_in(v):
    return bytes.fromhex(v) if v else None


def _tuples(v):
    return [tuple(x) for x in v]


_CODECS = {
    KernelSpec: {"macros": ("macros", dict, dict), "language_version": ("language_version", int, int)},
    BufferSpec: {"init": ("init_hex", lambda b: b.hex() if b is not None else None, _hex_in),
                 "file_offset": ("file_offset", int, int)},
    OpSpec: {"bindings": ("bindings", _tuples, _tuples), "grid": ("grid", tuple, tuple),
             "threadgroup": ("threadgroup", tuple, tuple), "threadgroup_memory": ("threadgroup_memory", _tuples, _tuples),
             "meta": ("meta", dict, dict)},
}


def _encode(spec) -> dict:
    codec = _CODECS.get(type(spec), {})
    out = {}
    for f in fields(spec):
        key, to_json, _ = codec.get(f.name, (f.name, None, None))
        v = getattr(spec, f.name)
        out[key] = to_json(v) if to_json is not None else v
    return out


def _decode(cls, d: Mapping[str, object]):
    codec = _CODECS.get(cls, {})
    kw = {}
    for f in fields(cls):
        key, _, from_json = codec.get(f.name, (f.name, None, None))
        if key in d:
            kw[f.name] = from_json(d[key]) if from_json is not None else d[key]
    return cls(**kw)


@dataclass
class Program:
    kernels: Dict[str, KernelSpec]
    buffers: Dict[str, BufferSpec]
    ops: List[OpSpec]
    step_state: str = "step_state"
    ring: str = "ring"                   # 8-byte slots, (sequence << 32) | token
    ring_capacity: int = 4096
    layout: StepStateLayout = field(default_factory=StepStateLayout)
    context_capacity: int = 0
    backend_id: str = "common"
    config_digest: str = ""

    _SCALARS = ("step_state", "ring", "ring_capacity", "context_capacity", "backend_id", "config_digest")

    def to_dict(self) -> dict:
        d = {"version": 1}
        d.update({k: getattr(self, k) for k in self._SCALARS})
        d["layout"] = {"t_max": self.layout.t_max, "gamma_max": self.layout.gamma_max}
        d["kernels"] = {name: _encode(k) for name, k in self.kernels.items()}
        d["buffers"] = {name: _encode(b) for name, b in self.buffers.items()}
        d["ops"] = [_encode(o) for o in self.ops]
        return d

    def to_json(self) -> str:
        return json.dumps(self.to_dict(), indent=1)

    @classmethod
    def from_dict(cls, d: Mapping[str, object]) -> "Program":
        if d.get("version") != 1:
            raise ValueError(f"program.json version {d.get('version')!r}: this runtime reads version 1")
        lay = d["layout"]
        extra = {k: d[k] for k in cls._SCALARS if k in d}
        return cls(kernels={n: _decode(KernelSpec, v) for n, v in d["kernels"].items()},
                   buffers={n: _decode(BufferSpec, v) for n, v in d["buffers"].items()},
                   ops=[_decode(OpSpec, o) for o in d["ops"]],
                   layout=StepStateLayout(int(lay["t_max"]), int(lay["gamma_max"])), **extra)

    @classmethod
    def from_json(cls, text: str) -> "Program":
        return cls.from_dict(json.loads(text))

    def save(self, path) -> None:
        Path(path).write_text(self.to_json())

    @classmethod
    def load(cls, path) -> "Program":
        return cls.from_json(Path(path).read_text())
