"""Element types of graph values (``monolith/core/dtypes.py``): the same members, short names and sizes, so a
value's byte size is computed the same way on both sides. Packed weight formats are not dtypes: a weight value
carries its format by name and the storage byte as its dtype."""

from __future__ import annotations

from enum import Enum


class DType(Enum):
    BF16 = ("bf16", 2)
    F16 = ("f16", 2)
    F32 = ("f32", 4)
    I32 = ("i32", 4)
    U32 = ("u32", 4)
    I64 = ("i64", 8)
    U8 = ("u8", 1)
    BOOL = ("bool", 1)

    def __init__(self, short: str, itemsize: int) -> None:
        self.short = short
        self.itemsize = itemsize

    @classmethod
    def parse(cls, name: str) -> "DType":
        key = name.lower()
        for d in cls:
            if key in (d.short, d.name.lower()):
                return d
        raise ValueError(f"unknown dtype {name!r}")

    def __str__(self) -> str:
        return self.short
