"""Checkpoint packing for the gfx950 kernels: safetensors input, format detection, the T16 weight pack with its
manifest, and the reader that uploads slabs."""

from .checkpoint import Group, group_tensors, logical_shape, storage_format
from .packer import ALIGN, Packer, PackFile, Segment
from .safetensors_io import Checkpoint, read_header, write

__all__ = ["ALIGN", "Checkpoint", "Group", "PackFile", "Packer", "Segment", "group_tensors", "logical_shape",
           "read_header", "storage_format", "write"]
