"""Runtime: the ctypes binding of ``libmi355.so`` (device, buffers, streams, events, graphs, kernels)."""

from . import hip  # noqa: F401
