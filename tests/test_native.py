"""The native runtime surface (``runtime/src/native.mm:13-95``): run-time compiled libraries, dispatches, queues,
ICB replay and file-backed buffers, after the reference's runtime tests (``tests/runtime/test_native.py`` style:
compile a small kernel, bind buffers and bytes, run, read back; errors surface as exceptions or ``RunResult.error``).

CPU tests: compiling needs no GPU (hiprtc), the argument packing is host logic. GPU tests run the kernels.
"""

import os
import struct

import numpy as np
import pytest

from monolith_mi355.runtime import hip, native

SRC = r"""
struct Params { float a; int n; };
extern "C" __global__ void axpy(float* y, const float* x, Params p) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < p.n) y[i] = p.a * x[i] + y[i] + BIAS;
}
extern "C" __global__ void block_sum(float* out, const float* x, int n) {
  extern __shared__ float part[];
  float s = 0.0f;
  for (int i = threadIdx.x; i < n; i += blockDim.x) s += x[i];
  part[threadIdx.x] = s;
  __syncthreads();
  if (threadIdx.x == 0) {
    float t = 0.0f;
    for (int i = 0; i < (int)blockDim.x; ++i) t += part[i];
    out[blockIdx.x] = t;
  }
}
"""


def test_compile_without_gpu():
    code = native.compile_source(SRC, {"BIAS": "0.0f"})
    assert len(code) > 1000
    assert code[:4] == b"\x7fELF" or code.startswith(b"__CLANG_OFFLOAD_BUNDLE__")


def test_compile_error_carries_the_log():
    with pytest.raises(hip.MiError) as e:
        native.compile_source("extern \"C\" __global__ void k() { undefined_name(); }")
    assert "undefined_name" in str(e.value)


def test_macros_reach_the_preprocessor():
    src = "#ifndef FLAG\n#error FLAG is missing\n#endif\nextern \"C\" __global__ void k(int* p) { p[0] = FLAG; }"
    native.compile_source(src, {"FLAG": "7"})
    with pytest.raises(hip.MiError, match="FLAG is missing"):
        native.compile_source(src)


class _FakeBuf:
    def __init__(self, addr, n):
        self.gpu_address, self.nbytes = addr, n


def test_kernarg_layout():
    """Slots in index order at their natural alignment: the HIP parameter list (ptr, ptr, struct{float,int})."""
    d = native.Dispatch()
    d.buffer(1, _FakeBuf(0x2000, 64), 16).buffer(0, _FakeBuf(0x1000, 64))
    d.bytes(2, struct.pack("<fi", 2.0, 5))
    raw = d.kernargs()
    assert len(raw) == 24
    assert struct.unpack_from("<QQfi", raw) == (0x1000, 0x2010, 2.0, 5)
    d2 = native.Dispatch().bytes(0, struct.pack("<i", 3)).bytes(1, struct.pack("<i", 4)).buffer(2, _FakeBuf(8, 8))
    raw2 = d2.kernargs()                                   # int, int, ptr → 0, 4, 8
    assert struct.unpack("<iiQ", raw2) == (3, 4, 8)
    d3 = native.Dispatch().bytes(0, b"\x01\x02").buffer(1, _FakeBuf(16, 8))   # short at 0, ptr at 8
    assert d3.kernargs() == b"\x01\x02" + b"\0" * 6 + (16).to_bytes(8, "little")


@pytest.mark.gpu
def test_library_dispatch_queue(torch_gpu):
    dev = native.Device(0)
    info = dev.info()
    assert info.arch.startswith("gfx950") and info.gpu_cores >= 256
    lib = native.Library(dev, SRC, {"BIAS": "0.5f"})
    axpy = native.Pipeline(lib, "axpy")
    assert axpy.thread_execution_width == 64 and axpy.max_threads_per_threadgroup >= 256
    with pytest.raises(hip.MiError, match="no kernel named nope"):
        native.Pipeline(lib, "nope")
    n = 1000
    rng = np.random.default_rng(3)
    x = rng.standard_normal(n).astype(np.float32)
    y0 = rng.standard_normal(n).astype(np.float32)
    bx, by = native.Buffer(dev, x.tobytes()), native.Buffer(dev, y0.tobytes())
    d = (native.Dispatch().pipeline(axpy).buffer(0, by).buffer(1, bx).bytes(2, struct.pack("<fi", 3.0, n))
         .grid((n + 255) // 256).threadgroup(256))
    q = native.Queue(dev)
    r = q.run([d])
    assert r.error == "" and r.gpu_ms > 0 and r.wall_ms >= r.gpu_ms * 0.5
    y = np.frombuffer(by.read(0, 4 * n), np.float32)
    want = ((3.0 * x.astype(np.float64) + y0).astype(np.float32) + np.float32(0.5))   # a·x + y contracts to an FMA
    np.testing.assert_allclose(y, want, rtol=0, atol=2e-6)
    # profile: one (start, end) pair per dispatch, in order
    prof = q.profile([d, d, d])
    assert len(prof) == 3 and all(e >= s for s, e in prof) and prof[1][0] >= prof[0][1] - 1e-3
    # dynamic LDS through threadgroup_memory
    bs = native.Pipeline(lib, "block_sum")
    out = native.Buffer(dev, 4)
    d2 = (native.Dispatch().pipeline(bs).buffer(0, out).buffer(1, bx).bytes(2, struct.pack("<i", n))
          .threadgroup_memory(0, 128 * 4).grid(1).threadgroup(128))
    assert q.run([d2]).error == ""
    got = struct.unpack("<f", out.read(0, 4))[0]
    assert abs(got - float(x.astype(np.float64).sum())) < 1e-3
    # an invalid launch comes back in RunResult.error, as the reference's command-buffer error
    bad = native.Dispatch().pipeline(axpy).grid(1).threadgroup(2048)
    assert "1024" in q.run([bad]).error


@pytest.mark.gpu
def test_icb_replay(torch_gpu):
    dev = native.Device(0)
    lib = native.Library(dev, SRC, {"BIAS": "0.0f"})
    axpy = native.Pipeline(lib, "axpy")
    n = 4096
    x = np.arange(n, dtype=np.float32)
    bx, by = native.Buffer(dev, x.tobytes()), native.Buffer(dev, n * 4)
    d = (native.Dispatch().pipeline(axpy).buffer(0, by).buffer(1, bx).bytes(2, struct.pack("<fi", 1.0, n))
         .grid(n // 256).threadgroup(256))
    icb = native.Icb(dev, [d, d])
    assert icb.count == 2
    for rep in range(1, 4):
        icb.launch()
        icb.synchronize()
        y = np.frombuffer(by.read(0, 4 * n), np.float32)
        np.testing.assert_array_equal(y, x * np.float32(2 * rep))


@pytest.mark.gpu
def test_buffer_from_file_and_bounds(torch_gpu, tmp_path):
    dev = native.Device(0)
    page = os.sysconf("SC_PAGESIZE")
    data = np.random.default_rng(5).integers(0, 256, 5 * page, dtype=np.uint8).tobytes()
    path = tmp_path / "weights.bin"
    path.write_bytes(data)
    b = native.Buffer.from_file(dev, str(path), page, 3 * page)
    assert b.nbytes == 3 * page and b.read(0, 3 * page) == data[page:4 * page]
    with pytest.raises(hip.MiError, match="page-aligned"):
        native.Buffer.from_file(dev, str(path), 100, page)
    with pytest.raises(hip.MiError, match="window ends"):
        native.Buffer.from_file(dev, str(path), 4 * page, 2 * page)
    with pytest.raises(IndexError):
        b.read(page, 3 * page)
    with pytest.raises(IndexError):
        b.write(b"x" * 8, 3 * page - 4)
    b.write(b"\x01\x02\x03", 10)
    assert b.read(9, 5) == data[page + 9:page + 10] + b"\x01\x02\x03" + data[page + 13:page + 14]
    b.fill(0xAB)
    assert b.read(0, 16) == b"\xab" * 16
    z = native.Buffer(dev, 64)
    assert z.read(0, 64) == b"\0" * 64 and z.read() == b""
