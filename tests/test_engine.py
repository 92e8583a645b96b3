"""The program format and the Engine, after the reference's toy-program gate (``tests/runtime/test_toy_program.py``):
a two-op self-advancing program replayed from one capture for 1,000 steps with tokens drained from the ring,
replay ≡ re-encode, early exit after ``done``, ring wrap and overflow, the JSON round trip, the pipeline cache,
per-op profiles and file-backed weights. The kernels are the toy's, written in HIP."""

import os
import struct

import numpy as np
import pytest

from monolith_mi355.runtime import hip
from monolith_mi355.runtime.program import BufferSpec, KernelSpec, OpSpec, Program, StepStateLayout

LAYOUT = StepStateLayout(t_max=8, gamma_max=7)
H = 4096

SRC = LAYOUT.to_hip() + r"""
struct Params { unsigned n_stop, ring_cap, width, pad; };
// op A (map): every element of h advances with the step; returns at once when the program is done
extern "C" __global__ void toy_map(float* h, const StepState* st, const Params* p) {
  if (st->done) return;
  const unsigned i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < p->width) h[i] = h[i] * 0.5f + float(st->step + 1);
}
// op B (serial, one thread): consume h[0], emit a token, advance the state, stop at n_stop
extern "C" __global__ void toy_serial(const float* h, StepState* st, const Params* p, unsigned long long* ring) {
  if (threadIdx.x != 0 || blockIdx.x != 0 || st->done) return;
  const unsigned s = st->step + 1, head = st->ring_head;
  if (head - st->ring_tail >= p->ring_cap) { st->error = 1; st->done = 1; return; }
  const int token = int(s * 7u) + (h[0] > 0.0f ? 0 : 1000000);
  ring[head % p->ring_cap] = ((unsigned long long)(head + 1u) << 32) | (unsigned)token;
  st->ring_head = head + 1u;
  st->step = s;
  st->position = st->position + 1;
  if (s >= p->n_stop) st->done = 1;
}
"""


def _program(n_stop: int, ring_cap: int = 256) -> Program:
    params = struct.pack("<IIII", n_stop, ring_cap, H, 0)
    return Program(
        kernels={"toy": KernelSpec(SRC, "toy_map"), "toy_serial": KernelSpec(SRC, "toy_serial")},
        buffers={"h": BufferSpec(H * 4, np.ones(H, np.float32).tobytes(), "arena"),
                 "step_state": BufferSpec(LAYOUT.size, LAYOUT.pack({}), "step_state"),
                 "params": BufferSpec(16, params, "params"),
                 "ring": BufferSpec(ring_cap * 8, None, "ring")},
        ops=[OpSpec("toy", [(0, "h", 0), (1, "step_state", 0), (2, "params", 0)], (H // 384 + 1, 1, 1), (384, 1, 1),
                    True, name="map"),
             OpSpec("toy_serial", [(0, "h", 0), (1, "step_state", 0), (2, "params", 0), (3, "ring", 0)], (1, 1, 1),
                    (64, 1, 1), True, name="advance")],
        ring_capacity=ring_cap, layout=LAYOUT)


def _expected_h(steps: int) -> float:
    h = 1.0
    for s in range(steps):
        h = h * 0.5 + (s + 1)
    return h


# ---- CPU -------------------------------------------------------------------------------------------------------
def test_layout_matches_the_c_abi_state():
    """mi_step_state is the layout at t_max = 16, gamma_max = 15: same offsets, same size."""
    lay = StepStateLayout(16, 15)
    assert lay.size == C_sizeof_state()
    for name, _ in hip.MiStepState._fields_:
        if name != "pad_":
            assert lay.offset(name) == getattr(hip.MiStepState, name).offset, name


def C_sizeof_state():
    import ctypes
    return ctypes.sizeof(hip.MiStepState)


def test_layout_reference_offsets_and_pack():
    """The reference's default layout (t_max 8, gamma_max 7): 8 pending tokens, 7 drafts / confidences."""
    lay = StepStateLayout()
    assert lay.offset("pending_tokens") == 16 and lay.offset("rng_lo") == 48 and lay.offset("draft_tokens") == 64
    assert lay.offset("confidence") == 92 and lay.offset("verify_len") == 120 and lay.offset("n_chain") == 164
    assert lay.size == 176
    v = {"step": 3, "pending_tokens": [5, -1], "confidence": [0.5], "done": 1}
    u = lay.unpack(lay.pack(v))
    assert u["step"] == 3 and u["pending_tokens"][:3] == [5, -1, 0] and u["confidence"][0] == 0.5 and u["done"] == 1
    with pytest.raises(ValueError):
        lay.pack({"pending_tokens": list(range(9))})
    with pytest.raises(ValueError):
        StepStateLayout(t_max=4, gamma_max=7)


def test_program_json_roundtrip(tmp_path):
    p = _program(5)
    p.save(tmp_path / "program.json")
    q = Program.load(tmp_path / "program.json")
    assert q.to_json() == p.to_json() and q.ops[1].name == "advance" and q.buffers["params"].init == p.buffers["params"].init
    with pytest.raises(ValueError, match="version"):
        Program.from_json('{"version": 2}')


def test_toy_sources_compile_without_gpu():
    from monolith_mi355.runtime import native
    assert len(native.compile_source(SRC)) > 1000


# ---- GPU -------------------------------------------------------------------------------------------------------
@pytest.mark.gpu
def test_replay_1000_steps_from_one_capture(torch_gpu):
    from monolith_mi355.runtime.engine import Engine
    eng = Engine(_program(n_stop=1000))
    rep = eng.run(1000, steps_per_cb=25, in_flight=3)
    assert rep.steps == 1000 and rep.done and rep.command_buffers == 40
    assert rep.tokens == [7 * s for s in range(1, 1001)]
    st = eng.state()
    assert st["step"] == 1000 and st["position"] == 1000 and st["ring_head"] == 1000
    h = np.frombuffer(eng.read("h"), dtype=np.float32)
    assert np.allclose(h, _expected_h(1000), rtol=1e-6)
    assert rep.host_fraction < 0.9
    print(f"\n1000 steps: gpu {rep.gpu_ms:.2f} ms, wall {rep.wall_ms:.2f} ms, host busy {rep.host_busy_ms:.2f} ms")


@pytest.mark.gpu
def test_reencode_matches_replay(torch_gpu):
    from monolith_mi355.runtime.engine import Engine
    a = Engine(_program(n_stop=300)); ra = a.run(300, steps_per_cb=10, in_flight=2, reencode=False)
    b = Engine(_program(n_stop=300)); rb = b.run(300, steps_per_cb=10, in_flight=2, reencode=True)
    sa, sb = a.state(), b.state()
    sa.pop("ring_tail"), sb.pop("ring_tail")      # host-written: the tail drained when the last batch was queued
    assert ra.tokens == rb.tokens == [7 * s for s in range(1, 301)] and sa == sb
    assert a.read("h") == b.read("h")


@pytest.mark.gpu
def test_early_exit_after_done_and_ring_wrap(torch_gpu):
    from monolith_mi355.runtime.engine import Engine
    eng = Engine(_program(n_stop=100, ring_cap=64))
    rep = eng.run(1000, steps_per_cb=4, in_flight=2)
    assert rep.done and rep.steps <= 100 + 4 * 2 and eng.state()["step"] == 100 and eng.state()["error"] == 0
    assert rep.tokens == [7 * s for s in range(1, 101)]
    h = np.frombuffer(eng.read("h"), dtype=np.float32)
    assert np.allclose(h, _expected_h(100), rtol=1e-6)


@pytest.mark.gpu
def test_pipeline_cache_survives_engine_replacement(torch_gpu):
    from monolith_mi355.runtime import native as nt
    from monolith_mi355.runtime.engine import Engine
    device, cache = nt.Device(), {}
    first = Engine(_program(2), device, pipeline_cache=cache)
    pipelines = dict(first.pipelines)
    assert first.run(2).tokens == [7, 14]
    del first
    second = Engine(_program(3), device, pipeline_cache=cache)
    assert all(second.pipelines[name] is p for name, p in pipelines.items())
    assert second.run(3).tokens == [7, 14, 21]
    assert len(cache) == 2
    changed = Engine(_program(1), device, fast_math=True, pipeline_cache=cache)
    assert all(changed.pipelines[name] is not p for name, p in pipelines.items())
    assert changed.run(1).tokens == [7] and len(cache) == 4


@pytest.mark.gpu
def test_ring_overflow_is_an_error_not_corruption(torch_gpu):
    from monolith_mi355.runtime.engine import Engine
    eng = Engine(_program(n_stop=1000, ring_cap=16))
    rep = eng.run(1000, steps_per_cb=25, in_flight=3)
    st = eng.state()
    assert st["error"] == 1 and st["done"] == 1
    assert rep.tokens == [7 * s for s in range(1, len(rep.tokens) + 1)] and len(rep.tokens) <= 16


@pytest.mark.gpu
def test_profile_gives_per_op_gpu_times(torch_gpu):
    from monolith_mi355.runtime.engine import Engine
    eng = Engine(_program(n_stop=50))
    eng.run(5, steps_per_cb=5, in_flight=1)
    runs = eng.profile(3)
    assert len(runs) == 3 and all(len(r) == 2 for r in runs)
    for (s0, e0), (s1, e1) in runs:
        assert 0 <= s0 <= e0 <= s1 + 1e-3 and s1 <= e1 and e1 - s0 < 5.0 and e0 > s0


@pytest.mark.gpu
def test_runner_reports_host_phases(torch_gpu):
    from monolith_mi355.runtime.engine import Engine
    eng = Engine(_program(n_stop=20))
    report = eng.run(20, steps_per_cb=5, in_flight=2)
    assert report.tokens == [7 * s for s in range(1, 21)]
    assert report.encode_ms >= 0 and report.wait_ms >= 0
    assert report.encode_ms + report.commit_ms + report.wait_ms <= report.wall_ms + 0.1


@pytest.mark.gpu
def test_file_weights_survive_engine_recreation(torch_gpu, tmp_path):
    from monolith_mi355.runtime.engine import Engine
    path = tmp_path / "weights.pack"
    page = os.sysconf("SC_PAGESIZE")
    values = np.arange(page // 4, dtype=np.uint32)
    path.write_bytes(bytes(page) + values.tobytes())
    source = r"""extern "C" __global__ void copy_weights(const unsigned* w, unsigned* out) {
      const unsigned i = blockIdx.x * blockDim.x + threadIdx.x; out[i] = w[i] + 7u; }"""
    program = _program(1)
    program.buffers["weights"] = BufferSpec(page, role="weights", file=str(path), file_offset=page)
    program.buffers["out"] = BufferSpec(page, role="arena")
    program.kernels["copy"] = KernelSpec(source, "copy_weights")
    program.ops = [OpSpec("copy", [(0, "weights", 0), (1, "out", 0)], (page // 4 // 128, 1, 1), (128, 1, 1), True)]
    for _ in range(2):
        engine = Engine(program)
        engine.run(1, steps_per_cb=1, in_flight=1)
        np.testing.assert_array_equal(np.frombuffer(engine.read("out"), dtype=np.uint32), values + 7)
        del engine
    assert path.read_bytes() == bytes(page) + values.tobytes()
