"""``program.json`` and ``Engine`` on a program small enough to predict exactly on the host.

The program ("mixer"): a map op stirs an integer vector with the step counter (``x[i] = 5·x[i] + step + i``, mod
2^32), then a one-thread op reads two of its words, emits their digest as the step's token into the ring (tagged with
its 1-based sequence number), advances the step state and sets ``done`` after ``stop`` steps; both ops return at once
once ``done`` is set, and the emit op turns a full ring (the host's tail not keeping up) into ``error = 1``. Integer
arithmetic makes every step's token and the final vector exact, so the checks are equalities.

Acceptance criteria (the reference's runtime gate, ``tests/runtime/test_toy_program.py``, in this file's own
harness): 1,000 steps replayed from one capture with every token drained in order; graph replay and op-by-op
re-encoding agree bit for bit; submission stops early once ``done`` is set; the ring wraps; an overrun is an error,
never a corrupted token; the JSON round trip; compiled kernels reused across engines; per-op GPU times; weights read
from a file window.
"""

import os
import struct

import numpy as np
import pytest

from monolith_mi355.runtime import hip
from monolith_mi355.runtime.program import BufferSpec, KernelSpec, OpSpec, Program, StepStateLayout

LAYOUT = StepStateLayout(t_max=8, gamma_max=7)
N = 4096
MASK = np.uint64(0xFFFFFFFF)

MIXER = LAYOUT.to_hip() + r"""
struct Knobs { unsigned stop, ring_slots, n, unused; };
extern "C" __global__ void mixer_stir(unsigned* x, const StepState* st, const Knobs* k) {
  if (st->done) return;
  const unsigned i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < k->n) x[i] = x[i] * 5u + st->step + i;
}
extern "C" __global__ void mixer_emit(const unsigned* x, StepState* st, const Knobs* k, unsigned long long* ring) {
  if (threadIdx.x != 0 || blockIdx.x != 0 || st->done) return;
  const unsigned head = st->ring_head;
  if (head - st->ring_tail >= k->ring_slots) { st->error = 1u; st->done = 1u; return; }
  const unsigned token = (x[0] ^ (x[k->n - 1] >> 7)) & 0xFFFFFu;
  ring[head % k->ring_slots] = ((unsigned long long)(head + 1u) << 32) | token;
  st->ring_head = head + 1u;
  st->step += 1u;
  st->position += 1u;
  if (st->step >= k->stop) st->done = 1u;
}
"""


def mixer(stop: int, ring_slots: int = 256) -> Program:
    """The two-op program, its vector starting at ``x[i] = 2654435761·i`` (mod 2^32)."""
    x0 = (np.arange(N, dtype=np.uint64) * np.uint64(2654435761) & MASK).astype(np.uint32)
    return Program(
        kernels={"stir": KernelSpec(MIXER, "mixer_stir"), "emit": KernelSpec(MIXER, "mixer_emit")},
        buffers={"x": BufferSpec(N * 4, x0.tobytes(), "arena"),
                 "step_state": BufferSpec(LAYOUT.size, LAYOUT.pack({}), "step_state"),
                 "knobs": BufferSpec(16, struct.pack("<IIII", stop, ring_slots, N, 0), "params"),
                 "ring": BufferSpec(ring_slots * 8, None, "ring")},
        ops=[OpSpec("stir", [(0, "x", 0), (1, "step_state", 0), (2, "knobs", 0)], (N // 256, 1, 1), (256, 1, 1),
                    True, name="stir"),
             OpSpec("emit", [(0, "x", 0), (1, "step_state", 0), (2, "knobs", 0), (3, "ring", 0)], (1, 1, 1),
                    (64, 1, 1), True, name="emit")],
        ring_capacity=ring_slots, layout=LAYOUT)


def predicted(steps: int):
    """(tokens, final vector) of ``steps`` steps, computed on the host in uint64 and reduced mod 2^32."""
    i = np.arange(N, dtype=np.uint64)
    x = (i * np.uint64(2654435761)) & MASK
    tokens = []
    for s in range(steps):
        x = (x * np.uint64(5) + np.uint64(s) + i) & MASK
        tokens.append(int((x[0] ^ (x[N - 1] >> np.uint64(7))) & np.uint64(0xFFFFF)))
    return tokens, x.astype(np.uint32)


# ---- CPU -------------------------------------------------------------------------------------------------------
def test_c_abi_state_is_the_layout_at_16_and_15():
    import ctypes
    lay = StepStateLayout(16, 15)
    assert lay.size == ctypes.sizeof(hip.MiStepState)
    for name, _ in hip.MiStepState._fields_:
        if name != "pad_":
            assert lay.offset(name) == getattr(hip.MiStepState, name).offset, name


def test_default_layout_offsets_and_packing():
    """t_max 8 / gamma_max 7: 8 pending tokens, 7 drafts and confidences, 176 bytes; pack / unpack invert."""
    lay = StepStateLayout()
    assert (lay.offset("pending_tokens"), lay.offset("rng_lo"), lay.offset("draft_tokens")) == (16, 48, 64)
    assert (lay.offset("confidence"), lay.offset("verify_len"), lay.offset("n_chain"), lay.size) == (92, 120, 164, 176)
    fields = {"step": 9, "pending_tokens": [4, -2], "confidence": [0.25], "error": 2}
    back = lay.unpack(lay.pack(fields))
    assert back["step"] == 9 and back["pending_tokens"][:3] == [4, -2, 0] and back["confidence"][0] == 0.25
    assert back["error"] == 2
    with pytest.raises(ValueError):
        lay.pack({"pending_tokens": list(range(9))})
    with pytest.raises(ValueError):
        StepStateLayout(t_max=4, gamma_max=7)


def test_json_round_trip(tmp_path):
    p = mixer(5)
    p.save(tmp_path / "program.json")
    q = Program.load(tmp_path / "program.json")
    assert q.to_json() == p.to_json()
    assert [o.name for o in q.ops] == ["stir", "emit"] and q.buffers["x"].init == p.buffers["x"].init
    with pytest.raises(ValueError, match="version"):
        Program.from_json('{"version": 2}')


def test_mixer_compiles_without_a_gpu():
    from monolith_mi355.runtime import native
    assert len(native.compile_source(MIXER)) > 1000


def test_host_prediction_is_self_consistent():
    a, xa = predicted(10)
    b, xb = predicted(11)
    assert a == b[:10] and len(set(b)) > 5 and not np.array_equal(xa, xb)


# ---- GPU -------------------------------------------------------------------------------------------------------
def _run(stop, steps, ring_slots=256, **kw):
    from monolith_mi355.runtime.engine import Engine
    eng = Engine(mixer(stop, ring_slots))
    return eng, eng.run(steps, **kw)


@pytest.mark.gpu
def test_thousand_steps_from_one_capture(torch_gpu):
    eng, rep = _run(1000, 1000, steps_per_cb=25, in_flight=3)
    tokens, x = predicted(1000)
    assert rep.steps == 1000 and rep.done and rep.command_buffers == 40
    assert rep.tokens == tokens
    st = eng.state()
    assert (st["step"], st["position"], st["ring_head"]) == (1000, 1000, 1000)
    assert np.array_equal(np.frombuffer(eng.read("x"), np.uint32), x)
    assert rep.host_fraction < 0.9
    print(f"\n1000 steps: gpu {rep.gpu_ms:.2f} ms, wall {rep.wall_ms:.2f} ms, host busy {rep.host_busy_ms:.2f} ms")


@pytest.mark.gpu
def test_graph_replay_equals_op_by_op(torch_gpu):
    a, ra = _run(300, 300, steps_per_cb=10, in_flight=2)
    b, rb = _run(300, 300, steps_per_cb=10, in_flight=2, reencode=True)
    sa, sb = a.state(), b.state()
    sa.pop("ring_tail"), sb.pop("ring_tail")      # host-written: where the drain stood when the last batch was queued
    assert ra.tokens == rb.tokens == predicted(300)[0] and sa == sb
    assert a.read("x") == b.read("x")


@pytest.mark.gpu
def test_stops_at_done_and_wraps_the_ring(torch_gpu):
    eng, rep = _run(100, 1000, ring_slots=64, steps_per_cb=4, in_flight=2)
    st = eng.state()
    assert rep.done and rep.steps <= 100 + 4 * 2 and st["step"] == 100 and st["error"] == 0
    tokens, x = predicted(100)
    assert rep.tokens == tokens
    assert np.array_equal(np.frombuffer(eng.read("x"), np.uint32), x)    # the steps past done changed nothing


@pytest.mark.gpu
def test_ring_overrun_is_an_error(torch_gpu):
    """A ring of 16 slots drained only between batches of 25 steps: the emit op refuses to overwrite an undrained
    slot, flags error 1 and stops; every token that arrived is the right one, in order."""
    eng, rep = _run(1000, 1000, ring_slots=16, steps_per_cb=25, in_flight=3)
    st = eng.state()
    assert st["error"] == 1 and st["done"] == 1
    assert 0 < len(rep.tokens) <= 16 and rep.tokens == predicted(len(rep.tokens))[0]


@pytest.mark.gpu
def test_compiled_kernels_are_shared_through_the_cache(torch_gpu):
    from monolith_mi355.runtime import native as nt
    from monolith_mi355.runtime.engine import Engine
    device, cache = nt.Device(), {}
    first = Engine(mixer(2), device, pipeline_cache=cache)
    kept = dict(first.pipelines)
    assert first.run(2).tokens == predicted(2)[0]
    del first
    second = Engine(mixer(3), device, pipeline_cache=cache)
    assert all(second.pipelines[name] is p for name, p in kept.items())
    assert second.run(3).tokens == predicted(3)[0] and len(cache) == 2
    fast = Engine(mixer(1), device, fast_math=True, pipeline_cache=cache)     # other options: compiled anew
    assert all(fast.pipelines[name] is not p for name, p in kept.items())
    assert fast.run(1).tokens == predicted(1)[0] and len(cache) == 4


@pytest.mark.gpu
def test_per_op_gpu_times(torch_gpu):
    from monolith_mi355.runtime.engine import Engine
    eng = Engine(mixer(50))
    eng.run(5, steps_per_cb=5, in_flight=1)
    runs = eng.profile(3)
    assert len(runs) == 3 and all(len(r) == 2 for r in runs)
    for (s0, e0), (s1, e1) in runs:                # stir, then emit, in order, each a positive span
        assert 0 <= s0 < e0 <= s1 + 1e-3 and s1 <= e1 and e1 - s0 < 5.0


@pytest.mark.gpu
def test_runner_host_phases_add_up(torch_gpu):
    _, rep = _run(20, 20, steps_per_cb=5, in_flight=2)
    assert rep.tokens == predicted(20)[0]
    assert rep.encode_ms >= 0 and rep.wait_ms >= 0
    assert rep.encode_ms + rep.commit_ms + rep.wait_ms <= rep.wall_ms + 0.1


@pytest.mark.gpu
def test_weights_from_a_file_window(torch_gpu, tmp_path):
    """A weights buffer mapped from page 1 of a file (page 0 is zeros): a kernel reads it, a second engine reads it
    again, the file is never written."""
    from monolith_mi355.runtime.engine import Engine
    page = os.sysconf("SC_PAGESIZE")
    words = (np.arange(page // 4, dtype=np.uint32) * np.uint32(40503)) ^ np.uint32(0x5A5A5A5A)
    path = tmp_path / "weights.pack"
    path.write_bytes(bytes(page) + words.tobytes())
    src = r"""extern "C" __global__ void xor_in(const unsigned* w, unsigned* out) {
      const unsigned i = blockIdx.x * blockDim.x + threadIdx.x; out[i] = w[i] ^ 0xFFu; }"""
    p = mixer(1)
    p.buffers["w"] = BufferSpec(page, role="weights", file=str(path), file_offset=page)
    p.buffers["out"] = BufferSpec(page, role="arena")
    p.kernels["xor"] = KernelSpec(src, "xor_in")
    p.ops = [OpSpec("xor", [(0, "w", 0), (1, "out", 0)], (page // 4 // 64, 1, 1), (64, 1, 1), True)]
    for _ in range(2):
        eng = Engine(p)
        eng.run(1, steps_per_cb=1, in_flight=1)
        assert np.array_equal(np.frombuffer(eng.read("out"), np.uint32), words ^ np.uint32(0xFF))
        del eng
    assert path.read_bytes() == bytes(page) + words.tobytes()
