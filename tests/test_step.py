"""CPU tests of the serial step ops' oracle and the step-state contract (the ``-m gpu`` twins are in
``test_step_gpu.py``)."""

import ctypes as C

import numpy as np
import pytest

from oracle import step as O

# the reference's StepStateLayout field order (core/step_state.py:38-63), counts at t_max = 16, gamma_max = 15
REFERENCE_FIELDS = [("step", 1), ("position", 1), ("kv_len", 1), ("t_this_step", 1), ("pending_tokens", 16),
                    ("rng_lo", 1), ("rng_hi", 1), ("anchor", 1), ("gamma", 1), ("draft_tokens", 15),
                    ("confidence", 15), ("verify_len", 1), ("accepted", 1), ("checkpoint_index", 1),
                    ("drafter_ctx_len", 1), ("done", 1), ("error", 1), ("ring_head", 1), ("ring_tail", 1),
                    ("prefill_left", 1), ("n_inject", 1), ("stop_at", 1), ("n_chain", 1)]


def test_step_state_layout_is_the_reference_order():
    from monolith_mi355.runtime import hip
    off = 0
    for name, count in REFERENCE_FIELDS:
        assert getattr(hip.MiStepState, name).offset == off, name
        off += 4 * count
    assert C.sizeof(hip.MiStepState) == (off + 15) // 16 * 16 == 272


def test_argmax_oracle_matches_numpy(rng):
    x = rng.standard_normal((6, 1000)).astype(np.float32)
    x[1, 5] = x[1, 7] = 50.0                        # tie: the lowest index
    x[2] = -np.abs(x[2]) - 1
    assert O.argmax(x).tolist() == np.argmax(x, axis=1).tolist()
    assert O.argmax(x)[1] == 5


def test_argmax_oracle_nan_and_inf_brute_force(rng):
    vals = np.array([np.nan, -np.inf, np.inf, 0.0, -1.0, 1.0], np.float32)
    for _ in range(500):
        row = rng.choice(vals, size=5)
        got = int(O.argmax(row[None])[0])
        if np.isnan(row).all():
            assert got == -1
        else:                                        # the largest (value, -index) pair among the numbers
            assert got == -max((float(v), -i) for i, v in enumerate(row) if not np.isnan(v))[1]


@pytest.mark.parametrize("token,stops,done", [(2, [2, 9, 11], 1), (9, [2, 9, 11], 1), (11, [2, 9, 11], 1),
                                              (7, [2, 9, 11], 0), (9, [], 0), (9, [-1], 0), (9, [9], 1)])
def test_advance_oracle_stop_tokens(token, stops, done):
    """The reference's ``tests/kernels/test_eos_set.py`` table."""
    st = O.new_state(t_this_step=1, position=5)
    ring = np.zeros(16, np.uint64)
    O.advance(st, [token], ring, eos=stops)
    assert st["done"] == done and st["ring_head"] == 1 and st["position"] == 6
    assert int(ring[0]) & 0xFFFFFFFF == token and int(ring[0]) >> 32 == 1


def _chain(tok, vocab):
    return (tok * 7 + 3) % vocab


def test_advance_oracle_ring_wrap_and_overflow():
    vocab, ring = 97, np.zeros(16, np.uint64)
    st, tail, got, tok = O.new_state(stop_at=100), 0, [], 1
    for s in range(1000):
        tok = _chain(tok, vocab)
        O.advance(st, [tok], ring)
        if s % 8 == 7:
            tail = O.drain(ring, tail, got)
            st["ring_tail"] = tail
    O.drain(ring, tail, got)
    want, t = [], 1
    for _ in range(100):
        t = _chain(t, vocab)
        want.append(t)
    assert got == want and st["step"] == 100 and st["done"] == 1 and st["error"] == 0
    # nobody drains: the 17th step overflows, nothing is corrupted
    ring = np.zeros(16, np.uint64)
    st, got = O.new_state(), []
    for s in range(40):
        O.advance(st, [s], ring)
    assert st["error"] == 1 and st["done"] == 1 and st["step"] == 16
    O.drain(ring, 0, got)
    assert got == list(range(16))


def test_advance_oracle_prefill_and_context():
    ring = np.zeros(4, np.uint64)
    st = O.new_state(t_this_step=8, position=0, prefill_left=1)
    O.advance(st, [0] * 8, ring)
    assert st["position"] == 8 and st["ring_head"] == 0 and not st["done"]
    st = O.new_state(position=9)
    O.advance(st, [3], ring, ctx_cap=10)
    assert st["error"] == 2 and st["done"] == 1 and st["ring_head"] == 1


def test_embed_oracle_out_of_range_reads_row_zero(rng):
    table = rng.standard_normal((5, 8)).astype(np.float32)
    h = O.embed(table, [3, -1, 5, 0])
    assert np.array_equal(h, table[[3, 0, 0, 0]])
