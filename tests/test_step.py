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


# ---- the speculative round's serial ops: the reference's known answers (tests/kernels/test_draft_ops.py:280-317,
#      378-420 and tests/kernels/test_eos_set.py:27-42) ----------------------------------------------------------------

DRAFTS, CONF = [11, 12, 13, 14, 15], [0.9, 0.6, 0.4, 0.8, 0.1]
SELECT_BASE = {"anchor": 7, "drafter_ctx_len": 10, "n_inject": 3, "t_this_step": 1}


def _select(base=SELECT_BASE, **kw):
    st = O.new_state(**base)
    O.verify_select(st, DRAFTS, CONF, gamma=5, **kw)
    return st


def test_verify_select_oracle_known_answers():
    s = _select(threshold=0.0)
    assert s["drafter_ctx_len"] == 13 and s["n_inject"] == 0 and s["gamma"] == 5 and s["verify_len"] == 5
    assert s["t_this_step"] == 6 and s["pending_tokens"][:8] == [7, 11, 12, 13, 14, 15, 0, 0]
    assert s["draft_tokens"][:5] == DRAFTS and s["confidence"][:5] == pytest.approx(CONF)
    s = _select(threshold=0.5)
    assert s["verify_len"] == 2 and s["t_this_step"] == 3 and s["pending_tokens"][:4] == [7, 11, 12, 0]
    s = _select(threshold=0.0, t_max=3)
    assert s["verify_len"] == 2 and s["t_this_step"] == 3
    s = _select(dict(SELECT_BASE, prefill_left=2, t_this_step=8, pending_tokens=[1, 2, 3, 4, 5, 6, 7, 8]))
    assert s["drafter_ctx_len"] == 13 and s["n_inject"] == 0 and s["t_this_step"] == 8
    assert s["pending_tokens"][:8] == [1, 2, 3, 4, 5, 6, 7, 8]
    s = _select(dict(SELECT_BASE, done=1))
    assert s["drafter_ctx_len"] == 10 and s["n_inject"] == 3
    cost = [1.0, 1.28, 1.535, 1.79, 2.67, 3.55, 4.4, 5.3]
    assert _select(mode=1, cost=cost)["verify_len"] == 2
    log = np.zeros((4, 16), np.float32)
    s = _select(dict(SELECT_BASE, step=6), threshold=2.0, mode=2, conf_log=log)
    assert s["verify_len"] == 2 and log[6 % 4, :5].tolist() == pytest.approx(CONF)
    assert _select(threshold=9.0, mode=2)["verify_len"] == 5 and _select(threshold=9.0, t_max=4, mode=2)["verify_len"] == 3
    at = dict(SELECT_BASE, position=10)
    s = _select(at, ctx_cap=13)
    assert s["verify_len"] == 2 and s["t_this_step"] == 3 and s["error"] == 0 and s["done"] == 0
    s = _select(at, ctx_cap=11)
    assert s["verify_len"] == 0 and s["t_this_step"] == 1 and s["error"] == 0
    s = _select(at, ctx_cap=10)
    assert s["error"] == 2 and s["done"] == 1 and s["t_this_step"] == 1
    assert _select(at, ctx_cap=64)["verify_len"] == 5


ACCEPT_BASE = dict(position=40, step=5, ring_head=3, ring_tail=1, anchor=9, t_this_step=4, verify_len=3,
                   pending_tokens=[9, 21, 22, 23])


def accept_case(case):
    """(state fields, tokens, eos, ctx_cap) of the reference's ``test_accept_scan`` cases; ring capacity 16."""
    st, tokens, eos, ctx_cap = dict(ACCEPT_BASE), [21, 22, 23, 24], [], 0
    if case == "context_full":
        ctx_cap = 44
    elif case == "context_room":
        ctx_cap = 45
    elif case == "partial":
        tokens = [21, 50, 23, 24]
    elif case == "none":
        tokens = [51, 22, 23, 24]
    elif case == "eos_draft":
        eos = [22]
    elif case == "eos_bonus":
        tokens, eos = [21, 50, 23, 24], [50]
    elif case == "first_token":
        st.update(t_this_step=3, verify_len=0, pending_tokens=[101, 102, 103], ring_head=0, ring_tail=0)
        tokens = [31, 32, 33]
    elif case == "overflow":
        st.update(ring_head=17, ring_tail=0)
    elif case == "wrap":
        st.update(ring_head=15, ring_tail=13)
    return st, tokens, eos, ctx_cap


ACCEPT_CASES = ["all", "partial", "none", "eos_draft", "eos_bonus", "first_token", "overflow", "wrap",
                "context_full", "context_room"]


@pytest.mark.parametrize("case", ACCEPT_CASES)
def test_accept_scan_oracle_known_answers(case):
    fields, tokens, eos, ctx_cap = accept_case(case)
    st, ring, log = O.new_state(**fields), np.zeros(16, np.uint64), np.zeros(64, np.uint32)
    O.accept_scan(st, tokens, ring, eos=eos, log=log, ctx_cap=ctx_cap)
    vals = [int(v) & 0xFFFFFFFF for v in ring if v]
    if case == "context_full":
        assert st["error"] == 2 and st["done"] == 1 and st["position"] == 44 and st["ring_head"] == 7 and len(vals) == 4
    if case == "context_room":
        assert st["error"] == 0 and st["done"] == 0 and st["position"] == 44
    if case == "all":
        assert st["accepted"] == 3 and st["position"] == 44 and st["anchor"] == 24 and st["n_inject"] == 4
        assert st["ring_head"] == 7 and log[5] == (4 << 16) | (3 << 8) | 3
    if case == "partial":
        assert st["accepted"] == 1 and st["position"] == 42 and st["anchor"] == 50 and st["n_inject"] == 2
        assert vals == [21, 50]
    if case == "eos_draft":
        assert st["done"] == 1 and st["ring_head"] == 5 and st["anchor"] == 22 and st["position"] == 42
    if case == "first_token":
        assert st["position"] == 43 and st["n_inject"] == 3 and st["anchor"] == 33 and st["ring_head"] == 1
        assert st["step"] == 6
    if case == "overflow":
        assert st["error"] == 1 and st["done"] == 1 and not vals
    if case == "wrap":                                   # slots 15 and 0 hold sequences 16 and 17
        assert int(ring[15]) >> 32 == 16 and int(ring[0]) >> 32 == 17 and st["ring_head"] == 19
    # a prefill chunk only advances and marks its rows for injection
    st = O.new_state(**dict(fields, prefill_left=2, t_this_step=4))
    O.accept_scan(st, tokens, np.zeros(16, np.uint64), eos=eos, log=log, ctx_cap=ctx_cap)
    assert st["position"] == fields["position"] + 4 and st["n_inject"] == 4 and st["n_chain"] == 0
    assert log[fields["step"] % 64] == (4 << 16) | 0xFFFF


@pytest.mark.parametrize("token,stops,done", [(2, [2, 9, 11], 1), (9, [2, 9, 11], 1), (7, [2, 9, 11], 0), (9, [], 0)])
def test_accept_scan_oracle_stop_tokens(token, stops, done):
    st = O.new_state(t_this_step=1, position=5)
    O.accept_scan(st, [token], np.zeros(16, np.uint64), eos=stops)
    assert st["done"] == done and st["ring_head"] == 1 and st["position"] == 6


def test_accept_scan_oracle_stops_after_the_first_eos():
    st = O.new_state(t_this_step=4, verify_len=3, position=5, pending_tokens=[1, 7, 9, 8])
    ring = np.zeros(16, np.uint64)
    O.accept_scan(st, [7, 9, 8, 12], ring, eos=[2, 9])
    assert st["done"] == 1 and st["ring_head"] == 2 and st["position"] == 7 and st["checkpoint_index"] == 2
    assert [int(v) & 0xFFFFFFFF for v in ring[:3]] == [7, 9, 0]


# ---- the sampler's oracle ----------------------------------------------------------------------------------------

def test_splitmix64_known_answers():
    """The published splitmix64 sequence for seed 0 (state advanced by the golden gamma before each mix)."""
    g = 0x9E3779B97F4A7C15
    assert O.splitmix64_mix(g) == 0xE220A8397B1DCDAF
    assert O.splitmix64_mix(2 * g & 0xFFFFFFFFFFFFFFFF) == 0x6E789E6AA1B965F4
    # the noise hashes seed + step·gamma + …: seed 0, step 1, row 0, index 0 is that first output
    u = ((0xE220A8397B1DCDAF >> 41) + 0.5) / 8388608.0
    assert O.gumbel_noise(0, 1, 0, [0])[0] == np.float32(-np.log(-np.log(np.float32(u))))


def _bf16_logits(rng, t, vocab, scale):
    from oracle.fp import rbf
    return rbf((rng.standard_normal((t, vocab)) * scale).astype(np.float32))


def test_thresholds_match_the_hf_warpers():
    """τ keeps exactly what the Hugging Face warpers keep (the reference's tests/kernels/test_sampling.py check)."""
    torch = pytest.importorskip("torch")
    tf = pytest.importorskip("transformers")
    rng = np.random.default_rng(3)
    lf = _bf16_logits(rng, 2, 4096, 3.0)
    cases = [(dict(top_k=25), tf.TopKLogitsWarper(25)), (dict(top_p=0.8), tf.TopPLogitsWarper(0.8)),
             (dict(min_p=0.1), tf.MinPLogitsWarper(0.1)),
             (dict(top_k=25, top_p=0.8, topp_in_topk=True),
              lambda ids, sc: tf.TopPLogitsWarper(0.8)(ids, tf.TopKLogitsWarper(25)(ids, sc)))]
    for opts, warper in cases:
        for i in range(2):
            tau = O.thresholds(lf[i], temperature=1.0, **opts)
            hf = warper(None, torch.from_numpy(lf[i:i + 1]).clone())[0].numpy()
            assert np.array_equal(np.isfinite(hf), lf[i] >= tau), (opts, i)


def test_sample_oracle_follows_the_warped_softmax():
    rng = np.random.default_rng(11)
    lf = np.full(512, -60.0, np.float32)
    lf[:16] = rng.standard_normal(16) * 1.5
    from oracle.fp import rbf
    lf = rbf(lf)
    n = 3000
    counts = np.zeros(512)
    for step in range(n):
        counts[O.sample(lf, seed=99, step=step, temperature=0.9)] += 1
    p = O.warped_probabilities(lf, temperature=0.9)
    sigma = np.sqrt(p * (1 - p) / n)
    assert np.all(np.abs(counts / n - p)[:16] <= 4 * sigma[:16] + 1e-9) and counts[16:].sum() == 0


def test_accept_scan_oracle_guards_an_inconsistent_state():
    """A verify length longer than the step (a state the host left stale) is read as the step allows: t = 1 means
    the anchor row alone, whatever verify_len says (this build's guard; the kernel then never indexes outside the
    step's rows)."""
    st = O.new_state(t_this_step=1, verify_len=7, position=10, pending_tokens=[3, 4, 5])
    ring = np.zeros(8, np.uint64)
    O.accept_scan(st, [42] + [0] * 15, ring)
    assert st["ring_head"] == 1 and int(ring[0]) & 0xFFFFFFFF == 42 and st["position"] == 11 and st["accepted"] == 0
