"""The GPU-resident token loop on the MI355X: ``embed`` / ``argmax`` / ``advance`` against the oracle, the native
pump over a captured step graph (the reference's ``tests/runtime/test_toy_program.py`` cases: many steps from one
capture, graph ≡ eager, early exit with ring wrap, overflow as an error), and a decoder with Gated DeltaNet and
attention layers whose replayed tokens equal a launch-by-launch host loop."""

import numpy as np
import pytest

from helpers import from_dev_bf16, to_dev_bf16
from oracle import step as O

pytestmark = pytest.mark.gpu


def _say(*a):
    print(*a, flush=True)


@pytest.mark.parametrize("vocab", [248320, 1000, 300])
@pytest.mark.parametrize("f32", [True, False])
def test_argmax(torch_gpu, vocab, f32):
    torch = torch_gpu
    from monolith_mi355 import kernels
    _say("argmax", vocab, f32)
    rng = np.random.default_rng(vocab)
    x = rng.standard_normal((5, vocab)).astype(np.float32) * 4
    x[0, vocab - 1] = 100.0
    x[1, 5] = x[1, 7] = 50.0
    x[2] = -np.abs(x[2]) - 1
    x[3, ::3] = np.nan
    x[3, 11] = 60.0
    x[4] = np.nan
    x[4, vocab // 2] = -np.inf
    if f32:
        logits = torch.from_numpy(x).cuda()
        ref = O.argmax(x)
    else:
        logits = to_dev_bf16(torch, x)
        ref = O.argmax(from_dev_bf16(logits))
    got = kernels.argmax(logits).cpu().numpy()
    assert got.tolist() == ref.tolist()
    assert got[1] == 5 and got[0] == vocab - 1 and got[3] == 11 and got[4] == vocab // 2


def test_argmax_all_nan_row(torch_gpu):
    torch = torch_gpu
    from monolith_mi355 import kernels
    x = torch.full((2, 300), float("nan"), device="cuda")
    x[1, 17] = 0.0
    assert kernels.argmax(x).cpu().tolist() == [-1, 17]


def test_argmax_repeated_calls_and_caller_workspace(torch_gpu):
    """The arrival counters return to zero: consecutive calls (rows, vocab and dtype varying) stay exact, also with
    a caller-owned zeroed workspace."""
    torch = torch_gpu
    import ctypes as C
    from monolith_mi355 import kernels
    from monolith_mi355.runtime import hip
    rng = np.random.default_rng(9)
    for i, (t, v) in enumerate([(1, 248320), (16, 70000), (3, 4097), (8, 248320), (1, 5)]):
        x = rng.standard_normal((t, v)).astype(np.float32)
        logits = torch.from_numpy(x).cuda() if i % 2 == 0 else to_dev_bf16(torch, x)
        ref = O.argmax(x if i % 2 == 0 else from_dev_bf16(logits))
        assert kernels.argmax(logits).cpu().numpy().tolist() == ref.tolist(), (t, v)
    x = torch.randn(4, 100000, device="cuda")
    ids = torch.empty(4, dtype=torch.int32, device="cuda")
    d = hip.MiArgmaxDesc(t=4, vocab=100000, logits=hip.ptr(x), ld=100000, f32=1, ids=hip.ptr(ids))
    need = hip.load().mi_argmax_workspace_bytes(C.byref(d))
    ws = torch.zeros(need, dtype=torch.uint8, device="cuda")
    d.workspace, d.workspace_bytes = hip.ptr(ws), need
    for _ in range(3):
        x.normal_()
        hip.call("mi_argmax", C.byref(d), hip.stream_handle(None))
        assert ids.cpu().tolist() == O.argmax(x.cpu().numpy()).tolist()
    assert int(ws[:64].view(torch.int32).abs().sum()) == 0          # counters back at zero
    d.workspace_bytes = need - 1
    with pytest.raises(hip.MiError):
        hip.call("mi_argmax", C.byref(d), hip.stream_handle(None))


def test_embed(torch_gpu):
    torch = torch_gpu
    from monolith_mi355 import kernels
    rng = np.random.default_rng(3)
    table = rng.standard_normal((1000, 5120)).astype(np.float32)
    tdev = to_dev_bf16(torch, table)
    ids = [999, -3, 1000, 0, 17, 512]
    out = kernels.embed(tdev, torch.tensor(ids, dtype=torch.int32, device="cuda"))
    assert np.array_equal(from_dev_bf16(out), O.embed(from_dev_bf16(tdev), ids))


def _advance_once(torch, state, token, **kw):
    """One advance over 16 token rows (``tokens[t_this_step - 1]`` is read), all holding ``token``."""
    from monolith_mi355 import kernels
    tokens = torch.full((16,), token, dtype=torch.int32, device="cuda")
    kernels.advance(state.buf, tokens, state.ring.addr, state.ring_capacity, host_ctl=state.ctl.addr, **kw)
    torch.cuda.synchronize()


@pytest.mark.parametrize("token,stops,done", [(2, [2, 9, 11], 1), (9, [2, 9, 11], 1), (11, [2, 9, 11], 1),
                                              (7, [2, 9, 11], 0), (9, [], 0), (9, [-1], 0), (9, [9], 1)])
def test_advance_stop_tokens(torch_gpu, token, stops, done):
    """The reference's ``tests/kernels/test_eos_set.py`` table, through the kernel."""
    from monolith_mi355.runtime.step import StepState
    st = StepState(ring_capacity=16)
    st.write(t_this_step=1, position=5)
    _advance_once(torch_gpu, st, token, eos=stops)
    got = st.read()
    assert got["done"] == done and got["ring_head"] == 1 and got["position"] == 6 and got["step"] == 1
    assert int(st.ring.array[0]) & 0xFFFFFFFF == token and int(st.ring.array[0]) >> 32 == 1
    assert got["pending_tokens"][0] == token and st.done == bool(done) and st.error == 0


def test_advance_matches_oracle_over_a_sequence(torch_gpu):
    """Prefill chunk, tokens, ring wrap with drains, stop_at, then context capacity: field by field."""
    torch = torch_gpu
    from monolith_mi355.runtime.step import StepState
    st = StepState(ring_capacity=8)
    st.write(t_this_step=4, position=0, prefill_left=1, stop_at=30)
    ref, ring_ref, tail_ref = O.new_state(t_this_step=4, position=0, prefill_left=1, stop_at=30), np.zeros(8, np.uint64), 0
    got_tokens, ref_tokens = [], []
    for s in range(40):
        if s == 1:
            st.write(prefill_left=0)
            ref["prefill_left"] = 0
        tok = (s * 37 + 5) % 101
        _advance_once(torch, st, tok, ctx_cap=64)
        O.advance(ref, [tok] * 16, ring_ref, ctx_cap=64)
        if s % 3 == 2:
            st.drain(got_tokens)
            st.write(ring_tail=int(st.ctl.array[0]))
            tail_ref = O.drain(ring_ref, tail_ref, ref_tokens)
            ref["ring_tail"] = tail_ref
        g = st.read()
        for k in ("step", "position", "t_this_step", "done", "error", "ring_head"):
            assert g[k] == ref[k], (s, k)
    st.drain(got_tokens)
    O.drain(ring_ref, tail_ref, ref_tokens)
    assert got_tokens == ref_tokens and len(got_tokens) == 30


def test_advance_context_capacity(torch_gpu):
    from monolith_mi355.runtime.step import StepState
    st = StepState(ring_capacity=4)
    st.write(t_this_step=1, position=9)
    _advance_once(torch_gpu, st, 3, ctx_cap=10)
    g = st.read()
    assert g["error"] == 2 and g["done"] == 1 and st.error == 2 and st.done


# ---- the pump over a captured graph: a toy program of this library's own ops --------------------------------------

class _ToyModel:
    """No layers; the embedding table's row v is one-hot at f(v) = (7·v + 3) mod V and the LM head is the identity,
    so the step maps token v to f(v) (the RMSNorm of a one-hot row keeps its argmax)."""

    def __init__(self, torch, vocab=256):
        from monolith_mi355 import kernels
        from monolith_mi355.formats import device as DV
        self.layers, self.eps = [], 1e-6
        t = torch.zeros(vocab, vocab, device="cuda")
        t[torch.arange(vocab), (torch.arange(vocab) * 7 + 3) % vocab] = 1.0
        self.embed_table = t.to(torch.bfloat16)
        self.norm_w = torch.ones(vocab, device="cuda")
        eye = torch.eye(vocab, device="cuda").to(torch.bfloat16)
        self.lm_head = kernels.PackedWeight("bf16", vocab, vocab, 1, DV.pack_bf16(eye), None)
        self.vocab = vocab

    def chain(self, tok, n):
        out = []
        for _ in range(n):
            tok = (tok * 7 + 3) % self.vocab
            out.append(tok)
        return out


def _toy_program(torch, *, ring=256, stop_at=0, steps_per_graph=2):
    from monolith_mi355.runtime.step import StepProgram, StepState
    model = _ToyModel(torch)
    st = StepState(ring_capacity=ring)
    prog = StepProgram(model, st, steps_per_graph=steps_per_graph)
    return model, st, prog


def test_pump_replays_1000_steps_from_one_capture(torch_gpu):
    torch = torch_gpu
    _say("pump 1000")
    model, st, prog = _toy_program(torch, stop_at=0)
    st.start(position=0, token=1, stop_at=1)
    prog.step_eager(1)                                   # grows the workspaces; emits one token
    st.start(position=0, token=1, stop_at=1000)
    prog.capture()
    rep = prog.run(1000, launches_per_batch=25, in_flight=3)
    assert rep.done and rep.error == 0 and rep.steps_submitted == 1000 and rep.batches == 20
    assert rep.tokens == model.chain(1, 1000)
    g = st.read()
    assert g["step"] == 1000 and g["position"] == 1000 and g["ring_head"] == 1000
    _say(f"1000 steps: gpu {rep.gpu_ms:.2f} ms wall {rep.wall_ms:.2f} ms host busy {rep.host_busy_ms:.2f} ms")


def test_pump_matches_eager(torch_gpu):
    torch = torch_gpu
    model, st, prog = _toy_program(torch)
    st.start(position=0, token=5)
    eager = prog.step_eager(60)
    st.start(position=0, token=5)
    rep = prog.run(60, launches_per_batch=5, in_flight=2)
    assert eager == rep.tokens == model.chain(5, 60)


def test_pump_early_exit_and_ring_wrap(torch_gpu):
    torch = torch_gpu
    model, st, prog = _toy_program(torch, ring=64)
    st.start(position=0, token=2)
    prog.step_eager(1)
    st.start(position=0, token=2, stop_at=100)
    rep = prog.run(1000, launches_per_batch=2, in_flight=2)
    g = st.read()
    assert rep.done and rep.steps_submitted <= 100 + 2 * 2 * 2 and g["step"] == 100 and g["error"] == 0
    assert rep.tokens == model.chain(2, 100)


def test_pump_ring_overflow_is_an_error_not_corruption(torch_gpu):
    torch = torch_gpu
    model, st, prog = _toy_program(torch, ring=16)
    st.start(position=0, token=3)
    prog.step_eager(1)
    st.start(position=0, token=3)
    rep = prog.run(1000, launches_per_batch=25, in_flight=3)     # 50 steps per batch: the GPU outruns the host
    g = st.read()
    assert g["error"] == 1 and g["done"] == 1 and rep.error == 1
    assert rep.tokens == model.chain(3, len(rep.tokens)) and len(rep.tokens) == 16


def test_pump_max_tokens(torch_gpu):
    torch = torch_gpu
    model, st, prog = _toy_program(torch)
    st.start(position=0, token=4)
    prog.step_eager(1)
    st.start(position=0, token=4)
    rep = prog.run(200, launches_per_batch=4, in_flight=1, max_tokens=20)
    assert 20 <= len(rep.tokens) < 40 and rep.tokens == model.chain(4, len(rep.tokens)) and not rep.done


# ---- a decoder: GDN + attention layers, graph replay ≡ a launch-by-launch host loop --------------------------------

def _decoder(torch, seed):
    from monolith_mi355.layers import AttnDecoderLayer, DecoderModel, GdnDecoderLayer
    hidden = 1024
    layers = [GdnDecoderLayer(hidden=hidden, k_heads=2, v_heads=4, inter=1024, seed=seed),
              AttnDecoderLayer(hidden=hidden, heads=4, kv_heads=1, ctx=256, inter=1024, seed=seed + 1)]
    gen = torch.Generator(device="cuda")
    gen.manual_seed(seed)
    layers[1].fill_cache(40, gen)
    return DecoderModel(layers, vocab=4096, hidden=hidden, seed=seed)


def test_decoder_program_matches_host_loop(torch_gpu):
    """Model A: host loop with int positions, the oracle's argmax of the BF16 logits. Model B (same seeds): two eager
    steps then graph replay through the pump. Same tokens; B's state matches A's step count and position."""
    torch = torch_gpu
    from monolith_mi355 import kernels
    from monolith_mi355.runtime.step import StepProgram, StepState
    _say("decoder program")
    steps = 24
    a = _decoder(torch, 11)
    tok, pos, host = 7, 40, []
    for _ in range(steps):
        h = kernels.embed(a.embed_table, torch.tensor([tok], dtype=torch.int32, device="cuda"))
        for layer in a.layers:
            h = layer.step(h, pos=pos)
        logits = kernels.gemv(a.lm_head, h, norm_w=a.norm_w, eps=a.eps)            # BF16, as the program's
        tok = int(O.argmax(from_dev_bf16(logits))[0])
        host.append(tok)
        pos += 1
    b = _decoder(torch, 11)
    st = StepState(ring_capacity=64)
    prog = StepProgram(b, st, ctx_cap=256, steps_per_graph=2)
    st.start(position=40, token=7)
    first = prog.step_eager(2)
    rep = prog.run(steps - 2, launches_per_batch=3, in_flight=2)
    assert first + rep.tokens == host
    g = st.read()
    assert g["step"] == steps and g["position"] == 40 + steps and g["error"] == 0


def test_decoder_program_stops_at_context_capacity(torch_gpu):
    torch = torch_gpu
    from monolith_mi355.runtime.step import StepProgram, StepState
    b = _decoder(torch, 5)
    st = StepState(ring_capacity=64)
    prog = StepProgram(b, st, ctx_cap=50, steps_per_graph=2)
    st.start(position=40, token=1)
    prog.step_eager(2)
    rep = prog.run(40, launches_per_batch=2, in_flight=2)
    g = st.read()
    assert g["error"] == 2 and g["done"] == 1 and g["position"] == 50 and len(rep.tokens) == 8


# ---- the speculative round's serial ops through the kernels, state compared field by field with the oracle ---------

from test_step import ACCEPT_CASES, CONF, DRAFTS, SELECT_BASE, accept_case  # noqa: E402


def _fresh(fields, ring=16):
    from monolith_mi355.runtime.step import StepState
    st = StepState(ring_capacity=ring)
    st.write(**O.new_state(**fields))
    return st


def _same_state(got, ref):
    for k, v in ref.items():
        g = got[k]
        if k == "confidence":
            assert np.array_equal(np.float32(g), np.float32(v)), k
        else:
            assert g == v, k


SELECT_CALLS = [(SELECT_BASE, dict(threshold=0.0)), (SELECT_BASE, dict(threshold=0.5)),
                (SELECT_BASE, dict(threshold=0.0, t_max=3)),
                (dict(SELECT_BASE, prefill_left=2, t_this_step=8, pending_tokens=[1, 2, 3, 4, 5, 6, 7, 8]), {}),
                (dict(SELECT_BASE, done=1), {}),
                (SELECT_BASE, dict(mode=1, cost=[1.0, 1.28, 1.535, 1.79, 2.67, 3.55, 4.4, 5.3])),
                (dict(SELECT_BASE, step=6), dict(threshold=2.0, mode=2, log=True)),
                (SELECT_BASE, dict(threshold=9.0, t_max=4, mode=2)),
                (dict(SELECT_BASE, position=10), dict(ctx_cap=13)), (dict(SELECT_BASE, position=10), dict(ctx_cap=10)),
                (dict(SELECT_BASE, position=30), dict(lm=True)),
                (dict(SELECT_BASE, position=30, prefill_left=1), dict(lm=True))]


@pytest.mark.parametrize("i", range(len(SELECT_CALLS)))
def test_verify_select_matches_oracle(torch_gpu, i):
    torch = torch_gpu
    from monolith_mi355 import kernels
    base, kw = SELECT_CALLS[i]
    kw = dict(kw)
    want_log = kw.pop("log", False)
    st = _fresh(base)
    log = torch.zeros(4, 16, dtype=torch.float32, device="cuda") if want_log else None
    kernels.verify_select(st.buf, torch.tensor(DRAFTS, dtype=torch.int32, device="cuda"),
                          torch.tensor(CONF, dtype=torch.float32, device="cuda"), gamma=5, conf_log=log, **kw)
    torch.cuda.synchronize()
    ref = O.new_state(**base)
    ref_log = np.zeros((4, 16), np.float32) if want_log else None
    O.verify_select(ref, DRAFTS, CONF, gamma=5, conf_log=ref_log, **kw)
    _same_state(st.read(), ref)
    if want_log:
        assert np.array_equal(log.cpu().numpy(), ref_log)


@pytest.mark.parametrize("case", ACCEPT_CASES + ["prefill", "stop_at", "lm"])
def test_accept_scan_matches_oracle(torch_gpu, case):
    torch = torch_gpu
    from monolith_mi355 import kernels
    fields, tokens, eos, ctx_cap = accept_case(case if case in ACCEPT_CASES else "all")
    lm = case == "lm"
    if case == "prefill":
        fields = dict(fields, prefill_left=2)
    if case == "stop_at":
        fields = dict(fields, stop_at=5)
    if lm:
        fields = dict(fields, drafter_ctx_len=41)
    st = _fresh(fields)
    log = torch.zeros(64, dtype=torch.int32, device="cuda")
    kernels.accept_scan(st.buf, torch.tensor(tokens, dtype=torch.int32, device="cuda"), st.ring.addr, 16, eos=eos,
                        log=log, ctx_cap=ctx_cap, lm=lm, host_ctl=st.ctl.addr)
    torch.cuda.synchronize()
    ref, ring, ref_log = O.new_state(**fields), np.zeros(16, np.uint64), np.zeros(64, np.uint32)
    O.accept_scan(ref, tokens, ring, eos=eos, log=ref_log, ctx_cap=ctx_cap, lm=lm)
    _same_state(st.read(), ref)
    assert np.array_equal(st.ring.array, ring) and np.array_equal(log.cpu().numpy().view(np.uint32), ref_log)
    assert st.done == bool(ref["done"]) and st.error == ref["error"]


# ---- stochastic sampling: draws equal to the oracle's (same hash, same thresholds) -------------------------------

SAMPLE_OPTS = [dict(temperature=1.0), dict(temperature=0.7, top_k=40), dict(temperature=1.0, top_p=0.9),
               dict(temperature=1.3, min_p=0.05), dict(temperature=0.8, top_k=50, top_p=0.95, min_p=0.02),
               dict(temperature=0.8, top_k=50, top_p=0.9, topp_in_topk=True)]


@pytest.mark.parametrize("vocab", [248320, 1000])
@pytest.mark.parametrize("oi", range(len(SAMPLE_OPTS)))
def test_sample_draws_equal_the_oracle(torch_gpu, vocab, oi):
    """The reference's tests/kernels/test_sampling.py case: three rows, steps 0, 1, 7; every token equals the host
    restatement's draw."""
    torch = torch_gpu
    from monolith_mi355 import kernels
    opts = SAMPLE_OPTS[oi]
    _say("sample", vocab, opts)
    rng = np.random.default_rng(vocab + len(opts))
    lb = to_dev_bf16(torch, (rng.standard_normal((3, vocab)) * 4.0).astype(np.float32))
    lf = from_dev_bf16(lb)
    for step in (0, 1, 7):
        tok = kernels.sample(lb, seed=12345, step=step, **opts).cpu().tolist()
        for i in range(3):
            assert tok[i] == O.sample(lf[i], seed=12345, step=step, t=i, **opts), (step, i)


def test_sample_distribution_determinism_and_device_seed(torch_gpu):
    torch = torch_gpu
    from monolith_mi355 import kernels
    from monolith_mi355.runtime.step import StepState
    from oracle.fp import rbf
    rng = np.random.default_rng(11)
    lf = np.full(512, -60.0, np.float32)
    lf[:16] = rng.standard_normal(16) * 1.5
    lf = rbf(lf)
    lb = to_dev_bf16(torch, lf[None, :])
    n = 2000
    counts = np.zeros(512)
    out = torch.empty(1, dtype=torch.int32, device="cuda")
    for step in range(n):
        kernels.sample(lb, seed=99, step=step, temperature=0.9, out=out)
        counts[int(out.item())] += 1
    p = O.warped_probabilities(lf, temperature=0.9)
    sigma = np.sqrt(p * (1 - p) / n)
    assert np.all(np.abs(counts / n - p)[:16] <= 4 * sigma[:16] + 1e-9) and counts[16:].sum() == 0
    a = kernels.sample(lb, seed=99, step=5, temperature=0.9).item()
    assert a == kernels.sample(lb, seed=99, step=5, temperature=0.9).item() == O.sample(lf, seed=99, step=5,
                                                                                           temperature=0.9)
    # seed and step from a step state, read on the device
    st = StepState(ring_capacity=4)
    seed = 0x0123456789ABCDEF
    st.write(rng_lo=seed & 0xFFFFFFFF, rng_hi=seed >> 32, step=17)
    lb3 = to_dev_bf16(torch, (rng.standard_normal((3, 5000)) * 3).astype(np.float32))
    got = kernels.sample(lb3, state=st.buf, temperature=1.1, top_k=100).cpu().tolist()
    l3 = from_dev_bf16(lb3)
    assert got == [O.sample(l3[i], seed=seed, step=17, t=i, temperature=1.1, top_k=100) for i in range(3)]


def test_decoder_program_sampling_matches_host_loop(torch_gpu):
    """The program with a sampler: the host loop draws each token with the oracle from the same BF16 logits, seed
    and step; the replayed program (seed in the state's rng words, step from the state) draws the same tokens."""
    torch = torch_gpu
    from monolith_mi355 import kernels
    from monolith_mi355.runtime.step import StepProgram, StepState
    steps, seed = 12, 0xFEEDFACE12345
    opts = dict(temperature=0.9, top_k=64, top_p=0.95)
    a = _decoder(torch, 21)
    tok, pos, host = 3, 40, []
    for s in range(steps):
        h = kernels.embed(a.embed_table, torch.tensor([tok], dtype=torch.int32, device="cuda"))
        for layer in a.layers:
            h = layer.step(h, pos=pos)
        logits = from_dev_bf16(kernels.gemv(a.lm_head, h, norm_w=a.norm_w, eps=a.eps))
        tok = O.sample(logits[0], seed=seed, step=s, t=0, **opts)
        host.append(tok)
        pos += 1
    b = _decoder(torch, 21)
    st = StepState(ring_capacity=64)
    prog = StepProgram(b, st, ctx_cap=256, steps_per_graph=2, sampling=opts)
    st.start(position=40, token=3)
    st.write(rng_lo=seed & 0xFFFFFFFF, rng_hi=seed >> 32)
    first = prog.step_eager(2)
    rep = prog.run(steps - 2, launches_per_batch=2, in_flight=2)
    assert first + rep.tokens == host


# ---- the speculative round: graph replay of verify → accept → commit → select ------------------------------------

def _spec_run(torch, table, steps, *, eager_steps=2, ctx_cap=240):
    from monolith_mi355.runtime.step import SpecProgram, StepState
    model = _decoder(torch, 31)
    st = StepState(ring_capacity=512)
    prog = SpecProgram(model, st, gamma=7, draft_table=table, ctx_cap=ctx_cap, steps_per_graph=2)
    st.start(position=40, token=9)
    first = prog.step_eager(eager_steps)
    rep = prog.run(steps - eager_steps, launches_per_batch=2, in_flight=2)
    return first + rep.tokens, st.read(), prog


def test_spec_program_accepted_drafts_change_nothing_but_the_step_count(torch_gpu):
    """Run A: random drafts (all but never accepted) — one token per step. Run B: the drafts are A's own tokens —
    up to eight per step. Every row of the verify pass computes exactly what a one-token step computes at that
    position (GEMV, recurrence, cache appends and attention are per-row), so B's tokens are A's, in far fewer
    steps; the committed state (position, ring) follows the tokens."""
    torch = torch_gpu
    _say("spec program")
    rng = np.random.default_rng(5)
    ctx = 256
    rand = torch.from_numpy(rng.integers(0, 4096, size=(ctx, 7), dtype=np.int32)).cuda()
    a, st_a, _ = _spec_run(torch, rand, 40)
    assert len(a) >= 40 and st_a["error"] == 0
    seq = [9] + a                                            # the token at position 40 + i
    perfect = np.zeros((ctx, 7), np.int32)
    for p in range(40, ctx):
        for j in range(7):
            i = p - 40 + 1 + j
            perfect[p, j] = seq[i] if i < len(seq) else 0
    b, st_b, prog = _spec_run(torch, torch.from_numpy(perfect).cuda(), 8)
    assert len(b) >= 40 and b[:40] == a[:40], (a, b)
    assert st_b["step"] == 8 and st_b["position"] == 40 + len(b) and st_b["ring_head"] == len(b)
    log = [((e >> 16), (e >> 8) & 0xFF, e & 0xFF) for e in prog.acceptance()[:8]]
    assert log[0] == (1, 0, 0) and all(x == (8, 7, 7) for x in log[1:5]), log   # whole blocks accepted


def test_start_resets_the_speculative_fields_and_the_scan_guards_a_stale_state(torch_gpu):
    """Regression: a program restarted with StepState.start after speculative steps kept verify_len, and the accept
    scan then indexed rows below the step. start() clears every speculative field; the scan also keeps L <= t - 1."""
    torch = torch_gpu
    from monolith_mi355 import kernels
    from monolith_mi355.runtime.step import StepState
    st = StepState(ring_capacity=8)
    st.write(t_this_step=8, verify_len=7, accepted=5, checkpoint_index=6, n_inject=6, gamma=7,
             draft_tokens=[1] * 15, confidence=[0.5] * 15, drafter_ctx_len=3, n_chain=1)
    st.start(position=10, token=3)
    g = st.read()
    for k in ("verify_len", "accepted", "checkpoint_index", "n_inject", "gamma", "drafter_ctx_len", "n_chain"):
        assert g[k] == 0, k
    assert g["draft_tokens"] == [0] * 15 and g["confidence"] == [0.0] * 15 and g["t_this_step"] == 1
    st.write(verify_len=7)                                   # stale, as before the fix
    ids = torch.full((16,), 42, dtype=torch.int32, device="cuda")
    kernels.accept_scan(st.buf, ids, st.ring.addr, 8, host_ctl=st.ctl.addr)
    torch.cuda.synchronize()
    g = st.read()
    assert g["ring_head"] == 1 and g["position"] == 11 and g["accepted"] == 0
    assert int(st.ring.array[0]) & 0xFFFFFFFF == 42


def test_decoder_program_stop_inside_a_graph_leaves_the_state_of_the_emitted_steps(torch_gpu):
    """stop_at = 5 with four steps per graph: the stop falls on the first step of the second launch's pair, so the
    steps queued after it in the same graph still run. They must take no token: the Gated DeltaNet recurrent and conv
    state and the attention KV cache equal those of a host loop over exactly the five emitted steps (bit for bit),
    and nothing is appended at the sixth position."""
    torch = torch_gpu
    from monolith_mi355 import kernels
    from monolith_mi355.runtime.step import StepProgram, StepState
    _say("decoder program: stop inside a graph")
    emitted = 5
    a = _decoder(torch, 13)
    tok, pos, host = 7, 40, []
    for _ in range(emitted):
        h = kernels.embed(a.embed_table, torch.tensor([tok], dtype=torch.int32, device="cuda"))
        for layer in a.layers:
            h = layer.step(h, pos=pos)
        logits = kernels.gemv(a.lm_head, h, norm_w=a.norm_w, eps=a.eps)
        tok = int(O.argmax(from_dev_bf16(logits))[0])
        host.append(tok)
        pos += 1
    b = _decoder(torch, 13)
    st = StepState(ring_capacity=64)
    prog = StepProgram(b, st, ctx_cap=256, steps_per_graph=4)
    st.start(position=40, token=7, stop_at=emitted)
    first = prog.step_eager(2)                     # steps 1, 2 eagerly; then graphs of steps 3-6 and 7-10
    rep = prog.run(8, launches_per_batch=1, in_flight=1)
    torch.cuda.synchronize()
    assert first + rep.tokens == host and rep.done
    g = st.read()
    assert g["step"] == emitted and g["position"] == 40 + emitted and g["done"] == 1
    ga, gb = a.layers[0], b.layers[0]
    assert torch.equal(ga.rec, gb.rec), "GDN recurrent state moved after the stop"
    assert torch.equal(ga.conv_state[ga.parity], gb.conv_state[gb.parity]), "GDN conv state moved after the stop"
    ca, cb = a.layers[1].cache, b.layers[1].cache
    for name in ("k_codes", "v_codes", "k_scales", "v_scales"):
        assert torch.equal(getattr(ca, name), getattr(cb, name)), f"KV cache {name} differs after the stop"
    assert int(cb.k_scales[:, 40 + emitted].abs().sum()) == 0
