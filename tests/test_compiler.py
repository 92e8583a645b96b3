"""The compiler side of the operator API for gfx950: backend selection by profile, the handler table, emission of a
decode step (GDN + attention layers, LM head, argmax, advance) into program.json, and — on the GPU — that program
replayed by Engine gives the tokens and states of the hand-built StepProgram on a twin model, bit for bit."""

import numpy as np
import pytest


def _decoder(torch, seed, device):
    from monolith_mi355.layers import AttnDecoderLayer, DecoderModel, GdnDecoderLayer
    hidden = 1024
    layers = [GdnDecoderLayer(hidden=hidden, k_heads=2, v_heads=4, inter=1024, seed=seed, device=device),
              AttnDecoderLayer(hidden=hidden, heads=4, kv_heads=1, ctx=256, inter=1024, seed=seed + 1, device=device)]
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    layers[1].fill_cache(40, gen)
    return DecoderModel(layers, vocab=4096, hidden=hidden, seed=seed, device=device)


def _entries(program):
    return [program.kernels[o.kernel].function for o in program.ops]


def test_emit_decode_step_program():
    import torch
    from monolith_mi355.compiler import Profile, compile_program
    from monolith_mi355.runtime.program import Program
    model = _decoder(torch, 3, "cpu")
    prof = Profile(ring_capacity=64, ctx_cap=256, eos=(2,))
    p = compile_program(model, prof)
    assert p.backend_id == "gfx950" and p.config_digest == prof.fingerprint
    names = [o.name for o in p.ops]
    assert names[0] == "embed" and names[-3:] == ["lm_head", "argmax", "advance"]
    assert names[1:6] == ["layers.0.in_proj", "layers.0.gdn", "layers.0.out_proj", "layers.0.mlp.gate_up",
                          "layers.0.mlp.down"]
    assert names[6:11] == ["layers.1.qkv", "layers.1.gqa", "layers.1.o_proj", "layers.1.mlp.gate_up",
                           "layers.1.mlp.down"]
    assert set(_entries(p)) == {"lib:mi_embed", "lib:mi_gemv", "lib:mi_gdn_step", "lib:mi_gqa_decode",
                                "lib:mi_argmax", "lib:mi_advance"}
    # the step state feeds the device-side fields: the GDN parity and stop flag, attention's position
    from monolith_mi355.runtime import hip
    gdn = p.ops[2]
    fields = {[f for f, _ in hip.MiGdnDesc._fields_][i]: (b, off) for i, b, off in gdn.bindings}
    assert fields["step"] == ("step_state", p.layout.offset("step"))
    assert fields["done"] == ("step_state", p.layout.offset("done"))
    gqa = p.ops[7]
    gf = {[f for f, _ in hip.MiGqaDesc._fields_][i]: (b, off) for i, b, off in gqa.bindings}
    assert gf["pos_dev"] == ("step_state", p.layout.offset("position")) and gqa.meta["desc"]["workspace_bytes"] > 0
    # the out_proj's gated norm reads z inside the projection output: same buffer, the projection's row stride
    op = p.ops[3]
    of = {[f for f, _ in hip.MiGemvDesc._fields_][i]: (b, off) for i, b, off in op.bindings}
    assert of["gnorm_z"][0] == dict((f, v) for f, v in ((([f for f, _ in hip.MiGemvDesc._fields_][i]), b)
                                                        for i, b, _ in p.ops[1].bindings))["y"]
    assert op.meta["desc"]["ld_gnorm_z"] == model.layers[0].n_proj
    # the model's own tensors are bound, not copied
    assert len(p.bound_tensors) > 10 and all(p.buffers[n].role in ("weights", "state") for n in p.bound_tensors)
    q = Program.from_json(p.to_json())
    assert q.to_json() == p.to_json()


def test_backend_selection_and_coverage():
    from monolith_mi355.compiler import Graph, Profile, Value, emit_program, get_backend, register_backend
    from monolith_mi355.compiler.context import Gfx950Backend
    from monolith_mi355.ops import CoverageError
    g = Graph()
    x = Value("x", (1, 256), "bf16")
    g.add("no_such_op", [x], [x])
    with pytest.raises(CoverageError):
        emit_program(g, Profile())
    with pytest.raises(ValueError, match="unknown backend"):
        emit_program(Graph(), Profile(backend="nope"))

    class Tagged(Gfx950Backend):                      # a chip backend that wraps the shared emission
        id = "gfx950-tagged"

        def emit(self, shared_emit, *args, **kwargs):
            p = shared_emit(*args, **kwargs)
            p.context_capacity = 1234
            return p
    register_backend(Tagged())
    p = emit_program(Graph(), Profile(backend="gfx950-tagged"))
    assert p.backend_id == "gfx950-tagged" and p.context_capacity == 1234
    assert get_backend("gfx950").id == "gfx950"


@pytest.mark.gpu
def test_emitted_program_equals_step_program(torch_gpu):
    """Model A: the hand-built StepProgram (graph replay through the pump). Model B, the same seeds: the program
    emitted by compile_program, run by Engine. Same tokens; the same GDN recurrent and conv state and KV cache."""
    torch = torch_gpu
    from monolith_mi355.compiler import Profile, compile_program
    from monolith_mi355.runtime.engine import Engine, bound_buffers
    from monolith_mi355.runtime.step import StepProgram, StepState
    steps = 12
    a = _decoder(torch, 21, "cuda")
    st = StepState(ring_capacity=64)
    prog = StepProgram(a, st, ctx_cap=256, steps_per_graph=2)
    st.start(position=40, token=7)
    tok_a = prog.step_eager(2)
    tok_a += prog.run(steps - 2, launches_per_batch=2, in_flight=2).tokens
    torch.cuda.synchronize()

    b = _decoder(torch, 21, "cuda")
    p = compile_program(b, Profile(ring_capacity=64, ctx_cap=256))
    eng = Engine(p, buffers=bound_buffers(p))
    lay = p.layout
    st_b = eng.buffers[p.step_state]
    st_b.write(lay.pack(dict(position=40, kv_len=40, t_this_step=1, pending_tokens=[7], anchor=7)), 0)
    rep = eng.run(steps, steps_per_cb=4, in_flight=2)
    torch.cuda.synchronize()
    assert rep.tokens == tok_a, (rep.tokens, tok_a)
    s = eng.state()
    assert s["step"] == steps and s["position"] == 40 + steps
    ga, gb = a.layers[0], b.layers[0]
    assert torch.equal(ga.rec_state, gb.rec_state)
    assert torch.equal(ga.conv_state[ga.parity], gb.conv_state[s["step"] & 1])
    ca, cb = a.layers[1].cache, b.layers[1].cache
    for name in ("k_codes", "v_codes", "k_scales", "v_scales"):
        assert torch.equal(getattr(ca, name), getattr(cb, name)), name
    # the re-encoded (op by op) run continues the same sequence
    rep2 = eng.run(4, steps_per_cb=2, in_flight=1, reencode=True)
    assert len(rep2.tokens) == 4 and eng.state()["step"] == steps + 4
    # per-op timings of the emitted step (library calls profiled like run-time kernels)
    times = eng.profile(1)[0]
    assert len(times) == len(p.ops) and all(e >= s0 for s0, e in times)


@pytest.mark.gpu
def test_emitted_program_survives_json(torch_gpu):
    """program.json round trip: the reloaded program, given the same bound buffers (its names are stable), emits
    the same tokens as the original on a twin model."""
    torch = torch_gpu
    from monolith_mi355.compiler import Profile, compile_program
    from monolith_mi355.runtime.engine import Engine, bound_buffers
    from monolith_mi355.runtime.program import Program
    runs = []
    for reload in (False, True):
        m = _decoder(torch, 41, "cuda")
        p = compile_program(m, Profile(ring_capacity=64, ctx_cap=256))
        q = Program.from_json(p.to_json()) if reload else p
        eng = Engine(q, buffers=bound_buffers(p))
        eng.buffers[q.step_state].write(q.layout.pack(dict(position=40, kv_len=40, t_this_step=1,
                                                           pending_tokens=[5], anchor=5)), 0)
        runs.append(eng.run(6, steps_per_cb=2, in_flight=2).tokens)
        torch.cuda.synchronize()
    assert runs[0] == runs[1] and len(runs[0]) == 6


@pytest.mark.gpu
def test_emitted_moe_program_equals_step_program(torch_gpu):
    """A hybrid MoE decoder (the GDN layer's MLP replaced by a 64-expert top-8 block with a shared expert): the
    emitted program (router, route, grouped expert GEMVs, combine) against the hand-built StepProgram, bit for bit."""
    torch = torch_gpu
    from monolith_mi355.compiler import Profile, compile_program
    from monolith_mi355.layers import MoeBlock
    from monolith_mi355.runtime.engine import Engine, bound_buffers
    from monolith_mi355.runtime.step import StepProgram, StepState

    def model(seed):
        m = _decoder(torch, seed, "cuda")
        m.layers[0].mlp = MoeBlock(hidden=1024, experts=64, top_k=8, inter=512, shared_inter=512, device="cuda",
                                   seed=seed + 5)
        return m
    steps = 8
    a = model(31)
    st = StepState(ring_capacity=64)
    prog = StepProgram(a, st, ctx_cap=256, steps_per_graph=2)
    st.start(position=40, token=3)
    tok_a = prog.step_eager(2) + prog.run(steps - 2, launches_per_batch=1, in_flight=2).tokens
    b = model(31)
    p = compile_program(b, Profile(ring_capacity=64, ctx_cap=256))
    names = [o.name for o in p.ops]
    # one token: the expert gate|up launch routes for itself (no route op); the combine takes the shared slot
    assert "layers.0.mlp.route" not in names and "layers.0.mlp.combine" in names
    assert "layers.0.mlp.experts_gate_up" in names
    eng = Engine(p, buffers=bound_buffers(p))
    eng.buffers[p.step_state].write(p.layout.pack(dict(position=40, kv_len=40, t_this_step=1, pending_tokens=[3],
                                                       anchor=3)), 0)
    rep = eng.run(steps, steps_per_cb=2, in_flight=2)
    torch.cuda.synchronize()
    assert rep.tokens == tok_a, (rep.tokens, tok_a)
    assert torch.equal(a.layers[0].rec_state, b.layers[0].rec_state)
