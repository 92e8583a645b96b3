"""The compiler side of the operator API for gfx950, against the reference's op contract.

The graphs come from ``golden/graph_<model>.json``: what the reference's own ``Qwen3_5Model`` / ``Qwen3_5MoeModel``
lower at a small geometry (a Gated DeltaNet and a gated-attention layer, dense or MoE feed-forwards; written by
``golden/make_graph_golden.py``). On the CPU: this package's graph builders (``monolith_mi355.nn``) write those
graphs value for value and op for op; the layout the names stand for (row permutations, RoPE tables) matches
``golden/graph_layout.npz``; ``emit_program`` turns them, with weights mapped from a pack by name, into programs
of library calls with the launches the hand-built layers make. On the GPU: the program emitted from the reference's
graph and a pack of a model's weights, replayed by ``Engine``, gives the tokens and the states (GDN recurrent and
conv state, KV cache) of the hand-built ``StepProgram`` / ``SpecProgram`` on a twin model, bit for bit.
"""

import json
from pathlib import Path

import numpy as np
import pytest

from helpers import graph_from_json

GOLDEN = Path(__file__).resolve().parent / "golden"
HIDDEN, VOCAB, CTX = 1024, 4096, 256


def _fixture(tag):
    return graph_from_json(json.loads((GOLDEN / f"graph_{tag}.json").read_text()))


def _spec(moe=False):
    from monolith_mi355 import nn as NN
    return NN.HybridDecoder(vocab=VOCAB, hidden=HIDDEN, layer_types=["gdn", "attention"], inter=1024,
                            gdn=dict(k_heads=2, v_heads=4), moe=dict(experts=64, top_k=8, inter=512, shared_inter=512),
                            attention=dict(heads=4, kv_heads=1, head_dim=128, rotary_dim=64, theta=1e6),
                            moe_layers=[0, 1] if moe else [], max_context=CTX)


def _decoder(torch, seed, device, *, kv="bf16", moe=False):
    """The fixture's geometry as hand-built layers (attention in the reference's packed layout)."""
    from monolith_mi355.layers import AttnDecoderLayer, DecoderModel, GdnDecoderLayer, MoeBlock
    layers = [GdnDecoderLayer(hidden=HIDDEN, k_heads=2, v_heads=4, inter=1024, seed=seed, device=device),
              AttnDecoderLayer(hidden=HIDDEN, heads=4, kv_heads=1, ctx=CTX, inter=1024, seed=seed + 1, device=device,
                               layout="packed", kv_dtype=kv)]
    if moe:
        for i, l in enumerate(layers):
            l.mlp = MoeBlock(hidden=HIDDEN, experts=64, top_k=8, inter=512, shared_inter=512, device=device,
                             seed=seed + 5 + i)
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    layers[1].fill_cache(40, gen)
    return DecoderModel(layers, vocab=VOCAB, hidden=HIDDEN, seed=seed, device=device)


def _norm(x):
    if isinstance(x, (tuple, list)):
        return [_norm(v) for v in x]
    if isinstance(x, dict):
        return {k: _norm(v) for k, v in x.items()}
    return x


def _fields(desc_cls, op):
    names = [f for f, _ in desc_cls._fields_]
    return {names[i]: (b, off) for i, b, off in op.bindings}


# ---- the contract ------------------------------------------------------------------------------------------------
@pytest.mark.parametrize("tag,moe", [("qwen3_5", False), ("qwen3_5_moe", True)])
def test_builders_write_the_reference_graph(tag, moe):
    from monolith_mi355.core import Graph
    ref, ref_token = _fixture(tag)
    g = Graph("step")
    token = _spec(moe).lower(g)
    g.check()
    assert token.name == ref_token.name
    assert [op.kind for op in g.ops] == [op.kind for op in ref.ops]
    for a, b in zip(ref.ops, g.ops):
        assert [v.name for v in a.inputs] == [v.name for v in b.inputs], a.kind
        assert [v.name for v in a.outputs] == [v.name for v in b.outputs], a.kind
        assert _norm(a.attrs) == _norm(b.attrs), (a.kind, a.attrs, b.attrs)
        assert (a.domain.kind, str(a.domain.n_blocks), a.klass.value) == (b.domain.kind, str(b.domain.n_blocks),
                                                                          b.klass.value)

    def meta(vals):
        return {n: (tuple(map(str, v.shape)), str(v.dtype), v.format, v.is_input, v.is_weight, v.is_state, v.is_const,
                    v.view_of) for n, v in vals.items()}
    assert meta(ref.values) == meta(g.values)


def test_layout_matches_the_reference():
    """The row permutations of the stacked slabs (the RoPE head-dim permutation on q and k with the gate rows last;
    the gate|up chunk interleave) and the pack's permuted RoPE tables, bit for bit."""
    from monolith_mi355.formats.fp import f32_to_bf16
    from monolith_mi355 import nn as NN
    lay = np.load(GOLDEN / "graph_layout.npz")
    spec = _spec()
    perms = {}
    for blk in spec.blocks:
        for lin in blk.mixer.linears() + blk.mlp.linears():
            grp = lin.slab_groups()[0]
            if grp.row_perm is not None:
                perms[grp.name] = grp.row_perm
    keys = {k[5:] for k in lay.files if k.startswith("perm:")}
    assert keys == set(perms)
    for name, perm in perms.items():
        assert np.array_equal(perm, lay[f"perm:{name}"]), name
    for name, (dtype, arr) in spec.tables().items():
        assert dtype == "BF16" and np.array_equal(arr, lay[f"table:{name}"]), name
    cos, _ = NN.rope_tables_permuted(1e6, 128, 64, CTX)
    assert np.array_equal(f32_to_bf16(cos), lay["table:rope_cos"])


# ---- emission ----------------------------------------------------------------------------------------------------
def _emit(tag, model, tmp_path, **kw):
    from monolith_mi355.compiler import Profile, emit_program, write_pack
    g, token = _fixture(tag)
    pack = write_pack(model, tmp_path / "pack")
    prof = kw.pop("profile", None) or Profile(ring_capacity=64, kv_cache=kw.pop("kv", "bf16"))
    return emit_program(g, pack=pack, profile=prof, token=token, **kw), pack


def test_emit_reference_graph(tmp_path):
    """The reference's dense hybrid graph at T = 1: the launches of the hand-built layers (the sibling GEMVs
    merged over their slab, the norms fused, the GDN norm moved onto the output projection, attention core and
    merge in one), weights as file windows of the pack, step-state fields bound."""
    import torch
    from monolith_mi355.runtime import hip
    from monolith_mi355.runtime.program import Program
    p, pack = _emit("qwen3_5", _decoder(torch, 3, "cpu"), tmp_path)
    assert p.backend_id == "gfx950"
    names = [o.name for o in p.ops]
    assert names[0] == "embed" and names[-3:] == ["lm_head", "argmax", "advance"]
    pre0, pre1 = "gemv:layers.0.", "gemv:layers.1."
    assert names[1:6] == [pre0 + "linear_attn.in_proj.in_proj_z+in_proj_qkv+in_proj_a+in_proj_b", "gdn_mixer",
                          pre0 + "linear_attn.out_proj.out_proj", pre0 + "mlp.gate_up.gate_proj+up_proj",
                          pre0 + "mlp.down.down_proj"]
    assert names[6:11] == [pre1 + "self_attn.qkv.q_proj+k_proj+v_proj", "gqa_decode", pre1 + "self_attn.o_proj.o_proj",
                           pre1 + "mlp.gate_up.gate_proj+up_proj", pre1 + "mlp.down.down_proj"]
    assert p.plan_report == {"merge_row_ranges": 2, "fuse_norm_stat": 5, "fuse_gdn": 1, "fold_gdn_conv": 1,
                             "fuse_gqa": 1}
    # weights come from the pack file, by name
    weights = {n: b for n, b in p.buffers.items() if b.role == "weights"}
    assert weights and all(b.file == str(pack.dir / "weights.pack") for b in weights.values())
    # the merged projection: the whole slab; the step reads z | q | k | v | a | b at their columns
    proj = p.ops[1]
    assert proj.meta["desc"]["n"] == 4 * 128 + 2 * 256 + 4 * 128 + 2 * 4 and proj.meta["desc"]["m"] == 1
    gdn = p.ops[2]
    d = gdn.meta["desc"]
    assert (d["z_off"], d["q_off"], d["k_off"], d["v_off"], d["a_off"], d["b_off"]) == (0, 512, 768, 1024, 1536, 1540)
    f = _fields(hip.MiGdnDesc, gdn)
    assert f["step"] == ("step_state", p.layout.offset("step")) and f["done"] == ("step_state", p.layout.offset("done"))
    assert f["rec_in"] == f["rec_out"] and d["defer_norm"] == 1
    # at one token the projection runs the conv (rows 512.. of its output) and the step reads the result
    pf = _fields(hip.MiGemvDesc, proj)
    assert proj.meta["desc"]["conv_row0"] == 512 and proj.meta["desc"]["conv_channels"] == 1024
    assert pf["conv_out"] == f["pre"] and pf["conv_in"][0] == "layers.0.linear_attn.conv_state"
    assert pf["conv_step"] == ("step_state", p.layout.offset("step")) and d["ld_pre"] == 1024
    # the out_proj applies the gated norm to z, read in the projection's buffer at its row stride
    of = _fields(hip.MiGemvDesc, p.ops[3])
    assert of["gnorm_z"] == _fields(hip.MiGemvDesc, proj)["y"] and p.ops[3].meta["desc"]["ld_gnorm_z"] == 1544
    # attention: q | k | v at the front of the merged projection, the gate rows after them
    gq = p.ops[7]
    gf = _fields(hip.MiGqaDesc, gq)
    assert gf["pos_dev"] == ("step_state", p.layout.offset("position"))
    py = _fields(hip.MiGemvDesc, p.ops[6])["y"]
    assert gf["proj"] == py and gf["gate_src"] == (py[0], py[1] + 2 * 6 * 128)
    assert gq.meta["desc"]["rotary_dim"] == 128 and gq.meta["desc"]["kv_dtype"] == hip.MI_KV_BF16
    assert p.context_capacity == CTX
    q = Program.from_json(p.to_json())
    assert q.to_json() == p.to_json()


def test_emit_reference_moe_graph(tmp_path):
    """The reference's MoE hybrid: the router and the shared-expert gate (back to back in the pack) become one
    launch, the shared expert joins the grouped expert launches as slot k, and at one token the gate|up launch
    routes for itself (no route op); at T = 8 the route runs, two pairs per record."""
    import torch
    model = _decoder(torch, 3, "cpu", moe=True)
    p, _ = _emit("qwen3_5_moe", model, tmp_path)
    names = [o.name for o in p.ops]
    assert "moe_route" not in names and names.count("moe_combine") == 2
    assert p.plan_report["fuse_shared_expert"] == 2 and p.plan_report["merge_adjacent_slabs"] == 2
    router = next(o for o in p.ops if o.name == "gemv:layers.0.mlp.router.gate")
    assert router.meta["desc"]["n"] == 65
    gu = next(o for o in p.ops if o.name == "moe_gemv:layers.0.mlp.experts_gate_up")
    assert gu.meta["desc"]["top_k"] == 9 and gu.meta["desc"]["shared_expert"] == 64
    assert gu.meta["desc"]["route_experts"] == 64 and gu.meta["desc"]["route_gate_col"] == 64
    p8, _ = _emit("qwen3_5_moe", model, tmp_path / "t8", t=8)
    route = [o for o in p8.ops if o.name == "moe_route"]
    assert len(route) == 2 and route[0].meta["desc"]["pairs_per_record"] == 2
    assert route[0].meta["desc"]["max_groups"] == 8 * 9


def test_emit_without_adjacency_keeps_the_reference_split(tmp_path):
    """Without the stacking passes (a pack whose shared expert is not stored after the routed experts): the shared
    expert runs as its own two GEMVs and the combine adds it with its gate — the reference's op split, on the
    library's entry points."""
    import torch
    from monolith_mi355.compiler import Profile, emit_program, write_pack
    model = _decoder(torch, 3, "cpu", moe=True)
    pack = write_pack(model, tmp_path / "pack")
    g, token = _fixture("qwen3_5_moe")
    from monolith_mi355.compiler.plan import PASSES, fuse_shared_expert, merge_adjacent_slabs
    passes = [f for f in PASSES if f not in (fuse_shared_expert, merge_adjacent_slabs)]
    p = emit_program(g, pack=pack, profile=Profile(ring_capacity=64), token=token, passes=passes)
    names = [o.name for o in p.ops]
    assert names.count("moe_route") == 2
    assert "gemv:layers.0.mlp.shared_gate_up.gate_proj+up_proj" in names
    assert "gemv:layers.0.mlp.shared_gate.shared_expert_gate" in names
    comb = next(o for o in p.ops if o.name == "moe_combine")
    assert comb.meta["desc"]["top_k"] == 8 and comb.meta["desc"]["ld_gate"] > 0


def test_emit_speculative_round(tmp_path):
    """The speculative program (T = 1 + γ): the verify pass writes the GDN state's second slot, then the accept scan,
    the commit pass (in place, the accepted count from the step state), the draft lookup and the verify select."""
    import torch
    from monolith_mi355.compiler import Profile, compile_decoder
    from monolith_mi355.runtime import hip
    model = _decoder(torch, 3, "cpu")
    table = np.zeros((CTX, 8), np.int32)
    p, _, images = compile_decoder(model, tmp_path, Profile(ring_capacity=64, ctx_cap=240), gamma=7, verify_length=7,
                                   tables={"draft_table": (table, "I32")})
    names = [o.name for o in p.ops]
    assert names[-5:] == ["argmax", "accept_scan", "gdn_commit", "embed", "verify_select"]
    assert all(o.meta["desc"].get("m", 8) == 8 for o in p.ops if o.name.startswith("gemv"))
    mix, com = p.ops[names.index("gdn_mixer")], p.ops[names.index("gdn_commit")]
    fm, fc = _fields(hip.MiGdnDesc, mix), _fields(hip.MiGdnDesc, com)
    slot = 4 * 128 * 128 * 4
    assert fm["rec_out"] == (fm["rec_in"][0], fm["rec_in"][1] + slot) and fc["rec_out"] == fc["rec_in"] == fm["rec_in"]
    assert fc["t_dev"] == ("step_state", p.layout.offset("checkpoint_index"))
    assert p.ops[-1].meta["desc"]["mode"] == 2 and p.ops[-1].meta["desc"]["threshold"] == 7.0
    assert p.context_capacity == 240
    assert set(images) == set(p.state_names)
    # T = 8: each layer's residual GEMV writes the next norm's rows (the next layer's input, then the LM head's), and
    # the GEMVs that read them apply no norm of their own
    handing = [o for o in p.ops if o.name.startswith("gemv") and o.meta["desc"].get("ld_next_x", 0) > 0]
    assert len(handing) >= 2, [o.name for o in handing]
    lm = p.ops[names.index("lm_head")]
    assert "norm_w" not in _fields(hip.MiGemvDesc, lm)


def test_backend_selection_and_coverage():
    from monolith_mi355.compiler import Profile, emit_program, get_backend, register_backend
    from monolith_mi355.compiler.context import Gfx950Backend
    from monolith_mi355.core import BlockDomain, DType, Graph, OpClass
    from monolith_mi355.ops import CoverageError
    g = Graph()
    x = g.input("x", (1, 256), DType.BF16)
    y = g.value("y", (1, 256), DType.BF16)
    g.op("no_such_op", [x], [y], domain=BlockDomain("rows", 1), klass=OpClass.MAP)
    with pytest.raises(CoverageError):
        emit_program(g, profile=Profile(), tail=None)
    with pytest.raises(ValueError, match="unknown backend"):
        emit_program(Graph(), profile=Profile(backend="nope"), tail=None)

    class Tagged(Gfx950Backend):                      # a chip backend that wraps the shared emission
        id = "gfx950-tagged"

        def emit(self, shared_emit, *args, **kwargs):
            p = shared_emit(*args, **kwargs)
            p.context_capacity = 1234
            return p
    register_backend(Tagged())
    p = emit_program(Graph(), profile=Profile(backend="gfx950-tagged"), tail=None)
    assert p.backend_id == "gfx950-tagged" and p.context_capacity == 1234
    assert get_backend("gfx950").id == "gfx950"


# ---- on the GPU: the emitted programs against the hand-built ones ------------------------------------------------
def _engine(p, images):
    from monolith_mi355.compiler import load_states
    from monolith_mi355.runtime.engine import Engine
    eng = Engine(p)
    load_states(eng, images)
    return eng


def _state_equal(torch, a, eng, p, step):
    """Model A's layer states against the program's state buffers after ``step`` steps."""
    ga = a.layers[0]
    rec = np.frombuffer(eng.read("layers.0.linear_attn.rec_state"), np.float32)[: ga.rec.numel()]
    assert np.array_equal(rec, ga.rec.cpu().numpy().ravel())
    conv = np.frombuffer(eng.read("layers.0.linear_attn.conv_state"), np.uint16).reshape(2, -1)[step & 1]
    assert np.array_equal(conv, ga.conv_state[ga.parity].view(torch.int16).cpu().numpy().view(np.uint16).ravel())
    c = a.layers[1].cache
    for name, t in (("k_cache", c.k_codes), ("v_cache", c.v_codes)):
        got = np.frombuffer(eng.read(f"layers.1.self_attn.{name}"), np.uint8)[: t.numel() * t.element_size()]
        assert np.array_equal(got, t.contiguous().view(torch.uint8).cpu().numpy().ravel()), name
    if c.k_scales is not None:
        for name, t in (("k_cache.scales", c.k_scales), ("v_cache.scales", c.v_scales)):
            got = np.frombuffer(eng.read(f"layers.1.self_attn.{name}"), np.uint8)
            assert np.array_equal(got, t.contiguous().view(torch.uint8).cpu().numpy().ravel()), name


def _step_program(torch, model, steps, token=7):
    from monolith_mi355.runtime.step import StepProgram, StepState
    st = StepState(ring_capacity=64)
    prog = StepProgram(model, st, ctx_cap=CTX, steps_per_graph=2)
    st.start(position=40, token=token)
    out = prog.step_eager(2) + prog.run(steps - 2, launches_per_batch=2, in_flight=2).tokens
    torch.cuda.synchronize()
    return out


def _start(eng, p, token):
    eng.buffers[p.step_state].write(p.layout.pack(dict(position=40, kv_len=40, t_this_step=1, pending_tokens=[token],
                                                       anchor=token)), 0)


@pytest.mark.gpu
@pytest.mark.parametrize("kv", ["bf16", "int8"])
def test_reference_graph_program_equals_step_program(torch_gpu, tmp_path, kv):
    """Model A: the hand-built StepProgram. Model B (same seeds): the reference's lowered graph emitted from a pack of
    B's weights, run by Engine. Same tokens; the same recurrent and conv state and KV cache, bit for bit."""
    torch = torch_gpu
    from monolith_mi355.compiler import Profile, emit_program, state_images, write_pack
    steps = 12
    print(f"reference graph vs StepProgram kv={kv}", flush=True)
    a = _decoder(torch, 21, "cuda", kv=kv)
    tok_a = _step_program(torch, a, steps)
    b = _decoder(torch, 21, "cuda", kv=kv)
    g, token = _fixture("qwen3_5")
    p = emit_program(g, pack=write_pack(b, tmp_path), profile=Profile(ring_capacity=64, kv_cache=kv), token=token)
    eng = _engine(p, state_images(b))
    _start(eng, p, 7)
    rep = eng.run(steps, steps_per_cb=4, in_flight=2)
    torch.cuda.synchronize()
    assert rep.tokens == tok_a, (rep.tokens, tok_a)
    s = eng.state()
    assert s["step"] == steps and s["position"] == 40 + steps
    _state_equal(torch, a, eng, p, steps)
    rep2 = eng.run(4, steps_per_cb=2, in_flight=1, reencode=True)     # op by op continues the same sequence
    assert len(rep2.tokens) == 4 and eng.state()["step"] == steps + 4


@pytest.mark.gpu
def test_reference_moe_graph_program_equals_step_program(torch_gpu, tmp_path):
    """The reference's MoE hybrid graph (both layers sparse, 64 experts top-8 + a shared expert) against the
    hand-built StepProgram on a twin model: tokens and states bit for bit."""
    torch = torch_gpu
    from monolith_mi355.compiler import Profile, emit_program, state_images, write_pack
    steps = 8
    print("reference MoE graph vs StepProgram", flush=True)
    a = _decoder(torch, 31, "cuda", moe=True)
    tok_a = _step_program(torch, a, steps, token=3)
    b = _decoder(torch, 31, "cuda", moe=True)
    g, token = _fixture("qwen3_5_moe")
    p = emit_program(g, pack=write_pack(b, tmp_path), profile=Profile(ring_capacity=64), token=token)
    assert "moe_route" not in [o.name for o in p.ops]
    eng = _engine(p, state_images(b))
    _start(eng, p, 3)
    rep = eng.run(steps, steps_per_cb=2, in_flight=2)
    torch.cuda.synchronize()
    assert rep.tokens == tok_a, (rep.tokens, tok_a)
    _state_equal(torch, a, eng, p, steps)


@pytest.mark.gpu
@pytest.mark.parametrize("moe", [False, True])
def test_speculative_program_equals_spec_program(torch_gpu, tmp_path, moe):
    """The speculative round compiled from the reference's graph (verify block of 8 rows, accept scan, commit, the
    draft table, a fixed verify length) against the hand-built SpecProgram: the same tokens, the same states. The
    drafts are the one-token decode's own tokens, so whole blocks are accepted and the commit replays 8 rows. With
    MoE feed-forwards the hand-built verify pass hands each layer's input norm over through the MoE combine."""
    torch = torch_gpu
    from monolith_mi355.compiler import Profile, compile_decoder
    from monolith_mi355.runtime.step import SpecProgram, StepState
    print(f"speculative program vs SpecProgram moe={moe}", flush=True)
    seq = [9] + _step_program(torch, _decoder(torch, 41, "cuda", moe=moe), 60, token=9)
    table = np.zeros((CTX, 8), np.int32)
    for pos in range(40, CTX):
        for j in range(7):
            i = pos - 40 + 1 + j
            table[pos, j] = seq[i] if i < len(seq) else 0
    steps = 8
    a = _decoder(torch, 41, "cuda", moe=moe)
    st = StepState(ring_capacity=512)
    prog = SpecProgram(a, st, gamma=7, draft_table=torch.from_numpy(table).cuda(), ctx_cap=240, steps_per_graph=2)
    st.start(position=40, token=9)
    tok_a = prog.step_eager(2) + prog.run(steps - 2, launches_per_batch=2, in_flight=2).tokens
    torch.cuda.synchronize()
    b = _decoder(torch, 41, "cuda", moe=moe)
    p, _, images = compile_decoder(b, tmp_path, Profile(ring_capacity=512, ctx_cap=240), gamma=7, verify_length=7,
                                   tables={"draft_table": (table, "I32")})
    eng = _engine(p, images)
    _start(eng, p, 9)
    rep = eng.run(steps, steps_per_cb=2, in_flight=2)
    torch.cuda.synchronize()
    assert len(tok_a) > steps and rep.tokens == tok_a, (rep.tokens, tok_a)
    assert tok_a == seq[1: 1 + len(tok_a)]
    s = eng.state()
    assert s["position"] == 40 + len(tok_a)
    _state_equal(torch, a, eng, p, s["step"])


@pytest.mark.gpu
def test_emitted_program_survives_json(torch_gpu, tmp_path):
    """program.json round trip: the reloaded program (buffers by name, weights from the same pack file) emits the
    same tokens as the original on a twin model."""
    torch = torch_gpu
    from monolith_mi355.compiler import Profile, emit_program, state_images, write_pack
    from monolith_mi355.runtime.program import Program
    runs = []
    for reload in (False, True):
        m = _decoder(torch, 41, "cuda")
        g, token = _fixture("qwen3_5")
        p = emit_program(g, pack=write_pack(m, tmp_path / str(reload)), profile=Profile(ring_capacity=64), token=token)
        q = Program.from_json(p.to_json()) if reload else p
        eng = _engine(q, state_images(m))
        _start(eng, q, 5)
        runs.append(eng.run(6, steps_per_cb=2, in_flight=2).tokens)
        torch.cuda.synchronize()
    assert runs[0] == runs[1] and len(runs[0]) == 6
