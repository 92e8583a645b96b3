"""Whole decode layers (``h += mixer(norm1(h)); h += mlp(norm2(h))``, ``nn/decoder.py:14-26``) built from the HIP
kernels against the same layer composed from the oracle's functions on the exactly dequantized weights: the Gated
DeltaNet layer and the gated-GQA layer over the int8 KV cache, at the 27B geometry (hidden 5120) and a small one,
M = 1 and 8, two consecutive steps (state carried).

Bars: every stage of the layer (the norm-fused projection, the mixer, the output projection with its residual, the
gate|up and down GEMVs) against the oracle fed the device's own input to that stage, element-wise within 1e-2
relative / 1e-3 absolute — the attention core within its kernel test's bar; and the whole
layer end to end from the oracle's own chain with the reference's composite layer bar
(``tests/kernels/test_gqa_decode.py:347``: cosine > 0.9999, max |error| ≤ 1e-2 of the output's largest magnitude),
on the output and on the GDN recurrent state. End to end, each GEMV's BF16 rounding can flip against the oracle's and
the flip propagates (the stage bars show each kernel is within tolerance of the oracle on its own input), so the
element-wise fraction outside 1e-2 / 1e-3 is bounded by a per-case ceiling about 1.5x the worst measured on MI355X
(``E2E_CEILING``) rather than asserted at zero: the layers are deterministic, so a regression in any stage shows
up as a fraction above it. Measured worst (of two steps, both M): GDN small 0.01 %, GDN 27B 5.4 %, attention small
0.9 %, attention 27B 13.4 % (its output sums an MLP of K = 17408 over an attention output of ~1/sqrt(4000) scale,
so its ULP flips move the most elements past 1e-2 of a small reference value); the recurrent state 0."""

import numpy as np
import pytest

from helpers import from_dev_bf16, to_dev_bf16
from oracle import formats as OF
from oracle import nn as ON
from oracle.fp import rbf
from oracle.gates import check_against_oracle, tolerance_violations

pytestmark = pytest.mark.gpu
EPS = 1e-6
# end-to-end element-wise ceiling per (mixer, geometry): about 1.5x the worst fraction measured on MI355X
E2E_CEILING = {("gdn", "small"): 0.005, ("gdn", "27b"): 0.08, ("attn", "small"): 0.015, ("attn", "27b"): 0.20,
               ("state", "small"): 0.0, ("state", "27b"): 0.0}


def _deq(q):
    return OF.dequantize_rows({"format": "nvfp4", "weight": q["weight"], "weight_scale": q["weight_scale"],
                               "row_scale": q["row_scale"], "weight_scale_2": 1.0})


def _deq_gate_up(q):
    w = _deq(q)
    inter = w.shape[0] // 2
    out = np.empty_like(w)
    out[ON.interleave_chunks(inter, inter, 8)] = w                  # back to [gate; up]
    return out


def _bar(got, ref, what, ceiling):
    """The end-to-end layer bar: cosine and max error norm-wise (the reference's layer bar), and the element-wise
    fraction outside 1e-2 / 1e-3 at most ``ceiling`` — each GEMV's BF16 rounding can flip against the oracle's, and
    a flip moves every later stage by up to an ULP, so element-wise exactness is asserted per stage (``_stage``)."""
    g, r = got.astype(np.float64).ravel(), ref.astype(np.float64).ravel()
    cos = float(g @ r / (np.linalg.norm(g) * np.linalg.norm(r) + 1e-30))
    err, scale = float(np.abs(g - r).max()), float(np.abs(r).max())
    assert cos > 0.9999 and err <= 1e-2 * scale, (what, cos, err, scale)
    bad = tolerance_violations(g, r)
    print(f"  {what} end to end: {bad} of {g.size} outside 1e-2/1e-3 (cos {cos:.7f})", flush=True)
    assert bad <= ceiling * g.size, (what, bad, g.size, ceiling)


def _stage(got, ref, what):
    """One stage of the layer given the device's own input to it: the north-star bar element-wise (every element
    within 1e-3 + 1e-2·|ref|) and the reference's ``ok_rounded``."""
    chk = check_against_oracle(got, ref)
    print(f"  {what}: {chk.tol_violations} of {chk.n} outside 1e-2/1e-3", flush=True)
    assert chk.within and chk.ok_rounded(), (what, chk)


def _mlp(h1, ex):
    x2 = ON.rms_norm(h1, ex["norm2"], EPS, one_plus=False)
    act = ON.linear(x2, _deq_gate_up(ex["gate_up"]), epilogue="silu_mul")
    return ON.linear(act, _deq(ex["down"]), epilogue="residual", residual=h1)


def _mlp_stages(layer, m, h1_dev, ex):
    """The MLP's two GEMVs, each against the oracle fed the device's own input."""
    _, _, _, act, h2 = layer.buffers(m)
    act_d, h2_d = from_dev_bf16(act), from_dev_bf16(h2)
    x2 = ON.rms_norm(h1_dev, ex["norm2"], EPS, one_plus=False)
    _stage(act_d, ON.linear(x2, _deq_gate_up(ex["gate_up"]), epilogue="silu_mul"), "gate|up silu·mul")
    _stage(h2_d, ON.linear(act_d, _deq(ex["down"]), epilogue="residual", residual=h1_dev), "down + residual")


@pytest.mark.parametrize("geom", ["small", "27b"])
@pytest.mark.parametrize("m", [1, 8])
def test_gdn_decoder_layer(torch_gpu, geom, m):
    torch = torch_gpu
    from monolith_mi355.layers import GdnDecoderLayer
    kw = dict(hidden=1024, k_heads=2, v_heads=6, inter=1536) if geom == "small" else {}
    layer = GdnDecoderLayer(seed=3, **kw)
    ex = layer.export()
    conv, rec = ex["conv_state"], ex["rec_state"]
    w_in, w_out = _deq(ex["w_in"]), _deq(ex["w_out"])
    hv = layer.hv
    gdn_kw = dict(conv_w=ex["conv_w"], a_log=ex["a_log"], dt_bias=ex["dt_bias"], norm_w=ex["gdn_norm_w"],
                  k_heads=layer.hk, v_heads=hv, dk=128, dv=128, eps=EPS)
    rng = np.random.default_rng(m)
    for step in range(2):
        print(f"gdn layer {geom} m={m} step {step}", flush=True)
        dev_state = layer.export()                      # the device's state before this step
        h = rbf(rng.standard_normal((m, layer.hidden)))
        got = from_dev_bf16(layer.step(to_dev_bf16(torch, h)))
        # stage by stage, each fed the device's own input
        proj_d, o_dev, h1_dev = (from_dev_bf16(b) for b in layer.buffers(m)[:3])
        xn = ON.rms_norm(h, ex["norm1"], EPS, one_plus=False)
        _stage(proj_d, ON.linear(xn, w_in), "in_proj (norm fused)")
        y_ref, _, _ = ON.gdn_mix(proj_d, dev_state["conv_state"], dev_state["rec_state"], **gdn_kw)
        if layer.defers_norm(m):                        # o holds the read-out; the norm rides on out_proj
            o_dev = ON.gated_rms_norm(o_dev.reshape(m * hv, 128), proj_d[:, : hv * 128].reshape(m * hv, 128),
                                      ex["gdn_norm_w"], EPS).reshape(m, hv * 128)
        _stage(o_dev, y_ref, "gdn mixer (gated norm)")
        _stage(h1_dev, ON.linear(o_dev, w_out, epilogue="residual", residual=h), "out_proj + residual")
        _mlp_stages(layer, m, h1_dev, ex)
        # end to end from the oracle's own chain
        xn = ON.rms_norm(h, ex["norm1"], EPS, one_plus=False)
        proj = ON.linear(xn, w_in)
        o, conv, rec = ON.gdn_mix(proj, conv, rec, **gdn_kw)
        h1 = ON.linear(o, w_out, epilogue="residual", residual=h)
        _bar(got, _mlp(h1, ex), "layer output", E2E_CEILING[("gdn", geom)])
        _bar(layer.rec_state.cpu().numpy(), rec, "recurrent state", E2E_CEILING[("state", geom)])


@pytest.mark.parametrize("geom,ctx,pos", [("small", 1024, 300), ("27b", 4096, 4000)])
@pytest.mark.parametrize("m", [1, 8])
def test_attention_decoder_layer(torch_gpu, geom, ctx, pos, m):
    torch = torch_gpu
    from monolith_mi355.layers import AttnDecoderLayer
    kw = dict(hidden=1024, heads=8, kv_heads=2, inter=1536) if geom == "small" else {}
    layer = AttnDecoderLayer(ctx=ctx, seed=4, **kw)
    gen = torch.Generator(device="cuda")
    gen.manual_seed(5)
    layer.fill_cache(pos, gen)
    ex = layer.export()
    kc, ks = ex["k_codes"].transpose(1, 0, 2).copy(), ex["k_scales"].T.copy()
    vc, vs = ex["v_codes"].transpose(1, 0, 2).copy(), ex["v_scales"].T.copy()
    w_qkv, w_o = _deq(ex["w_qkv"]), _deq(ex["w_o"])
    cfg = dict(heads=layer.heads, kv_heads=layer.kv, head_dim=128, rotary_dim=64, theta=1e6, eps=EPS, gate=True,
               qk_norm=True, q_norm=ex["q_norm"] - 1, k_norm=ex["k_norm"] - 1, tables=(ex["cos"], ex["sin"]))
    rng = np.random.default_rng(m + 10)
    for step in range(2):
        print(f"attn layer {geom} m={m} step {step} pos={pos}", flush=True)
        h = rbf(rng.standard_normal((m, layer.hidden)))
        dev = layer.export()                            # the device's cache before this step
        got = from_dev_bf16(layer.step(to_dev_bf16(torch, h), pos))
        proj_d, o_dev, h1_dev = (from_dev_bf16(b) for b in layer.buffers(m)[:3])
        xn = ON.rms_norm(h, ex["norm1"], EPS, one_plus=False)
        _stage(proj_d, ON.linear(xn, w_qkv), "qkv proj (norm fused)")
        o_ref = ON.gqa_mix(proj_d, dev["k_codes"].transpose(1, 0, 2).copy(), dev["k_scales"].T.copy(),
                           dev["v_codes"].transpose(1, 0, 2).copy(), dev["v_scales"].T.copy(), pos, **cfg)
        # the kernel test's bar: none outside at a long cache (4K), at most 0.5 % over a few hundred keys (an output
        # formed by a few cancelling keys carries P's rounding before normalisation against the oracle's after)
        bad = tolerance_violations(o_dev, o_ref)
        print(f"  attention core: {bad} of {o_dev.size} outside 1e-2/1e-3", flush=True)
        assert bad <= (0 if geom == "27b" else 0.005 * o_dev.size), bad     # 27b: 4000+ keys
        _stage(h1_dev, ON.linear(o_dev, w_o, epilogue="residual", residual=h), "o_proj + residual")
        _mlp_stages(layer, m, h1_dev, ex)
        proj = ON.linear(xn, w_qkv)
        o = ON.gqa_mix(proj, kc, ks, vc, vs, pos, **cfg)
        h1 = ON.linear(o, w_o, epilogue="residual", residual=h)
        _bar(got, _mlp(h1, ex), "layer output", E2E_CEILING[("attn", geom)])
        pos += m


@pytest.mark.parametrize("kind", ["gdn", "attn"])
@pytest.mark.parametrize("m", [3, 8])
def test_layer_norm_hand_over(torch_gpu, kind, m):
    """At M ≥ 3 consecutive layers hand the input norm over: a layer given its normalized input (``x_in``) and asked
    for the next one's (``next_norm``, written by the MLP's split-K reduction) gives the same output and state, bit
    for bit, as the same layer normalizing its own input, and the x_next it writes is ``norm_apply`` of its output."""
    torch = torch_gpu
    from monolith_mi355 import kernels
    from monolith_mi355.layers import AttnDecoderLayer, GdnDecoderLayer

    def make():
        if kind == "gdn":
            return GdnDecoderLayer(seed=3)
        layer = AttnDecoderLayer(ctx=4096, seed=4)
        gen = torch.Generator(device="cuda")
        gen.manual_seed(5)
        layer.fill_cache(4000, gen)
        return layer

    a, b = make(), make()
    w_next = torch.from_numpy((1.0 + np.random.default_rng(9).standard_normal(a.hidden) * 0.1).astype(np.float32)).cuda()
    xn = torch.empty(m, a.hidden, dtype=torch.bfloat16, device="cuda")
    rng = np.random.default_rng(m + 20)
    pos = 4000
    for step in range(2):
        print(f"norm hand-over {kind} m={m} step {step}", flush=True)
        h = to_dev_bf16(torch, rbf(rng.standard_normal((m, a.hidden))))
        args = (pos,) if kind == "attn" else ()
        y_a = a.step(h, *args).clone()
        x_in = kernels.norm_apply(h, b.norm_w, eps=b.eps)
        xn.fill_(3.0)
        y_b = b.step(h, *args, x_in=x_in, next_norm=(w_next, xn, 1e-6)).clone()
        torch.cuda.synchronize()
        assert torch.equal(y_a.view(torch.int16), y_b.view(torch.int16)), step
        assert torch.equal(xn.view(torch.int16), kernels.norm_apply(y_b, w_next, eps=1e-6).view(torch.int16)), step
        if kind == "gdn":
            assert torch.equal(a.rec, b.rec) and torch.equal(a.conv_state, b.conv_state)
        else:
            assert torch.equal(a.cache.k_codes, b.cache.k_codes) and torch.equal(a.cache.v_codes, b.cache.v_codes)
        pos += m
