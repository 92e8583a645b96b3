"""Whole decode layers (``h += mixer(norm1(h)); h += mlp(norm2(h))``, ``nn/decoder.py:14-26``) built from the HIP
kernels against the same layer composed from the oracle's functions on the exactly dequantized weights: the Gated
DeltaNet layer and the gated-GQA layer over the int8 KV cache, at the 27B geometry (hidden 5120) and a small one,
M = 1 and 8, two consecutive steps (state carried). Bar: the reference's composite layer bar
(``tests/kernels/test_gqa_decode.py:347``: cosine > 0.9999, max |error| ≤ 1e-2 of the output's largest magnitude) —
each GEMV's BF16 rounding can flip against the oracle's and the flip propagates — on the output and on the GDN
recurrent state."""

import numpy as np
import pytest

from helpers import from_dev_bf16, to_dev_bf16
from oracle import formats as OF
from oracle import nn as ON
from oracle.fp import rbf

pytestmark = pytest.mark.gpu
EPS = 1e-6


def _deq(q):
    return OF.dequantize_rows({"format": "nvfp4", "weight": q["weight"], "weight_scale": q["weight_scale"],
                               "row_scale": q["row_scale"], "weight_scale_2": 1.0})


def _deq_gate_up(q):
    w = _deq(q)
    inter = w.shape[0] // 2
    out = np.empty_like(w)
    out[ON.interleave_chunks(inter, inter, 8)] = w                  # back to [gate; up]
    return out


def _bar(got, ref):
    g, r = got.astype(np.float64).ravel(), ref.astype(np.float64).ravel()
    cos = float(g @ r / (np.linalg.norm(g) * np.linalg.norm(r) + 1e-30))
    err, scale = float(np.abs(g - r).max()), float(np.abs(r).max())
    assert cos > 0.9999 and err <= 1e-2 * scale, (cos, err, scale)


def _mlp(h1, ex):
    x2 = ON.rms_norm(h1, ex["norm2"], EPS, one_plus=False)
    act = ON.linear(x2, _deq_gate_up(ex["gate_up"]), epilogue="silu_mul")
    return ON.linear(act, _deq(ex["down"]), epilogue="residual", residual=h1)


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
    rng = np.random.default_rng(m)
    for step in range(2):
        print(f"gdn layer {geom} m={m} step {step}", flush=True)
        h = rbf(rng.standard_normal((m, layer.hidden)))
        got = from_dev_bf16(layer.step(to_dev_bf16(torch, h)))
        xn = ON.rms_norm(h, ex["norm1"], EPS, one_plus=False)
        proj = ON.linear(xn, w_in)
        o, conv, rec = ON.gdn_mix(proj, conv, rec, conv_w=ex["conv_w"], a_log=ex["a_log"], dt_bias=ex["dt_bias"],
                                  norm_w=ex["gdn_norm_w"], k_heads=layer.hk, v_heads=layer.hv, dk=128, dv=128, eps=EPS)
        h1 = ON.linear(o, w_out, epilogue="residual", residual=h)
        _bar(got, _mlp(h1, ex))
        _bar(layer.rec_state.cpu().numpy(), rec)


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
        got = from_dev_bf16(layer.step(to_dev_bf16(torch, h), pos))
        xn = ON.rms_norm(h, ex["norm1"], EPS, one_plus=False)
        proj = ON.linear(xn, w_qkv)
        o = ON.gqa_mix(proj, kc, ks, vc, vs, pos, **cfg)
        h1 = ON.linear(o, w_o, epilogue="residual", residual=h)
        _bar(got, _mlp(h1, ex))
        pos += m
