"""Writes the golden vectors that pin the oracle to the reference's own CPU oracle.

Run in a container that has the reference checkout (``/root/reference`` or ``$LITHOS_REFERENCE``):
``python tests/golden/make_golden.py``. It imports the reference's ``monolith.formats`` (numpy) and the torch
``forward`` oracles of ``monolith.nn`` — the functions whose last-ulp behaviour no closed form or known answer pins
(the torch GDN mixer, attention step, MoE routing and forward, RMSNorm, the gated MLP, the quantizers) — on small
seeded inputs, and saves inputs and outputs as ``.npz`` fixtures next to this script. The fixtures are data; the
reference code itself is not needed (and not present) where the tests run.
"""

from __future__ import annotations

import os
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
REF = Path(os.environ.get("LITHOS_REFERENCE", "/root/reference"))


def bf16_bits(t):
    import torch
    return t.to(torch.bfloat16).view(torch.int16).numpy().astype(np.uint16)


def main():
    sys.path.insert(0, str(REF))
    import torch

    from monolith.formats import FORMATS
    from monolith.formats.fp import f32_to_bf16, f32_to_e2m1, f32_to_e4m3
    from monolith.nn import oracle
    from monolith.nn.attention import GQAAttention
    from monolith.nn.gdn import GatedDeltaNet
    from monolith.nn.mlp import GatedMLP
    from monolith.nn.moe import SparseMoE
    from monolith.nn.norm import RMSNorm

    torch.manual_seed(0)
    rng = np.random.default_rng(20261201)
    bf = torch.bfloat16

    # ---- codecs and quantizers --------------------------------------------------------------------------------
    v = np.concatenate([rng.standard_normal(500).astype(np.float32) * 3,
                        np.array([0.0, -0.0, 1.0625, 1.1875, 448, 500, -500, 2.0 ** -10, 0.25, 0.75, 2.5, 5.0, 7.0,
                                  1 + 2 ** -8, 1 + 3 * 2 ** -8, -1.5], np.float32)]).astype(np.float32)
    w_nv = (rng.standard_normal((32, 256)) * 0.02).astype(np.float32)
    w_nv[3, :16] = 0.0
    nv = FORMATS.get("nvfp4").quantize(w_nv)
    w_i4 = (rng.standard_normal((32, 256)) * 0.02).astype(np.float32)
    i4 = FORMATS.get("int4_affine").quantize(w_i4)
    np.savez_compressed(HERE / "formats.npz", codec_in=v, e4m3=f32_to_e4m3(v), e2m1=f32_to_e2m1(np.clip(v, -6, 6)),
                        bf16=f32_to_bf16(v), nv_w=w_nv, nv_codes=nv.tensors["weight"], nv_scales=nv.tensors["weight_scale"],
                        nv_s2=np.float32(nv.params["weight_scale_2"]), nv_deq=FORMATS.get("nvfp4").dequantize(nv),
                        i4_w=w_i4, i4_codes=i4.tensors["weight"], i4_scales=i4.tensors["scales"],
                        i4_biases=i4.tensors["biases"], i4_deq=FORMATS.get("int4_affine").dequantize(i4))

    # ---- RMSNorm and the gated MLP ------------------------------------------------------------------------------
    hidden, inter = 64, 48
    h = torch.randn(3, hidden).to(bf)
    nw = (torch.randn(hidden) * 0.2).to(bf)
    norm = RMSNorm(hidden, 1e-6, "x.norm.weight")
    norm.set_param("weight", nw)
    mlp = GatedMLP(hidden, inter, hf_prefix="x.mlp.")
    wg, wu, wd = [(torch.randn(r, c) * 0.05).to(bf) for r, c in ((inter, hidden), (inter, hidden), (hidden, inter))]
    mlp.gate_up.set_param("gate_proj", wg)
    mlp.gate_up.set_param("up_proj", wu)
    mlp.down.set_param("down_proj", wd)
    with torch.no_grad():
        xn = norm.forward(h)
        y = mlp.forward(xn, h)
    np.savez_compressed(HERE / "mlp.npz", h=bf16_bits(h), norm_w=bf16_bits(nw), xn=bf16_bits(xn), wg=bf16_bits(wg),
                        wu=bf16_bits(wu), wd=bf16_bits(wd), y=bf16_bits(y), eps=np.float32(1e-6))

    # ---- Gated DeltaNet mixer -----------------------------------------------------------------------------------
    for tag, (hk, hv, dk, dv, t, zero_gates) in {"gdn_t1": (2, 6, 32, 32, 1, False), "gdn_t3": (2, 6, 32, 32, 3, False),
                                                  "gdn_cfg": (2, 6, 32, 32, 2, True)}.items():
        m = GatedDeltaNet(64, hk, hv, dk, dv, 4, 1e-6, hf_prefix="x.", prefix="l.")
        conv_dim = 2 * hk * dk + hv * dv
        conv_w = (torch.randn(conv_dim, 1, 4) * 0.3).to(bf)
        a_log = torch.zeros(hv).to(bf) if zero_gates else torch.from_numpy(rng.uniform(-2, 1, hv).astype(np.float32)).to(bf)
        dt_bias = torch.zeros(hv).to(bf) if zero_gates else torch.randn(hv).to(bf)
        norm_w = (1 + torch.randn(dv) * 0.2).to(bf)
        for k_, v_ in (("conv_w", conv_w), ("a_log", a_log), ("dt_bias", dt_bias), ("norm_w", norm_w)):
            m.set_param(k_, v_)
        n1 = m.in_proj.n
        proj = torch.randn(t, n1).to(bf)
        conv_state = (torch.randn(conv_dim, 3) * 0.5).to(bf)
        rec_state = torch.randn(hv, dk, dv) * 0.1
        state = {"l.conv_state": conv_state.clone(), "l.rec_state": rec_state.clone()}
        with torch.no_grad():
            out = m.mix(proj, state)
        np.savez_compressed(HERE / f"{tag}.npz", hk=hk, hv=hv, dk=dk, dv=dv, proj=bf16_bits(proj),
                            conv_w=bf16_bits(conv_w.reshape(conv_dim, 4)), a_log=bf16_bits(a_log),
                            dt_bias=bf16_bits(dt_bias), norm_w=bf16_bits(norm_w), conv_state=bf16_bits(conv_state),
                            rec_state=rec_state.numpy(), out=bf16_bits(out),
                            new_conv=bf16_bits(state["l.conv_state"]), new_rec=state["l.rec_state"].numpy())

    # ---- attention step -----------------------------------------------------------------------------------------
    for tag, (t, qk_norm, pos) in {"attn_t1": (1, False, 5), "attn_t3": (3, False, 5), "attn_qknorm": (3, True, 9)}.items():
        heads, kv, d, rot, ctx = 4, 2, 32, 16, 16
        a = GQAAttention(64, heads, kv, d, rot, 1e6, 1e-6, hf_prefix="x.", prefix="l.", max_context=ctx, qk_norm=qk_norm)
        qn, kn = (torch.randn(d) * 0.1).to(bf), (torch.randn(d) * 0.1).to(bf)
        if qk_norm:
            a.set_param("q_norm", qn)
            a.set_param("k_norm", kn)
        n1 = heads * 2 * d + 2 * kv * d
        proj = torch.randn(t, n1).to(bf)
        kc = torch.zeros(ctx, kv, d, dtype=bf)
        vc = torch.zeros(ctx, kv, d, dtype=bf)
        kc[:pos] = torch.randn(pos, kv, d).to(bf)
        vc[:pos] = torch.randn(pos, kv, d).to(bf)
        kc0, vc0 = kc.clone(), vc.clone()
        state = {"l.k_cache": kc, "l.v_cache": vc}
        with torch.no_grad():
            out = a.mix(proj, state, pos)
        np.savez_compressed(HERE / f"{tag}.npz", heads=heads, kv=kv, d=d, rot=rot, pos=pos, qk_norm=int(qk_norm),
                            theta=np.float64(1e6), q_norm=bf16_bits(qn), k_norm=bf16_bits(kn), proj=bf16_bits(proj),
                            k_cache=bf16_bits(kc0), v_cache=bf16_bits(vc0), out=bf16_bits(out),
                            new_k=bf16_bits(state["l.k_cache"]), new_v=bf16_bits(state["l.v_cache"]))

    # ---- MoE: routing (with a forced tie) and the forward -------------------------------------------------------
    hidden, e, k, inter = 64, 16, 4, 32
    moe = SparseMoE(hidden, e, k, inter, hf_prefix="x.", prefix="l.", shared_intermediate=inter)
    wr = (torch.randn(e, hidden) * 0.3).to(bf)
    moe.router.set_param("gate", wr)
    egu = []
    for i in range(e):
        g_, u_, d_ = [(torch.randn(r, c) * 0.05).to(bf) for r, c in ((inter, hidden), (inter, hidden), (hidden, inter))]
        moe.gate_up.slab.set_param(f"e{i}.gate_proj", g_)
        moe.gate_up.slab.set_param(f"e{i}.up_proj", u_)
        moe.down.slab.set_param(f"e{i}.down_proj", d_)
        egu.append((g_, u_, d_))
    sg, su, sd = [(torch.randn(r, c) * 0.05).to(bf) for r, c in ((inter, hidden), (inter, hidden), (hidden, inter))]
    sgate = (torch.randn(1, hidden) * 0.1).to(bf)
    moe.shared_gate_up.set_param("gate_proj", sg)
    moe.shared_gate_up.set_param("up_proj", su)
    moe.shared_down.set_param("down_proj", sd)
    moe.shared_gate.set_param("shared_expert_gate", sgate)
    x = torch.randn(5, hidden).to(bf)
    res = torch.randn(5, hidden).to(bf)
    with torch.no_grad():
        ids, wts = moe.route(x)
        y = moe.forward(x, res)
        logits = moe.router.forward(x)
    tie = torch.randn(3, e).to(bf)
    tie[0, 7] = tie[0].max()                                   # a tie at the top: the lower index first
    tie[1, 2] = tie[1, 9] = tie[1].max() + 0.5
    probs = torch.softmax(tie.float(), dim=-1)
    tv, ti = torch.topk(probs, k, dim=-1)
    np.savez_compressed(HERE / "moe.npz", x=bf16_bits(x), res=bf16_bits(res), wr=bf16_bits(wr),
                        gate=np.stack([bf16_bits(a_) for a_, _, _ in egu]), up=np.stack([bf16_bits(b_) for _, b_, _ in egu]),
                        down=np.stack([bf16_bits(c_) for _, _, c_ in egu]), sg=bf16_bits(sg), su=bf16_bits(su),
                        sd=bf16_bits(sd), sgate=bf16_bits(sgate), logits=bf16_bits(logits), ids=ids.numpy().astype(np.int32),
                        wts=bf16_bits(wts), y=bf16_bits(y), top_k=k, tie_logits=bf16_bits(tie),
                        tie_ids=ti.numpy().astype(np.int32))
    # the attention step on BF16 caches directly (the helper the layer oracle calls)
    q = torch.randn(2, 4, 32).to(bf)
    kn_, vn_ = torch.randn(2, 2, 32).to(bf), torch.randn(2, 2, 32).to(bf)
    kc = torch.zeros(8, 2, 32, dtype=bf); vc = torch.zeros(8, 2, 32, dtype=bf)
    kc[:3], vc[:3] = torch.randn(3, 2, 32).to(bf), torch.randn(3, 2, 32).to(bf)
    kc0, vc0 = kc.clone(), vc.clone()
    with torch.no_grad():
        o = oracle.attention_step(q, kn_, vn_, kc, vc, 3, 32 ** -0.5)
    np.savez_compressed(HERE / "attention_step.npz", q=bf16_bits(q), k_new=bf16_bits(kn_), v_new=bf16_bits(vn_),
                        k_cache=bf16_bits(kc0), v_cache=bf16_bits(vc0), pos=3, out=bf16_bits(o))
    print("golden vectors written to", HERE)


if __name__ == "__main__":
    main()
