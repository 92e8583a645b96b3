"""Execute one op through the C ABI: ``run(kind, *inputs, **attrs)`` with the reference op's inputs and attrs
(the handler table of ``monolith/compiler/emit.py:1381-1386``, here calling the typed kernels of
:mod:`monolith_mi355.kernels` instead of encoding Metal dispatches). A kind without a gfx950 binding raises
:class:`~monolith_mi355.ops.coverage.CoverageError`; a fused op (``norm_apply`` into ``gemv`` …) must be run through
the op that carries it."""

from __future__ import annotations

from .. import kernels
from .coverage import CoverageError, check_coverage
from .registry import OPS, PROFILE


def _gemv(x, w, *, norm_w=None, eps=1e-6, epilogue=None, residual=None, out=None, stream=None, **_):
    return kernels.gemv(w, x, epilogue=epilogue, residual=residual, norm_w=norm_w, eps=eps, out=out, stream=stream)


def _lm_head(x, w, *, norm_w=None, eps=1e-6, out=None, stream=None, **_):
    return kernels.gemv(w, x, norm_w=norm_w, eps=eps, out=out, stream=stream, out_f32=True)


def _gqa(proj, cache, *, position, heads, rope_cos, rope_sin, gate=True, q_norm=None, k_norm=None, eps=1e-6,
         scaling=None, out=None, stream=None, **_):
    return kernels.gqa_decode(proj, cache, position, heads=heads, rope_cos=rope_cos, rope_sin=rope_sin, gate=gate,
                              q_norm=q_norm, k_norm=k_norm, eps=eps, scaling=scaling, out=out, stream=stream)


def _gdn(proj, conv_in, conv_out, rec_in, rec_out, *, conv_w, neg_exp_a, dt_bias, norm_w, k_heads, v_heads, dk=128,
         dv=128, conv_width=4, eps=1e-6, ab=None, offsets=None, out=None, stream=None, **_):
    return kernels.gdn_step(proj, conv_in, conv_out, rec_in, rec_out, conv_w=conv_w, neg_exp_a=neg_exp_a,
                            dt_bias=dt_bias, norm_w=norm_w, k_heads=k_heads, v_heads=v_heads, dk=dk, dv=dv,
                            conv_width=conv_width, eps=eps, ab=ab, offsets=offsets, out=out, stream=stream)


def _gdn_commit(proj, conv_in, conv_out, rec_in, rec_out, *, conv_w, neg_exp_a, dt_bias, norm_w, k_heads, v_heads,
                dk=128, dv=128, conv_width=4, eps=1e-6, ab=None, offsets=None, committed=None, stream=None, **_):
    """``committed``: the accept scan's count of committed tokens as a device int32 (None: every row of proj)."""
    return kernels.gdn_step(proj, conv_in, conv_out, rec_in, rec_out, conv_w=conv_w, neg_exp_a=neg_exp_a,
                            dt_bias=dt_bias, norm_w=norm_w, k_heads=k_heads, v_heads=v_heads, dk=dk, dv=dv,
                            conv_width=conv_width, eps=eps, ab=ab, offsets=offsets, commit=True, t_dev=committed,
                            stream=stream)


def _route(logits, *, top_k, renorm=True, stream=None, **_):
    return kernels.moe_route(logits, top_k, renorm=renorm, stream=stream)


def _moe_gemv(x, w, groups, *, tokens, top_k, x_per_slot=False, epilogue=None, norm_w=None, eps=1e-6, out=None,
              stream=None, **_):
    return kernels.moe_gemv(w, x, groups, tokens=tokens, top_k=top_k, x_per_slot=x_per_slot, epilogue=epilogue,
                            norm_w=norm_w, eps=eps, out=out, stream=stream)


def _combine(h, weights, shared=None, shared_gate=None, residual=None, *, top_k, out=None, stream=None, **_):
    return kernels.moe_combine(h, weights, top_k=top_k, shared=shared, shared_gate=shared_gate, residual=residual,
                               out=out, stream=stream)


def _embed(tokens, table, *, t=None, out=None, stream=None, **_):
    return kernels.embed(table, tokens, t=t, out=out, stream=stream)


def _argmax(logits, *, out=None, stream=None, **_):
    return kernels.argmax(logits, out=out, stream=stream)


def _sample(logits, *, temperature=1.0, top_k=0, top_p=0.0, min_p=0.0, topp_in_topk=False, seed=0, step=0,
            state=None, out=None, stream=None, **_):
    return kernels.sample(logits, temperature=temperature, top_k=top_k, top_p=top_p, min_p=min_p,
                          topp_in_topk=topp_in_topk, seed=seed, step=step, state=state, out=out, stream=stream)


def _verify_select(drafts, conf, *, state, gamma, threshold=0.0, t_max=8, mode=0, cost=None, conf_log=None, ctx_cap=0,
                   lm=False, stream=None, **_):
    return kernels.verify_select(state, drafts, conf, gamma=gamma, threshold=threshold, t_max=t_max, mode=mode,
                                 cost=cost, conf_log=conf_log, ctx_cap=ctx_cap, lm=lm, stream=stream)


def _accept_scan(token, *, state, ring, ring_cap, eos=(), log=None, ctx_cap=0, lm=False, host_ctl=None, stream=None,
                 **_):
    return kernels.accept_scan(state, token, ring, ring_cap, eos=eos, log=log, ctx_cap=ctx_cap, lm=lm,
                               host_ctl=host_ctl, stream=stream)


HANDLERS = {"embed": _embed, "argmax": _argmax, "sample": _sample, "verify_select": _verify_select, "accept_scan": _accept_scan, "gemv": _gemv, "lm_head": _lm_head, "gqa_decode": _gqa, "gdn_mixer": _gdn, "gdn_commit": _gdn_commit,
            "moe_route": _route, "moe_gemv": _moe_gemv, "moe_combine": _combine}


def run(kind: str, *inputs, **attrs):
    check_coverage([kind])
    binding = OPS[kind].binding_for(PROFILE)
    carrier = binding.function_constants.get("fused_into")
    if carrier is not None:
        raise CoverageError(PROFILE, [(kind, OPS[kind])]) from ValueError(
            f"{kind} runs inside {carrier} on this backend ({binding.kernel}); run {carrier} with its inputs")
    return HANDLERS[kind](*inputs, **attrs)
