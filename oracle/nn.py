"""The layer math of the reference's torch oracles, restated in numpy float32 (float64 for matmul accumulation).

BF16 tensors are carried as float32 arrays holding BF16-representable values; every ``.to(bfloat16)`` of the
reference is an explicit :func:`rbf`. Sources: ``monolith/nn/oracle.py:20-134`` (helpers), ``nn/linear.py:114-135``
(projections and epilogues), ``nn/mlp.py:25-26``, ``nn/gdn.py:61-93``, ``nn/attention.py:212-243``,
``nn/moe.py:327-410``, ``nn/decoder.py:20-22``, ``nn/rope.py:19-64``, ``packs/transforms.py:16-24``.
"""

from __future__ import annotations

import numpy as np

from .fp import f16_round, rbf

F32 = np.float32


# ---- scalar helpers (torch semantics on float32) --------------------------------------------------------------------
def sigmoid(x):
    x = np.asarray(x, F32)
    return (F32(1) / (F32(1) + np.exp(-x))).astype(F32)


def silu(x):
    x = np.asarray(x, F32)
    return (x / (F32(1) + np.exp(-x))).astype(F32)


def softplus(x):
    """``F.softplus`` with ``beta = 1, threshold = 20``: ``x`` above the threshold, else ``log1p(exp(x))``."""
    x = np.asarray(x, F32)
    return np.where(x > 20, x, np.log1p(np.exp(np.minimum(x, 20)))).astype(F32)


def rsqrt(x):
    return (F32(1) / np.sqrt(np.asarray(x, F32))).astype(F32)


# ---- projections ---------------------------------------------------------------------------------------------------
def matmul_acc(x, w) -> np.ndarray:
    """``x @ wᵀ`` accumulated in float64 and returned as float32 (the fp32-accumulating GEMV, before rounding)."""
    return (np.asarray(x, np.float64) @ np.asarray(w, np.float64).T).astype(F32)


def linear(x, w, *, epilogue=None, residual=None, round_silu=False) -> np.ndarray:
    """``Linear.forward`` (``nn/linear.py:114-135``): FP32 accumulation, one BF16 rounding; ``residual`` adds before
    it; ``silu_mul`` takes the first half of the output columns as the gate and the second half as up."""
    acc = matmul_acc(x, w)
    if epilogue == "residual":
        acc = (acc + np.asarray(residual, F32)).astype(F32)
    elif epilogue == "silu_mul":
        half = acc.shape[-1] // 2
        g, u = acc[..., :half], acc[..., half:]
        if round_silu:                                  # the experts' two BF16 linears (nn/moe.py:333-336)
            g, u = rbf(g), rbf(u)
            return rbf(silu(g) * u)
        acc = (silu(g) * u).astype(F32)
    return rbf(acc)


def interleave_chunks(n_a: int, n_b: int, chunk: int) -> np.ndarray:
    """Row order of a ``gate|up`` slab: ``chunk`` gate rows, then the same ``chunk`` up rows, repeated
    (``packs/transforms.py:16-24``). ``perm[new] = old``."""
    if n_a != n_b or n_a % chunk:
        raise ValueError("interleave_chunks: need n_a == n_b, a multiple of chunk")
    idx = np.arange(n_a).reshape(-1, chunk)
    return np.concatenate([idx, idx + n_a], axis=1).reshape(-1)


# ---- norms and activations -----------------------------------------------------------------------------------------
def rms_norm(x, w, eps, *, one_plus=True) -> np.ndarray:
    """``oracle.rms_norm`` (``nn/oracle.py:25-32``): ``bf16(x · rsqrt(mean(x²) + eps) · (1 + w))`` in FP32."""
    xf = np.asarray(x, F32)
    y = (xf * rsqrt(np.mean(xf * xf, axis=-1, keepdims=True, dtype=F32) + F32(eps))).astype(F32)
    scale = (F32(1) + np.asarray(w, F32)) if one_plus else np.asarray(w, F32)
    return rbf(y * scale)


def gated_rms_norm(o, z, w, eps) -> np.ndarray:
    """``oracle.gated_rms_norm`` (``nn/oracle.py:35-41``): ``n = bf16(o·rsqrt(mean(o²)+eps))``, ``n = bf16(w·n)``,
    ``bf16(n · silu(z))``."""
    of = np.asarray(o, F32)
    n = rbf(of * rsqrt(np.mean(of * of, axis=-1, keepdims=True, dtype=F32) + F32(eps)))
    n = rbf(rbf(w) * n)
    return rbf(n * silu(z))


def l2norm(x, eps=1e-6) -> np.ndarray:
    x = np.asarray(x, F32)
    return (x * rsqrt(np.sum(x * x, axis=-1, keepdims=True, dtype=F32) + F32(eps))).astype(F32)


# ---- Gated DeltaNet --------------------------------------------------------------------------------------------------
def causal_conv1d(x, conv_state, w):
    """``oracle.causal_conv1d`` (``nn/oracle.py:76-88``): ``x [T, C]``, ``conv_state [C, W-1]``, ``w [C, W]`` →
    ``(bf16(silu(bf16(conv))) [T, C], new_state [C, W-1])``; taps accumulate in FP32 in order ``j = 0..W-1``."""
    x = np.asarray(x, F32)
    t, c = x.shape
    width = w.shape[-1]
    xs = np.concatenate([np.asarray(conv_state, F32), x.T], axis=-1)         # [C, W-1+T]
    y = np.zeros((c, t), F32)
    for j in range(width):
        y = (y + np.asarray(w, F32)[:, j:j + 1] * xs[:, j:j + t]).astype(F32)
    y = rbf(silu(rbf(y)))
    return np.ascontiguousarray(y.T), np.ascontiguousarray(xs[:, -(width - 1):])


def gated_delta_rule(q, k, v, g, beta, state):
    """``oracle.gated_delta_rule`` (``nn/oracle.py:91-109``): ``q, k [T, Hv, dk]``, ``v [T, Hv, dv]``,
    ``g, beta [T, Hv]``, ``state [Hv, dk, dv]`` FP32. Per token: ``S ← S·e^g``; ``Δ = (v − Σ_k S·k)·β``;
    ``S += k ⊗ Δ``; ``o = Σ_k S·q``. q is L2-normed and scaled by ``dk^-½``, k L2-normed. Returns
    ``(bf16 o [T, Hv, dv], new state)``."""
    qf = (l2norm(q) / F32(np.sqrt(F32(q.shape[-1])))).astype(F32)
    kf = l2norm(k)
    vf = np.asarray(v, F32)
    s = np.array(state, dtype=F32, copy=True)
    outs = []
    for i in range(qf.shape[0]):
        s = (s * np.exp(np.asarray(g[i], F32))[:, None, None]).astype(F32)
        kv_mem = np.sum(s * kf[i][:, :, None], axis=-2, dtype=F32)
        delta = ((vf[i] - kv_mem) * np.asarray(beta[i], F32)[:, None]).astype(F32)
        s = (s + kf[i][:, :, None] * delta[:, None, :]).astype(F32)
        outs.append(np.sum(s * qf[i][:, :, None], axis=-2, dtype=F32))
    return rbf(np.stack(outs)), s


def gdn_mix(proj, conv_state, rec_state, *, conv_w, a_log, dt_bias, norm_w, k_heads, v_heads, dk, dv, eps):
    """``GatedDeltaNet.mix`` (``nn/gdn.py:64-93``): ``proj [T, N1]`` in part order ``z | q | k | v | a | b``; returns
    ``(out [T, Hv·dv] bf16, new conv state, new rec state)``. ``beta = bf16(σ(b))``,
    ``g = −exp(A_log)·softplus(a + dt_bias)`` in FP32."""
    proj = np.asarray(proj, F32)
    t = proj.shape[0]
    kd, vd = k_heads * dk, v_heads * dv
    conv_dim = 2 * kd + vd
    z = proj[:, :vd]
    qkv = proj[:, vd: vd + conv_dim]
    a = proj[:, vd + conv_dim: vd + conv_dim + v_heads]
    b = proj[:, vd + conv_dim + v_heads: vd + conv_dim + 2 * v_heads]
    qkv, new_conv = causal_conv1d(qkv, conv_state, conv_w)
    q = qkv[:, :kd].reshape(t, k_heads, dk)
    k = qkv[:, kd: 2 * kd].reshape(t, k_heads, dk)
    v = qkv[:, 2 * kd:].reshape(t, v_heads, dv)
    beta = rbf(sigmoid(b))
    g = (-np.exp(np.asarray(a_log, F32)) * softplus(a + np.asarray(dt_bias, F32))).astype(F32)
    rep = v_heads // k_heads
    if rep > 1:
        q, k = np.repeat(q, rep, axis=1), np.repeat(k, rep, axis=1)
    o, new_rec = gated_delta_rule(q, k, v, g, beta, rec_state)
    y = gated_rms_norm(o.reshape(t * v_heads, dv), z.reshape(t * v_heads, dv), norm_w, eps)
    return y.reshape(t, vd), new_conv, new_rec


# ---- RoPE and attention ----------------------------------------------------------------------------------------------
def rope_tables(theta, rotary_dim, positions):
    """``cos``/``sin`` ``[P, rotary_dim]`` in FP32, ``cat(freqs, freqs)`` (``nn/oracle.py:49-55``)."""
    inv = (F32(1) / (F32(theta) ** (np.arange(0, rotary_dim, 2, dtype=F32) / F32(rotary_dim)))).astype(F32)
    freqs = (np.asarray(positions, F32)[:, None] * inv[None, :]).astype(F32)
    emb = np.concatenate([freqs, freqs], axis=-1)
    return np.cos(emb).astype(F32), np.sin(emb).astype(F32)


def apply_partial_rope(x, cos, sin):
    """``apply_partial_rope`` on BF16 tensors (``nn/oracle.py:58-69``): ``x [T, H, D]``, tables ``[T, r]`` already
    BF16; each elementwise op rounds to BF16 as torch's bf16 arithmetic does."""
    r = cos.shape[-1]
    c, s = cos[:, None, :], sin[:, None, :]
    xr, xp = x[..., :r], x[..., r:]
    h = r // 2
    rot = np.concatenate([-xr[..., h:], xr[..., :h]], axis=-1)
    return np.concatenate([rbf(rbf(xr * c) + rbf(rot * s)), xp], axis=-1)


def attention_step(q, k_new, v_new, k_cache, v_cache, pos, scaling):
    """``oracle.attention_step`` (``nn/oracle.py:112-134``): caches ``[ctx_max, Hkv, D]`` updated in place at
    ``pos..pos+T``; scores ``bf16(bf16(q·k)·scaling)``, causal inside the step, softmax FP32 → BF16, ``P·V`` FP32 →
    BF16. Returns ``[T, H, D]``."""
    t, h, d = q.shape
    hkv = k_new.shape[1]
    k_cache[pos: pos + t] = k_new
    v_cache[pos: pos + t] = v_new
    n = pos + t
    rep = h // hkv
    ks = np.repeat(np.asarray(k_cache[:n], np.float64), rep, axis=1)
    vs = np.repeat(np.asarray(v_cache[:n], np.float64), rep, axis=1)
    scores = np.einsum("thd,nhd->htn", np.asarray(q, np.float64), ks).astype(F32)
    scores = rbf(rbf(scores) * F32(scaling))
    if t > 1:
        causal = np.arange(n)[None, :] > (pos + np.arange(t))[:, None]
        scores = np.where(causal[None], -np.inf, scores).astype(F32)
    m = scores.max(-1, keepdims=True)
    e = np.exp((scores - m).astype(F32)).astype(F32)
    p = rbf(e / e.sum(-1, keepdims=True, dtype=F32))
    return rbf(np.einsum("htn,nhd->thd", p.astype(np.float64), vs).astype(F32))


def kv_quantize(x):
    """The build's int8 KV codec (the reference caches BF16, ``nn/attention.py:207-209``): per (token, head) row of
    ``D`` values, ``scale = f16(absmax / 127)``, ``code = clip(rint(x / scale), -127, 127)`` (0 when absmax = 0).
    Returns ``(codes int8 [..., D], scales float16 [...])``."""
    x = np.asarray(x, F32)
    amax = np.abs(x).max(axis=-1)
    scale = (amax / F32(127)).astype(F32).astype(np.float16)
    sf = scale.astype(F32)[..., None]
    q = np.where(sf > 0, np.rint(np.divide(x, sf, out=np.zeros_like(x), where=sf > 0)), 0)
    return np.clip(q, -127, 127).astype(np.int8), scale


def kv_dequantize(codes, scales):
    """``code · scale`` in FP32 (exact: 8-bit code × 11-bit scale)."""
    return (np.asarray(codes, F32) * np.asarray(scales, np.float16).astype(F32)[..., None]).astype(F32)


def gqa_prepare(proj, pos, *, heads, kv_heads, head_dim, rotary_dim, theta, eps, gate=True, qk_norm=False,
                q_norm=None, k_norm=None, tables=None):
    """The first half of ``GQAAttention.mix`` (``nn/attention.py:222-238``): split ``proj [T, N1]`` (checkpoint
    column order: ``q|gate`` per head, then ``k``, ``v``), optional q/k RMSNorm(1 + w), partial RoPE with BF16 tables.
    ``tables`` = BF16 ``(cos, sin) [ctx, rotary_dim]`` to use instead of numpy's (torch's FP32 ``cos``/``sin`` of
    large arguments differ from numpy's in the last bit, which flips a few BF16 roundings).
    Returns ``(q [T,H,D], k [T,Hkv,D], v [T,Hkv,D], gate [T,H,D] or None)``."""
    proj = np.asarray(proj, F32)
    t = proj.shape[0]
    d = head_dim
    q_rows = heads * (2 if gate else 1) * d
    if gate:
        qg = proj[:, :q_rows].reshape(t, heads, 2 * d)
        q, g = qg[..., :d], qg[..., d:]
    else:
        q, g = proj[:, :q_rows].reshape(t, heads, d), None
    k = proj[:, q_rows: q_rows + kv_heads * d].reshape(t, kv_heads, d)
    v = proj[:, q_rows + kv_heads * d: q_rows + 2 * kv_heads * d].reshape(t, kv_heads, d)
    if qk_norm:
        q = rms_norm(q, q_norm, eps)
        k = rms_norm(k, k_norm, eps)
    if tables is None:
        cos, sin = rope_tables(theta, rotary_dim, np.arange(pos, pos + t))
        cos, sin = rbf(cos), rbf(sin)
    else:
        cos, sin = (np.asarray(tb, F32)[pos: pos + t] for tb in tables)
    return apply_partial_rope(q, cos, sin), apply_partial_rope(k, cos, sin), v, g


def _gate(o, g, heads, head_dim):
    if g is not None:
        o = rbf(o * rbf(sigmoid(g)))
    return o.reshape(o.shape[0], heads * head_dim)


def gqa_mix_bf16(proj, k_cache, v_cache, pos, **cfg):
    """``GQAAttention.mix`` over BF16 caches ``[ctx_max, Hkv, D]`` (updated in place) — the reference's layer."""
    q, k, v, g = gqa_prepare(proj, pos, **cfg)
    o = attention_step(q, k, v, k_cache, v_cache, pos, cfg["head_dim"] ** -0.5)
    return _gate(o, g, cfg["heads"], cfg["head_dim"])


def gqa_mix(proj, k_codes, k_scales, v_codes, v_scales, pos, **cfg):
    """The same layer over the build's int8 cache (codes ``[ctx_max, Hkv, D]`` int8, scales ``[ctx_max, Hkv]`` f16,
    updated in place): the fresh k/v are quantized into the cache at ``pos..pos+T`` and the step attends over the
    dequantized cache, new tokens included."""
    q, k, v, g = gqa_prepare(proj, pos, **cfg)
    t = q.shape[0]
    kc, ks = kv_quantize(k)
    vc, vs = kv_quantize(v)
    k_codes[pos: pos + t], k_scales[pos: pos + t] = kc, ks
    v_codes[pos: pos + t], v_scales[pos: pos + t] = vc, vs
    n = pos + t
    kd = kv_dequantize(k_codes[:n], k_scales[:n])
    vd = kv_dequantize(v_codes[:n], v_scales[:n])
    o = attention_step(q, kd[pos:n], vd[pos:n], kd.copy(), vd.copy(), pos, cfg["head_dim"] ** -0.5)
    return _gate(o, g, cfg["heads"], cfg["head_dim"])


# ---- MoE -------------------------------------------------------------------------------------------------------------
def moe_route(logits, top_k, renorm=True):
    """``SparseMoE.route`` (``nn/moe.py:383-393``) / ``moe_route.metal``: softmax in FP32 over BF16 logits, top-k with
    ties to the lowest index, optional renormalization, weights rounded to BF16. Returns ``(ids int32, weights)``."""
    lg = np.asarray(logits, F32)
    e = np.exp((lg - lg.max(-1, keepdims=True)).astype(F32)).astype(F32)
    p = (e / e.sum(-1, keepdims=True, dtype=F32)).astype(F32)
    order = np.argsort(-p, axis=-1, kind="stable")[:, :top_k]          # stable: equal probabilities keep index order
    ids = order.astype(np.int32)
    w = np.take_along_axis(p, order, axis=-1).astype(F32)
    if renorm:
        w = (w / w.sum(-1, keepdims=True, dtype=F32)).astype(F32)
    return ids, rbf(w)


def expert_forward(x, w_gate_up, w_down):
    """``Experts.forward_expert`` for the gate|up then down slabs (``nn/moe.py:327-337``): two BF16-rounded linears,
    ``bf16(silu(gate)·up)``, then the down linear rounded to BF16. ``w_gate_up`` is ``[gate; up]`` (un-interleaved)."""
    act = linear(x, w_gate_up, epilogue="silu_mul", round_silu=True)
    return linear(act, w_down)


def moe_forward(x, residual, logits, top_k, w_gate_up, w_down, *, renorm=True, shared=None):
    """``SparseMoE.forward`` (``nn/moe.py:395-410``). ``w_gate_up [E, 2I, H]``, ``w_down [E, H, I]`` dequantized
    float32; ``shared = (w_gate_up_s, w_down_s, w_gate_s [1, H])`` or None. Sum in FP32, one rounding."""
    ids, w = moe_route(logits, top_k, renorm)
    t = x.shape[0]
    out = np.zeros((t, w_down.shape[1]), F32)
    for tt in range(t):
        for j in range(top_k):
            e = int(ids[tt, j])
            d = expert_forward(x[tt: tt + 1], w_gate_up[e], w_down[e])
            out[tt] = (out[tt] + w[tt, j] * d[0]).astype(F32)
    if shared is not None:
        gu, dn, gw = shared
        s = linear(linear(x, gu, epilogue="silu_mul"), dn)
        gate = rbf(sigmoid(linear(x, gw)))
        out = (out + gate * s).astype(F32)
    return rbf(out + np.asarray(residual, F32)), ids, w


def moe_combine(h, weights, residual=None, shared=None, shared_gate=None):
    """``moe_combine`` (``kernels/common/moe_combine.metal:19-49``): ``Σ_j w_j·h_j (+ bf16(σ(gate))·shared)
    (+ residual)`` in FP32, one rounding. ``h [T, k, H]``."""
    acc = np.einsum("tk,tkh->th", np.asarray(weights, np.float64), np.asarray(h, np.float64))
    if shared is not None:
        acc = acc + rbf(sigmoid(shared_gate)).astype(np.float64) * np.asarray(shared, np.float64)
    if residual is not None:
        acc = acc + np.asarray(residual, np.float64)
    return rbf(acc.astype(F32))


__all__ = [n for n in dir() if not n.startswith("_")] + ["f16_round"]
