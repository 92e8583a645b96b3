"""The HIP MoE path against the oracle (the reference's ``tests/kernels/test_moe_ops.py`` strategy and bars):

* ``moe_route``: ids bit-exact against the oracle's routing (ties to the lowest index, a forced tie included), weights
  BF16-valued and within 2^-8 of the largest weight (``test_moe_ops.py:66-67``), at the reference's test shapes and
  the BASELINE 256 experts / top-8; the expert groups cover every (token, slot) pair exactly once;
* the grouped expert GEMV (``moe_gemv``): every pair's row against a float64 matmul of that expert's exact
  dequantized matrix (per-slot and per-token inputs, plain and silu·mul), one BF16 ULP of its own magnitude;
* ``moe_combine`` within one BF16 ULP (``test_moe_ops.py:119-144``);
* the whole sparse MoE block at the BASELINE geometry (hidden 2048, expert intermediate 512, NVFP4 experts, top-8,
  a shared expert, fused input RMSNorm) for M = 1 and 8, against ``SparseMoE.forward``'s restatement fed the same
  router logits (``ok_rounded``).
"""

import numpy as np
import pytest

from helpers import from_dev_bf16, spec_of, to_dev_bf16
from oracle import formats as OF
from oracle import nn as ON
from oracle.fp import bf16_to_f32, f32_to_bf16, rbf
from oracle.gates import check_against_oracle

GROUP_REC = 18


def _check_groups(groups, ids, t, k):
    g = groups.cpu().numpy()
    ids = ids.cpu().numpy()
    seen = []
    for rec in g:
        e, cnt = int(rec[0]), int(rec[1])
        if cnt == 0:
            assert e == -1
            continue
        pairs = rec[2: 2 + cnt]
        assert np.all(np.diff(pairs) > 0)
        for p in pairs:
            assert ids[p // k, p % k] == e
        seen += list(pairs)
    assert sorted(seen) == list(range(t * k))
    used = [int(r[0]) for r in g if r[1] > 0]
    assert len(used) == len(set(used)) == len(np.unique(ids))


@pytest.mark.gpu
@pytest.mark.parametrize("n_experts,k,renorm", [(8, 2, True), (60, 4, False), (128, 8, True), (5, 5, False),
                                                (256, 8, True), (256, 8, False)])
@pytest.mark.parametrize("t", [1, 5, 8, 16])
def test_moe_route(torch_gpu, n_experts, k, renorm, t):
    from monolith_mi355 import kernels
    rng = np.random.default_rng(n_experts * 10 + t)
    logits = rbf(rng.standard_normal((t, n_experts)) * 2)
    if t > 1:
        logits[1, 3] = logits[1, 0]                         # a tie: the lower index wins
    ids, w, groups = kernels.moe_route(to_dev_bf16(torch_gpu, logits), k, renorm=renorm)
    ref_ids, ref_w = ON.moe_route(logits, k, renorm)
    got_w = w.cpu().numpy()
    assert np.array_equal(ids.cpu().numpy(), ref_ids)
    assert np.allclose(got_w, ref_w, rtol=0, atol=2 ** -8 * ref_w.max()) and np.array_equal(got_w, rbf(got_w))
    _check_groups(groups, ids, t, k)


@pytest.mark.gpu
def test_moe_route_tied_logits_and_underflow(torch_gpu):
    """Exact ties among the top probabilities and probabilities that underflow to 0 both resolve by index."""
    from monolith_mi355 import kernels
    logits = np.zeros((3, 256), np.float32)
    logits[0, [6, 7, 9]] = 1.0                                # three-way tie at the top
    logits[1, :] = -120.0
    logits[1, 2] = logits[1, 9] = 0.0                         # everything else underflows to p = 0
    logits[2] = rbf(np.linspace(-3, 3, 256))[::-1]
    logits = rbf(logits)
    ids, w, _ = kernels.moe_route(to_dev_bf16(torch_gpu, logits), 8, renorm=False)
    ref_ids, ref_w = ON.moe_route(logits, 8, renorm=False)
    assert np.array_equal(ids.cpu().numpy(), ref_ids)
    assert list(ids.cpu().numpy()[1, :4]) == [2, 9, 0, 1]


@pytest.mark.gpu
@pytest.mark.parametrize("t", [1, 8, 16])
def test_moe_route_512_experts_with_the_shared_expert_last(torch_gpu, t):
    """The largest expert table (512) with the shared expert at index 512: ids and weights match the oracle, the
    shared slot carries bf16(σ(gate logit)), and the groups cover every pair once — the grouping's per-expert LDS
    tables hold index 512 (one past the routed experts)."""
    from monolith_mi355 import kernels
    torch = torch_gpu
    rng = np.random.default_rng(512 + t)
    e, k = 512, 8
    logits = rbf(rng.standard_normal((t, e + 1)) * 2)        # column 512: the shared expert's gate logit
    for ppr in (0, 2):
        ids, w, groups = kernels.moe_route(to_dev_bf16(torch, logits)[:, :e], k, renorm=True, shared_expert=e,
                                           shared_gate=e, pairs_per_record=ppr)
        ref_ids, ref_w = ON.moe_route(logits[:, :e], k, True)
        got_ids, got_w = ids.cpu().numpy(), w.cpu().numpy()
        assert np.array_equal(got_ids[:, :k], ref_ids)
        assert np.all(got_ids[:, k] == e)
        assert np.allclose(got_w[:, :k], ref_w, rtol=0, atol=2 ** -8 * ref_w.max())
        sg = 1.0 / (1.0 + np.exp(-logits[:, e].astype(np.float64)))
        assert np.array_equal(got_w[:, k], rbf(got_w[:, k])) and np.all(np.abs(got_w[:, k] - sg) <= 2 ** -8)
        g = groups.cpu().numpy()
        seen = sorted(int(p) for rec in g if rec[1] > 0 for p in rec[2: 2 + rec[1]])
        assert seen == list(range(t * (k + 1)))
        for rec in g:
            for p in rec[2: 2 + rec[1]]:
                assert got_ids[p // (k + 1), p % (k + 1)] == rec[0]
        assert sum(int(rec[1]) for rec in g if rec[0] == e) == t


def _experts(rng, n_exp, inter, hidden):
    """Per expert: gate|up slab (chunk-interleaved by 8, per-row tensor scales) and down, plus their exact
    dequantized float32 matrices ([gate; up] un-interleaved)."""
    perm = ON.interleave_chunks(inter, inter, 8)
    gu_specs, gu_scales, dn_specs, dn_scales, w_gu, w_dn = [], [], [], [], [], []
    for _ in range(n_exp):
        gate, up, down = OF.nvfp4_random(inter, hidden, rng), OF.nvfp4_random(inter, hidden, rng), OF.nvfp4_random(hidden, inter, rng)
        slab = OF.permute_rows(OF.stack_rows([gate, up]), perm)
        gu_specs.append(spec_of(dict(slab, weight_scale_2=1.0)))
        gu_scales.append(slab["row_scale"])
        dn_specs.append(spec_of(dict(down, weight_scale_2=1.0)))
        dn_scales.append(np.full(hidden, down["weight_scale_2"], np.float32))
        w_gu.append(np.concatenate([OF.dequantize(gate), OF.dequantize(up)]))
        w_dn.append(OF.dequantize(down))
    return gu_specs, gu_scales, dn_specs, dn_scales, np.stack(w_gu), np.stack(w_dn)


@pytest.mark.gpu
@pytest.mark.parametrize("x_per_slot,epilogue", [(False, None), (True, None), (False, "silu_mul_rounded"),
                                                 (False, "silu_mul")])
@pytest.mark.parametrize("t", [1, 3, 8])
def test_moe_gemv_pairs_stream_the_chosen_experts(torch_gpu, x_per_slot, epilogue, t):
    torch = torch_gpu
    from monolith_mi355 import kernels
    rng = np.random.default_rng(t + 7 * x_per_slot)
    n_exp, inter, hidden, k = 6, 64, 256, 2
    gu_specs, gu_scales, _, _, w_gu, _ = _experts(rng, n_exp, inter, hidden)
    w = kernels.upload(gu_specs, row_scales=gu_scales)
    ids = rng.integers(0, n_exp, (t, k)).astype(np.int32)
    for row in ids:                                           # distinct experts per token, as top-k gives
        while row[0] == row[1]:
            row[1] = rng.integers(0, n_exp)
    logits = np.full((t, n_exp), -4.0, np.float32)            # route logits that pick exactly `ids`
    for tt in range(t):
        logits[tt, ids[tt, 0]], logits[tt, ids[tt, 1]] = 2.0, 1.0
    rid, _, groups = kernels.moe_route(to_dev_bf16(torch, rbf(logits)), k, renorm=False)
    assert np.array_equal(rid.cpu().numpy(), ids)
    x = rbf(rng.uniform(-1, 1, (t * k if x_per_slot else t, hidden)))
    got = from_dev_bf16(kernels.moe_gemv(w, to_dev_bf16(torch, x), groups, tokens=t, top_k=k, x_per_slot=x_per_slot,
                                         epilogue=epilogue))
    for p in range(t * k):
        e = ids[p // k, p % k]
        xr = x[p] if x_per_slot else x[p // k]
        if epilogue:
            ref = ON.linear(xr[None], w_gu[e], epilogue="silu_mul", round_silu=epilogue == "silu_mul_rounded")[0]
        else:
            ref = ON.linear(xr[None], np.concatenate([w_gu[e][ON.interleave_chunks(inter, inter, 8)]]))[0]
        chk = check_against_oracle(got[p], ref)
        assert chk.ok_rounded() and chk.within and chk.max_ulp_elementwise <= 1, (p, chk)


@pytest.mark.gpu
@pytest.mark.parametrize("shared,residual", [(False, True), (True, True), (True, False), (False, False)])
def test_moe_combine(torch_gpu, shared, residual):
    torch = torch_gpu
    from monolith_mi355 import kernels
    rng = np.random.default_rng(3)
    t, k, hidden = 4, 3, 96
    h = rbf(rng.standard_normal((t * k, hidden)))
    w = rbf(rng.uniform(0, 1, (t, k)))
    sh = rbf(rng.standard_normal((t, hidden)))
    gate = rbf(rng.standard_normal((t, 1)))
    res = rbf(rng.standard_normal((t, hidden)))
    got = from_dev_bf16(kernels.moe_combine(to_dev_bf16(torch, h), torch.from_numpy(w).cuda(), top_k=k,
                                            shared=to_dev_bf16(torch, sh) if shared else None,
                                            shared_gate=to_dev_bf16(torch, gate) if shared else None,
                                            residual=to_dev_bf16(torch, res) if residual else None))
    ref = ON.moe_combine(h.reshape(t, k, hidden), w, residual=res if residual else None,
                         shared=sh if shared else None, shared_gate=gate if shared else None)
    chk = check_against_oracle(got, ref)
    assert chk.ok_rounded() and chk.within and chk.max_ulp_elementwise <= 1, chk


@pytest.mark.gpu
@pytest.mark.parametrize("t", [1, 8])
def test_sparse_moe_block_baseline_geometry(torch_gpu, t):
    """hidden 2048, expert intermediate 512 (NVFP4), top-8 of 32 experts (256 in the routing tests: the grouped GEMV
    streams only the chosen experts, so E changes nothing but the slab size), shared expert 512, fused RMSNorm."""
    torch = torch_gpu
    from monolith_mi355 import kernels
    rng = np.random.default_rng(100 + t)
    n_exp, k, inter, hidden, si, eps = 32, 8, 512, 2048, 512, 1e-6
    gu_specs, gu_scales, dn_specs, dn_scales, w_gu, w_dn = _experts(rng, n_exp, inter, hidden)
    w_gu_d = kernels.upload(gu_specs, row_scales=gu_scales)
    w_dn_d = kernels.upload(dn_specs, row_scales=dn_scales)
    sgu_specs, sgu_scales, sdn_specs, sdn_scales, s_gu, s_dn = _experts(rng, 1, si, hidden)
    s_gu_d = kernels.upload(sgu_specs, row_scales=sgu_scales)
    s_dn_d = kernels.upload(sdn_specs, row_scales=sdn_scales)
    router = {"format": "bf16", "weight": f32_to_bf16((rng.standard_normal((n_exp, hidden)) * 0.02).astype(np.float32))}
    sgate = {"format": "bf16", "weight": f32_to_bf16((rng.standard_normal((1, hidden)) * 0.02).astype(np.float32))}
    r_d, sg_d = kernels.upload(spec_of(router)), kernels.upload(spec_of(sgate))
    h = rbf(rng.standard_normal((t, hidden)))
    wn = rbf(rng.standard_normal(hidden) * 0.1)
    nw = torch.from_numpy((1 + wn).astype(np.float32)).cuda()
    hd = to_dev_bf16(torch, h)

    logits = kernels.gemv(r_d, hd, norm_w=nw, eps=eps)
    ids, wts, groups = kernels.moe_route(logits, k, renorm=True)
    act = kernels.moe_gemv(w_gu_d, hd, groups, tokens=t, top_k=k, x_per_slot=False, epilogue="silu_mul_rounded",
                           norm_w=nw, eps=eps)
    hk = kernels.moe_gemv(w_dn_d, act, groups, tokens=t, top_k=k, x_per_slot=True)
    s_act = kernels.gemv(s_gu_d, hd, epilogue="silu_mul", norm_w=nw, eps=eps)
    s_out = kernels.gemv(s_dn_d, s_act)
    s_gate = kernels.gemv(sg_d, hd, norm_w=nw, eps=eps)
    y = kernels.moe_combine(hk, wts, top_k=k, shared=s_out, shared_gate=s_gate, residual=hd)
    torch.cuda.synchronize()

    xn = ON.rms_norm(h, wn, eps)
    got_logits = from_dev_bf16(logits)
    chk = check_against_oracle(got_logits, ON.linear(xn, bf16_to_f32(router["weight"])))
    assert chk.ok_rounded() and chk.within, chk
    ref, ref_ids, _ = ON.moe_forward(xn, h, got_logits, k, w_gu, w_dn, renorm=True,
                                     shared=(s_gu[0], s_dn[0], bf16_to_f32(sgate["weight"])))
    assert np.array_equal(ids.cpu().numpy(), ref_ids)
    chk = check_against_oracle(from_dev_bf16(y), ref)
    assert chk.ok_rounded() and chk.within, chk


@pytest.mark.gpu
@pytest.mark.parametrize("t", [1, 5, 16])
def test_moe_route_with_the_shared_expert_slot(torch_gpu, t):
    """``shared_expert``: the routed slots exactly as without it; slot k = the shared expert (index E) with weight
    bf16(σ(logit of the gate column)); the groups hold every pair once, one record for the shared expert with the t
    pairs p = tok·(k + 1) + k, and the routed experts' records in the same first-use order as without it."""
    torch = torch_gpu
    from monolith_mi355 import kernels
    rng = np.random.default_rng(t)
    e, k = 64, 8
    lg = rbf(rng.standard_normal((t, 72)))               # E logits, then the shared gate's column, padding
    dev = to_dev_bf16(torch, lg)
    ids, w, groups = kernels.moe_route(dev[:, :e], k, renorm=True, shared_expert=e, shared_gate=e)
    ids, w, groups = ids.cpu().numpy(), w.cpu().numpy(), groups.cpu().numpy()
    ref_ids, ref_w = ON.moe_route(lg[:, :e], k, True)
    assert np.array_equal(ids[:, :k], ref_ids) and np.array_equal(w[:, :k], ref_w)
    assert (ids[:, k] == e).all() and np.array_equal(w[:, k], rbf(ON.sigmoid(lg[:, e])))
    recs = groups[groups[:, 1] > 0]
    sh = recs[recs[:, 0] == e]
    assert len(sh) == 1 and list(sh[0, 2: 2 + t]) == [tok * (k + 1) + k for tok in range(t)]
    pairs = sorted(int(p) for r in recs for p in r[2: 2 + r[1]])
    assert pairs == list(range(t * (k + 1)))
    # the routed experts' records: the same experts, in the same first-use order, as without the shared slot
    plain = kernels.moe_route(dev[:, :e], k, renorm=True)[2].cpu().numpy()
    assert list(recs[recs[:, 0] != e, 0]) == list(plain[plain[:, 1] > 0, 0])


@pytest.mark.gpu
@pytest.mark.parametrize("nan_row", [False, True])
def test_moe_gemv_routes_for_itself_at_one_token(torch_gpu, nan_row):
    """At one token the expert gate|up launch routes for itself (``route=``): the same ids and weights as
    ``moe_route`` bit for bit, the group records slot by slot (one pair each), and the same activations as the
    launch fed ``moe_route``'s groups; a NaN logits row routes nowhere (experts -1, weight 0, no group computes)."""
    torch = torch_gpu
    from monolith_mi355 import kernels
    from monolith_mi355.layers import MoeBlock
    blk = MoeBlock(experts=64, seed=7)
    e, k = 64, 8
    rng = np.random.default_rng(3)
    h = to_dev_bf16(torch, rbf(rng.standard_normal((1, 2048))))
    lg = rbf(rng.standard_normal((1, 72)))
    if nan_row:
        lg[0, :e] = np.nan
    logits = to_dev_bf16(torch, lg)
    ids_a, w_a, g_a = kernels.moe_route(logits[:, :e], k, renorm=True, shared_expert=e, shared_gate=e)
    act_a = kernels.moe_gemv(blk.gate_up_s, h, g_a, tokens=1, top_k=k + 1, x_per_slot=False,
                             epilogue="silu_mul_rounded", norm_w=blk.norm_w, shared_expert=e,
                             shared_epilogue="silu_mul")
    ids_b = torch.full((1, k + 1), -7, dtype=torch.int32, device="cuda")
    w_b = torch.zeros(1, k + 1, dtype=torch.float32, device="cuda")
    g_b = torch.full((k + 1, kernels.GROUP_REC), -7, dtype=torch.int32, device="cuda")
    act_b = torch.zeros_like(act_a)
    kernels.moe_gemv(blk.gate_up_s, h, g_b, tokens=1, top_k=k + 1, x_per_slot=False, epilogue="silu_mul_rounded",
                     norm_w=blk.norm_w, shared_expert=e, shared_epilogue="silu_mul", out=act_b,
                     route=dict(logits=logits[:, :e], ids=ids_b, weights=w_b, top_k=k, renorm=True, gate_col=e))
    torch.cuda.synchronize()
    assert torch.equal(ids_a, ids_b) and torch.equal(w_a.view(torch.int32), w_b.view(torch.int32))
    gb = g_b.cpu().numpy()
    ib = ids_b.cpu().numpy()[0]
    assert list(gb[:, 0]) == list(ib) and list(gb[:, 1]) == [int(x >= 0) for x in ib] and list(gb[:, 2]) == list(range(k + 1))
    rows = [r for r in range(k + 1) if ib[r] >= 0]                   # slots with an expert were computed
    assert torch.equal(act_a[rows], act_b[rows])
    if nan_row:
        assert (ib[:k] == -1).all() and ib[k] == e and len(rows) == 1


def test_moe_rejects_bad_descriptors():
    import ctypes as C
    from monolith_mi355.runtime import hip
    lib = hip.load()
    base = dict(t=2, n_experts=256, top_k=8, renorm=1, logits=256, ld_logits=256, ids=256, weights=256, groups=0,
                max_groups=0)
    for kw in (dict(t=0), dict(t=17), dict(n_experts=513), dict(top_k=17), dict(top_k=0), dict(ld_logits=100),
               dict(groups=256, max_groups=10), dict(logits=0), dict(shared_expert=100, shared_gate_col=256),
               dict(shared_expert=200, shared_gate_col=0)):
        assert lib.mi_moe_route(C.byref(hip.MiMoeRouteDesc(**{**base, **kw})), None) == 1, kw
        assert hip.last_error().startswith("mi_moe_route")
    cb = dict(t=2, hidden=2048, top_k=8, h=256, ldh=2048, weights=256, out=256, ldo=2048)
    for kw in (dict(hidden=2044), dict(ldh=2047), dict(h=8), dict(shared=256, ld_shared=2048), dict(out=0)):
        assert lib.mi_moe_combine(C.byref(hip.MiMoeCombineDesc(**{**cb, **kw})), None) == 1, kw
        assert hip.last_error().startswith("mi_moe_combine")


class _LazyExperts:
    """``[E, rows, cols]`` dequantized expert matrices, each decoded on first use (256 experts of C5 would take
    3 GB of host memory dense; a step touches at most 64)."""

    def __init__(self, decode, n, shape):
        self.decode, self.shape, self.cache = decode, (n, *shape), {}

    def __getitem__(self, e):
        e = int(e)
        if e not in self.cache:
            self.cache[e] = self.decode(e)
        return self.cache[e]


@pytest.mark.gpu
@pytest.mark.parametrize("t", [1, 8])
@pytest.mark.parametrize("n_exp", [32, 256])
def test_moe_block_layer(torch_gpu, t, n_exp):
    """layers.MoeBlock (the bench's MoE workload; 256 experts is C5) against the oracle's SparseMoE forward, with its
    own weights dequantized bit-exactly on the device (gate|up rows un-interleaved): route ids equal — from the
    device's router logits, where those equal the oracle's router GEMV bit for bit from the oracle's, and on every
    row from the oracle's router logits routed by the device — output
    within the bars (``ok_rounded`` and 1e-2 relative / 1e-3 absolute element-wise)."""
    torch = torch_gpu
    from monolith_mi355 import kernels
    from monolith_mi355.layers import MoeBlock
    print(f"moe block t={t} experts={n_exp}", flush=True)
    blk = MoeBlock(experts=n_exp, seed=3)
    rng = np.random.default_rng(40 + t)
    h = rbf(rng.standard_normal((t, 2048)))
    hd = to_dev_bf16(torch, h)
    y = from_dev_bf16(blk(hd))
    both = from_dev_bf16(blk.buffers(t)[0])           # router logits | the shared gate's logit, one GEMV
    logits, gate = both[:, :n_exp], both[:, n_exp:n_exp + 1]
    ids_all = blk.buffers(t)[1][0].cpu().numpy()
    ids = ids_all[:, :8]
    if blk.fused_shared:                               # the shared expert: slot 8 of every token, weight bf16(σ(gate))
        assert (ids_all[:, 8] == n_exp).all()
        w_all = blk.buffers(t)[1][1].cpu().numpy()
        assert np.array_equal(w_all[:, 8], rbf(ON.sigmoid(gate[:, 0])))

    def dense(w, expert=0, gate_up=False):
        d = kernels.dequant(w, expert=expert).cpu().numpy()
        if gate_up:
            n, k = d.shape
            d = d.reshape(n // 16, 2, 8, k)
            d = np.concatenate([d[:, 0].reshape(-1, k), d[:, 1].reshape(-1, k)])
        return d

    w_gu = _LazyExperts(lambda e: dense(blk.gate_up, e, True), n_exp, (1024, 2048))
    w_dn = _LazyExperts(lambda e: dense(blk.down, e), n_exp, (2048, 512))
    s_gu, s_dn = dense(blk.shared_gate_up.packed, 0, True), dense(blk.shared_down.packed)
    wn = (blk.norm_w.cpu().numpy() - 1.0).astype(np.float32)
    xn = ON.rms_norm(h, wn, 1e-6)
    from oracle.fp import bf16_to_f32
    rw = bf16_to_f32(blk.router_w.view(torch.int16).cpu().numpy().astype(np.uint16))
    gw = bf16_to_f32(blk.shared_gate_w.view(torch.int16).cpu().numpy().astype(np.uint16))
    ref_logits = ON.linear(xn, rw)
    chk_l = check_against_oracle(logits, ref_logits)
    assert chk_l.ok_rounded() and chk_l.within, chk_l
    chk_g = check_against_oracle(gate, ON.linear(xn, gw))
    assert chk_g.ok_rounded() and chk_g.within, chk_g
    ref, ref_ids, _ = ON.moe_forward(xn, h, logits, 8, w_gu, w_dn, renorm=True, shared=(s_gu, s_dn, gw))
    assert np.array_equal(ids, ref_ids)
    same = np.all(logits.view(np.uint32) == rbf(ref_logits).view(np.uint32), axis=1)
    oracle_ids, _ = ON.moe_route(rbf(ref_logits), 8, True)
    assert np.array_equal(ids[same], oracle_ids[same])         # end to end from the oracle's own router GEMV
    print(f"  router rows bit-identical to the oracle's: {int(same.sum())} of {t}", flush=True)
    # every row, whatever the GEMV's last-ulp agreement: the oracle's own router logits routed by the device
    dev_ids, _, _ = kernels.moe_route(to_dev_bf16(torch, rbf(ref_logits)), 8, renorm=True)
    assert np.array_equal(dev_ids.cpu().numpy(), oracle_ids)
    chk = check_against_oracle(y, ref)
    assert chk.ok_rounded() and chk.within, chk


@pytest.mark.gpu
def test_moe_route_nan_row_routes_nowhere(torch_gpu):
    """A row of NaN logits has no finite probability: its slots get expert -1 with weight 0 and join no expert
    group (so no grouped GEMV reads past the expert table); the other rows route as usual."""
    torch = torch_gpu
    from monolith_mi355 import kernels
    rng = np.random.default_rng(5)
    lg = rbf(rng.standard_normal((3, 256)))
    lg[1] = np.nan
    ids, w, groups = kernels.moe_route(to_dev_bf16(torch, lg), 8, renorm=True)
    ids, w, groups = ids.cpu().numpy(), w.cpu().numpy(), groups.cpu().numpy()
    assert (ids[1] == -1).all() and (w[1] == 0).all()
    ref_ids, ref_w = ON.moe_route(lg[[0, 2]], 8, True)
    assert np.array_equal(ids[[0, 2]], ref_ids) and np.array_equal(w[[0, 2]], ref_w)
    recs = groups[groups[:, 1] > 0]
    pairs = sorted(int(p) for r in recs for p in r[2: 2 + r[1]])
    assert pairs == [p for p in range(24) if p // 8 != 1]
    assert ((recs[:, 0] >= 0) & (recs[:, 0] < 256)).all()


@pytest.mark.gpu
@pytest.mark.parametrize("t,nan_row", [(3, False), (8, False), (16, False), (5, True)])
def test_moe_route_records_of_two_pairs(torch_gpu, t, nan_row):
    """``moe_route(pairs_per_record=2)``: every pair in exactly one record; a record holds one expert's pairs,
    ascending, at most two; an expert's records consecutive and the experts in order of first use (the unsplit
    records, cut in twos); the grouped gate|up and down GEMVs over them (``group_max_pairs=2``, one pass per
    record) give the same outputs bit for bit as over the unsplit records. Tied logits force big groups; a NaN row
    leaves a token with its shared-expert pair only."""
    torch = torch_gpu
    from monolith_mi355 import kernels
    from monolith_mi355.layers import MoeBlock
    blk = MoeBlock(experts=64, seed=13)
    e, k = 64, 8
    rng = np.random.default_rng(21 + t)
    lg = rbf(rng.standard_normal((t, 72)))
    lg[: t // 2, :e] = lg[0, :e]                    # half the tokens route identically: groups of t / 2 pairs
    if nan_row:
        lg[t - 1, :e] = np.nan                      # a token that routes nowhere: only its shared-expert pair
    logits = to_dev_bf16(torch, lg)
    ids, w, g1 = kernels.moe_route(logits[:, :e], k, renorm=True, shared_expert=e, shared_gate=e)
    ids2, w2, g2 = kernels.moe_route(logits[:, :e], k, renorm=True, shared_expert=e, shared_gate=e,
                                     pairs_per_record=2)
    torch.cuda.synchronize()
    assert torch.equal(ids, ids2) and torch.equal(w.view(torch.int32), w2.view(torch.int32))
    a, b = g1.cpu().numpy(), g2.cpu().numpy()
    assert b.shape[0] == t * (k + 1)
    cut = []                                         # the unsplit records cut into twos, in order
    for rec in a:
        if rec[1] <= 0:
            continue
        pairs = list(rec[2: 2 + rec[1]])
        cut += [(int(rec[0]), pairs[i: i + 2]) for i in range(0, len(pairs), 2)]
    got = [(int(r[0]), list(r[2: 2 + r[1]])) for r in b if r[1] > 0]
    assert got == cut
    assert all(r[0] == -1 and r[1] == 0 for r in b[len(got):])
    h = to_dev_bf16(torch, rbf(rng.standard_normal((t, 2048))))
    kw = dict(tokens=t, top_k=k + 1, shared_expert=e, shared_epilogue="silu_mul")
    act1 = kernels.moe_gemv(blk.gate_up_s, h, g1, x_per_slot=False, epilogue="silu_mul_rounded", norm_w=blk.norm_w,
                            **kw)
    act2 = kernels.moe_gemv(blk.gate_up_s, h, g2, x_per_slot=False, epilogue="silu_mul_rounded", norm_w=blk.norm_w,
                            group_max_pairs=2, **kw)
    torch.cuda.synchronize()
    ok = torch.from_numpy(ids.cpu().numpy().reshape(-1) >= 0).cuda()   # a pair without an expert writes no row
    assert torch.equal(act1.view(torch.int16)[ok], act2.view(torch.int16)[ok])
    y1 = kernels.moe_gemv(blk.down_s, act1, g1, tokens=t, top_k=k + 1, x_per_slot=True)
    y2 = kernels.moe_gemv(blk.down_s, act1, g2, tokens=t, top_k=k + 1, x_per_slot=True, group_max_pairs=2)
    torch.cuda.synchronize()
    assert torch.equal(y1.view(torch.int16)[ok], y2.view(torch.int16)[ok])


@pytest.mark.gpu
@pytest.mark.parametrize("m", [1, 3, 8])
def test_moe_block_norm_hand_over(torch_gpu, m):
    """A MoE block given its normalized input (``x_in``, M ≥ 3) and asked for the next layer's (``next_norm``, written
    by the combine) gives the same output bit for bit as the block normalizing its own input, and x_next is
    ``norm_apply`` of that output."""
    torch = torch_gpu
    from monolith_mi355 import kernels
    from monolith_mi355.layers import MoeBlock
    a, b = MoeBlock(seed=81), MoeBlock(seed=81)
    rng = np.random.default_rng(m + 30)
    w_next = torch.from_numpy((1.0 + rng.standard_normal(a.hidden) * 0.1).astype(np.float32)).cuda()
    xn = torch.empty(m, a.hidden, dtype=torch.bfloat16, device="cuda")
    for step in range(2):
        print(f"moe norm hand-over m={m} step {step}", flush=True)
        h = torch.from_numpy(rng.standard_normal((m, a.hidden)).astype(np.float32)).cuda().to(torch.bfloat16)
        y_a = a(h).clone()
        x_in = kernels.norm_apply(h, b.norm_w, eps=b.eps) if m >= 3 else None
        xn.fill_(3.0)
        y_b = b(h, x_in=x_in, next_norm=(w_next, xn, 1e-6)).clone()
        torch.cuda.synchronize()
        assert torch.equal(y_a.view(torch.int16), y_b.view(torch.int16)), step
        assert torch.equal(xn.view(torch.int16), kernels.norm_apply(y_b, w_next, eps=1e-6).view(torch.int16)), step
