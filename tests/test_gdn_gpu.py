"""The HIP Gated DeltaNet decode step against the oracle's ``GatedDeltaNet.mix`` (pinned to the reference by
golden vectors), with the reference's own bars (``tests/kernels/test_gdn_mixer.py:161-175``): conv state exact,
recurrent state within 8 FP32 ULP of its largest value, output within ``ok_rounded`` — at the 27B geometry
(hk 16, hv 48, dk = dv = 128) and smaller ones, T = 1 / 4 / 8, two consecutive steps (continuation, conv state
ping-pong), a|b in a second buffer, the BASELINE gates (A_log = dt_bias = 0), bit-identical repeats."""

import numpy as np
import pytest

from helpers import from_dev_bf16, to_dev_bf16
from oracle import nn as ON
from oracle.fp import rbf
from oracle.gates import check_against_oracle

pytestmark = pytest.mark.gpu
EPS = 1e-6


def _params(rng, hk, hv, zero_gates=False):
    conv_dim = 2 * hk * 128 + hv * 128
    return dict(conv_w=rbf(rng.standard_normal((conv_dim, 4)) * 0.3),
                a_log=np.zeros(hv, np.float32) if zero_gates else rbf(rng.uniform(-2, 1, hv)),
                dt_bias=np.zeros(hv, np.float32) if zero_gates else rbf(rng.standard_normal(hv)),
                norm_w=rbf(1 + rng.standard_normal(128) * 0.2))


def _dev_params(torch, p):
    return dict(conv_w=to_dev_bf16(torch, p["conv_w"]),
                neg_exp_a=torch.from_numpy((-np.exp(p["a_log"])).astype(np.float32)).cuda(),
                dt_bias=torch.from_numpy(p["dt_bias"].astype(np.float32)).cuda(),
                norm_w=torch.from_numpy(p["norm_w"].astype(np.float32)).cuda())


def _check(got, ref, conv_got, conv_ref, rec_got, rec_ref):
    assert np.array_equal(conv_got, conv_ref), np.argwhere(conv_got != conv_ref)[:4]
    scale = float(np.abs(rec_ref).max())
    err = float(np.abs(rec_got - rec_ref).max())
    assert err <= 8 * 2.0 ** -23 * scale, (err, scale)
    chk = check_against_oracle(got, ref)
    assert chk.ok_rounded() and chk.within, chk


@pytest.mark.parametrize("hk,hv", [(16, 48), (4, 4), (2, 6)])
@pytest.mark.parametrize("t", [1, 3, 4, 8, 16])
def test_gdn_step_matches_oracle(torch_gpu, hk, hv, t):
    torch = torch_gpu
    from monolith_mi355 import kernels
    rng = np.random.default_rng(hk * 100 + hv + t)
    p = _params(rng, hk, hv)
    dp = _dev_params(torch, p)
    conv_dim = 2 * hk * 128 + hv * 128
    n1 = hv * 128 + conv_dim + 2 * hv
    conv = rbf(rng.standard_normal((conv_dim, 3)) * 0.5)
    rec = (rng.standard_normal((hv, 128, 128)) * 0.1).astype(np.float32)
    bufs = [to_dev_bf16(torch, conv), torch.empty(conv_dim, 3, dtype=torch.bfloat16, device="cuda")]
    rec_d = torch.from_numpy(rec).cuda()
    for step in range(2):                                     # a step on the filled state, then its continuation
        proj = rbf(rng.standard_normal((t, n1)))
        ref, conv, rec = ON.gdn_mix(proj, conv, rec, k_heads=hk, v_heads=hv, dk=128, dv=128, eps=EPS, **p)
        y = kernels.gdn_step(to_dev_bf16(torch, proj), bufs[step & 1], bufs[(step + 1) & 1], rec_d, rec_d,
                             k_heads=hk, v_heads=hv, eps=EPS, **dp)
        torch.cuda.synchronize()
        _check(from_dev_bf16(y), ref, from_dev_bf16(bufs[(step + 1) & 1]), conv, rec_d.cpu().numpy(), rec)


def test_gdn_separate_ab_and_baseline_gates(torch_gpu):
    torch = torch_gpu
    from monolith_mi355 import kernels
    rng = np.random.default_rng(11)
    hk, hv, t = 16, 48, 8
    p = _params(rng, hk, hv, zero_gates=True)                 # C4: g = −softplus(a), A_log = dt_bias = 0
    dp = _dev_params(torch, p)
    conv_dim = 2 * hk * 128 + hv * 128
    conv = rbf(rng.standard_normal((conv_dim, 3)) * 0.5)
    rec = (rng.standard_normal((hv, 128, 128)) * 0.1).astype(np.float32)
    proj = rbf(rng.standard_normal((t, hv * 128 + conv_dim + 2 * hv)))
    ref, conv_ref, rec_ref = ON.gdn_mix(proj, conv, rec, k_heads=hk, v_heads=hv, dk=128, dv=128, eps=EPS, **p)
    main = proj[:, : hv * 128 + conv_dim]
    ab = np.ascontiguousarray(proj[:, hv * 128 + conv_dim:])
    vd, kd = hv * 128, hk * 128
    cin, cout = to_dev_bf16(torch, conv), torch.empty(conv_dim, 3, dtype=torch.bfloat16, device="cuda")
    rin = torch.from_numpy(rec).cuda()
    rout = torch.empty_like(rin)
    y = kernels.gdn_step(to_dev_bf16(torch, main), cin, cout, rin, rout, k_heads=hk, v_heads=hv, eps=EPS,
                         ab=to_dev_bf16(torch, ab), offsets=(0, vd, vd + kd, vd + 2 * kd, 0, hv), **dp)
    torch.cuda.synchronize()
    _check(from_dev_bf16(y), ref, from_dev_bf16(cout), conv_ref, rout.cpu().numpy(), rec_ref)
    assert torch.equal(rin, torch.from_numpy(rec).cuda())     # the input state is untouched when out ≠ in
    y2 = kernels.gdn_step(to_dev_bf16(torch, main), cin, cout, rin, torch.empty_like(rin), k_heads=hk, v_heads=hv,
                          eps=EPS, ab=to_dev_bf16(torch, ab), offsets=(0, vd, vd + kd, vd + 2 * kd, 0, hv), **dp)
    assert torch.equal(y, y2)                                 # bit-identical repeat


def test_gdn_rejects_aliased_conv_state(torch_gpu):
    torch = torch_gpu
    from monolith_mi355 import kernels
    from monolith_mi355.runtime.hip import MiError
    rng = np.random.default_rng(0)
    p = _dev_params(torch, _params(rng, 2, 2))
    conv = torch.zeros(2 * 256 + 256, 3, dtype=torch.bfloat16, device="cuda")
    rec = torch.zeros(2, 128, 128, device="cuda")
    proj = torch.zeros(1, 256 + 768 + 4, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(MiError):
        kernels.gdn_step(proj, conv, conv, rec, rec, k_heads=2, v_heads=2, **p)


@pytest.mark.parametrize("t", [1, 8])
def test_gdn_deferred_norm_read_out(torch_gpu, t):
    """defer_norm: y holds the BF16 read-out o; the oracle's gated RMSNorm of it is the mixer output."""
    torch = torch_gpu
    from monolith_mi355 import kernels
    hk, hv = 4, 12
    rng = np.random.default_rng(7 + t)
    p = _params(rng, hk, hv)
    dp = _dev_params(torch, p)
    conv_dim = 2 * hk * 128 + hv * 128
    n1 = hv * 128 + conv_dim + 2 * hv
    conv = rbf(rng.standard_normal((conv_dim, 3)) * 0.5)
    rec = (rng.standard_normal((hv, 128, 128)) * 0.1).astype(np.float32)
    proj = rbf(rng.standard_normal((t, n1)))
    ref, conv_ref, rec_ref = ON.gdn_mix(proj, conv, rec, k_heads=hk, v_heads=hv, dk=128, dv=128, eps=EPS, **p)
    rec_d = torch.from_numpy(rec).cuda()
    conv_out = torch.empty(conv_dim, 3, dtype=torch.bfloat16, device="cuda")
    o = kernels.gdn_step(to_dev_bf16(torch, proj), to_dev_bf16(torch, conv), conv_out, rec_d, rec_d, k_heads=hk,
                         v_heads=hv, eps=EPS, defer_norm=True, **dp)
    torch.cuda.synchronize()
    o = from_dev_bf16(o).reshape(t, hv, 128)
    z = proj[:, : hv * 128].reshape(t, hv, 128)
    got = ON.gated_rms_norm(o, z, p["norm_w"], EPS).reshape(t, hv * 128)
    _check(got, ref, from_dev_bf16(conv_out), conv_ref, rec_d.cpu().numpy(), rec_ref)


@pytest.mark.parametrize("n_commit,via_device", [(3, True), (8, True), (0, True), (5, False)])
def test_gdn_commit_replays_the_accepted_prefix(torch_gpu, n_commit, via_device):
    """``gdn_commit`` (ops/gdn.py:13-17): after a verify step of 8 tokens wrote the output slot, the commit pass
    recomputes the state for the first n accepted tokens from the step's input slot — the output slot then equals
    the oracle's state after those n tokens, conv window included, and no read-out is written."""
    torch = torch_gpu
    from monolith_mi355 import kernels
    hk, hv, t = 4, 12, 8
    rng = np.random.default_rng(100 + n_commit)
    p = _params(rng, hk, hv)
    dp = _dev_params(torch, p)
    conv_dim = 2 * hk * 128 + hv * 128
    n1 = hv * 128 + conv_dim + 2 * hv
    conv = rbf(rng.standard_normal((conv_dim, 3)) * 0.5)
    rec = (rng.standard_normal((hv, 128, 128)) * 0.1).astype(np.float32)
    proj = rbf(rng.standard_normal((t, n1)))
    conv_a, conv_b = to_dev_bf16(torch, conv), torch.empty(conv_dim, 3, dtype=torch.bfloat16, device="cuda")
    rec_a, rec_b = torch.from_numpy(rec).cuda(), torch.empty(hv, 128, 128, device="cuda")
    pd = to_dev_bf16(torch, proj)
    kernels.gdn_step(pd, conv_a, conv_b, rec_a, rec_b, k_heads=hk, v_heads=hv, eps=EPS, **dp)    # the verify step
    if via_device:
        tdev = torch.tensor([n_commit], dtype=torch.int32, device="cuda")
        r = kernels.gdn_step(pd, conv_a, conv_b, rec_a, rec_b, k_heads=hk, v_heads=hv, eps=EPS, commit=True,
                             t_dev=tdev, **dp)
    else:
        r = kernels.gdn_step(pd[:n_commit], conv_a, conv_b, rec_a, rec_b, k_heads=hk, v_heads=hv, eps=EPS,
                             commit=True, **dp)
    torch.cuda.synchronize()
    assert r is None
    if n_commit:
        _, conv_ref, rec_ref = ON.gdn_mix(proj[:n_commit], conv, rec, k_heads=hk, v_heads=hv, dk=128, dv=128,
                                          eps=EPS, **p)
    else:
        conv_ref, rec_ref = conv, rec
    assert np.array_equal(from_dev_bf16(conv_b), conv_ref)
    got = rec_b.cpu().numpy()
    assert float(np.abs(got - rec_ref).max()) <= 8 * 2.0 ** -23 * float(np.abs(rec_ref).max())
    assert np.array_equal(rec_a.cpu().numpy(), rec)                          # the input slot is untouched


def test_gdn_commit_in_place_equals_two_slots(torch_gpu):
    """The commit pass may write the recurrent state over its input (each workgroup holds its state columns from
    the first load to the last store): in place gives what writing a second slot gives, bit for bit."""
    torch = torch_gpu
    from monolith_mi355 import kernels
    hk, hv, t = 2, 6, 4
    rng = np.random.default_rng(3)
    dp = _dev_params(torch, _params(rng, hk, hv))
    conv_dim = 2 * hk * 128 + hv * 128
    proj = to_dev_bf16(torch, rbf(rng.standard_normal((t, hv * 128 + conv_dim + 2 * hv))))
    rec = torch.from_numpy((rng.standard_normal((hv, 128, 128)) * 0.1).astype(np.float32)).cuda()
    conv = to_dev_bf16(torch, rbf(rng.standard_normal((conv_dim, 3)) * 0.5))
    n = torch.tensor([2], dtype=torch.int32, device="cuda")
    other, in_place = torch.zeros_like(rec), rec.clone()
    c1, c2 = (torch.zeros(conv_dim, 3, dtype=torch.bfloat16, device="cuda") for _ in range(2))
    kernels.gdn_step(proj, conv, c1, rec, other, k_heads=hk, v_heads=hv, commit=True, t_dev=n, eps=EPS, **dp)
    kernels.gdn_step(proj, conv, c2, in_place, in_place, k_heads=hk, v_heads=hv, commit=True, t_dev=n, eps=EPS, **dp)
    torch.cuda.synchronize()
    assert torch.equal(other, in_place) and torch.equal(c1, c2) and not torch.equal(in_place, rec)


@pytest.mark.parametrize("t", [1, 2])
@pytest.mark.parametrize("parity", [False, True])
def test_gdn_conv_in_the_projection_epilogue(torch_gpu, t, parity):
    """The short conv run by the input projection (``gemv(conv=…)``, the step reading ``pre``) against the conv inside
    the step: projection, read-out, both conv slots and the recurrent state bit for bit, over three steps — slots
    named explicitly or chosen by the step counter — and a fourth with the stop flag set (the state passes to the
    other slot unchanged, nothing else is written)."""
    torch = torch_gpu
    from monolith_mi355 import kernels
    from monolith_mi355.layers import nvfp4_matrix
    hk, hv, hidden = 4, 8, 1024
    rng = np.random.default_rng(50 + t + 2 * parity)
    p = _params(rng, hk, hv)
    dp = _dev_params(torch, p)
    conv_dim = 2 * hk * 128 + hv * 128
    n1 = hv * 128 + conv_dim + 2 * hv
    gen = torch.Generator(device="cuda")
    gen.manual_seed(5)
    w = nvfp4_matrix(n1, hidden, gen, "cuda").packed
    norm_w = torch.from_numpy((1 + rng.standard_normal(hidden) * 0.1).astype(np.float32)).cuda()
    conv0 = to_dev_bf16(torch, rbf(rng.standard_normal((conv_dim, 3)) * 0.5))
    rec0 = torch.from_numpy((rng.standard_normal((hv, 128, 128)) * 0.1).astype(np.float32)).cuda()
    slots = {k: torch.zeros(2, conv_dim, 3, dtype=torch.bfloat16, device="cuda") for k in "ab"}
    for k in "ab":
        slots[k][0] = conv0
    rec = {k: rec0.clone() for k in "ab"}
    step = torch.zeros(1, dtype=torch.int32, device="cuda")
    done = torch.zeros(1, dtype=torch.int32, device="cuda")
    pre = torch.empty(t, conv_dim, dtype=torch.bfloat16, device="cuda")
    for s in range(4):
        if s == 3:
            done.fill_(1)
        h = to_dev_bf16(torch, rbf(rng.standard_normal((t, hidden))))
        outs = {}
        for k in "ab":
            proj = torch.empty(t, n1, dtype=torch.bfloat16, device="cuda")
            y = torch.zeros(t, hv * 128, dtype=torch.bfloat16, device="cuda")
            if parity:
                cin, cout, st = slots[k], None, dict(step=step)
            else:
                cin, cout, st = slots[k][s & 1], slots[k][(s + 1) & 1], {}
            conv = None
            if k == "b":
                conv = dict(w=dp["conv_w"], state=cin, out_state=cout, out=pre, row0=hv * 128, done=done, **st)
            kernels.gemv(w, h, norm_w=norm_w, eps=EPS, out=proj, conv=conv)
            kernels.gdn_step(proj, cin, cout, rec[k], rec[k], k_heads=hk, v_heads=hv, eps=EPS, out=y, done=done,
                             pre=pre if k == "b" else None, **st, **dp)
            outs[k] = (proj, y)
        torch.cuda.synchronize()
        assert torch.equal(outs["a"][0], outs["b"][0]), s
        assert torch.equal(outs["a"][1], outs["b"][1]), s
        assert torch.equal(slots["a"], slots["b"]) and torch.equal(rec["a"], rec["b"]), s
        step += 1


def test_gdn_conv_slots_by_step_parity(torch_gpu):
    """With the step counter (``step``): one call shape serves every step — the conv window is read from slot
    ``step & 1`` of ``[2, conv_dim, 3]`` and written to the other. Three steps with the counter advanced on the device
    equal the same steps with the slots named explicitly, bit for bit (outputs, both slots, recurrent state)."""
    torch = torch_gpu
    from monolith_mi355 import kernels
    hk, hv, t = 4, 8, 1
    rng = np.random.default_rng(77)
    p = _params(rng, hk, hv)
    dp = _dev_params(torch, p)
    conv_dim = 2 * hk * 128 + hv * 128
    n1 = hv * 128 + conv_dim + 2 * hv
    conv = rbf(rng.standard_normal((conv_dim, 3)) * 0.5)
    rec = (rng.standard_normal((hv, 128, 128)) * 0.1).astype(np.float32)
    slots = torch.zeros(2, conv_dim, 3, dtype=torch.bfloat16, device="cuda")
    slots[0] = to_dev_bf16(torch, conv)
    explicit = slots.clone()
    rec_a, rec_b = torch.from_numpy(rec).cuda(), torch.from_numpy(rec).cuda()
    step = torch.zeros(1, dtype=torch.int32, device="cuda")
    for s in range(3):
        pd = to_dev_bf16(torch, rbf(rng.standard_normal((t, n1))))
        ya = kernels.gdn_step(pd, slots, None, rec_a, rec_a, k_heads=hk, v_heads=hv, eps=EPS, step=step, **dp)
        yb = kernels.gdn_step(pd, explicit[s & 1], explicit[(s + 1) & 1], rec_b, rec_b, k_heads=hk, v_heads=hv,
                              eps=EPS, **dp)
        step += 1
        torch.cuda.synchronize()
        assert torch.equal(ya, yb) and torch.equal(slots, explicit) and torch.equal(rec_a, rec_b), s
    with pytest.raises(ValueError, match="conv_out is None"):
        kernels.gdn_step(pd, slots, explicit[0], rec_a, rec_a, k_heads=hk, v_heads=hv, eps=EPS, step=step, **dp)
