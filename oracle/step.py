"""CPU restatement of the serial ops that close a decode step — TEST INFRASTRUCTURE ONLY.

``embed`` (``kernels/common/embed.metal:1-12``, row-major BF16 table), ``argmax`` (``kernels/common/argmax.metal:1-99``),
``advance`` (``kernels/common/advance.metal:1-37``), the speculative round's ``verify_select`` and ``accept_scan``
(``kernels/common/spec_ops.metal:108-195``) and the host ring drain (``runtime/src/metal_core.mm:304-318``),
over a step state held as a dict with the reference's field names (``core/step_state.py:38-63``).

Pinning: ``argmax`` against ``numpy.argmax`` (first occurrence on ties) on NaN-free rows and brute force over tiny
rows with NaN / ±inf; ``advance`` against the known answers of the reference's ``tests/kernels/test_eos_set.py``
(stop-token table: done, ring head 1, position 6, slot token) and the toy-program invariants of
``tests/runtime/test_toy_program.py`` (every token once, in order; overflow → error 1 with a clean prefix);
``verify_select`` and ``accept_scan`` against the known answers of the reference's ``tests/kernels/test_draft_ops.py``
(``test_verify_select``'s lengths, tokens and bookkeeping; ``test_accept_scan``'s per-case fields) and
``tests/kernels/test_eos_set.py``'s EOS cases; the sampler's ``thresholds`` against the Hugging Face logits warpers
(``TopKLogitsWarper``, ``TopPLogitsWarper``, ``MinPLogitsWarper``, as the reference's ``tests/kernels/test_sampling.py``
does), ``splitmix64_mix`` against the published splitmix64 output for seed 0, and ``sample``'s draws against the
warped softmax in distribution.
"""

from __future__ import annotations

from typing import Dict, List, Sequence

import numpy as np


def embed(table: np.ndarray, tokens: Sequence[int]) -> np.ndarray:
    """``h[t] = table[tokens[t]]``; an id outside ``[0, vocab)`` reads row 0 (``embed.metal:6``)."""
    vocab = table.shape[0]
    rows = [int(t) if 0 <= int(t) < vocab else 0 for t in tokens]
    return table[rows]


def argmax(logits: np.ndarray) -> np.ndarray:
    """Per row the index of the largest value; ties → the lowest index; NaN never wins (``v > best`` is false for
    it); a row without a number → -1 (``argmax.metal:19-21,95-98``)."""
    logits = np.asarray(logits, np.float32)
    out = np.full(logits.shape[0], -1, np.int32)
    for r, row in enumerate(logits):
        ok = ~np.isnan(row)
        if ok.any():
            best = row[ok].max()
            out[r] = int(np.flatnonzero(ok & (row == best))[0])
    return out


STATE_FIELDS = {"step": 0, "position": 0, "kv_len": 0, "t_this_step": 0, "pending_tokens": [0] * 16, "rng_lo": 0,
                "rng_hi": 0, "anchor": 0, "gamma": 0, "draft_tokens": [0] * 15, "confidence": [0.0] * 15,
                "verify_len": 0, "accepted": 0, "checkpoint_index": 0, "drafter_ctx_len": 0, "done": 0, "error": 0,
                "ring_head": 0, "ring_tail": 0, "prefill_left": 0, "n_inject": 0, "stop_at": 0, "n_chain": 0}


def new_state(**fields) -> Dict[str, object]:
    """A step state with every field of the reference's layout (zero unless given; t_this_step defaults to 1)."""
    st = {k: (list(v) if isinstance(v, list) else v) for k, v in STATE_FIELDS.items()}
    st["t_this_step"] = 1
    for k, v in fields.items():
        if isinstance(st[k], list):
            v = list(v) + [0] * (len(st[k]) - len(v))
        st[k] = v
    return st


def advance(st: Dict[str, object], tokens: Sequence[int], ring: np.ndarray, *, eos: Sequence[int] = (),
            ctx_cap: int = 0) -> None:
    """``advance.metal:15-37``: publish the last row's token as ``((head + 1) << 32) | token`` unless the ring is
    full (error 1), make it the pending token, move position / step, stop at ``stop_at``, an EOS id or ``ctx_cap``."""
    if st["done"]:
        return
    t = min(max(st["t_this_step"], 1), 16)          # this build's guard: rows stay inside the step's 16
    if st["prefill_left"] > 0:
        st["position"] += t
        st["step"] += 1
        if ctx_cap and st["position"] >= ctx_cap:
            st["error"], st["done"] = 2, 1
        return
    tok = int(tokens[t - 1])
    head = st["ring_head"]
    cap = ring.shape[0]
    if head - st["ring_tail"] >= cap:
        st["error"], st["done"] = 1, 1
        return
    ring[head % cap] = np.uint64(((head + 1) << 32) | (tok & 0xFFFFFFFF))
    st["ring_head"] = head + 1
    if st["stop_at"] and st["ring_head"] >= st["stop_at"]:
        st["done"] = 1
    st["pending_tokens"][0] = tok
    st["position"] += t
    st["step"] += 1
    st["t_this_step"] = 1
    if tok in set(int(e) for e in eos):
        st["done"] = 1
    if ctx_cap and st["position"] >= ctx_cap:
        st["error"], st["done"] = 2, 1


def drain(ring: np.ndarray, tail: int, out: List[int]) -> int:
    """Take slots while the next expected 1-based sequence number is present; return the new tail."""
    cap = ring.shape[0]
    while True:
        v = int(ring[tail % cap])
        if (v >> 32) != tail + 1:
            return tail
        out.append(int(np.uint32(v & 0xFFFFFFFF).view(np.int32)))
        tail += 1


def verify_select(st: Dict[str, object], drafts: Sequence[int], conf: Sequence[float], *, gamma: int,
                  threshold: float = 0.0, t_max: int = 8, mode: int = 0, cost: Sequence[float] = (),
                  conf_log: np.ndarray = None, ctx_cap: int = 0, lm: bool = False) -> None:
    """``spec_ops.metal:108-146``: the drafter's bookkeeping, then the verify length and the next step's tokens.
    ``conf`` is taken as float32 (the kernel's arithmetic)."""
    if st["done"]:
        return
    f32 = np.float32
    if lm:
        st["drafter_ctx_len"] = st["position"] + (0 if st["prefill_left"] > 0 else gamma)
    else:
        st["drafter_ctx_len"] += st["n_inject"]
    st["n_inject"] = 0
    if st["prefill_left"] > 0:
        return
    c = [f32(v) for v in conf]
    for k in range(gamma):
        st["draft_tokens"][k] = int(drafts[k])
        st["confidence"][k] = float(c[k])
        if conf_log is not None and conf_log.shape[0]:
            conf_log[st["step"] % conf_log.shape[0], k] = c[k]
    lmax = min(gamma, t_max - 1)
    if ctx_cap:
        if st["position"] >= ctx_cap:
            st["error"], st["done"] = 2, 1
            return
        lmax = min(lmax, ctx_cap - st["position"] - 1)
    L = 0
    if mode == 2:
        L = min(int(max(f32(threshold), f32(0))), lmax)
    elif mode == 1:
        a, e = f32(1), f32(1)
        best = f32(1) / f32(cost[0])
        for l in range(1, lmax + 1):
            a = f32(a * c[l - 1])
            e = f32(e + a)
            score = f32(e / f32(cost[l]))
            if score > best:
                best, L = score, l
    elif f32(threshold) <= 0:
        L = lmax
    else:
        while L < lmax and c[L] >= f32(threshold):
            L += 1
    st["gamma"], st["verify_len"] = gamma, L
    st["pending_tokens"][0] = st["anchor"]
    for k in range(L):
        st["pending_tokens"][k + 1] = int(drafts[k])
    st["t_this_step"] = 1 + L


def accept_scan(st: Dict[str, object], tokens: Sequence[int], ring: np.ndarray, *, eos: Sequence[int] = (),
                log: np.ndarray = None, ctx_cap: int = 0, lm: bool = False) -> None:
    """``spec_ops.metal:148-195``: commit the matching prefix of the drafts and the bonus token, advance the state."""
    if st["done"]:
        return
    t = min(max(st["t_this_step"], 1), 16)          # this build's guard: rows stay inside the step's 16
    cap = ring.shape[0]
    log_cap = 0 if log is None else log.shape[0]
    if st["prefill_left"] > 0:
        if log_cap:
            log[st["step"] % log_cap] = (t << 16) | 0xFFFF
        st["position"] += t
        st["step"] += 1
        st["n_inject"] = st["checkpoint_index"] = t
        st["n_chain"] = 0
        if ctx_cap and st["position"] >= ctx_cap:
            st["error"], st["done"] = 2, 1
        return
    L = min(st["verify_len"], t - 1)                # this build's guard (the reference kernel trusts the state)
    base = t - 1 - L
    acc = 0
    while acc < L and int(tokens[base + acc]) == st["pending_tokens"][base + acc + 1]:
        acc += 1
    bonus = int(tokens[base + acc])
    head = st["ring_head"]
    if head + acc + 1 - st["ring_tail"] > cap:
        st["error"], st["done"] = 1, 1
        return
    stops = set(int(e) for e in eos)
    committed, last, stop = 0, bonus, False
    for k in range(acc + 1):
        tok = st["pending_tokens"][base + k + 1] if k < acc else bonus
        ring[head % cap] = np.uint64(((head + 1) << 32) | (tok & 0xFFFFFFFF))
        head += 1
        committed += 1
        last = tok
        if tok in stops:
            stop = True
            break
    if log_cap:
        log[st["step"] % log_cap] = (committed << 16) | (L << 8) | acc
    st["ring_head"] = head
    if st["stop_at"] and head >= st["stop_at"]:
        stop = True
    st["accepted"], st["anchor"] = acc, last
    st["position"] += base + committed
    st["step"] += 1
    st["verify_len"], st["t_this_step"] = 0, 1
    st["n_inject"] = st["checkpoint_index"] = base + committed
    st["n_chain"] = 1
    if lm:
        st["n_inject"] = st["position"] - st["drafter_ctx_len"] if st["position"] > st["drafter_ctx_len"] else 0
    if stop:
        st["done"] = 1
    if ctx_cap and st["position"] >= ctx_cap:
        st["error"], st["done"] = 2, 1


# ---- stochastic sampling (nn/sampling_ref.py:19-71, kernels/common/sample.metal:22-30) ------------------------------

_M64 = 0xFFFFFFFFFFFFFFFF


def splitmix64_mix(x: int) -> int:
    """The splitmix64 finalizer (Steele, Lea & Flood 2014; ``sample.metal:25``)."""
    x &= _M64
    x ^= x >> 30
    x = (x * 0xBF58476D1CE4E5B9) & _M64
    x ^= x >> 27
    x = (x * 0x94D049BB133111EB) & _M64
    return x ^ (x >> 31)


def gumbel_noise(seed: int, step: int, t: int, idx) -> np.ndarray:
    """``−log(−log u)`` per index, ``u = ((h >> 41) + 0.5) / 2^23`` with ``h`` the finalizer of
    ``seed + step·φ64 + t·c2 + i·c3`` (``sampling_ref.py:44-55``); float32 arithmetic."""
    idx = np.asarray(idx, np.uint64)
    with np.errstate(over="ignore"):
        x = (np.uint64(seed & _M64) + np.uint64(step) * np.uint64(0x9E3779B97F4A7C15)
             + np.uint64(t) * np.uint64(0xC2B2AE3D27D4EB4F) + idx * np.uint64(0x165667B19E3779F9))
        x ^= x >> np.uint64(30)
        x *= np.uint64(0xBF58476D1CE4E5B9)
        x ^= x >> np.uint64(27)
        x *= np.uint64(0x94D049BB133111EB)
        x ^= x >> np.uint64(31)
    u = ((x >> np.uint64(41)) & np.uint64(0x7FFFFF)).astype(np.float32)
    u = (u + np.float32(0.5)) * np.float32(1.0 / 8388608.0)
    return (-np.log(-np.log(u))).astype(np.float32)


def thresholds(logits, *, temperature: float = 1.0, top_k: int = 0, top_p: float = 0.0, min_p: float = 0.0,
               topp_in_topk: bool = False) -> float:
    """The logit threshold τ (``sampling_ref.py:19-41``): the largest of the enabled top-k (k-th largest value, ties
    kept), top-p (the distinct value at which the descending cumulative softmax mass of v / T first reaches p of the
    total — of the top-k set with ``topp_in_topk``) and min-p (max + T·log min_p); −inf when none is enabled."""
    v = np.asarray(logits, np.float32)
    taus = []
    tau_k = -np.inf
    if top_k > 0:
        tau_k = float(np.sort(v)[::-1][min(top_k, v.size) - 1])
        taus.append(tau_k)
    if 0.0 < top_p < 1.0:
        vals = np.unique(v)[::-1]
        counts = np.array([(v == x).sum() for x in vals], np.float64)
        cum = np.cumsum(counts * np.exp((vals.astype(np.float64) - vals[0]) / temperature))
        total = cum[vals >= tau_k][-1] if topp_in_topk and top_k > 0 else cum[-1]
        taus.append(float(vals[int(np.argmax(cum >= top_p * total))]))
    if min_p > 0.0:
        taus.append(float(v.max() + temperature * np.log(min_p)))
    return max(taus) if taus else -np.inf


def sample(logits, *, seed: int, step: int, t: int = 0, temperature: float = 1.0, **opts) -> int:
    """The token drawn for one row (``sampling_ref.py:58-64``): argmax over the kept logits of v / T + noise."""
    v = np.asarray(logits, np.float32)
    tau = thresholds(v, temperature=temperature, **opts)
    keys = v * np.float32(1.0 / temperature) + gumbel_noise(seed, step, t, np.arange(v.size))
    keys = np.where(v >= tau, keys, -np.inf).astype(np.float32)
    return int(np.argmax(keys))


def warped_probabilities(logits, *, temperature: float = 1.0, **opts) -> np.ndarray:
    """The distribution the draws follow: the softmax of v / T over the kept logits (``sampling_ref.py:67-71``)."""
    v = np.asarray(logits, np.float64)
    tau = thresholds(v.astype(np.float32), temperature=temperature, **opts)
    z = np.where(v >= tau, (v - v.max()) / temperature, -np.inf)
    p = np.exp(z)
    return p / p.sum()
