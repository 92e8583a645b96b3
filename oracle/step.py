"""CPU restatement of the serial ops that close a decode step — TEST INFRASTRUCTURE ONLY.

``embed`` (``kernels/common/embed.metal:1-12``, row-major BF16 table), ``argmax`` (``kernels/common/argmax.metal:1-99``),
``advance`` (``kernels/common/advance.metal:1-37``) and the host ring drain (``runtime/src/metal_core.mm:304-318``),
over a step state held as a dict with the reference's field names (``core/step_state.py:38-63``).

Pinning: ``argmax`` against ``numpy.argmax`` (first occurrence on ties) on NaN-free rows and brute force over tiny
rows with NaN / ±inf; ``advance`` against the known answers of the reference's ``tests/kernels/test_eos_set.py``
(stop-token table: done, ring head 1, position 6, slot token) and the toy-program invariants of
``tests/runtime/test_toy_program.py`` (every token once, in order; overflow → error 1 with a clean prefix).
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


def new_state(**fields) -> Dict[str, object]:
    st = {"step": 0, "position": 0, "t_this_step": 1, "pending_tokens": [0] * 16, "done": 0, "error": 0,
          "ring_head": 0, "ring_tail": 0, "prefill_left": 0, "stop_at": 0}
    st.update(fields)
    return st


def advance(st: Dict[str, object], tokens: Sequence[int], ring: np.ndarray, *, eos: Sequence[int] = (),
            ctx_cap: int = 0) -> None:
    """``advance.metal:15-37``: publish the last row's token as ``((head + 1) << 32) | token`` unless the ring is
    full (error 1), make it the pending token, move position / step, stop at ``stop_at``, an EOS id or ``ctx_cap``."""
    if st["done"]:
        return
    t = st["t_this_step"]
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
