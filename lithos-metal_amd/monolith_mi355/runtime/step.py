"""The GPU-resident token loop: a captured step replayed as a HIP graph, its varying state in device memory, its
tokens returned through a sequence-tagged ring in pinned host memory.

This is the counterpart of the reference's ``Engine`` / ``Runner`` (``runtime/engine.py:47-122``,
``runtime/src/metal_core.mm:256-386``): there the step is a pre-encoded Metal indirect command buffer replayed in
command buffers of ``steps_per_cb`` steps with ``in_flight`` of them queued; here it is a ``hipGraphExec`` holding
``steps_per_graph`` steps, replayed by the native pump ``mi_runner_run`` in batches of launches. Everything that
changes between steps lives in :class:`StepState` (the reference's StepState layout, ``core/step_state.py:28-73``)
and is written by the serial ops that close a step (``argmax``, ``advance``), so the graph never changes.

A step of :class:`StepProgram`: ``embed(pending_tokens) → layers → lm_head (final RMSNorm fused, BF16 logits as
the reference's argmax and sampler take them) → argmax or sample → advance``. Attention layers read the position from the step state (``pos_dev``); Gated DeltaNet layers
ping-pong their conv state between two buffers, so a graph holds an even number of steps.
"""

from __future__ import annotations

import ctypes as C
from dataclasses import dataclass, field
from typing import Dict, List, Optional, Sequence

import numpy as np

from . import hip
from .. import kernels


def _torch():
    import torch
    return torch


STATE_BYTES = C.sizeof(hip.MiStepState)
STATE_WORDS = STATE_BYTES // 4
T_MAX = 16


def field_offset(name: str) -> int:
    """Byte offset of a step-state field (the layout contract shared with the kernels)."""
    return getattr(hip.MiStepState, name).offset


class HostBuffer:
    """Pinned, device-accessible host memory (``mi_host_alloc``: coherent ``hipHostMalloc``) viewed as numpy."""

    def __init__(self, nbytes: int, dtype=np.uint8):
        lib = hip.load()
        self.nbytes = nbytes
        self.addr = lib.mi_host_alloc(nbytes)
        if not self.addr:
            raise hip.MiError(f"mi_host_alloc({nbytes}) failed: {hip.last_error()}")
        C.memset(self.addr, 0, nbytes)
        self.array = np.ctypeslib.as_array((C.c_uint8 * nbytes).from_address(self.addr)).view(dtype)

    def close(self):
        if self.addr:
            self.array = None
            hip.call("mi_host_free", self.addr)
            self.addr = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class StepState:
    """The device step state (``mi_step_state``, 272 bytes) with the token ring and the host control words.

    ``ring``: ``ring_capacity`` slots of ``(sequence << 32) | token`` (1-based sequence); ``ctl``: ``[0]`` the host's
    ring tail, ``[1]`` done, ``[2]`` error — the advance mirrors the last two there every step."""

    def __init__(self, *, ring_capacity: int = 4096, device="cuda"):
        torch = _torch()
        if ring_capacity < 1:
            raise ValueError("ring_capacity must be >= 1")
        self.ring_capacity = ring_capacity
        self.buf = torch.zeros(STATE_WORDS, dtype=torch.int32, device=device)
        self.ring = HostBuffer(8 * ring_capacity, np.uint64)
        self.ctl = HostBuffer(16, np.uint32)

    def view(self, name: str, n: int = 1):
        """A device int32 view of ``n`` words of field ``name`` (kernels read or write through it)."""
        off = field_offset(name) // 4
        return self.buf[off: off + n]

    def read(self) -> Dict[str, object]:
        """The fields as Python values (a synchronous copy: the caller orders it after the work it observes)."""
        raw = self.buf.cpu().numpy().tobytes()
        st = hip.MiStepState.from_buffer_copy(raw)
        out = {}
        for name, _ in hip.MiStepState._fields_:
            if name == "pad_":
                continue
            v = getattr(st, name)
            out[name] = list(v) if not isinstance(v, (int, float)) else v
        return out

    def write(self, **fields):
        """Set fields (read-modify-write of the whole struct; the device must be idle on this state)."""
        torch = _torch()
        st = hip.MiStepState.from_buffer_copy(self.buf.cpu().numpy().tobytes())
        for name, v in fields.items():
            cur = getattr(st, name)
            if isinstance(cur, (int, float)):
                setattr(st, name, v)
            else:
                vals = list(v)
                for i in range(len(cur)):
                    cur[i] = vals[i] if i < len(vals) else 0
        host = torch.frombuffer(bytearray(bytes(st)), dtype=torch.int32)
        self.buf.copy_(host)
        torch.cuda.synchronize(self.buf.device)

    def start(self, *, position: int, token: int, stop_at: int = 0, prefill_left: int = 0):
        """Begin a sequence: the step at ``position`` embeds ``token``; the ring, the stop flags and every
        speculative field (verify length, drafts, acceptance, injection counts) restart; the RNG words are kept."""
        self.ring.array[:] = 0
        self.ctl.array[:] = 0
        self.write(step=0, position=position, kv_len=position, t_this_step=1, pending_tokens=[token], anchor=token,
                   gamma=0, draft_tokens=[], confidence=[], verify_len=0, accepted=0, checkpoint_index=0,
                   drafter_ctx_len=0, done=0, error=0, ring_head=0, ring_tail=0, prefill_left=prefill_left,
                   n_inject=0, stop_at=stop_at, n_chain=0)

    def drain(self, tokens: List[int]) -> int:
        """Take ring slots in sequence order (the host pump does this natively; here for eager loops)."""
        tail = int(self.ctl.array[0])
        n = 0
        while True:
            v = int(self.ring.array[tail % self.ring_capacity])
            if (v >> 32) != tail + 1:
                break
            tokens.append(int(np.uint32(v & 0xFFFFFFFF).view(np.int32)))
            tail += 1
            n += 1
        self.ctl.array[0] = tail
        return n

    @property
    def done(self) -> bool:
        return bool(self.ctl.array[1])

    @property
    def error(self) -> int:
        return int(self.ctl.array[2])


@dataclass
class StepReport:
    """``Engine.run``'s report (``runtime/engine.py:97-106``): steps submitted, graph launches, GPU / wall / host
    busy milliseconds, the stop flag and the tokens drained during the run."""

    steps_submitted: int
    launches: int
    batches: int
    gpu_ms: float
    wall_ms: float
    host_busy_ms: float
    done: bool
    error: int
    tokens: List[int] = field(default_factory=list)
    launch_ms: float = 0.0
    wait_ms: float = 0.0


class StepProgram:
    """One decode step of ``model`` over ``state``, captured ``steps_per_graph`` times into a HIP graph.

    ``model`` provides ``embed_table`` (BF16 [vocab, hidden]), ``layers`` (objects with ``step(h, pos=, out=)``),
    ``norm_w`` (the final RMSNorm's (1 + w) FP32 weight), ``lm_head`` (a packed weight [vocab, hidden]) and ``eps``.
    """

    def __init__(self, model, state: StepState, *, eos: Sequence[int] = (), ctx_cap: int = 0,
                 steps_per_graph: int = 2, stream=None, sampling: Optional[dict] = None):
        """``sampling``: ``dict(temperature=…, top_k=…, top_p=…, min_p=…, topp_in_topk=…)`` draws each token with
        :func:`kernels.sample`, seeded by the state's ``rng_lo``/``rng_hi`` and its step (set them with
        ``state.write``); None (or temperature 0) is greedy."""
        torch = _torch()
        if steps_per_graph < 1:
            raise ValueError("steps_per_graph must be >= 1")
        if any(getattr(l, "ping_pong", False) for l in model.layers) and steps_per_graph % 2:
            raise ValueError("a program with Gated DeltaNet layers captures an even number of steps per graph")
        self.model, self.state, self.eos, self.ctx_cap = model, state, list(eos), ctx_cap
        self.steps_per_graph = steps_per_graph
        dev = state.buf.device
        self.stream = stream if stream is not None else torch.cuda.Stream(device=dev)
        vocab, hidden = model.embed_table.shape
        self.h0 = torch.empty(1, hidden, dtype=torch.bfloat16, device=dev)
        self.logits = torch.empty(1, vocab, dtype=torch.bfloat16, device=dev)
        self.sampling = dict(sampling) if sampling and sampling.get("temperature", 1.0) > 0 else None
        self.ids = torch.empty(T_MAX, dtype=torch.int32, device=dev)
        self.graph: Optional[hip.Graph] = None

    def enqueue_step(self):
        """Enqueue one step on the program's stream (eager, or recorded while capturing)."""
        m, st = self.model, self.state
        s = self.stream
        kernels.embed(m.embed_table, st.view("pending_tokens", 1), t=1, out=self.h0, stream=s)
        h = self.h0
        pos = st.view("position")
        torch = _torch()
        with torch.cuda.stream(s):
            for layer in m.layers:
                h = layer.step(h, pos=pos, done=st.view("done"))
        kernels.gemv(m.lm_head, h, norm_w=m.norm_w, eps=m.eps, out=self.logits, stream=s)
        if self.sampling:
            kernels.sample(self.logits, state=st.buf, out=self.ids, stream=s, **self.sampling)
        else:
            kernels.argmax(self.logits, out=self.ids, stream=s)
        kernels.advance(st.buf, self.ids, st.ring.addr, st.ring_capacity, eos=self.eos, ctx_cap=self.ctx_cap,
                        host_ctl=st.ctl.addr, stream=s)

    def step_eager(self, n: int = 1) -> List[int]:
        """Run ``n`` steps eagerly (launch by launch) and return the tokens they emitted."""
        torch = _torch()
        for _ in range(n):
            self.enqueue_step()
        self.stream.synchronize()
        out: List[int] = []
        self.state.drain(out)
        return out

    def capture(self):
        """Record ``steps_per_graph`` steps into a graph. Run at least one eager step first: the library grows its
        workspaces on first use, which a capture cannot do."""
        self.stream.synchronize()
        g = hip.Graph(self.stream)
        with g:
            for _ in range(self.steps_per_graph):
                self.enqueue_step()
        self.graph = g
        return g

    def run(self, max_steps: int, *, launches_per_batch: int = 4, in_flight: int = 2, max_tokens: int = 0,
            token_capacity: Optional[int] = None) -> StepReport:
        """Replay the graph up to ``max_steps`` steps (rounded up to whole graphs) through the native pump; stop
        submitting at done, at ``max_tokens`` drained tokens (queued batches still complete) or when full."""
        if self.graph is None:
            self.capture()
        st = self.state
        launches = -(-max_steps // self.steps_per_graph)
        per_step = getattr(self, "t", 1)                     # tokens a step can emit
        cap = token_capacity if token_capacity is not None else launches * self.steps_per_graph * per_step + 16
        tokens = np.zeros(max(cap, 1), np.int32)
        d = hip.MiRunnerDesc(graph_exec=self.graph.exec, stream=self.graph.stream, state=hip.ptr(st.buf),
                             ring=st.ring.addr, ring_capacity=st.ring_capacity, host_ctl=st.ctl.addr,
                             max_launches=launches, launches_per_batch=launches_per_batch, in_flight=in_flight,
                             max_tokens=max_tokens, tokens=tokens.ctypes.data, tokens_capacity=cap, n_tokens=0)
        stats = hip.MiRunnerStats()
        hip.call("mi_runner_run", C.byref(d), C.byref(stats))
        return StepReport(stats.launches * self.steps_per_graph, stats.launches, stats.batches, stats.gpu_ms,
                          stats.wall_ms, stats.host_busy_ms, bool(stats.done), int(stats.error),
                          tokens[: d.n_tokens].tolist(), stats.launch_ms, stats.wait_ms)


class SpecProgram(StepProgram):
    """The speculative decode round on a static ``1 + gamma``-row step (the reference's DSpark program,
    ``compiler/emit.py:1392-1470`` with ``speculative=True``, minus the drafter): ``embed(pending_tokens) → layers at
    M = 1 + gamma (Gated DeltaNet layers verify into their second state slot, attention appends every row) → lm_head
    → argmax per row → accept_scan (the matching prefix + bonus token to the ring) → gdn_commit per GDN layer (replay
    of the committed rows) → draft source → verify_select (the next step's rows)``. Every count the round needs
    (verify length, committed rows, position) stays on the device, so the step replays as a graph. Rows past the
    step's ``t_this_step`` are computed and discarded; their cache entries are overwritten by later steps.

    The drafter itself is outside this build: ``draft_table`` (int32 ``[ctx, ≥ gamma]``) stands in for it — row p
    holds the drafts proposed after a token at position p — read by ``embed`` at the step state's position."""

    def __init__(self, model, state: StepState, *, gamma: int, draft_table, eos: Sequence[int] = (), ctx_cap: int = 0,
                 steps_per_graph: int = 2, stream=None):
        torch = _torch()
        if not 1 <= gamma <= 15:
            raise ValueError("gamma must be in 1..15")
        super().__init__(model, state, eos=eos, ctx_cap=ctx_cap, steps_per_graph=steps_per_graph, stream=stream)
        self.gamma, self.t = gamma, gamma + 1
        dev = state.buf.device
        vocab, hidden = model.embed_table.shape
        self.h0 = torch.empty(self.t, hidden, dtype=torch.bfloat16, device=dev)
        # at M >= 3 each layer writes the next one's normalized input (two buffers: a layer reads one while its
        # reduction writes the other); the last writes the final norm's, so the LM head reads it as is
        self.xn = [torch.empty(self.t, hidden, dtype=torch.bfloat16, device=dev) for _ in range(2)]
        self.logits = torch.empty(self.t, vocab, dtype=torch.bfloat16, device=dev)
        w = -(-gamma // 4) * 4                               # drafts per table row, padded to 16 bytes
        if draft_table.dtype != torch.int32 or draft_table.dim() != 2 or draft_table.shape[1] < gamma:
            raise ValueError("draft_table must be int32 [ctx, >= gamma]")
        tbl = torch.zeros(draft_table.shape[0], w, dtype=torch.int32, device=dev)
        tbl[:, :gamma] = draft_table[:, :gamma]
        self.draft_rows = tbl.view(torch.bfloat16)           # [ctx, 2w] 16-bit words: embed copies them verbatim
        self.draft_buf = torch.zeros(1, 2 * w, dtype=torch.bfloat16, device=dev)
        self.drafts = self.draft_buf.view(torch.int32).view(-1)
        self.conf = torch.ones(gamma, dtype=torch.float32, device=dev)
        self.log = torch.zeros(64, dtype=torch.int32, device=dev)

    def enqueue_step(self):
        torch = _torch()
        m, st, s, t = self.model, self.state, self.stream, self.t
        kernels.embed(m.embed_table, st.view("pending_tokens", t), t=t, out=self.h0, stream=s)
        h = self.h0
        pos = st.view("position")
        hand_over = t >= 3
        x = None
        with torch.cuda.stream(s):
            for i, layer in enumerate(m.layers):
                kw = {}
                if hand_over:
                    nxt = m.layers[i + 1] if i + 1 < len(m.layers) else None
                    w, eps = (nxt.norm_w, nxt.eps) if nxt is not None else (m.norm_w, m.eps)
                    kw = dict(x_in=x, next_norm=(w, self.xn[i % 2], eps))
                if getattr(layer, "ping_pong", False):
                    h = layer.step(h, pos=pos, verify=True, done=st.view("done"), **kw)
                else:
                    h = layer.step(h, pos=pos, done=st.view("done"), **kw)
                x = self.xn[i % 2] if hand_over else None
        if x is not None:
            kernels.gemv(m.lm_head, x, out=self.logits, stream=s)
        else:
            kernels.gemv(m.lm_head, h, norm_w=m.norm_w, eps=m.eps, out=self.logits, stream=s)
        kernels.argmax(self.logits, out=self.ids, stream=s)
        kernels.accept_scan(st.buf, self.ids, st.ring.addr, st.ring_capacity, eos=self.eos, log=self.log,
                            ctx_cap=self.ctx_cap, host_ctl=st.ctl.addr, stream=s)
        with torch.cuda.stream(s):
            for layer in m.layers:
                if getattr(layer, "ping_pong", False):
                    layer.commit(st.view("checkpoint_index"), done=st.view("done"))
        kernels.embed(self.draft_rows, st.view("position"), t=1, out=self.draft_buf, stream=s)
        kernels.verify_select(st.buf, self.drafts, self.conf, gamma=self.gamma, threshold=float(self.gamma),
                              t_max=t, mode=2, ctx_cap=self.ctx_cap, stream=s)

    def acceptance(self) -> List[int]:
        """The accept scan's per-step log entries ``(committed << 16) | (L << 8) | accepted`` of the last 64 steps."""
        return self.log.cpu().tolist()
