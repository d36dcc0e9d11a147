"""The caller of the paged path: the engine's scheduling over ``PagedModel``.

Restates ``yaxus_model::engine::Engine`` (crates/yaxus-model/src/engine/mod.rs) for the
parts that decide which rows form a pass and how the KV cache is reserved, grown and
rolled back: admission with the page-reservation rule (``admit``, :398-473), prompt
chunks alternating with decode passes (``step_async``, :336-385; ``prefill_step``,
:477-528), round-robin decode batches of at most ``decode_rows`` (:530-551),
cancellation (:309-333), the split between a failed request and a failed backend
(:825-849), and speculative verification: ``verify`` runs ``[next, props...]`` as one
multi-row pass and ``rewind`` truncates to ``base + 1 + accepted`` (:555-636).

Out of scope (not on the KV path): the draft model, the hint cursor's matching and the
draft-length tuner (engine/{hint,tuning}.rs), and the response cache (engine/cache.rs).
Proposals come from ``Request.hint`` read from the current output position. Tokens
come from ``token_fn(pass_rows, outputs) -> [token per row]`` (the test backend gives
token 0 for every row, as the reference's ``NullBackend`` does).
"""

from __future__ import annotations

from collections import deque
from dataclasses import dataclass, field
from enum import Enum

from .kv import KvError
from .model import ModelError


class Finish(Enum):  # engine/mod.rs:59-67
    STOP = "stop"
    LENGTH = "length"
    CANCELLED = "cancelled"


@dataclass
class Request:  # engine/mod.rs:42-57
    id: int
    prompt: list
    max_new_tokens: int
    stop: list = field(default_factory=list)
    hint: list = field(default_factory=list)


@dataclass
class EngineConfig:  # engine/mod.rs:77-110 (defaults of :97-110)
    max_streams: int = 16
    decode_rows: int = 8
    busy_prefill_rows: int = 64
    draft_k: int = 7
    spec_max_streams: int = 1
    hint_k: int = 7


@dataclass
class Stream:  # engine/mod.rs:134-148
    req: Request
    ts: int
    phase: tuple  # ("prefill", done) or ("decode", next)
    reserved: int
    reused: int
    generated: int = 0
    out: list = field(default_factory=list)
    outcome: object = None  # None (running), Finish, or ("failed", message)

    def running(self):
        return self.outcome is None


class BackendFailure(Exception):
    """A failure of the backend itself: the whole step fails (engine/mod.rs:825-849)."""


class Engine:
    def __init__(self, model, cfg=None, token_fn=None):
        cfg = cfg or EngineConfig()
        if cfg.decode_rows < 1 or cfg.max_streams < 1 or cfg.busy_prefill_rows < 1:
            raise ValueError("decode_rows, max_streams and busy_prefill_rows must be at least 1")
        self.m, self.cfg = model, cfg
        self.token_fn = token_fn or (lambda pr, outs: [0] * len(pr.meta.pos))
        self.waiting = deque()
        self.streams = []
        self.rr = 0
        self.prefill_turn = False
        self.pending = []
        self.passes = []  # (kind, rows) of every pass, for inspection

    # engine/mod.rs:285-333
    def submit(self, req):
        self.waiting.append(req)

    def active(self):
        return len(self.streams)

    def is_idle(self):
        return not self.waiting and not self.streams and not self.pending

    def cancel(self, rid):
        for i, r in enumerate(self.waiting):
            if r.id == rid:
                del self.waiting[i]
                self.pending.append(("done", rid, Finish.CANCELLED, 0))
                return True
        for s in self.streams:
            if s.req.id == rid and s.running():
                s.outcome = Finish.CANCELLED
                return True
        return False

    def _forward(self, items, all_rows):
        """Model::forward + argmax: request errors raise ModelError/KvError."""
        pr, outs = self.m.forward(items, self.m_inputs)
        toks = self.token_fn(pr, outs)
        if all_rows:
            return toks
        return [toks[i] for i in pr.last]

    m_inputs = None  # per-layer (k, v, q) supplier handed to PagedModel.forward

    # engine/mod.rs:336-385
    def step(self, emit=lambda ev: True):
        cancelled = bool(self.pending) or any(isinstance(s.outcome, Finish) for s in self.streams)
        for ev in self.pending:
            emit(ev)
        self.pending = []
        self._sweep(emit)
        self._admit(emit)
        if not self.streams:
            return cancelled
        decoding = [i for i, s in enumerate(self.streams) if s.phase[0] == "decode"]
        prefilling = [i for i, s in enumerate(self.streams) if s.phase[0] == "prefill"]
        if prefilling and (not decoding or self.prefill_turn):
            self.prefill_turn = False
            self._prefill_step(prefilling, bool(decoding), emit)
        else:
            self.prefill_turn = True
            spec = len(decoding) <= self.cfg.spec_max_streams and all(
                self.streams[i].req.hint for i in decoding)
            if spec:
                for i in decoding:
                    try:
                        self._spec_round(i, emit)
                    except (ModelError, KvError) as e:
                        self.streams[i].outcome = ("failed", str(e))
            else:
                n = min(len(decoding), self.cfg.decode_rows)
                start = self.rr % len(decoding)
                self.rr += n
                picked = [decoding[(start + j) % len(decoding)] for j in range(n)]
                try:
                    self._decode_step(picked, emit)
                except (ModelError, KvError) as e:
                    for i in picked:
                        self.streams[i].outcome = ("failed", str(e))
        self._sweep(emit)
        return True

    # engine/mod.rs:398-473
    def _admit(self, emit):
        total, max_pos = self.m.arena()
        P = self.m.page
        while len(self.streams) < self.cfg.max_streams and self.waiting:
            req = self.waiting[0]
            if not req.prompt or req.max_new_tokens == 0:
                self.waiting.popleft()
                emit(("done", req.id, Finish.LENGTH, 0))
                continue
            need = -(-min(len(req.prompt) + req.max_new_tokens, max_pos) // P)
            if len(req.prompt) > max_pos or need > total:
                self.waiting.popleft()
                if len(req.prompt) > max_pos:
                    msg = (f"the prompt has {len(req.prompt)} tokens, more than the {max_pos} "
                           "positions the model's KV covers")
                else:
                    msg = f"the request needs {need} KV pages, more than the {total} the arena has"
                emit(("error", req.id, msg))
                continue
            if sum(s.reserved for s in self.streams) + need > total:
                break
            self.waiting.popleft()
            try:
                ts, reused = self.m.begin(req.prompt)
            except KvError as e:
                emit(("error", req.id, str(e)))
                continue
            self.streams.append(Stream(req, ts, ("prefill", reused), need, reused))

    # engine/mod.rs:477-528
    def _prefill_step(self, prefilling, busy, emit):
        budget = self.cfg.busy_prefill_rows if busy else self.m.chunk
        plan = []
        for i in prefilling:
            if budget == 0:
                break
            done = self.streams[i].phase[1]
            n = min(len(self.streams[i].req.prompt) - done, budget)
            budget -= n
            plan.append((i, done, done + n))
        items = [(self.streams[i].ts, self.streams[i].req.prompt[a:b]) for i, a, b in plan]
        self.passes.append(("prefill", sum(b - a for _, a, b in plan)))
        try:
            toks = self._forward(items, False)
        except (ModelError, KvError) as e:
            for i, _, _ in plan:
                self.streams[i].outcome = ("failed", str(e))
            return
        for i, _, to in plan:
            self.streams[i].phase = ("prefill", to)
        for j, (i, _, to) in enumerate(plan):
            if to == len(self.streams[i].req.prompt):
                self._on_token(i, toks[j], emit)

    # engine/mod.rs:530-551
    def _decode_step(self, picked, emit):
        items = [(self.streams[i].ts, [self.streams[i].phase[1]]) for i in picked]
        self.passes.append(("decode", len(items)))
        toks = self._forward(items, False)
        for i, t in zip(picked, toks):
            self._on_token(i, t, emit)

    # engine/mod.rs:555-583 (hint proposals only), verify :616-626, rewind :629-636
    def _spec_round(self, i, emit):
        s = self.streams[i]
        nxt = s.phase[1]
        left = s.req.max_new_tokens - s.generated
        at = len(s.out)
        props = s.req.hint[at + 1:at + 1 + min(self.cfg.hint_k, left)]
        if not props:
            return self._decode_step([i], emit)
        base = self.m.seq_len(s.ts)
        self.passes.append(("verify", 1 + len(props)))
        g = self._forward([(s.ts, [nxt] + list(props))], True)
        acc = 0
        while acc < len(props) and props[acc] == g[acc]:
            acc += 1
        self.m.truncate(s.ts, base + 1 + acc)  # rewind
        for t in list(props[:acc]) + [g[acc]]:
            self._on_token(i, t, emit)
            if not s.running():
                break

    # engine/mod.rs:674-691
    def _on_token(self, i, tok, emit):
        s = self.streams[i]
        if tok in s.req.stop:
            s.outcome = Finish.STOP
            return
        s.generated += 1
        s.out.append(tok)
        if not emit(("token", s.req.id, tok)):
            s.outcome = Finish.CANCELLED
        elif s.generated >= s.req.max_new_tokens:
            s.outcome = Finish.LENGTH
        else:
            s.phase = ("decode", tok)

    # engine/mod.rs:693-723
    def _sweep(self, emit):
        i = 0
        while i < len(self.streams):
            s = self.streams[i]
            if s.running():
                i += 1
                continue
            self.streams[i] = self.streams[-1]
            self.streams.pop()
            if isinstance(s.outcome, tuple):
                self.m.free_seq(s.ts)
                emit(("error", s.req.id, s.outcome[1]))
            else:
                self.m.finish(s.ts)
                emit(("done", s.req.id, s.outcome, s.generated))

    def run_all(self):
        """Steps until idle; returns [(id, Finish or error message)] in end order."""
        ended = []

        def emit(ev):
            if ev[0] == "done":
                ended.append((ev[1], ev[2]))
            elif ev[0] == "error":
                ended.append((ev[1], ev[2]))
            return True

        while self.step(emit):
            pass
        return ended
