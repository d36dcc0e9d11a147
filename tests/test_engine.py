"""The engine's scheduling over the paged KV path with a do-nothing backend: the
reference's engine tests (crates/yaxus-model/src/engine/mod.rs:928-1037) restated, and
speculative verify + rewind at the KV level."""

import pytest

from yaxus_amd.engine import Engine, EngineConfig, Finish, Request
from yaxus_amd.model import PagedModel


class NullBackend:
    """lib.rs:597-654: tensors are row counts; nothing is computed."""

    def new_kv(self, layers, pages, page, hkv):
        return None

    def copy_pages(self, kv, copies):
        self.copies = getattr(self, "copies", 0) + len(copies)

    def begin_pass(self, meta):
        self.rows = len(meta.pos)

    def attend_append(self, *a, **k):
        return None


def model(pages, max_pos=8192):
    """lib.rs:667-672: one layer, PAGE = 128."""
    return PagedModel(NullBackend(), pages, max_pos=max_pos, page=128)


def request(rid, prompt_len, max_new):
    """engine/mod.rs:948-951: distinct prompts, so no prefix is shared."""
    return Request(rid, [t + rid * 1000 for t in range(prompt_len)], max_new)


def test_a_waiting_request_is_cancelled_before_it_starts():
    eng = Engine(model(2))
    eng.submit(request(1, 130, 3))
    eng.submit(request(2, 130, 3))
    eng.step()
    assert (eng.active(), len(eng.waiting)) == (1, 1)
    assert eng.cancel(2)
    assert not eng.cancel(2)
    assert not eng.cancel(99)
    ended = eng.run_all()
    assert (2, Finish.CANCELLED) in ended
    assert (1, Finish.LENGTH) in ended
    assert eng.is_idle()


def test_a_running_request_is_cancelled_and_its_pages_serve_the_next():
    eng = Engine(model(2))
    eng.submit(request(1, 130, 120))
    eng.submit(request(2, 130, 3))
    eng.step()
    assert eng.cancel(1)
    tokens_of_1, ended = 0, []

    def emit(ev):
        nonlocal tokens_of_1
        if ev[0] == "token" and ev[1] == 1:
            tokens_of_1 += 1
        if ev[0] == "done":
            ended.append((ev[1], ev[2]))
        return True

    while eng.step(emit):
        pass
    assert tokens_of_1 == 0
    assert ended == [(1, Finish.CANCELLED), (2, Finish.LENGTH)]
    assert eng.is_idle()


def test_a_request_waits_for_the_pages_of_the_others():
    eng = Engine(model(2))
    eng.submit(request(1, 130, 3))
    eng.submit(request(2, 130, 3))
    eng.step()
    assert (eng.active(), len(eng.waiting)) == (1, 1)
    assert eng.run_all() == [(1, Finish.LENGTH), (2, Finish.LENGTH)]


def test_requests_that_fit_together_run_together():
    eng = Engine(model(2))
    eng.submit(request(1, 100, 20))
    eng.submit(request(2, 100, 20))
    eng.step()
    assert (eng.active(), len(eng.waiting)) == (2, 0)


def test_a_request_that_cannot_fit_alone_fails_at_once_and_blocks_nobody():
    eng = Engine(model(2))
    eng.submit(request(1, 250, 10))
    eng.submit(request(2, 10, 3))
    ended = eng.run_all()
    assert len(ended) == 2
    assert ended[0][0] == 1 and "KV pages" in ended[0][1]
    assert ended[1] == (2, Finish.LENGTH)


def test_a_prompt_past_the_positions_of_the_model_fails_at_once():
    eng = Engine(model(4, max_pos=200))
    eng.submit(request(1, 201, 1))
    ended = eng.run_all()
    assert "positions" in ended[0][1]


def test_a_budget_past_the_positions_is_not_refused_when_the_output_ends_first():
    eng = Engine(model(4, max_pos=200))
    req = request(1, 150, 100)
    req.stop = [0]  # the test backend's first token
    eng.submit(req)
    assert eng.run_all() == [(1, Finish.STOP)]


def test_a_request_may_take_the_whole_arena():
    eng = Engine(model(2))
    eng.submit(request(1, 250, 6))
    assert eng.run_all() == [(1, Finish.LENGTH)]


def test_zero_row_budgets_are_rejected():
    with pytest.raises(ValueError):
        Engine(model(2), EngineConfig(busy_prefill_rows=0))
    Engine(model(2), EngineConfig())


def test_decode_passes_batch_round_robin_and_prefill_alternates():
    eng = Engine(model(64), EngineConfig(decode_rows=4))
    for r in range(6):
        eng.submit(request(r, 20 + r, 5))
    eng.run_all()
    kinds = [k for k, _ in eng.passes]
    # all prompts fit one chunk pass; then decode passes of at most 4 rows
    assert kinds[0] == "prefill" and eng.passes[0][1] == sum(20 + r for r in range(6))
    assert all(n <= 4 for k, n in eng.passes if k == "decode")
    assert sum(n for k, n in eng.passes if k == "decode") == 6 * 4


def test_verify_and_rewind_keep_the_kv_to_the_accepted_tokens():
    """A speculative round verifies [next, props...] in one pass and truncates the KV
    to base + 1 + accepted (engine/mod.rs:555-636): the test backend returns token 0,
    so a hint of zeros is accepted and one with a 5 is cut there."""
    m = model(16)
    eng = Engine(m)
    req = Request(1, list(range(40)), 12, hint=[0, 0, 0, 5, 0, 0, 0, 0, 0, 0, 0, 0, 0])
    eng.submit(req)
    seen = []
    eng.step(lambda ev: seen.append(ev) or True)  # prefill: first token 0
    s = eng.streams[0]
    base = m.seq_len(s.ts)
    eng.step(lambda ev: seen.append(ev) or True)  # verify [0, 0, 0, 5, ...]
    assert eng.passes[-1][0] == "verify"
    # one token is out after the prompt, so props = hint[2:9] = [0, 5, 0, ...]: one
    # accepted, then the target's own 0 in place of the 5
    assert m.seq_len(s.ts) == base + 1 + 1
    assert [e[2] for e in seen if e[0] == "token"] == [0, 0, 0]
