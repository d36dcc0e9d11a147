"""The engine driving the HIP path (reference vs_cpu.rs:163-208 `concurrent_matches_solo`,
restated at the attention level): requests run alone and together give the same
attention outputs per (request, position), and match the CPU oracle backend."""

import numpy as np
import pytest

from oracle.attn import OracleArena, normal
from tests.scenario import close
from yaxus_amd.engine import Engine, EngineConfig, Finish, Request
from yaxus_amd.model import PagedModel

pytestmark = pytest.mark.gpu
D, HQ, HKV, LAYERS, PAGE, PAGES = 128, 8, 2, 2, 16, 160


def inputs(layer, meta):
    """k, v, q of each row from (token, position, layer) only."""
    rows = len(meta.pos)
    k = np.empty((rows, HKV, D), np.float32)
    v = np.empty_like(k)
    q = np.empty((rows, HQ * D), np.float32)
    for r in range(rows):
        seed = int(meta.ids[r]) * 1000003 + int(meta.pos[r]) * 31 + layer
        x = normal((2 * HKV + HQ) * D, seed)
        k[r] = x[:HKV * D].reshape(HKV, D)
        v[r] = x[HKV * D:2 * HKV * D].reshape(HKV, D)
        q[r] = x[2 * HKV * D:]
    return k, v, q


def token_fn(pr, outs):
    return [(int(p) * 7 + 3) % 97 + 200 for p in pr.meta.pos]


class Recording(Engine):
    def __init__(self, *a, **k):
        super().__init__(*a, **k)
        self.m_inputs = inputs
        self.record = {}

    def _forward(self, items, all_rows):
        pr, outs = self.m.forward(items, self.m_inputs)
        owner = {s.ts: s.req.id for s in self.streams}
        r = 0
        for ts, toks in items:
            for _ in toks:
                for layer, o in enumerate(outs):
                    self.record[(owner[ts], int(pr.meta.pos[r]), layer)] = np.asarray(o)[r]
                r += 1
        toks = self.token_fn(pr, outs)
        return toks if all_rows else [toks[i] for i in pr.last]


class OracleModelBackend:
    def new_kv(self, layers, pages, page, hkv):
        return [OracleArena(pages, page, hkv, D) for _ in range(layers)]

    def copy_pages(self, kv, copies):
        for c in copies:
            for a in kv:
                a.copy_page(c.src, c.dst)

    def begin_pass(self, meta):
        self.meta = meta

    def attend_append(self, kv, layer, k, v, q, hq, window=None):
        m = self.meta
        kv[layer].store(m.kv_slot, k.reshape(len(m.pos), -1), v.reshape(len(m.pos), -1))
        return kv[layer].attend(q, hq, m.pos, m.pt_off, m.pages, window=window or 0)


def run(backend, reqs, together, passes=None):
    model = PagedModel(backend, PAGES, max_pos=4096, page=PAGE, layers=LAYERS, hkv=HKV, hq=HQ,
                       windows=[0, 64], chunk=96)
    eng = Recording(model, EngineConfig(decode_rows=4, busy_prefill_rows=32), token_fn=token_fn)
    if together:
        for r in reqs:
            eng.submit(r)
        eng.run_all()
    else:
        for r in reqs:
            eng.submit(r)
            eng.run_all()
    if passes is not None:
        passes.extend(eng.passes)
    return eng.record


def test_concurrent_matches_solo_and_the_oracle(hip):
    reqs = [Request(i, [(i * 37 + t) % 90 + 1 for t in range(n)], 6)
            for i, n in enumerate([150, 17, 64, 230, 5])]
    solo = run(hip, reqs, together=False)
    both = run(hip, reqs, together=True)
    orc = run(OracleModelBackend(), reqs, together=True)
    assert set(solo) == set(both) == set(orc)
    for key in both:
        assert close(both[key], solo[key]).all(), key
        assert close(both[key], orc[key]).all(), key


def test_speculative_matches_plain(hip):
    """Reference vs_cpu.rs:124-160 `speculative_matches_plain`, at the attention level:
    a request decoded with verify passes (hint proposals, some wrong, so rewinds happen)
    ends with the same attention outputs per (position, layer) as plain decoding."""
    f = lambda p: (p * 7 + 3) % 97 + 200  # the token the test model emits at position p
    prompt = [(t * 13) % 90 + 1 for t in range(70)]
    n_new = 12
    good = [f(len(prompt) - 1 + i) for i in range(n_new)]
    hint = list(good)
    hint[4] = 5  # rejected: the verify pass rewinds to before it
    hint[9] = 6
    plain = run(hip, [Request(0, prompt, n_new)], together=False)
    kinds = []
    spec = run(hip, [Request(0, prompt, n_new, hint=hint)], together=False, passes=kinds)
    verify = [n for kind, n in kinds if kind == "verify"]
    assert len(verify) >= 2 and max(verify) > 1, kinds  # multi-row verify passes ran
    assert set(plain) == set(spec)
    for key in plain:
        assert close(spec[key], plain[key]).all(), key


def test_cancelling_everything_leaves_a_clean_engine(hip):
    """Reference vs_cpu.rs:209-255 `cancelling_everything_leaves_a_clean_engine`, at the
    attention level: with two requests running and one waiting, cancelling all three
    ends each as cancelled, leaves no stream, no waiting request and every KV page
    free, and the engine then answers a request as it did before."""
    model = PagedModel(hip, PAGES, max_pos=4096, page=PAGE, layers=LAYERS, hkv=HKV, hq=HQ,
                       windows=[0, 64], chunk=96)
    model.set_prefix_cache(False)
    eng = Recording(model, EngineConfig(max_streams=2, decode_rows=4, busy_prefill_rows=32),
                    token_fn=token_fn)
    prompt = [(t * 11) % 90 + 1 for t in range(100)]

    def answer(rid):
        eng.record = {}
        eng.submit(Request(rid, prompt, 16))
        assert eng.run_all() == [(rid, Finish.LENGTH)]
        return {(p, layer): o for (r, p, layer), o in eng.record.items() if r == rid}

    before = answer(100)
    free = model.free_pages()
    for i in range(3):
        eng.submit(Request(i, prompt, 64))
    for _ in range(3):
        eng.step()
    assert eng.active() > 0 and len(eng.waiting) > 0
    for i in range(3):
        assert eng.cancel(i)
    ended = sorted(eng.run_all(), key=lambda e: e[0])
    assert ended == [(0, Finish.CANCELLED), (1, Finish.CANCELLED), (2, Finish.CANCELLED)]
    assert eng.is_idle()
    assert model.free_pages() == free
    after = answer(101)
    assert set(after) == set(before)
    for key in before:
        assert np.array_equal(after[key], before[key]), key  # deterministic kernels
