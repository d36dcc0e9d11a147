"""The shipped allocator (yaxus_amd/csrc/kv_cache.cpp) under AddressSanitizer and
UndefinedBehaviorSanitizer: seeded random operation sequences (begin with prefix reuse,
append, fork, truncate, finish, free; the mix of test_kv_host's differential test) are
run on the allocator oracle (oracle/kv_oracle.py, restating
crates/yaxus-model/src/kv.rs:49-353), written out as a script, and replayed by
tests/native/kv_replay.cpp built with kv_cache.cpp under the sanitizers
(``yaxus_amd.build.build_sanitized``). Every line the sanitized program prints (results,
copy lists, pass metadata, refcounts of every page, live page tables and tokens) must
equal the oracle's, and the program must exit cleanly: any out-of-bounds access, use
after free, leak or undefined operation aborts it."""

import os
import random
import subprocess

import pytest

from oracle.kv_oracle import KvError, OracleKvCache
from yaxus_amd import build

BIN = build.NATIVE_REPLAY_ASAN


@pytest.fixture(scope="module")
def replay():
    build.build_sanitized()
    return BIN


def _fmt(xs):
    return "".join(f" {x}" for x in xs)


def _copies(cp):
    return " C" + "".join(f" {s} {d}" for s, d in cp)


def _state(kv, pages, live):
    s = f"S {kv.free_pages()}" + _fmt(kv.pool.refs) + " L"
    for i in sorted(live):
        s += f" {i} {kv.seq_len(i)} P" + _fmt(kv.seq_pages(i)) + " T" + _fmt(kv.seq_tokens(i))
    return s


def _script(seed, trials, steps):
    """A script and the oracle's expected output lines."""
    rnd = random.Random(seed)
    ops, want = [], []
    for _ in range(trials):
        P = rnd.choice([16, 32, 128])
        pages = rnd.randint(2, 40)
        max_pos = rnd.choice([P * 3, 300, 4096])
        kv = OracleKvCache(pages, max_pos, P)
        ops.append(f"create {pages} {max_pos} {P}")
        live = set()
        vocab = rnd.randint(2, 5)
        for _ in range(steps):
            op = rnd.random()
            cp = []
            if op < 0.25 or not live:
                prompt = [rnd.randrange(vocab) for _ in range(rnd.randint(1, 3 * P))]
                if kv.seqs and rnd.random() < 0.6:
                    base = kv.seqs[rnd.choice(sorted(kv.seqs))].tokens
                    prompt = base[:rnd.randint(0, len(base))] + prompt[:rnd.randint(1, P)]
                ops.append(f"begin {len(prompt)}" + _fmt(prompt))
                try:
                    sid, reused = kv.begin(prompt, cp)
                    live.add(sid)
                    r = f"R {sid} {reused}"
                except KvError:
                    r = "E"
                want.append(r + _copies(cp))
            elif op < 0.6:
                items = [(s, [rnd.randrange(vocab) for _ in range(rnd.randint(1, P + 3))])
                         for s in rnd.sample(sorted(live), min(len(live), rnd.randint(1, 3)))]
                ops.append(f"append {len(items)}" + "".join(f" {s} {len(t)}" + _fmt(t) for s, t in items))
                try:
                    ids, pos, slot, off, pg, last = kv.append(items, cp)
                    r = "R" + " |".join(_fmt(x) for x in (ids, pos, slot, off, pg, last))
                except KvError:
                    r = "E"
                want.append(r + _copies(cp))
            elif op < 0.7:
                s = rnd.choice(sorted(live))
                n = rnd.randint(0, kv.seq_len(s))
                ops.append(f"fork {s} {n}")
                try:
                    f = kv.fork(s, n, cp)
                    live.add(f)
                    r = f"R {f}"
                except KvError:
                    r = "E"
                want.append(r + _copies(cp))
            elif op < 0.8:
                s = rnd.choice(sorted(live))
                n = rnd.randint(0, kv.seq_len(s))
                ops.append(f"truncate {s} {n}")
                kv.truncate(s, n)
                want.append("R")
            else:
                s = rnd.choice(sorted(live))
                live.discard(s)
                if op < 0.92:
                    ops.append(f"finish {s}")
                    kv.finish(s)
                else:
                    ops.append(f"free {s}")
                    kv.free_seq(s)
                want.append("R")
            want.append(_state(kv, pages, live))
    return "\n".join(ops) + "\n", want


@pytest.mark.parametrize("seed", [20241201, 7, 99])
def test_allocator_is_clean_under_asan_and_ubsan(replay, seed):
    script, want = _script(seed, trials=30, steps=120)
    env = dict(os.environ)
    env["ASAN_OPTIONS"] = "halt_on_error=1:detect_leaks=1:abort_on_error=0:exitcode=86"
    env["UBSAN_OPTIONS"] = "halt_on_error=1:print_stacktrace=1:exitcode=87"
    r = subprocess.run([replay], input=script, capture_output=True, text=True, env=env, timeout=300)
    assert r.returncode == 0, f"sanitized replay failed ({r.returncode}):\n{r.stderr[-4000:]}"
    assert "runtime error" not in r.stderr, r.stderr[-4000:]
    got = r.stdout.splitlines()
    assert len(got) == len(want)
    for i, (g, w) in enumerate(zip(got, want)):
        assert g == w, f"line {i}: sanitized allocator {g[:200]!r} != oracle {w[:200]!r}"


def test_the_sanitizer_is_really_on(replay):
    """The replay program is built with ASan (its runtime's symbols are linked in), so a
    clean run above means a checked run."""
    out = subprocess.run(["nm", "-D", "--undefined-only", replay], capture_output=True, text=True).stdout
    assert "__asan_init" in out or "__asan_report_load4" in out
    assert "__ubsan_handle" in out
