"""Benchmark of the paged decode path on one MI355X.

Workload (the headline benchmark): B=16 requests, each with ctx 4096 after appending one
token (4095 prior + 1), 16 query heads / 4 KV heads, head_dim 128, f16 KV with f32
accumulation, page size 16, pages scattered over an 8192-page pool by the host
allocator, 24 layers with distinct arenas (~6.4 GB, far beyond the 256 MB MALL). One
step = one decode pass over all 24 layers: per layer, the K/V append kernel and the
paged attention kernel, inputs resident in HBM. The pass metadata (page tables,
slots) is built by the host allocator and uploaded once before the timed region.

Prints one JSON line. ``value`` is GB/s of algorithmic bytes per layer-step
(K+V 134,217,728 + Q 131,072 + O 131,072 + page tables 16,384 + appended K/V 32,768)
over the measured time.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

B, CTX, HQ, HKV, D, PAGE, LAYERS, POOL = 16, 4096, 16, 4, 128, 16, 24, 8192
HBM_PEAK_GBS = 8000.0
KV_BYTES = B * CTX * HKV * D * 2 * 2
Q_BYTES = B * HQ * D * 4
O_BYTES = B * HQ * D * 4
PT_BYTES = B * (CTX // PAGE) * 4
APPEND_BYTES = B * HKV * D * 2 * 2
LAYER_STEP_BYTES = KV_BYTES + Q_BYTES + O_BYTES + PT_BYTES + APPEND_BYTES
ATTN_BYTES = LAYER_STEP_BYTES  # the fused kernel stores the appended K/V too
METRIC = "paged decode-attn GB/s (% HBM peak) + µs/layer-step at B=16, ctx 4096"
SEED = 0x59415855


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def build_pass(KvCache):
    """Host allocator: scatter the pool, lay out 16 sequences of 4095 tokens, then the
    decode pass appending one token to each. Returns (cache, PassRows)."""
    from yaxus_amd.data import permutation

    cache = KvCache(POOL, 1 << 20, PAGE)
    holders = [cache.new_seq() for _ in range(POOL)]
    for s in holders:
        cache.append([(s, [0] * PAGE)], [])
    for i in permutation(POOL, SEED):
        cache.free_seq(holders[int(i)])
    seqs = [cache.new_seq() for _ in range(B)]
    for s in seqs:
        cache.append([(s, [1] * (CTX - 1))], [])
    copies = []
    pr = cache.append([(s, [2]) for s in seqs], copies)
    assert not copies
    return cache, pr


BOX_CPU_SHARE = 16  # host threads one GPU's job may keep busy on the GPU boxes


def cpu_threads():
    """The reference CPU backend's pool size (crates/yaxus-backend-cpu/src/threads.rs:4-31):
    physical cores, SMT siblings counted once (distinct
    /sys/devices/system/cpu/cpuN/topology/thread_siblings_list), capped by the available
    parallelism (the affinity mask and a cgroup CPU quota, as Rust's
    std::thread::available_parallelism counts them); here also capped by the GPU box's
    CPU share for one GPU."""
    logical = len(os.sched_getaffinity(0))
    avail = logical
    try:  # cgroup v2 quota: "max 100000" or "<quota> <period>"
        with open("/sys/fs/cgroup/cpu.max") as f:
            quota, period = f.read().split()[:2]
        if quota != "max":
            avail = max(1, min(avail, -(-int(quota) // int(period))))
    except (OSError, ValueError):
        pass
    sib = set()
    base = "/sys/devices/system/cpu"
    try:
        for name in os.listdir(base):
            if name.startswith("cpu") and name[3:].isdigit():
                try:
                    with open(os.path.join(base, name, "topology", "thread_siblings_list")) as f:
                        sib.add(f.read().strip())
                except OSError:
                    pass
    except OSError:
        pass
    physical = len(sib) or None
    n = min(physical, avail) if physical else avail
    threads = min(n, BOX_CPU_SHARE)
    return {"physical_cores": physical, "logical_cpus": logical, "available_parallelism": avail,
            "threads": threads,
            "rule": "min(physical cores, available parallelism) as threads.rs:4-31, "
                    f"capped at the box's {BOX_CPU_SHARE}-thread share"}


def cpu_baseline(pr, budget_s=10.0):
    """The oracle's restatement of CpuBackend::attend (f16 KV, f32 math), threaded like
    the reference's rayon pool, on one layer-step of the same workload."""
    from oracle.attn import OracleArena, lib

    lib()
    cpu = cpu_threads()
    threads = cpu["threads"]
    arena = OracleArena(POOL, PAGE, HKV, D, f16=True)
    rng = np.random.default_rng(SEED)
    arena.k[:] = rng.standard_normal(arena.k.shape, dtype=np.float32).astype(np.float16).view(np.uint16)
    arena.v[:] = rng.standard_normal(arena.v.shape, dtype=np.float32).astype(np.float16).view(np.uint16)
    q = rng.standard_normal((B, HQ * D), dtype=np.float32)
    m = pr.meta
    reps, t0 = 0, time.perf_counter()
    while True:
        arena.attend(q, HQ, m.pos, m.pt_off, m.pages, threads=threads)
        reps += 1
        el = time.perf_counter() - t0
        if el >= budget_s:  # a bounded sample: about budget_s seconds of the host's cores
            break
    us = el / reps * 1e6
    return {
        "value": round(LAYER_STEP_BYTES / (us * 1e-6) / 1e9, 3),
        "unit": "GB/s",
        "us_per_layer_step": round(us, 1),
        "cores": threads,
        "physical_cores": cpu["physical_cores"],
        "logical_cpus": cpu["logical_cpus"],
        "available_parallelism": cpu["available_parallelism"],
        "threads": threads,
        "thread_rule": cpu["rule"],
        "kind": "port",
        "sample": f"{reps} layer-steps of B=16 ctx 4096 (1 layer, attend only) in {el:.1f} s",
    }


def _fill_arena(hip, kv, layers, seed):
    from yaxus_amd._lib import YX_K, YX_V

    f16 = not getattr(kv, "f32", False)
    per = kv.pages * kv.page_bytes // (2 if f16 else 4)
    for l in range(layers):
        hip.fill_normal(kv.layer_ptr(l, YX_K), per, f16, seed, (2 * l) * per)
        hip.fill_normal(kv.layer_ptr(l, YX_V), per, f16, seed, (2 * l + 1) * per)


def _scatter(cache, pool, seed):
    from yaxus_amd.data import permutation

    holders = [cache.new_seq() for _ in range(pool)]
    for s in holders:
        cache.append([(s, [0] * PAGE)], [])
    for i in permutation(pool, seed):
        cache.free_seq(holders[int(i)])


def _time_layers(hip, kv, pr, layers, hq, windows, steps, extra=None):
    """Times `steps` passes of `layers` fused append + attention launches on resident
    inputs (one HIP graph per pass); returns µs per pass."""
    from yaxus_amd.backend import DeviceTensor  # noqa: F401

    rows = len(pr.meta.pos)
    q = hip.tensor((rows, hq * D))
    k = hip.tensor((rows, kv.hkv * D))
    v = hip.tensor((rows, kv.hkv * D))
    out = hip.tensor((rows, hq * D))
    for i, t in enumerate((q, k, v)):
        hip.fill_normal(t.ptr, t.nbytes // 4, False, SEED + 99, i << 32)
    hip.begin_pass(pr.meta)

    def one():
        for l in range(layers):
            hip.attend_append(kv, l, k, v, q, hq, window=windows[l], out=out)

    one()
    hip.sync()
    hip.graph_begin()
    one()
    hip.graph_end()
    hip.graph_launch()
    hip.sync()
    hip.timer_start()
    for _ in range(steps):
        hip.graph_launch()
        if extra:
            extra()
    us = hip.timer_stop() * 1000.0 / steps
    for t in (q, k, v, out):
        t.free()
    return us


def _time_write_rows(hip, kv, pr, layers, steps):
    """write_rows (q/k RMSNorm + RoPE + K/V store) per layer for the pass `pr`:
    (us per layer, bytes per layer: qkv read, q written, K/V written)."""
    from yaxus_amd.rope import inv_freq, rope_table

    rows = len(pr.meta.pos)
    cols = (HQ + 2 * HKV) * D
    qkv = hip.tensor((rows, cols))
    hip.fill_normal(qkv.ptr, rows * cols, False, SEED + 77, 0)
    qn, kn = hip.tensor((D,)), hip.tensor((D,))
    hip.fill_normal(qn.ptr, D, False, SEED + 78, 0)
    hip.fill_normal(kn.ptr, D, False, SEED + 79, 0)
    table = rope_table(inv_freq(D, 10000.0), 1.0, int(max(pr.meta.pos)) + 1)
    cs = hip.tensor(table.shape).upload(table)
    q = hip.tensor((rows, HQ * D))
    hip.begin_pass(pr.meta)
    for l in range(layers):
        hip.qk_rope_append(kv, l, qkv, qn, kn, cs, 1e-6, HQ, out=q)
    hip.sync()
    hip.timer_start()
    for _ in range(steps):
        for l in range(layers):
            hip.qk_rope_append(kv, l, qkv, qn, kn, cs, 1e-6, HQ, out=q)
    us = hip.timer_stop() * 1000.0 / (steps * layers)
    for t in (qkv, qn, kn, cs, q):
        t.free()
    return us, rows * (cols * 4 + HQ * D * 4 + HKV * D * 2 * 2)


def _time_attention_kernel(hip, kv, pr, layers, hq, steps):
    """Average duration of the attention kernel alone (events around each launch of
    the same fused append + attention calls, not graph-replayed): µs per launch."""
    from yaxus_amd._lib import YX_KERNEL_ATTENTION

    rows = len(pr.meta.pos)
    q, out = hip.tensor((rows, hq * D)), hip.tensor((rows, hq * D))
    k, v = hip.tensor((rows, kv.hkv * D)), hip.tensor((rows, kv.hkv * D))
    for i, t in enumerate((q, k, v)):
        hip.fill_normal(t.ptr, t.nbytes // 4, False, SEED + 99, i << 32)
    hip.begin_pass(pr.meta)
    for l in range(layers):
        hip.attend_append(kv, l, k, v, q, hq, out=out)
    hip.sync()
    hip.profile(True)
    for _ in range(steps):
        for l in range(layers):
            hip.attend_append(kv, l, k, v, q, hq, out=out)
    hip.profile(False)
    ms, n = hip.profile_read(YX_KERNEL_ATTENTION)
    for t in (q, out, k, v):
        t.free()
    return ms * 1000.0 / max(n, 1)


def _time_backend_attention(hip, kv, pr, layers, steps):
    """Backend::attention in full (write_rows then attend) per layer for the pass `pr`,
    device inputs: (us one launch, us as write_rows + attention launches)."""
    from yaxus_amd.rope import inv_freq, rope_table

    rows = len(pr.meta.pos)
    cols = (HQ + 2 * HKV) * D
    qkv = hip.tensor((rows, cols))
    hip.fill_normal(qkv.ptr, rows * cols, False, SEED + 81, 0)
    qn, kn = hip.tensor((D,)), hip.tensor((D,))
    hip.fill_normal(qn.ptr, D, False, SEED + 82, 0)
    hip.fill_normal(kn.ptr, D, False, SEED + 83, 0)
    table = rope_table(inv_freq(D, 10000.0), 1.0, int(max(pr.meta.pos)) + 1)
    cs = hip.tensor(table.shape).upload(table)
    q, out = hip.tensor((rows, HQ * D)), hip.tensor((rows, HQ * D))
    hip.begin_pass(pr.meta)

    def one():
        for l in range(layers):
            hip.attention(kv, l, qkv, qn, kn, cs, 1e-6, HQ, out=out)

    def two():
        for l in range(layers):
            hip.qk_rope_append(kv, l, qkv, qn, kn, cs, 1e-6, HQ, out=q)
            hip.attend(kv, l, q, HQ, out=out)

    res = []
    for fn in (one, two):
        fn()
        hip.sync()
        hip.timer_start()
        for _ in range(steps):
            fn()
        res.append(hip.timer_stop() * 1000.0 / (steps * layers))
    for t in (qkv, qn, kn, cs, q, out):
        t.free()
    return res


def cfg2_pass(KvCache):
    """cfg2: 16 requests share a 1024-token prefix (64 refcounted pages); suffixes
    U[512, 3072]; the decode pass appending one token to each. (cache, pass, pool,
    suffix lengths)."""
    from yaxus_amd.data import uniform_ints

    pool = 4096
    cache = KvCache(pool, 1 << 20, PAGE)
    _scatter(cache, pool, SEED + 2)
    base = cache.new_seq()
    cache.append([(base, [1] * 1024)], [])
    suf = uniform_ints(B, 512, 3072, SEED + 2)
    seqs = [cache.fork(base, 1024, []) for _ in range(B)]
    for s, n in zip(seqs, suf):
        cache.append([(s, [1] * int(n))], [])
    pr = cache.append([(s, [2]) for s in seqs], [])
    return cache, pr, pool, suf


def cfg3_pass(KvCache):
    """cfg3: 16 requests append a 256-token chunk on contexts U[0, 2048] that leave a
    half-filled tail page (causal within the chunk). (cache, pass, pool, prior lengths)."""
    from yaxus_amd.data import uniform_ints

    pool = 4096
    cache = KvCache(pool, 1 << 20, PAGE)
    _scatter(cache, pool, SEED + 3)
    prior = [int(x) // 16 * 16 + 8 for x in uniform_ints(B, 0, 2040, SEED + 3)]
    seqs = [cache.new_seq() for _ in range(B)]
    for s, n in zip(seqs, prior):
        cache.append([(s, [1] * n)], [])
    pr = cache.append([(s, [2] * 256) for s in seqs], [])
    return cache, pr, pool, prior


def cfg4_pass(KvCache):
    """cfg4: 4 requests of 32768 tokens over a 65536-page pool, one decode step.
    (cache, pass, pool)."""
    pool = 65536
    cache = KvCache(pool, 1 << 20, PAGE)
    _scatter(cache, pool, SEED + 4)
    seqs = [cache.new_seq() for _ in range(4)]
    for s in seqs:
        cache.append([(s, [1] * 32767)], [])
    pr = cache.append([(s, [2]) for s in seqs], [])
    return cache, pr, pool


def cfg5_pass(KvCache):
    """cfg5: 16 requests of ctx 4096 (2048 shared) verifying 5 draft tokens (5 causal
    rows each). (cache, pass, pool, sequences)."""
    pool = 8192
    cache = KvCache(pool, 1 << 20, PAGE)
    _scatter(cache, pool, SEED + 5)
    base = cache.new_seq()
    cache.append([(base, [1] * 2048)], [])
    seqs = [cache.fork(base, 2048, []) for _ in range(B)]
    for s in seqs:
        cache.append([(s, [1] * (4096 - 2048 - 5))], [])
    pr = cache.append([(s, [2] * 5) for s in seqs], [])
    return cache, pr, pool, seqs


def bench_configs(hip, steps=10, include_long=True, only=None):
    """Benchmark configurations 2-5 at full size (one JSON object per configuration);
    `only`: a set of names among cfg2, cfg3, cfg4, cfg5, f32, long, step to run (all when None)."""
    from yaxus_amd import KvCache
    from yaxus_amd.data import uniform_ints

    def want(name):
        return only is None or name in only

    res = {}
    layers = 24
    if want('cfg2'):
        # cfg2: one decode step over 24 layers.
        cache, pr, pool, suf = cfg2_pass(KvCache)
        layers = 24
        kv = hip.new_kv(layers, pool, PAGE, HKV, D)
        _fill_arena(hip, kv, layers, SEED + 2)
        us = _time_layers(hip, kv, pr, layers, HQ, [0] * layers, steps) / layers
        ctx = [1024 + int(n) + 1 for n in suf]
        logical = sum(ctx) * HKV * D * 2 * 2
        unique = (1024 + int(sum(suf)) + B) * HKV * D * 2 * 2
        wr_us, wr_bytes = _time_write_rows(hip, kv, pr, layers, steps)
        ba_one, ba_two = _time_backend_attention(hip, kv, pr, layers, steps)
        res["cfg2_prefix_decode"] = {"us_per_layer_step": round(us, 2),
                                     "backend_attention_us_one_launch": round(ba_one, 2),
                                     "backend_attention_us_two_launches": round(ba_two, 2),
                                     "logical_GBs": round(logical / us / 1e3, 1),
                                     "unique_GBs": round(unique / us / 1e3, 1),
                                     "logical_bytes": logical, "unique_bytes": unique,
                                     "write_rows_us_per_layer": round(wr_us, 2)}
        kv.destroy()
    if want('cfg3'):
        # cfg3: the 256-row chunks over 24 layers.
        cache, pr, pool, prior = cfg3_pass(KvCache)
        kv = hip.new_kv(layers, pool, PAGE, HKV, D)
        _fill_arena(hip, kv, layers, SEED + 3)
        us = _time_layers(hip, kv, pr, layers, HQ, [0] * layers, max(2, steps // 2)) / layers
        flops = sum(4 * HQ * D * (256 * p + 256 * 257 // 2) for p in prior)
        wr_us, wr_bytes = _time_write_rows(hip, kv, pr, layers, max(2, steps // 2))
        k_us = _time_attention_kernel(hip, kv, pr, layers, HQ, max(2, steps // 2))
        ba_one, ba_two = _time_backend_attention(hip, kv, pr, layers, max(2, steps // 2))
        # us_per_layer_step: the K/V append launch plus the prefill kernel, graph-replayed;
        # attn_kernel_us: the prefill kernel alone (HIP events around each launch);
        # backend_attention_us: Backend::attention from qkv (write_rows' K/V part, then
        # the prefill kernel normalising and rotating its q heads itself).
        res["cfg3_chunked_prefill"] = {"us_per_layer_step": round(us, 2),
                                       "TFLOPs": round(flops / us / 1e6, 2),
                                       "mfma_util_vs_2.5PF": round(flops / us / 1e6 / 2500.0, 4),
                                       "attn_kernel_us": round(k_us, 2),
                                       "attn_kernel_TFLOPs": round(flops / k_us / 1e6, 2),
                                       "attn_kernel_mfma_util_vs_2.5PF": round(flops / k_us / 1e6 / 2500.0, 4),
                                       "flops_per_layer": flops,
                                       "write_rows_us_per_layer": round(wr_us, 2),
                                       "write_rows_GBs": round(wr_bytes / wr_us / 1e3, 1),
                                       "backend_attention_us": round(ba_one, 2),
                                       "write_rows_then_attention_us": round(ba_two, 2)}
        kv.destroy()
    if want('cfg5'):
        # cfg5: the verify pass over 24 layers; then 8 requests fork from a partly
        # filled tail page (copy on write) and roll back a seeded count in [0, 5].
        cache, pr, pool, seqs = cfg5_pass(KvCache)
        kv = hip.new_kv(layers, pool, PAGE, HKV, D)
        _fill_arena(hip, kv, layers, SEED + 5)
        us_verify = _time_layers(hip, kv, pr, layers, HQ, [0] * layers, steps) / layers
        ba_one, ba_two = _time_backend_attention(hip, kv, pr, layers, steps)
        t0 = time.perf_counter()
        copies = []
        forks = [cache.fork(s, cache.seq_len(s) - 3, copies) for s in seqs[:8]]
        back = uniform_ints(len(seqs) + len(forks), 0, 5, SEED + 55)
        for s, n in zip(seqs + forks, back):
            cache.truncate(s, cache.seq_len(s) - int(n))
        host_us = (time.perf_counter() - t0) * 1e6
        hip.timer_start()
        hip.copy_pages(kv, copies)
        copy_us = hip.timer_stop() * 1000.0
        bytes_verify = sum(4096 for _ in seqs) * HKV * D * 2 * 2
        res["cfg5_verify_fork"] = {"us_per_layer_step_verify": round(us_verify, 2),
                                   # yx_attention_qkv_dev (write_rows runs as its own
                                   # launch inside the call for passes of two tiles)
                                   # and the two calls made by the caller
                                   "backend_attention_us": round(ba_one, 2),
                                   "write_rows_then_attention_us": round(ba_two, 2),
                                   "verify_logical_GBs": round(bytes_verify / us_verify / 1e3, 1),
                                   "fork_copies": len(copies), "copy_us_all_layers": round(copy_us, 2),
                                   "host_fork_rollback_us": round(host_us, 1)}
        # The same host work through the allocator's C ABI from C++ (no Python per call).
        exe = os.path.join(ROOT, "tests", "native", "fork_rollback")
        if os.path.exists(exe):
            import subprocess
            r = subprocess.run([exe, "50"], capture_output=True, text=True, timeout=60)
            if r.returncode == 0:
                nat = json.loads(r.stdout.strip().splitlines()[-1])
                res["cfg5_verify_fork"]["host_fork_rollback_us_native"] = nat["host_fork_rollback_us_median"]
        kv.destroy()
    if want('f32'):
        # The headline's pass on an f32 arena (the reference's K/V precision): twice
        # the bytes, f32 MFMAs.
        _, pr = build_pass(KvCache)
        kv = hip.new_kv(layers, POOL, PAGE, HKV, D, f32=True)
        _fill_arena(hip, kv, layers, SEED)
        us = _time_layers(hip, kv, pr, layers, HQ, [0] * layers, steps) / layers
        nbytes = B * CTX * HKV * D * 4 * 2
        res["f32_arena_b16_ctx4096"] = {"us_per_layer_step": round(us, 2),
                                        "GBs": round(nbytes / us / 1e3, 1),
                                        "kv_bytes_per_layer": nbytes}
        kv.destroy()
        # cfg3's chunked prefill on an f32 arena: the f32 prefill kernel (exact f32
        # MFMA products), and the same pass through the f32 split-K decode kernel.
        cache, pr, pool, prior = cfg3_pass(KvCache)
        kv = hip.new_kv(layers, pool, PAGE, HKV, D, f32=True)
        _fill_arena(hip, kv, layers, SEED + 3)
        n = max(2, steps // 2)
        k_us = _time_attention_kernel(hip, kv, pr, layers, HQ, n)
        hip.set_option("prefill_min_rows", 1 << 20)
        k_split = _time_attention_kernel(hip, kv, pr, layers, HQ, n)
        hip.set_option("prefill_min_rows", 0)
        flops = sum(4 * HQ * D * (256 * p + 256 * 257 // 2) for p in prior)
        res["cfg3_chunked_prefill_f32"] = {"attn_kernel_us": round(k_us, 2),
                                           "TFLOPs": round(flops / k_us / 1e6, 2),
                                           "f32_mfma_util_vs_157.3TF": round(flops / k_us / 1e6 / 157.3, 4),
                                           "split_k_decode_kernel_us": round(k_split, 2)}
        kv.destroy()
    if want('long'):
        # Chunked prefill of one long sequence (256 rows after 32768 keys): too few tiles
        # to fill the GPU, so the prefill kernel splits them along keys; the same pass
        # with the split off, for comparison (prefill kernel alone, HIP events).
        pool = 2048 + 64
        cache = KvCache(pool, 1 << 20, PAGE)
        _scatter(cache, pool, SEED + 6)
        s = cache.new_seq()
        cache.append([(s, [1] * 32768)], [])
        pr = cache.append([(s, [2] * 256)], [])
        kv = hip.new_kv(4, pool, PAGE, HKV, D)
        _fill_arena(hip, kv, 4, SEED + 6)
        flops = 4 * HQ * D * (256 * 32768 + 256 * 257 // 2)
        n = max(2, steps // 2)
        k_split = _time_attention_kernel(hip, kv, pr, 4, HQ, n)
        hip.set_option("prefill_split", 0)
        k_whole = _time_attention_kernel(hip, kv, pr, 4, HQ, n)
        hip.set_option("prefill_split", 1)
        res["prefill_long_context"] = {"shape": "1 sequence, 256 rows after 32768 keys",
                                       "attn_kernel_us": round(k_split, 2),
                                       "TFLOPs": round(flops / k_split / 1e6, 1),
                                       "attn_kernel_us_unsplit": round(k_whole, 2),
                                       "flops_per_layer": flops}
        kv.destroy()
    if want('step'):
        # The step after attention at the headline's decode shape: o_proj (16 rows of
        # hq * 128 = 2048 against a bf16 [2048][2048] weight) and the greedy pick over a
        # 151936-token vocabulary.
        t, k, n, vocab = B, HQ * D, 2048, 151936
        x, w, o = hip.tensor((t, k)), hip.tensor((n, k), np.uint16), hip.tensor((t, n))
        hip.fill_normal(x.ptr, t * k, False, SEED + 61, 0)
        hip.fill_normal(w.ptr, n * k, True, SEED + 62, 0)  # N(0,1) binary16 bits, read as bf16
        logits, ids = hip.tensor((t, vocab)), hip.tensor((t,), np.uint32)
        hip.fill_normal(logits.ptr, t * vocab, False, SEED + 63, 0)
        def graph_us(fn, per_graph=24, reps=20):
            # A HIP graph of `per_graph` launches (as a decode step would hold them),
            # replayed: µs per launch, launch gaps inside the graph included.
            fn()
            hip.sync()
            hip.graph_begin()
            for _ in range(per_graph):
                fn()
            hip.graph_end()
            hip.graph_launch()
            hip.sync()
            hip.timer_start()
            for _ in range(reps):
                hip.graph_launch()
            return hip.timer_stop() * 1000.0 / (reps * per_graph)

        mm_us = graph_us(lambda: hip.matmul_bf16(x, w, out=o))
        am_us = graph_us(lambda: hip.argmax_rows(logits, out=ids))
        # The same launches over ROT distinct weights / logits buffers in turn (a graph of
        # ROT launches, 403 MB of weights and 467 MB of logits): beyond the 256 MB MALL,
        # so each launch reads its bytes from HBM, as 24 layers' distinct o_proj weights
        # do. The figures above replay one buffer, which the MALL then holds.
        ROT = 48
        ws = [hip.tensor((n, k), np.uint16) for _ in range(ROT)]
        ls = [hip.tensor((t, vocab)) for _ in range(ROT)]
        for i in range(ROT):
            hip.fill_normal(ws[i].ptr, n * k, True, SEED + 64, i * n * k)
            hip.fill_normal(ls[i].ptr, t * vocab, False, SEED + 65, i * t * vocab)
        it_w, it_l = iter(range(1 << 30)), iter(range(1 << 30))
        mm_hbm = graph_us(lambda: hip.matmul_bf16(x, ws[next(it_w) % ROT], out=o), per_graph=ROT)
        am_hbm = graph_us(lambda: hip.argmax_rows(ls[next(it_l) % ROT], out=ids), per_graph=ROT)
        for z in ws + ls:
            z.free()
        res["step_after_oproj_argmax"] = {
            "oproj_us": round(mm_us, 2), "oproj_weight_GBs": round(n * k * 2 / mm_us / 1e3, 1),
            "oproj_shape": [t, k, n], "argmax_us": round(am_us, 2),
            "argmax_GBs": round(t * vocab * 4 / am_us / 1e3, 1), "argmax_shape": [t, vocab],
            "same_buffer_note": "oproj_us / argmax_us replay one weight / logits buffer (MALL-resident)",
            "oproj_us_hbm": round(mm_hbm, 2), "oproj_weight_GBs_hbm": round(n * k * 2 / mm_hbm / 1e3, 1),
            "argmax_us_hbm": round(am_hbm, 2), "argmax_GBs_hbm": round(t * vocab * 4 / am_hbm / 1e3, 1),
            "hbm_note": f"{ROT} distinct buffers in turn, {ROT * n * k * 2 / 1e6:.0f} MB of weights and "
                        f"{ROT * t * vocab * 4 / 1e6:.0f} MB of logits: beyond the 256 MB MALL"}
        for z in (x, w, o, logits, ids):
            z.free()
    if include_long and want('cfg4'):
        # cfg4: 32 layers, 1 full then 3 sliding (window 2048), repeated.
        cache, pr, pool = cfg4_pass(KvCache)
        layers = 32
        kv = hip.new_kv(layers, pool, PAGE, HKV, D)
        _fill_arena(hip, kv, layers, SEED + 4)
        windows = [0 if l % 4 == 0 else 2048 for l in range(layers)]
        us_step = _time_layers(hip, kv, pr, layers, HQ, windows, max(2, steps // 2))
        nbytes = 4 * (8 * 32768 + 24 * 2048) * HKV * D * 2 * 2
        res["cfg4_long_sliding"] = {"us_per_step_32_layers": round(us_step, 1),
                                    "GBs": round(nbytes / us_step / 1e3, 1), "bytes_per_step": nbytes}
        kv.destroy()
    return res


def traffic_from_profiles():
    """HBM bytes per attention launch from the committed rocprof counter summary."""
    p = os.path.join(ROOT, "profiles", "attn_decode_b16_ctx4096_traffic.json")
    if not os.path.exists(p):
        return None
    with open(p) as f:
        return json.load(f).get("bytes_per_launch")


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--profile-run", action="store_true",
                    help="for rocprofv3: also run a 1 GiB device copy (the byte-counter "
                         "calibration point) and skip the CPU baseline")
    ap.add_argument("--only", default=None,
                    help="with --configs: comma-separated subset of cfg2,cfg3,cfg4,cfg5,f32,long,step")
    ap.add_argument("--configs", action="store_true",
                    help="also measure benchmark configurations 2-5 at full size (adds ~2 min)")
    ap.add_argument("--no-graph", action="store_true",
                    help="launch the 24 layers one call at a time instead of replaying a HIP graph")
    ap.add_argument("--set", action="append", default=[], metavar="KEY=VALUE",
                    help="a context option (yx_ctx_set_option, include/yaxus_hip.h) for every run "
                         "of this invocation, e.g. --set attn_cascade=0; repeatable")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path "
              "(the paged path shards by request and KV head without exchange)", file=sys.stderr)
        sys.exit(2)

    from yaxus_amd import KvCache
    from yaxus_amd._lib import YX_K, YX_KERNEL_APPEND, YX_KERNEL_ATTENTION, YX_KERNEL_COPY, YX_V
    from yaxus_amd.backend import HipBackend

    t_host = time.perf_counter()
    cache, pr = build_pass(KvCache)
    host_s = time.perf_counter() - t_host
    log(f"host allocator: {host_s:.2f} s for the pool, 16 prefills and the decode pass")

    hip = HipBackend(0)
    for kvp in args.set:
        key, val = kvp.split("=", 1)
        hip.set_option(key, int(val))
    kv = hip.new_kv(LAYERS, POOL, PAGE, HKV, D)
    per_layer = POOL * kv.page_bytes // 2
    for l in range(LAYERS):
        hip.fill_normal(kv.layer_ptr(l, YX_K), per_layer, True, SEED, (2 * l) * per_layer)
        hip.fill_normal(kv.layer_ptr(l, YX_V), per_layer, True, SEED, (2 * l + 1) * per_layer)
    qs = [hip.tensor((B, HQ * D)) for _ in range(LAYERS)]
    ks = [hip.tensor((B, HKV * D)) for _ in range(LAYERS)]
    vs = [hip.tensor((B, HKV * D)) for _ in range(LAYERS)]
    outs = [hip.tensor((B, HQ * D)) for _ in range(LAYERS)]
    base = 2 * LAYERS * per_layer
    for l in range(LAYERS):
        hip.fill_normal(qs[l].ptr, B * HQ * D, False, SEED, base + l * 3 * B * HQ * D)
        hip.fill_normal(ks[l].ptr, B * HKV * D, False, SEED, base + (l * 3 + 1) * B * HQ * D)
        hip.fill_normal(vs[l].ptr, B * HKV * D, False, SEED, base + (l * 3 + 2) * B * HQ * D)
    hip.begin_pass(pr.meta)
    hip.sync()

    def step():
        for l in range(LAYERS):
            hip.attend_append(kv, l, ks[l], vs[l], qs[l], HQ, out=outs[l])

    for _ in range(args.warmup):
        step()
    hip.sync()
    if not args.no_graph:
        # One decode step (24 layers) as a HIP graph, replayed per step.
        hip.graph_begin()
        step()
        hip.graph_end()
        hip.graph_launch()
        hip.sync()
    hip.timer_start()
    for _ in range(args.steps):
        if args.no_graph:
            step()
        else:
            hip.graph_launch()
    ms = hip.timer_stop()
    ms_per_step = ms / args.steps
    us_layer = ms_per_step * 1000.0 / LAYERS
    gbs = LAYER_STEP_BYTES / (us_layer * 1e-6) / 1e9
    o = outs[0].numpy()
    if not np.isfinite(o).all():
        raise RuntimeError("non-finite attention output")

    # Dominant kernel. A step launches nothing but the attention kernel (one fused
    # append + attention launch per layer): a pass with per-launch events checks that,
    # then the kernel's average duration is the graph-timed region above (HIP events on
    # the context's stream, the stream every launch is on) divided by its launches.
    # The per-launch event figure (each launch bracketed alone, event gaps included) is
    # reported beside it.
    hip.profile(True)
    for _ in range(args.steps):
        step()
    hip.profile(False)
    if args.profile_run:
        # Calibration for FETCH_SIZE / WRITE_SIZE: a plain copy of exactly 1 GiB (1 GiB
        # read, 1 GiB written), then a read-only pass over 1 GiB (yx_dev_checksum).
        src, dst = hip.tensor((1 << 30,), np.uint8), hip.tensor((1 << 30,), np.uint8)
        for _ in range(3):
            hip.L.yx_dev_copy(hip.ctx, dst.ptr, src.ptr, 1 << 30)
        hip.sync()
        for _ in range(3):
            hip.checksum(src.ptr, 1 << 30)
        src.free()
        dst.free()
    attn_ms, attn_n = hip.profile_read(YX_KERNEL_ATTENTION)
    other = [hip.profile_read(k)[1] for k in (YX_KERNEL_APPEND, YX_KERNEL_COPY)]
    if attn_n != args.steps * LAYERS or any(other):
        raise RuntimeError(f"a step launched {attn_n} attention and {other} other kernels")
    isolated_us = attn_ms / max(attn_n, 1) * 1000.0
    attn_us = us_layer
    achieved = ATTN_BYTES / (attn_us * 1e-6) / 1e9

    line = {
        "metric": METRIC,
        "value": round(gbs, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "us_per_layer_step": round(us_layer, 2),
        "pct_hbm_peak": round(100.0 * gbs / HBM_PEAK_GBS, 1),
        **({"options": dict(kv_.split("=", 1) for kv_ in args.set)} if args.set else {}),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "launch": "per-call" if args.no_graph else "hip-graph (one graph per 24-layer step)",
        "data": "synthetic (splitmix64/Box-Muller N(0,1), seed 0x59415855)",
        "config": {
            "workload": "batched paged decode: B=16, ctx 4096, 16q/4kv heads, d 128, "
                        "f16 KV, page 16, 24 layers (append + attention per layer, one launch)",
            "B": B, "ctx": CTX, "hq": HQ, "hkv": HKV, "head_dim": D, "page": PAGE,
            "layers": LAYERS, "pool_pages": POOL, "bytes_per_layer_step": LAYER_STEP_BYTES,
        },
        "roofline": {
            "bound": "hbm",
            "kernel": "paged_attn_decode_wide<1> (fused append + attention)",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "avg_launch_us": round(attn_us, 3),
            "avg_launch_us_isolated": round(isolated_us, 3),
            "bytes_per_launch": ATTN_BYTES,
            "traffic": traffic_from_profiles(),
            "traffic_source": "profiles/attn_decode_b16_ctx4096_traffic.json (rocprofv3 --pmc "
                              "FETCH_SIZE and WRITE_SIZE runs of bench.py --profile-run, committed)",
        },
        "cpu_baseline": None if (args.no_cpu or args.profile_run) else cpu_baseline(pr, args.cpu_seconds),
    }
    if args.configs:
        kv.destroy()
        line["configs"] = bench_configs(hip, only=set(args.only.split(",")) if args.only else None)
    print(json.dumps(line), flush=True)
    hip.close()


if __name__ == "__main__":
    main()
