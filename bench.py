"""Benchmark of the paged decode path on one MI355X.

Workload (BASELINE headline): B=16 requests, each with ctx 4096 after appending one
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


def cpu_baseline(pr, budget_s=10.0):
    """The oracle's restatement of CpuBackend::attend (f16 KV, f32 math), threaded like
    the reference's rayon pool, on one layer-step of the same workload."""
    from oracle.attn import OracleArena, lib

    lib()
    threads = len(os.sched_getaffinity(0))
    threads = min(threads, 16)
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
        if el >= budget_s or reps >= 200:
            break
    us = el / reps * 1e6
    return {
        "value": round(LAYER_STEP_BYTES / (us * 1e-6) / 1e9, 3),
        "unit": "GB/s",
        "us_per_layer_step": round(us, 1),
        "cores": threads,
        "kind": "port",
        "sample": f"{reps} layer-steps of B=16 ctx 4096 (1 layer, attend only) in {el:.1f} s",
    }


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
    ap.add_argument("--no-graph", action="store_true",
                    help="launch the 24 layers one call at a time instead of replaying a HIP graph")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path "
              "(the paged path shards by request; see DESIGN.md)", file=sys.stderr)
        sys.exit(2)

    from yaxus_amd import KvCache
    from yaxus_amd._lib import YX_K, YX_KERNEL_ATTENTION, YX_V
    from yaxus_amd.backend import HipBackend

    t_host = time.perf_counter()
    cache, pr = build_pass(KvCache)
    host_s = time.perf_counter() - t_host
    log(f"host allocator: {host_s:.2f} s for the pool, 16 prefills and the decode pass")

    hip = HipBackend(0)
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

    # Dominant kernel: the attention launches alone, each bracketed by HIP events on
    # the context's stream.
    hip.profile(True)
    for _ in range(args.steps):
        step()
    hip.profile(False)
    if args.profile_run:
        # Calibration for FETCH_SIZE / WRITE_SIZE: a plain copy of exactly 1 GiB.
        src, dst = hip.tensor((1 << 30,), np.uint8), hip.tensor((1 << 30,), np.uint8)
        for _ in range(3):
            hip.L.yx_dev_copy(hip.ctx, dst.ptr, src.ptr, 1 << 30)
        hip.sync()
        src.free()
        dst.free()
    attn_ms, attn_n = hip.profile_read(YX_KERNEL_ATTENTION)
    attn_us = attn_ms / max(attn_n, 1) * 1000.0
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
            "kernel": "paged_attn_decode<1,8> (fused append + attention)",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "avg_launch_us": round(attn_us, 3),
            "bytes_per_launch": ATTN_BYTES,
            "traffic": traffic_from_profiles(),
        },
        "cpu_baseline": None if (args.no_cpu or args.profile_run) else cpu_baseline(pr, args.cpu_seconds),
    }
    print(json.dumps(line), flush=True)
    hip.close()


if __name__ == "__main__":
    main()
