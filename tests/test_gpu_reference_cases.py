"""The reference GPU backend's own integration and kernel tests, restated at the
attention boundary (they need a model's weights in the reference; here the K/V and q
are seeded draws, and the CPU side is the oracle's restatement of `LayerPass::attend`).

- `tiled_attention_matches_cpu` / `tiled_attention_matches_per_row`
  (crates/yaxus-backend-gpu/tests/vs_cpu.rs:330-389): 40 rows after 2600 keys, attended
  per row (the split-K decode kernel), as tiles (the prefill kernel) and with the keys
  split finer, each against the CPU within 2e-3 and against each other.
- `decode_attention_matches_cpu` (vs_cpu.rs:433-462): contexts of 20, 600 and 2100
  tokens, 4 decode steps each, every step against the CPU.
- `kv_cache_for_a_single_kind_of_layer` (crates/yaxus-backend-gpu/tests/kernels.rs:
  343-362): an arena whose layers are all full or all sliding serves its passes.
- `failed_allocations_are_errors` (kernels.rs:365-374): a device allocation that cannot
  be made is an error, and the context works afterwards.
"""

import numpy as np
import pytest

from tests.scenario import D, Scenario, close

pytestmark = pytest.mark.gpu

HQ, HKV = 16, 4


def _opt(hip, key, value, default):
    class _Ctx:
        def __enter__(self):
            hip.set_option(key, value)

        def __exit__(self, *exc):
            hip.set_option(key, default)
    return _Ctx()


@pytest.mark.parametrize("f32", [False, True])
def test_tiled_attention_matches_per_row_and_cpu(hip, f32):
    sc = Scenario(hip, pages=2640 // 16 + 8, page=16, hkv=HKV, pool_seed=26, f32=f32)
    s = sc.cache.new_seq()
    sc.prefill({s: 2600})
    pr = sc.run_pass([(s, 40)])
    k, v = sc.store(pr)
    q = sc.draw(40 * HQ * D).reshape(40, HQ * D)
    want = sc.orc[0].attend(q, HQ, pr.meta.pos, pr.meta.pt_off, pr.meta.pages)
    with _opt(hip, "prefill_min_rows", 1, 0):
        tiled = hip.attend(sc.kv, 0, q, HQ)                   # prefill kernel
    with _opt(hip, "prefill_min_rows", 1 << 20, 0):
        per_row = hip.attend(sc.kv, 0, q, HQ)                 # split-K decode kernel
        with _opt(hip, "attn_target_waves", 1 << 14, 0):
            split = hip.attend(sc.kv, 0, q, HQ)               # the keys split finer
    before = hip.stat("prefill_plans")
    hip.attend(sc.kv, 0, q, HQ)
    assert hip.stat("prefill_plans") == before, "one 40-row chunk: decode items by default"
    for name, got in (("tiled", tiled), ("per-row", per_row), ("split keys", split)):
        err = np.abs(got - want).max()
        assert close(got, want).all(), f"{name}: max |gpu - cpu| = {err:.2e}"
        assert err < 2e-3, f"{name}: {err:.2e}"
        assert err < 2e-5, f"{name}: {err:.2e} (hi + lo products should stay near f32)"
    assert np.abs(tiled - per_row).max() < 2e-3
    assert np.abs(split - per_row).max() < 2e-3
    sc.kv.destroy()


@pytest.mark.parametrize("n", [20, 600, 2100])
def test_decode_attention_matches_cpu_over_steps(hip, n):
    sc = Scenario(hip, pages=(n + 4) // 16 + 8, page=16, hkv=HKV, pool_seed=n)
    s = sc.cache.new_seq()
    sc.prefill({s: n})
    worst = 0.0
    for _ in range(4):
        pr = sc.run_pass([(s, 1)])
        k = sc.draw(HKV * D).reshape(1, HKV, D)
        v = sc.draw(HKV * D).reshape(1, HKV, D)
        q = sc.draw(HQ * D).reshape(1, HQ * D)
        got = hip.attend_append(sc.kv, 0, k, v, q, HQ)
        sc.orc[0].store(pr.meta.kv_slot, k.reshape(1, -1), v.reshape(1, -1))
        want = sc.orc[0].attend(q, HQ, pr.meta.pos, pr.meta.pt_off, pr.meta.pages)
        assert close(got, want).all()
        worst = max(worst, float(np.abs(got - want).max()))
    assert worst < 2e-3, f"{n}-token context: worst {worst:.2e} over 4 decode steps"
    sc.kv.destroy()


@pytest.mark.parametrize("window", [0, 64])
def test_arena_of_a_single_kind_of_layer(hip, window):
    """Two layers, both full or both sliding (window 64)."""
    sc = Scenario(hip, pages=40, page=16, hkv=1, layers=2)
    s = sc.cache.new_seq()
    sc.prefill({s: 300})
    pr = sc.run_pass([(s, 1)])
    for layer in range(2):
        sc.store(pr, layer)
        q = sc.draw(2 * D).reshape(1, 2 * D)
        got = hip.attend(sc.kv, layer, q, 2, window=window)
        want = sc.orc[layer].attend(q, 2, pr.meta.pos, pr.meta.pt_off, pr.meta.pages, window=window)
        assert close(got, want).all()
    sc.kv.destroy()


def test_failed_allocations_are_errors(hip):
    with pytest.raises(RuntimeError):
        hip.new_kv(1, 1 << 24, 16, 8)        # 512 GiB per K array: beyond the device
    with pytest.raises(RuntimeError):
        hip.tensor((1 << 50,))                # 4 PiB
    # The context is still usable afterwards.
    logits = hip.tensor((1, 3)).upload(np.array([[0.0, 1.0, 0.5]], np.float32))
    assert list(hip.argmax_rows(logits).numpy()) == [1]
    logits.free()
    sc = Scenario(hip, pages=4, page=16, hkv=1)
    s = sc.cache.new_seq()
    sc.prefill({s: 20})
    pr = sc.run_pass([(s, 1)])
    sc.store(pr)
    q = sc.draw(D).reshape(1, D)
    assert close(hip.attend(sc.kv, 0, q, 1), sc.orc[0].attend(q, 1, pr.meta.pos, pr.meta.pt_off,
                                                               pr.meta.pages)).all()
    sc.kv.destroy()
