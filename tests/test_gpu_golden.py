"""The configurations on the GPU, through the C ABI, against the golden fixtures:
page tables, slots and copies bit-exact; K/V bytes of the pages each step wrote
bit-exact; attention within 2e-3 abs + 1e-3 rel. Configuration 1 runs on an f32
arena (the reference's K/V precision), configurations 2-5 on binary16 ones."""

import os

import numpy as np
import pytest

from tests.golden.configs import CONFIGS, run_config
from tests.scenario import close
from yaxus_amd.kv import KvCache, PageCopy

pytestmark = pytest.mark.gpu
HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


class HipAdapter:
    """HipBackend behind the scenario driver's backend protocol."""

    def __init__(self, hip, layers, pages, page, hkv, f32=False):
        self.hip, self.page, self.hkv = hip, page, hkv
        self.kv = hip.new_kv(layers, pages, page, hkv, f32=f32)

    def begin_pass(self, pos, slot, pt_off, pages):
        from yaxus_amd.kv import PassMeta

        n = len(pos)
        self.hip.begin_pass(PassMeta(np.zeros(n, np.uint32), pos, slot, pt_off, pages))

    def store(self, layer, k, v):
        self.hip.append(self.kv, layer, k, v)

    def attend_append(self, layer, k, v, q, hq, window):
        return self.hip.attend_append(self.kv, layer, k, v, q, hq, window=window)

    def copy_pages(self, copies):
        self.hip.copy_pages(self.kv, [PageCopy(s, d) for s, d in copies])

    def read_pages(self, layer, pages):
        k, v = self.kv.read_pages(layer, pages)
        if self.kv.f32:  # the fixture holds the oracle's f32 arena contents
            k, v = k.view(np.float32), v.view(np.float32)
        return k, v


@pytest.mark.parametrize("name", list(CONFIGS))
def test_config_matches_the_fixture(hip, name):
    c = CONFIGS[name]
    with np.load(os.path.join(HERE, name + ".npz"), allow_pickle=False) as z:
        want = {k: z[k] for k in z.files}
    be = HipAdapter(hip, c["layers"], c["pages"], c["page"], c["hkv"], f32=not c["f16"])
    try:
        got = run_config(name, KvCache(c["pages"], 1 << 20, c["page"]), be)
    finally:
        be.kv.destroy()
    assert got["inputs_sum"] == want["inputs_sum"], "inputs differ from the fixture's"
    for k in want:
        if "_attn" in k:
            err = np.abs(got[k] - want[k]).max()
            assert close(got[k], want[k]).all(), f"{name} {k}: max abs err {err}"
        elif want[k].dtype == np.float32:  # stored K/V: bit for bit
            assert np.array_equal(np.asarray(got[k]).view(np.uint32), want[k].view(np.uint32)), f"{name} {k}"
        else:
            assert np.array_equal(np.asarray(got[k]), want[k]), f"{name} {k}"
