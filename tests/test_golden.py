"""The golden fixtures (tests/golden/*.npz, made by make_golden.py from the oracle)
are re-derived on the CPU: by the oracle itself (the fixtures are current) and by the
shipped allocator driving the oracle arena (page tables, slots, copies, refcounts
and everything downstream of them equal bit for bit)."""

import os

import numpy as np
import pytest

from tests.golden.configs import CONFIGS, OracleBackend, oracle_pair, run_config
from yaxus_amd.kv import KvCache

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _load(name):
    with np.load(os.path.join(HERE, name + ".npz"), allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def _same(got, want):
    assert set(got) == set(want)
    for k in want:
        assert got[k].shape == want[k].shape, k
        assert np.array_equal(np.asarray(got[k]).view(np.uint8), want[k].view(np.uint8)), k


@pytest.mark.parametrize("name", list(CONFIGS))
def test_oracle_reproduces_the_fixture(name):
    _same(run_config(name, *oracle_pair(name)), _load(name))


@pytest.mark.parametrize("name", list(CONFIGS))
def test_shipped_allocator_reproduces_the_fixture(name):
    c = CONFIGS[name]
    cache = KvCache(c["pages"], 1 << 20, c["page"])
    be = OracleBackend(c["layers"], c["pages"], c["page"], c["hkv"], f16=c["f16"])
    _same(run_config(name, cache, be), _load(name))
