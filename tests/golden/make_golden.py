"""Writes the golden fixtures tests/golden/<config>.npz from the oracle (the CPU
restatements of kv.rs and of yaxus-backend-cpu's attention). Run from the repository
root: `python tests/golden/make_golden.py`. The reference publishes no numeric vectors
for this path (its attention tests need model weights), so these fixtures, made by the
pinned oracle, are the golden data; tests/test_golden.py re-derives them."""

import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

from tests.golden.configs import CONFIGS, oracle_pair, run_config  # noqa: E402


def main():
    here = os.path.dirname(os.path.abspath(__file__))
    for name in CONFIGS:
        out = run_config(name, *oracle_pair(name))
        np.savez_compressed(os.path.join(here, name + ".npz"), **out)
        print(name, {k: v.shape for k, v in out.items()})


if __name__ == "__main__":
    main()
