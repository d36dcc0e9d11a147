"""The decode loop of tests/native/decode_loop.cpp: the C ABIs driven from C++ alone (host
allocator, pass upload, one fused append + attention launch per layer, yx_sync), as a
native engine drives them."""

import json
import os
import subprocess

import pytest

pytestmark = pytest.mark.gpu
HERE = os.path.dirname(os.path.abspath(__file__))


def test_native_decode_loop_runs():
    exe = os.path.join(HERE, "native", "decode_loop")
    if not os.path.exists(exe):
        raise RuntimeError(f"{exe} is not built: run `python -m yaxus_amd.build`")
    r = subprocess.run([exe, "8", "16", "4000", "24"], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    d = json.loads(r.stdout.strip().splitlines()[-1])
    print(d)
    # One timed run of the launches against the median step that contains them: a 5%
    # allowance for the single sample's spread.
    assert 0 < d["attention_us_all_layers"] <= 1.05 * d["step_us_median"]
    assert 0 < d["host_us_median"] < d["step_us_median"]
