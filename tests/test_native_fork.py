"""cfg5's host-side fork and rollback through the allocator's C ABI alone
(tests/native/fork_rollback.cpp): 8 copy-on-write forks of a partly filled tail page and
24 rollbacks, timed natively. CPU only: the allocator is host code."""

import json
import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)


def test_native_fork_rollback_runs(tmp_path):
    lib_dir = os.path.join(ROOT, "yaxus_amd")
    assert os.path.exists(os.path.join(lib_dir, "libyaxus_kv.so")), "build the package first"
    exe = str(tmp_path / "fork_rollback")
    subprocess.run(["g++", "-O2", "-std=c++17", os.path.join(HERE, "native", "fork_rollback.cpp"),
                    "-L" + lib_dir, "-lyaxus_kv", "-Wl,-rpath," + lib_dir, "-o", exe], check=True)
    r = subprocess.run([exe, "5"], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    d = json.loads(r.stdout.strip().splitlines()[-1])
    print(d)
    # Each of the 8 forks copies its partly filled tail page once.
    assert d["copies"] == 8 and d["forks"] == 8 and d["rollbacks"] == 24
    assert 0 < d["fork_us_median"] <= d["host_fork_rollback_us_median"]
