"""Builds the package's native libraries in-tree.

- ``yaxus_amd/libyaxus_kv.so``  host page allocator (g++), C ABI of include/yaxus_kv_cache.h
- ``yaxus_amd/libyaxus_hip.so`` device path for gfx950 (hipcc), C ABI of include/yaxus_hip.h
- ``tests/native/*``            C++ programs over the C ABIs, one of them (``kv_replay_asan``)
  with the allocator built under ASan + UBSan

``python -m yaxus_amd.build`` compiles both; it always recompiles.
"""

from __future__ import annotations

import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

KV_LIB = os.path.join(HERE, "libyaxus_kv.so")
HIP_LIB = os.path.join(HERE, "libyaxus_hip.so")

# Packed-FP32 instructions are disabled for every HIP translation unit.
HIP_FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-shared",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-result",
]


def _run(cmd):
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in r.stdout.splitlines() if "packed-fp32-ops" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"build failed: {' '.join(cmd)}\n{out}")
    return out


def build_kv():
    _run(["g++", "-O2", "-std=c++17", "-fPIC", "-shared", "-Wall", "-Wextra",
          os.path.join(CSRC, "kv_cache.cpp"), "-o", KV_LIB])


def build_hip():
    srcs = [os.path.join(CSRC, "runtime.hip")]
    _run([HIPCC, *HIP_FLAGS, *srcs, "-o", HIP_LIB])


NATIVE_LOOP = os.path.join(ROOT, "tests", "native", "decode_loop")


NATIVE_FORK = os.path.join(ROOT, "tests", "native", "fork_rollback")


def build_native_tests():
    """The C++ programs over the C ABIs (tests/native), linked to the libraries above: the
    decode loop, and cfg5's fork and rollback (allocator only)."""
    _run(["g++", "-O2", "-std=c++17", "-Wall", "-Wextra", NATIVE_LOOP + ".cpp",
          "-L" + HERE, "-lyaxus_hip", "-lyaxus_kv", "-Wl,-rpath,$ORIGIN/../../yaxus_amd",
          "-o", NATIVE_LOOP])
    _run(["g++", "-O2", "-std=c++17", "-Wall", "-Wextra", NATIVE_FORK + ".cpp",
          "-L" + HERE, "-lyaxus_kv", "-Wl,-rpath,$ORIGIN/../../yaxus_amd", "-o", NATIVE_FORK])


NATIVE_REPLAY_ASAN = os.path.join(ROOT, "tests", "native", "kv_replay_asan")


def build_sanitized():
    """The allocator (kv_cache.cpp) compiled into the replay program of tests/native under
    AddressSanitizer and UndefinedBehaviorSanitizer, for the CPU tests: every out-of-bounds
    index, use after free, leak or undefined operation in its page-vector arithmetic
    aborts the run (halt_on_error)."""
    _run(["g++", "-O1", "-g", "-std=c++17", "-Wall", "-Wextra",
          "-fsanitize=address,undefined", "-fno-sanitize-recover=all", "-fno-omit-frame-pointer",
          NATIVE_REPLAY_ASAN.replace("_asan", "") + ".cpp", os.path.join(CSRC, "kv_cache.cpp"),
          "-o", NATIVE_REPLAY_ASAN])


def build_oracle():
    _run(["make", "-s", "-C", os.path.join(ROOT, "oracle"), "-B"])


def build_all():
    build_kv()
    build_hip()
    build_native_tests()
    build_sanitized()
    build_oracle()


if __name__ == "__main__":
    build_all()
    print("built", KV_LIB, HIP_LIB, file=sys.stderr)
