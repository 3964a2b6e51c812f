"""Runs the C++ host-layer tests (tests/cpp, built by __graft_entry__.build()).

test_memory: Tensor bf16 rules, BlockPool / PageTable known answers of the
reference (src/main.cpp Phase 3/4, tests/phase7_smoke.cpp) and random
alloc/append/free traces compared op for op with the oracle.
test_host_layer: Sampler configuration and RNG rules; its device sections
(DeviceBatch, device block tables, device pool copies) report themselves
skipped here and run in tests/test_gpu_host_cpp.py and, over host memory, in
tests/test_host_sanitizers.py.  CPU only.
"""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BIN = os.path.join(ROOT, "build", "bin")


def _run(name, timeout=120):
    exe = os.path.join(BIN, name)
    if not os.path.exists(exe):
        pytest.fail(f"{exe} is missing: run __graft_entry__.build() first")
    proc = subprocess.run([exe], stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True,
                          timeout=timeout)
    return proc.returncode, proc.stdout


def test_cpp_memory_and_tensor():
    rc, out = _run("test_memory")
    assert rc == 0, out


def test_cpp_host_layer_host_sections():
    rc, out = _run("test_host_layer")
    assert rc == 0, out
