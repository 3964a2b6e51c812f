"""The C++ host layer under AddressSanitizer + UndefinedBehaviorSanitizer.

build/asan/ (stratakv_amd/_build.py, target ``asan``) holds the host layer --
BlockPool, PageTable, DeviceBatch, the safetensors loader, Sampler, Generator,
Tensor -- and the host test programs compiled with
-fsanitize=address,undefined and linked against tests/cpp/abi_host_stand_in.cpp,
a host-memory implementation of the C ABI's memory, copy, event and scatter
entry points (kernel entry points report SKV_ERR_UNSUPPORTED).  Any sanitizer
report, leaks included, fails the program and so the test.  CPU only.
"""
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ASAN = os.path.join(ROOT, "build", "asan")
ENV = dict(os.environ,
           ASAN_OPTIONS="detect_leaks=1:halt_on_error=1:abort_on_error=0:exitcode=23",
           UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1")


def _exe(name):
    exe = os.path.join(ASAN, name)
    if not os.path.exists(exe):
        pytest.fail(f"{exe} is missing: run __graft_entry__.build() first")
    return exe


def _clean(out):
    return "ERROR: AddressSanitizer" not in out and "ERROR: LeakSanitizer" not in out \
        and "runtime error:" not in out


@pytest.mark.parametrize("name", ["test_memory", "test_host_layer"])
def test_host_programs_under_sanitizers(name):
    proc = subprocess.run([_exe(name)], stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True,
                          env=ENV, timeout=300)
    assert proc.returncode == 0 and _clean(proc.stdout), proc.stdout
    # The stand-in provides device memory, so every section ran.
    assert "all checks passed" in proc.stdout and "skipped" not in proc.stdout, proc.stdout


def test_loader_cases_under_sanitizers():
    """Every case of tests/test_model_loader.py (malformed headers, dtype
    decoding, require-mapped, the linear transpose) against the sanitized
    tool_model."""
    if not os.path.exists(os.path.join(ROOT, "oracle", "_ref", "libstratakv_ref.so")):
        pytest.skip("oracle/_ref is not built (the StrataKV sources are absent)")
    env = dict(ENV, SKV_TOOL_MODEL=_exe("tool_model"))
    proc = subprocess.run([sys.executable, "-m", "pytest", "-q", "-x", "-p", "no:cacheprovider",
                           os.path.join(ROOT, "tests", "test_model_loader.py")],
                          stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True, env=env, timeout=600,
                          cwd=ROOT)
    assert proc.returncode == 0, proc.stdout[-4000:]
    assert " passed" in proc.stdout and " skipped" not in proc.stdout, proc.stdout[-2000:]
