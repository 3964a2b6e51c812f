"""Build recipes for the native parts of stratakv_amd.

Everything is compiled in-tree so the built files travel with the source tree:

* ``stratakv_amd/libstratakv_amd.so`` -- the gfx950 HIP kernels, the C ABI
  (``include/stratakv_amd.h``) and the C++17 host layer (``include/stratakv/``),
  built with ``hipcc --offload-arch=gfx950``.
* ``stratakv_amd/libstratakv_amd_gemm.so`` -- the hipBLASLt projections of long
  prompt chunks (``include/stratakv_amd_gemm.h``), the only library that links
  hipBLASLt; it links the one above, whose host layer opens it on demand.
* ``build/bin/test_*`` -- the C++ test programs under ``tests/cpp``;
  ``build/bin/bench_*`` -- the C++ benchmark drivers under ``stratakv_amd/csrc/bench``.
* ``oracle/liboracle.so`` and, when the StrataKV sources are present,
  ``oracle/_ref/libstratakv_ref.so`` -- test infrastructure (``oracle/Makefile``).
* ``build/asan/`` -- test infrastructure: the C++ host layer and the host-side
  test programs built with AddressSanitizer and UndefinedBehaviorSanitizer
  (g++, no GPU code), linked against ``tests/cpp/abi_host_stand_in.cpp``
  instead of the library (``python -m stratakv_amd._build asan``).
"""
from __future__ import annotations

import glob
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "stratakv_amd")
CSRC = os.path.join(PKG, "csrc")
INCLUDE = os.path.join(ROOT, "include")
LIB = os.path.join(PKG, "libstratakv_amd.so")
GEMM_LIB = os.path.join(PKG, "libstratakv_amd_gemm.so")
BIN = os.path.join(ROOT, "build", "bin")
ORACLE = os.path.join(ROOT, "oracle")
REFERENCE = os.environ.get("STRATAKV_REFERENCE", "/root/reference")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
# Packed fp32 VALU forms are kept out of every kernel (the compiler otherwise
# forms v_pk_* from float2-shaped code); the host pass ignores the feature.
NO_PACKED_FP32 = ["-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]
HIP_FLAGS = ["-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}", "-Wall"] + NO_PACKED_FP32
# Per-file additions.  skv_layer_ops.hip: the matrix-core projections keep
# their MFMA accumulators in ordinary VGPRs (in AGPRs the allocator rotates
# them between unrolled stages with ~40 copies per loop iteration).
FILE_FLAGS = {"skv_layer_ops.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"]}


def _run(cmd: list[str], cwd: str | None = None) -> None:
    proc = subprocess.run(cmd, cwd=cwd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in proc.stdout.splitlines()
                    if "packed-fp32-ops' is not a recognized feature" not in l)
    if proc.returncode != 0:
        raise RuntimeError(f"build step failed ({proc.returncode}): {' '.join(cmd)}\n{out}")
    if out.strip():
        sys.stderr.write(out + "\n")


OBJ = os.path.join(ROOT, "build", "obj")
CXX = os.environ.get("CXX", "g++")


def _jobs() -> int:
    """Parallel compile jobs: MAX_JOBS when set, else the CPU count, at most 16."""
    try:
        return max(1, min(16, int(os.environ.get("MAX_JOBS", "0")) or (os.cpu_count() or 1)))
    except ValueError:
        return max(1, min(16, os.cpu_count() or 1))


def _run_all(cmds: list[list[str]]) -> None:
    from concurrent.futures import ThreadPoolExecutor
    with ThreadPoolExecutor(max_workers=_jobs()) as pool:
        for f in [pool.submit(_run, c) for c in cmds]:
            f.result()


def build_library() -> str:
    """Compile the HIP kernels and C ABI (hipcc, gfx950) and the C++ host
    layer (plain C++17; it reaches the GPU only through the C ABI) into one
    shared library."""
    os.makedirs(OBJ, exist_ok=True)
    objs, cmds = [], []
    for src in sorted(glob.glob(os.path.join(CSRC, "host", "*.cpp"))):
        obj = os.path.join(OBJ, os.path.basename(src) + ".o")
        cmds.append([CXX, "-O2", "-std=c++17", "-fPIC", "-Wall", "-Wextra", f"-I{INCLUDE}", "-c", src,
                     "-o", obj])
        objs.append(obj)
    for src in sorted(glob.glob(os.path.join(CSRC, "*.hip"))):
        obj = os.path.join(OBJ, os.path.basename(src) + ".o")
        extra = FILE_FLAGS.get(os.path.basename(src), [])
        cmds.append([HIPCC, *HIP_FLAGS, *extra, f"-I{INCLUDE}", f"-I{CSRC}", "-c", src, "-o", obj])
        objs.append(obj)
    gemm_src = os.path.join(CSRC, "gemm", "skv_prompt_gemm.hip")
    gemm_obj = os.path.join(OBJ, "gemm_" + os.path.basename(gemm_src) + ".o")
    cmds.append([HIPCC, *HIP_FLAGS, f"-I{INCLUDE}", f"-I{CSRC}", "-c", gemm_src, "-o", gemm_obj])
    _run_all(cmds)
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", *objs, "-Wl,-soname,libstratakv_amd.so", "-o", LIB + ".tmp"])
    os.replace(LIB + ".tmp", LIB)
    # The prompt-pass GEMMs on hipBLASLt, in their own library (found beside
    # libstratakv_amd.so through $ORIGIN).
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", gemm_obj, f"-L{PKG}", "-lstratakv_amd", "-lhipblaslt",
          "-Wl,-rpath,$ORIGIN", "-Wl,-soname,libstratakv_amd_gemm.so", "-o", GEMM_LIB + ".tmp"])
    os.replace(GEMM_LIB + ".tmp", GEMM_LIB)
    return LIB


def build_cpp_tests() -> list[str]:
    """Compile tests/cpp/*.cpp against the library (and the oracle, for traces)."""
    os.makedirs(BIN, exist_ok=True)
    outs, cmds = [], []
    srcs = glob.glob(os.path.join(ROOT, "tests", "cpp", "test_*.cpp")) + \
        glob.glob(os.path.join(ROOT, "tests", "cpp", "tool_*.cpp"))
    for src in sorted(srcs):
        exe = os.path.join(BIN, os.path.splitext(os.path.basename(src))[0])
        cmds.append([HIPCC, "-O2", "-std=c++17", f"-I{INCLUDE}", f"-I{ORACLE}", "-x", "c++", src,
                     f"-L{PKG}", "-lstratakv_amd", f"-Wl,-rpath,{PKG}",
                     f"-L{ORACLE}", "-loracle", f"-Wl,-rpath,{ORACLE}", "-o", exe])
        outs.append(exe)
    _run_all(cmds)
    return outs


def build_bench() -> list[str]:
    """Compile the C++ benchmark drivers (stratakv_amd/csrc/bench/*.cpp) into
    build/bin/bench_<name>; they use only the library's public headers."""
    os.makedirs(BIN, exist_ok=True)
    outs, cmds = [], []
    for src in sorted(glob.glob(os.path.join(CSRC, "bench", "*.cpp"))):
        exe = os.path.join(BIN, "bench_" + os.path.splitext(os.path.basename(src))[0])
        cmds.append([CXX, "-O2", "-std=c++17", "-Wall", f"-I{INCLUDE}", src, f"-L{PKG}", "-lstratakv_amd",
                     f"-Wl,-rpath,{PKG}", "-o", exe])
        outs.append(exe)
    _run_all(cmds)
    return outs


def build_oracle() -> None:
    """Test infrastructure: the C oracle, plus the reference checker when present."""
    _run(["make", "-B", "-C", ORACLE, "all"])
    if os.path.isdir(os.path.join(REFERENCE, "src")):
        _run(["make", "-B", f"-j{_jobs()}", "-C", ORACLE, "ref", f"REF={REFERENCE}"])


ASAN = os.path.join(ROOT, "build", "asan")
# Programs of tests/cpp whose code paths are host-only (or run over the host
# stand-in of the C ABI); test_gpu_layer needs the kernels and is left out.
ASAN_PROGRAMS = ("test_memory", "test_host_layer", "tool_model")
SANITIZE = ["-fsanitize=address,undefined", "-fno-sanitize-recover=undefined", "-fno-omit-frame-pointer"]


def build_sanitized() -> list[str]:
    """Test infrastructure: the host layer (BlockPool, PageTable, DeviceBatch,
    the safetensors loader, Sampler, Generator, Tensor) and the host test
    programs under AddressSanitizer + UndefinedBehaviorSanitizer.  Built with
    g++ alone; the C ABI comes from tests/cpp/abi_host_stand_in.cpp (host
    memory, copies and events; every kernel entry point reports
    SKV_ERR_UNSUPPORTED), so nothing here touches a GPU."""
    obj_dir = os.path.join(ASAN, "obj")
    os.makedirs(obj_dir, exist_ok=True)
    flags = ["-O1", "-g", "-std=c++17", "-Wall", *SANITIZE, f"-I{INCLUDE}", f"-I{ORACLE}"]
    objs, cmds = [], []
    for src in sorted(glob.glob(os.path.join(CSRC, "host", "*.cpp"))) + \
            [os.path.join(ROOT, "tests", "cpp", "abi_host_stand_in.cpp")]:
        obj = os.path.join(obj_dir, os.path.basename(src) + ".o")
        cmds.append([CXX, *flags, "-c", src, "-o", obj])
        objs.append(obj)
    oracle_obj = os.path.join(obj_dir, "oracle.c.o")
    cmds.append([os.environ.get("CC", "gcc"), "-O1", "-g", "-std=c11", *SANITIZE, "-c",
                 os.path.join(ORACLE, "oracle.c"), "-o", oracle_obj])
    tests = []
    for name in ASAN_PROGRAMS:
        obj = os.path.join(obj_dir, name + ".cpp.o")
        cmds.append([CXX, *flags, "-c", os.path.join(ROOT, "tests", "cpp", name + ".cpp"), "-o", obj])
        tests.append((name, obj))
    _run_all(cmds)
    outs = []
    link = []
    for name, obj in tests:
        exe = os.path.join(ASAN, name)
        link.append([CXX, *SANITIZE, obj, *objs, oracle_obj, "-lm", "-o", exe])
        outs.append(exe)
    _run_all(link)
    return outs


def build_all() -> None:
    build_library()
    build_bench()
    build_oracle()
    build_cpp_tests()
    build_sanitized()


if __name__ == "__main__":
    if sys.argv[1:] == ["asan"]:
        print("built", *build_sanitized())
    else:
        build_all()
        print("built", LIB)
