"""Build recipe for ``libturboquant_hip.so`` (gfx950, hipcc).

Every HIP translation unit under ``csrc/`` plus the C++ API
(``csrc/turboquant.cpp``) is compiled in-tree into one shared library next to
this file, so the library travels with the source tree.
"""
from __future__ import annotations

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
INCLUDE = os.path.join(ROOT, "include")
OBJDIR = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libturboquant_hip.so")
# gfx950 only: the decode kernels' split-K merge protocol rests on gfx950's
# memory behaviour (tq_sdpa_common.h refuses any other device target too).
ARCH = "gfx950"

HIP_SOURCES = ["tq_runtime.hip", "tq_quant.hip", "tq_sdpa.hip", "tq_sdpa_mfma.hip", "tq_sdpa_hc.hip",
               "tq_prefill.hip", "tq_polar.hip"]
CXX_SOURCES = ["turboquant.cpp"]

COMMON = ["-O3", "-fPIC", "-std=c++17", f"-I{INCLUDE}", f"-I{CSRC}", "-Wall",
          "-Wno-unused-function"]
# Keep hand-written float code off the packed-fp32 VALU forms (their results
# have proven unreliable on this fleet); hipcc's host pass warns and ignores.
HIP_FLAGS = [f"--offload-arch={ARCH}", "-Xclang", "-target-feature", "-Xclang",
             "-packed-fp32-ops", "-munsafe-fp-atomics"]


def _hipcc() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    return os.path.join(rocm, "bin", "hipcc")


def _compile(src: str) -> str:
    path = os.path.join(CSRC, src)
    obj = os.path.join(OBJDIR, src + ".o")
    if src.endswith(".hip"):
        cmd = [_hipcc(), *COMMON, *HIP_FLAGS, "-c", path, "-o", obj]
    else:
        rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
        cmd = [_hipcc(), *COMMON, "-x", "c++", "-D__HIP_PLATFORM_AMD__", f"-I{rocm}/include",
               "-c", path, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    errs = "\n".join(l for l in r.stderr.splitlines()
                     if "packed-fp32-ops" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"compile failed: {' '.join(cmd)}\n{errs}")
    if errs.strip():
        sys.stderr.write(errs + "\n")
    return obj


CPP_TESTS = ["test_sdpa_int4"]
CPP_TEST_DIR = os.path.join(os.path.dirname(HERE), "tests", "cpp")


def build_cpp_tests() -> list:
    """Compile the C++ API tests (tests/cpp/*.cpp) against the library, with
    an rpath to it, so the GPU box runs them without building."""
    outs = []
    for name in CPP_TESTS:
        src = os.path.join(CPP_TEST_DIR, name + ".cpp")
        exe = os.path.join(CPP_TEST_DIR, name)
        rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
        cmd = [_hipcc(), "-O2", "-std=c++17", f"-I{INCLUDE}", "-D__HIP_PLATFORM_AMD__",
               f"-I{rocm}/include", "-x", "c++", src, "-o", exe, f"-L{HERE}", "-lturboquant_hip",
               f"-L{rocm}/lib", "-lamdhip64", "-Wl,-rpath,$ORIGIN/../../gemma4metal_amd"]
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError(f"compile failed: {' '.join(cmd)}\n{r.stderr}")
        outs.append(exe)
    return outs


def build(verbose: bool = False) -> str:
    os.makedirs(OBJDIR, exist_ok=True)
    srcs = HIP_SOURCES + [s for s in CXX_SOURCES if os.path.exists(os.path.join(CSRC, s))]
    with ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        objs = list(ex.map(_compile, srcs))
    tmp = LIB + ".tmp"
    cmd = [_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed: {' '.join(cmd)}\n{r.stderr}")
    os.replace(tmp, LIB)
    build_cpp_tests()
    if verbose:
        print(f"built {LIB}")
    return LIB


if __name__ == "__main__":
    build(verbose=True)
