"""The C++ API (include/turboquant.h): exported from the library, and the
C++ test mirroring the reference's tests/test_sdpa_int4.cpp passes on GPU."""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(ROOT, "gemma4metal_amd", "libturboquant_hip.so")
EXE = os.path.join(ROOT, "tests", "cpp", "test_sdpa_int4")

CXX_API = ["turboquant::sdpa_int4(", "turboquant::sdpa_int4_into(", "turboquant::sdpa_int4_ragged(",
           "turboquant::sdpa_int4_workspace_size(",
           "turboquant::quantize(", "turboquant::dequantize(", "turboquant::kv_append_int4(",
           "turboquant::polar_quantize(", "turboquant::polar_dequantize(",
           "turboquant::polar_quantize_packed(", "turboquant::polar_dequantize_packed(",
           "turboquant::polar_dequantize_packed_fast(", "turboquant::polar_dequantize_fast(",
           "turboquant::compressed_sdpa(", "turboquant::compressed_score(",
           "turboquant::set_metallib_path("]


def test_cxx_api_exported():
    out = subprocess.run(["nm", "-DC", "--defined-only", LIB], capture_output=True, text=True,
                         check=True).stdout
    missing = [s for s in CXX_API if s not in out]
    assert not missing, missing


def test_cxx_test_links_against_library():
    assert os.path.exists(EXE), "run __graft_entry__.build() first"
    out = subprocess.run(["ldd", EXE], capture_output=True, text=True).stdout
    assert "libturboquant_hip.so" in out and "not found" not in out.split("libturboquant_hip.so")[1].splitlines()[0]


@pytest.mark.gpu
def test_cxx_sdpa_int4_matches_reference_composition():
    r = subprocess.run([EXE], capture_output=True, text=True, timeout=120)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
    assert r.stdout.count("PASS") == 6
