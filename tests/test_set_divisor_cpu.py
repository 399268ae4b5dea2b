"""The cache's division-free set / tag arithmetic (csrc/kernels/set_divisor.hpp,
used by every cache lookup kernel) against plain division and the reference's
rebuilt-key compare (ec_hash.h:36-60, ec_set_associative.cuh:46-80), brute
force on the host: tests/cpp/set_divisor_check.cpp over edge and random
divisors up to 2^32 - 1, dividends up to 2^64 - 1 and tags (the empty-way
sentinel among them), in 64 and 32 bits."""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++")
def test_set_divisor_matches_division_and_the_rebuilt_key_compare(tmp_path):
    exe = tmp_path / "set_divisor_check"
    subprocess.run(["g++", "-O2", "-std=c++17", "-D__HIP_PLATFORM_AMD__", "-I/opt/rocm/include",
                    "-I", os.path.join(ROOT, "nv-embedding-cache_amd", "csrc"), "-o", str(exe),
                    os.path.join(ROOT, "tests", "cpp", "set_divisor_check.cpp")], check=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True)
    assert out.returncode == 0 and out.stdout.startswith("ok"), out.stdout
    assert int(out.stdout.split()[1]) > 1_000_000


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++")
def test_planted_off_by_one_multiplier_is_caught(tmp_path):
    """The check has teeth: a multiplier one too small fails it."""
    src = open(os.path.join(ROOT, "tests", "cpp", "set_divisor_check.cpp")).read()
    src = src.replace("const SetDivisor s = nve_amd::make_set_divisor(d);",
                      "SetDivisor s = nve_amd::make_set_divisor(d); s.m64 -= 1;")
    f = tmp_path / "planted.cpp"
    f.write_text(src)
    exe = tmp_path / "planted"
    subprocess.run(["g++", "-O2", "-std=c++17", "-D__HIP_PLATFORM_AMD__", "-I/opt/rocm/include",
                    "-I", os.path.join(ROOT, "nv-embedding-cache_amd", "csrc"), "-o", str(exe), str(f)], check=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True)
    assert out.returncode != 0 and "FAIL div64" in out.stdout
