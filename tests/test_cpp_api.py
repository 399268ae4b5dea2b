"""The C++ surface: include/nve_amd.hpp gives a C++ host the reference's
layer and table classes (include/embedding_layer.hpp:34-213,
gpu_table.hpp:44-240, linear_embedding_layer.hpp:30-80,
host_embedding_layer.hpp) over the C ABI.  tests/cpp/cpp_api_check.cpp is such
a host, built next to the library by its Makefile; it checks its results bit
for bit (dyadic tables) and prints "<mode> ok"."""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BIN = os.path.join(ROOT, "nv-embedding-cache_amd", "cpp_api_check")


def run(mode):
    assert os.path.exists(BIN), "cpp_api_check is built by nv-embedding-cache_amd/Makefile (build())"
    p = subprocess.run([BIN, mode], capture_output=True, text=True, timeout=120)
    assert p.returncode == 0 and f"{mode} ok" in p.stdout, p.stdout + p.stderr


def test_host_layer_through_the_cpp_classes():
    run("host")


@pytest.mark.gpu
def test_gpu_and_uvm_layers_through_the_cpp_classes():
    run("gpu")
