"""Runs the C++ test mains of the host layer (soar.cpp_amd/host), the way
the reference registers its test executables with CTest."""
import os
import subprocess

import pytest

from conftest import ROOT

BUILD = os.environ.get("SOAR_HOST_BUILD") or os.path.join(ROOT, "soar.cpp_amd", "host", "build")


def run(name, timeout=300):
    exe = os.path.join(BUILD, name)
    assert os.path.exists(exe), f"{exe} is not built (run __graft_entry__.build())"
    r = subprocess.run([exe], capture_output=True, text=True, timeout=timeout)
    print(r.stdout, r.stderr)
    assert r.returncode == 0, r.stdout + r.stderr


def test_host_layer_cpu():
    run("test_host_cpu")


@pytest.mark.gpu
def test_host_layer_gpu(gpu):
    run("test_host_gpu")
