"""Runs the C++ host-mirror tests (tests/cpp/test_host.cpp): the reference's
own inline tests of attention.rs / cache_ops.rs / model_runner.rs restated
against rllm_amd/host/rllm_host.hpp, which calls the C ABI."""
import os
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
BIN = os.path.join(HERE, "cpp", "_build", "test_host")


def _binary():
    if not os.path.exists(BIN):   # normally built by __graft_entry__.build()
        subprocess.run(["make", "-s", "-C", os.path.join(HERE, "cpp")], check=True)
    return BIN


def test_host_mirror_cpu():
    r = subprocess.run([_binary(), "cpu"], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "0 failure(s)" in r.stdout


@pytest.mark.gpu
def test_host_mirror_gpu_kv_cache_and_decode():
    r = subprocess.run([_binary(), "gpu"], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "0 failure(s)" in r.stdout
