"""The C++ HipContext mirror (include/kraken/hip_context.hpp), driven by
tests/cpp/hip_context_check.cpp the way the reference runtime drives
toyllm::mps::MpsContext (mps_backend.hpp:76-428): Status codes and messages
without a GPU, and closed-form decode parity through the wrapper on one."""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BIN = os.path.join(ROOT, "kraken-infer_amd", "build", "hip_context_check")


def _binary():
    if not os.path.exists(BIN):
        subprocess.run(["make", "-C", os.path.join(ROOT, "kraken-infer_amd")], check=True,
                       capture_output=True)
    return BIN


def _run(mode):
    proc = subprocess.run([_binary(), mode], capture_output=True, text=True, timeout=120)
    print(proc.stdout)
    assert proc.returncode == 0, proc.stdout + proc.stderr
    assert "all checks passed" in proc.stdout
    return proc.stdout


def test_cpp_mirror_status_and_validation_without_gpu():
    import torch

    if torch.cuda.device_count() > 0:
        pytest.skip("a GPU is present: create() would succeed")
    out = _run("cpu")
    assert "heads % kv_heads != 0 rejected" in out


@pytest.mark.gpu
def test_cpp_mirror_decode_closed_form_on_gpu():
    out = _run("gpu")
    assert "zero-query decode equals the mean of V" in out
