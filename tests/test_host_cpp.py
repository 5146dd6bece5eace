"""Runs the C++ host-layer test program (minitensor_amd/cpp/tests/host_tests.cpp):
the reference API (Tensor<float>, matmul, bmm, conv2d, F::linear, Linear,
Conv2D, OpRegistry) on the CPU device -- pinned bit for bit to the reference's
own outputs in tests/golden/reference_vectors.bin -- and on the GPU against
the CPU device."""
import subprocess
from pathlib import Path

import pytest

EXE = Path(__file__).resolve().parents[1] / "minitensor_amd" / "lib" / "mt_host_tests"
GOLDEN = Path(__file__).resolve().parent / "golden" / "reference_vectors.bin"


def run(flag):
    assert EXE.exists(), f"{EXE} missing: run `python -m minitensor_amd.build`"
    r = subprocess.run([str(EXE), flag, "--golden", str(GOLDEN)], capture_output=True, text=True,
                       timeout=600)
    print(r.stdout[-6000:], r.stderr[-2000:])
    assert r.returncode == 0, f"host tests {flag} failed"
    assert " 0 failures" in r.stdout


def test_host_layer_cpu_device():
    run("--cpu")


@pytest.mark.gpu
def test_host_layer_gpu_device(dev):
    run("--gpu")
