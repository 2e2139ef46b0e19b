"""Test setup: import paths, the ``gpu`` marker, and helpers shared by the suites.

``-m "not gpu"`` runs on a CPU-only machine: the oracle against its pins, the host
logic (the reference's rejections), and the C ABI's exports.  ``-m gpu`` needs a
ROCm GPU and the built library; those tests call the kernels through the C ABI
(via the ``cpu_attention`` package) and compare with the CPU oracle.
"""

import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "cpu-attention_amd")
for p in (ROOT, PKG):
    if p not in sys.path:
        sys.path.insert(0, p)

LIB = os.path.join(PKG, "cpu_attention", "libcpu_attention_hip.so")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X) and the built kernel library")
    config.addinivalue_line("markers", "slow: larger shapes (full BASELINE sizes)")
    if not os.path.exists(LIB) and os.path.exists("/opt/rocm/bin/hipcc"):
        # A fresh checkout: build the kernel library once (seconds).
        subprocess.run([sys.executable, os.path.join(PKG, "build.py")], check=True)


def gpu_available():
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:  # noqa: BLE001
        return False


@pytest.fixture(scope="session")
def cuda():
    if not gpu_available():
        pytest.skip("no ROCm GPU")
    import torch
    return torch.device("cuda:0")
