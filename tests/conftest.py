"""Shared test setup.

Markers: ``gpu`` -- needs the built HIP extension and a visible MI355X; the
parity tests proper. Everything else runs on the CPU: the oracle against its
known answers and golden fixtures, the host contract, and the C-ABI library's
exported symbols.
"""

import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG_ROOT = os.path.join(ROOT, "int4-kv-cache-quantization-cuda-triton-pallas_amd")
for p in (ROOT, PKG_ROOT):
    if p not in sys.path:
        sys.path.insert(0, p)

GOLDEN = os.path.join(ROOT, "tests", "golden")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs the HIP extension and a GPU (MI355X)")


def _gpu_ready():
    try:
        import torch
        if not torch.cuda.is_available():
            return False
        from flash_decode_int4 import ops
        return ops.HAS_HIP
    except Exception:
        return False


def pytest_collection_modifyitems(config, items):
    if _gpu_ready():
        return
    skip = pytest.mark.skip(reason="needs the HIP extension and a visible GPU")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture(autouse=True)
def _print_case(request):
    """Name the case before a GPU test runs, so a crash still identifies it."""
    if "gpu" in request.keywords:
        print(f"\n[case] {request.node.nodeid}", flush=True)
    yield


def load_golden(name):
    return np.load(os.path.join(GOLDEN, name), allow_pickle=False)
