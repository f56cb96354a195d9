"""Test configuration: the `gpu` marker and import paths.

CPU tests (-m "not gpu") cover the oracle against the golden vectors and the
reference's known-answer tests, the host-side logic, and that the C-ABI
library loads and exports its symbols.  GPU tests (-m gpu) are the parity
tests proper and call the HIP kernels through the C ABI.
"""
import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
for path in (ROOT, ROOT / "ascend-int8-attention_amd"):
    if str(path) not in sys.path:
        sys.path.insert(0, str(path))

os.environ.setdefault("SKO_THREADS", "8")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device); parity tests through the C ABI")


def gpu_available():
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


def pytest_collection_modifyitems(config, items):
    if gpu_available():
        return
    skip = pytest.mark.skip(reason="no HIP device in this environment")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)
