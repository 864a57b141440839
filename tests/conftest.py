"""pytest configuration: the ``gpu`` marker and import paths.

The host package lives in ``flaggems-sglang_amd/`` (importable as
``flaggems_sglang``, the reference's own package name) and the CPU oracle in
``oracle/``; both are put on ``sys.path`` here.
"""

import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "flaggems-sglang_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")
    config.addinivalue_line("markers", "fused_moe: fused MoE operator tests")


def pytest_collection_modifyitems(config, items):
    # GPU tests are skipped (not failed) where no device is visible, so the
    # CPU suite can be run with or without `-m "not gpu"`.
    try:
        import torch

        has_gpu = torch.cuda.is_available()
    except Exception:  # pragma: no cover
        has_gpu = False
    if has_gpu:
        return
    skip = pytest.mark.skip(reason="no GPU visible")
    for it in items:
        if "gpu" in it.keywords:
            it.add_marker(skip)
