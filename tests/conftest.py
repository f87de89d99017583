"""Test configuration.

Markers: ``gpu`` — needs an MI355X (run with ``-m gpu``); everything else runs
on the CPU.  GPU tests are skipped when no GPU is visible.
"""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG_DIR = os.path.join(ROOT, "fused-logprob-entropy-cuda-kernel-for-llm-post-training_amd")
for p in (PKG_DIR, ROOT, os.path.join(ROOT, "tests")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X GPU (HIP kernels)")


def pytest_collection_modifyitems(config, items):
    import torch
    if torch.cuda.is_available():
        return
    skip = pytest.mark.skip(reason="no GPU visible")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture(scope="session")
def oracle():
    from oracle import klp_oracle
    return klp_oracle.get()
