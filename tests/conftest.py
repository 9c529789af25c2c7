"""pytest configuration: the `gpu` marker and import path.

Tests marked `gpu` need a real MI355X (HIP device). They are skipped, not
failed, when torch sees no GPU, so `-m "not gpu"` and a GPU-less run stay
green; on a GPU box they run and fail loudly if libveda_hip.so is missing.
"""

import pathlib
import sys

import pytest
import torch

ROOT = pathlib.Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line('markers', 'gpu: needs a HIP GPU (MI355X)')


def pytest_collection_modifyitems(config, items):
    if torch.cuda.is_available():
        return
    skip = pytest.mark.skip(reason='no GPU visible to torch')
    for item in items:
        if 'gpu' in item.keywords:
            item.add_marker(skip)
