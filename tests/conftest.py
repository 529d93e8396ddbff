"""Shared test setup: the `gpu` marker and repo-root imports.

GPU tests need a real MI355X (torch.cuda with the HIP runtime) and the built
libacorn_hip.so; without a GPU they are skipped.
"""
import os
import sys

import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X GPU and libacorn_hip.so")


def pytest_collection_modifyitems(config, items):
    if torch.cuda.is_available():
        return
    skip = pytest.mark.skip(reason="no GPU device")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)
