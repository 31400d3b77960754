"""Shared test setup.

Markers: `gpu` = needs a gfx950 GPU (run with -m gpu on the GPU box); every
other test runs on the CPU. GPU tests compare the HIP path with the CPU
oracle (oracle/), which only tests load.
"""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a gfx950 GPU and liblynnreal_amd.so")


def pytest_collection_modifyitems(config, items):
    import torch
    if torch.cuda.is_available():
        return
    skip = pytest.mark.skip(reason="no GPU in this process")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)
