"""Test configuration: markers and import paths.

``gpu`` tests need a ROCm device and the built ``libcnna.so``; everything else
runs on the CPU.  The package directory has a hyphenated name (it mirrors the
reference's flat module layout: ``from layers import MultiHeadConvNNAttention``),
so it is put on ``sys.path`` here.
"""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "convolutional-nearest-neighbor-attention_amd")
for p in (ROOT, PKG):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X / gfx950) and the built HIP library")
    config.addinivalue_line("markers", "slow: long-running")
