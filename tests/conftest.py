import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP (MI355X) device")
    config.addinivalue_line("markers", "slow: long-running CPU check")


def pytest_collection_modifyitems(config, items):
    import torch

    if torch.cuda.is_available():
        return
    skip = pytest.mark.skip(reason="no HIP device")
    for it in items:
        if "gpu" in it.keywords:
            it.add_marker(skip)


def seeded(*key):
    """Reproducible generator for a test case (stable across processes, unlike hash())."""
    import zlib

    return np.random.default_rng(zlib.crc32(repr(key).encode()))


def softmax_psf(rng, C, k, batch=1):
    """Seeded psf the way Converse2D initialises it: softmax over the k*k taps of N(0,1)."""
    w = rng.standard_normal((batch, C, k * k))
    w = np.exp(w - w.max(axis=-1, keepdims=True))
    w /= w.sum(axis=-1, keepdims=True)
    return w.reshape(batch, C, k, k).astype(np.float32)
