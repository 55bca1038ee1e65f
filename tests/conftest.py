"""Shared test setup.

Markers: ``gpu`` tests need a gfx950 device and run on the GPU host; every
other test runs on a CPU-only machine.  The package lives in
``breeze-engine_amd/`` (a directory name that is not importable), so it and
the repository root are put on ``sys.path`` here.
"""
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG_DIR = os.path.join(ROOT, "breeze-engine_amd")
for p in (ROOT, PKG_DIR):
    if p not in sys.path:
        sys.path.insert(0, p)

GOLDEN = os.path.join(ROOT, "tests", "golden")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def orc():
    """The C restatement of the reference arithmetic (built by __graft_entry__.build)."""
    from oracle import oracle
    return oracle.c_oracle()


@pytest.fixture(scope="session")
def hb():
    from breeze_amd import hip_backend
    return hip_backend


@pytest.fixture(scope="session")
def gpu(hb):
    """Torch on cuda:0 with the library's kernels usable; fails loudly if not."""
    import torch
    assert torch.cuda.is_available(), "GPU test on a machine without a GPU"
    assert hb.available(), f"kernel library missing: {hb._SO}"
    assert hb.device_available(), hb.last_error()
    return torch


@pytest.fixture
def hi_prec(hb):
    """Restore the default activation mode after each test."""
    yield hb
    hb.set_hi_prec(False)


def rng_weights(rng, N, K, bits, dtype=np.float32, explicit_zeros=False):
    """Random MatMulNBits weights with the edge bytes the reference tests force
    (tests/test_cpu_packing.py:33-53)."""
    blocks = K // 32
    qw = rng.integers(0, 256, (N, blocks, 4 * bits), dtype=np.uint8)
    qw.reshape(-1)[:8] = [0, 1, 7, 15, 127, 128, 254, 255]
    scales = rng.uniform(0.0001, 0.02, (N, blocks)).astype(dtype)
    zeros = None
    if explicit_zeros and bits == 4:
        zeros = rng.integers(0, 256, (N, (blocks + 1) // 2), dtype=np.uint8)
    return qw, scales, zeros


def bits_equal(a, b):
    a = np.asarray(a)
    b = np.asarray(b)
    return a.shape == b.shape and np.array_equal(a.view(np.uint32), b.view(np.uint32))
