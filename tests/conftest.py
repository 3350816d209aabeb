"""Shared fixtures: the `gpu` marker, library loading, tolerance helpers."""
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

# the attention path's tolerance for outputs against the fp32 oracle
ATOL = 2e-3
RTOL = 1e-3


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


def assert_close_f16(got_f16_bits, ref32, atol=ATOL, rtol=RTOL, what="output"):
    """|gpu - ref_fp32| <= atol + rtol*|ref_fp32| elementwise (fp16 gpu result)."""
    got = np.asarray(got_f16_bits).view(np.float16).astype(np.float32) \
        if np.asarray(got_f16_bits).dtype == np.uint16 else np.asarray(got_f16_bits, np.float32)
    ref = np.asarray(ref32, np.float32)
    assert got.shape == ref.shape, (got.shape, ref.shape)
    assert np.all(np.isfinite(got)), f"{what}: non-finite values"
    err = np.abs(got - ref)
    bound = atol + rtol * np.abs(ref)
    bad = err > bound
    if bad.any():
        i = np.unravel_index(np.argmax(err - bound), err.shape)
        raise AssertionError(
            f"{what}: {bad.sum()} of {bad.size} outside {atol}+{rtol}|ref|; worst at {i}: "
            f"got {got[i]} ref {ref[i]} (max abs err {err.max():.3g})")
    return float(err.max())


@pytest.fixture(scope="session")
def orc():
    import oracle
    oracle.lib()
    return oracle


@pytest.fixture(scope="session")
def cia():
    import cuda_inf_amd
    cuda_inf_amd.lib()
    return cuda_inf_amd


@pytest.fixture(scope="session")
def dev():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")
