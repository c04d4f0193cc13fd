"""Shared test helpers.  GPU tests are marked ``@pytest.mark.gpu`` and call the HIP library
through the package (C ABI); CPU tests cover the oracle, the golden fixtures, host logic and
the ABI surface of the built library."""
import os
import sys

import numpy as np
import pytest

ROOT = os.path.abspath(os.path.join(os.path.dirname(__file__), ".."))
sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (ROCm GPU) and the built HIP library")


def rel_err(a, b) -> float:
    """||a - b|| / ||b|| in float64 (the reference's rel_err, tests/conftest.py:53-55)."""
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / (np.linalg.norm(b) + 1e-30))


def assert_close(a, b, rtol=1e-5, atol=1e-6, what=""):
    """Elementwise |a - b| <= atol + rtol * |b| (fp32 tolerance of the north star), reporting the
    worst element."""
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    assert a.shape == b.shape, f"{what}: shape {a.shape} != {b.shape}"
    err = np.abs(a - b)
    bound = atol + rtol * np.abs(b)
    bad = err > bound
    if bad.any():
        i = np.unravel_index(np.argmax(err - bound), a.shape)
        raise AssertionError(f"{what}: {int(bad.sum())} of {a.size} elements outside rtol={rtol} atol={atol}; "
                             f"worst at {i}: got {a[i]!r} want {b[i]!r} (rel_err {rel_err(a, b):.2e})")


def assert_parity(got, want, mag, unc=None, rtol=1e-5, atol=1e-6, what=""):
    """The fp32 parity bar against the float64 oracle.

    * elementwise: |got - want| <= atol + rtol * mag + unc, where mag is the oracle's sum of
      |terms| of that output (fp32 summation error scales with it, not with |want|, when the
      terms cancel) and unc the contribution of relu masks an fp32 z may decide either way;
    * whole tensor: ||max(|got - want| - unc, 0)|| <= rtol * ||want|| (the reference's rel_err
      criterion, tests/conftest.py:53-55)."""
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    mag = np.asarray(mag, np.float64)
    unc = np.zeros_like(want) if unc is None else np.asarray(unc, np.float64)
    assert got.shape == want.shape, f"{what}: shape {got.shape} != {want.shape}"
    err = np.abs(got - want)
    bound = atol + rtol * mag + unc
    bad = err > bound
    if bad.any():
        i = np.unravel_index(np.argmax(err - bound), got.shape)
        raise AssertionError(f"{what}: {int(bad.sum())} of {got.size} elements outside the bound; worst at {i}: "
                             f"got {got[i]!r} want {want[i]!r} mag {mag[i]!r} unc {unc[i]!r}")
    resid = np.maximum(err - unc, 0.0)
    r = float(np.linalg.norm(resid) / (np.linalg.norm(want) + 1e-30))
    assert r <= rtol, f"{what}: relative error {r:.3e} > {rtol}"
    return r


def gpu_available() -> bool:
    try:
        import torch

        return torch.cuda.is_available()
    except Exception:
        return False


@pytest.fixture
def oracle():
    from oracle import oracle as o

    return o
