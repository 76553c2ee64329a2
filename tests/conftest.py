"""Shared pytest setup.

* ``gpu`` marks tests that launch HIP kernels; they are skipped when no GPU is
  visible (``python -m pytest -m "not gpu"`` runs the CPU tier, ``-m gpu`` the
  parity tier on an MI355X).
* ``oracle/`` (the CPU restatement of the reference path, test infrastructure
  only) is put on ``sys.path`` here; the package itself never imports it.
* The reference's metric, ``max|y - ref| / mean|ref|`` (tests/conftest.py:69-82
  in arvindcr4/nibblegemm), and the north-star metric ``max|y - ref| / rms(ref)``
  are provided as fixtures.
"""
from __future__ import annotations

import os
import sys

import numpy as np
import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "oracle")):
    if p not in sys.path:
        sys.path.insert(0, p)

HAS_GPU = torch.cuda.is_available()


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: launches HIP kernels; needs an AMD GPU")


def pytest_collection_modifyitems(config, items):
    if HAS_GPU:
        return
    skip = pytest.mark.skip(reason="no GPU visible")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture(scope="session", autouse=True)
def _exact_fp32_reference():
    """Keep torch fp32 matmuls (used by the package's reference_matmul) out of
    reduced-precision modes."""
    if HAS_GPU:
        torch.backends.cuda.matmul.allow_tf32 = False
    yield


@pytest.fixture(autouse=True)
def _seed():
    torch.manual_seed(0)


@pytest.fixture(scope="session")
def oracle():
    import oracle as O  # noqa: PLC0415

    O.lib()
    return O


@pytest.fixture(scope="session")
def ext():
    """The native binding; a GPU test fails (does not skip) if it is missing."""
    import nibblegemm_amd as ng  # noqa: PLC0415

    return ng.extension()


def _np(t):
    if isinstance(t, torch.Tensor):
        return t.detach().float().cpu().numpy().astype(np.float64)
    return np.asarray(t, dtype=np.float64)


@pytest.fixture(scope="session")
def rel_err():
    """``max|y - ref| / mean|ref|`` -- the reference suite's tolerance metric."""

    def _rel_err(y, ref) -> float:
        y, ref = _np(y), _np(ref)
        return float(np.abs(y - ref).max() / np.abs(ref).mean())

    return _rel_err


@pytest.fixture(scope="session")
def rms_err():
    """``max|y - ref| / rms(ref)`` -- the north-star bound is 1e-2."""

    def _rms_err(y, ref) -> float:
        y, ref = _np(y), _np(ref)
        return float(np.abs(y - ref).max() / np.sqrt(np.mean(ref * ref)))

    return _rms_err
