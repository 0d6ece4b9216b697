"""Shared pytest setup: the ``gpu`` marker, the native library, and the oracle as the
``"reference"`` backend for tests that compare against it."""

from __future__ import annotations

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config: pytest.Config) -> None:
    config.addinivalue_line("markers", "gpu: needs a gfx950 GPU (run with -m gpu)")
    lib = ROOT / "omniwave_amd" / "libomniwave_amd.so"
    if not lib.exists():  # build only when nothing is built yet
        from omniwave_amd import _build

        _build.build()


def oracle_reference_backend(*, x, plan, a_u, a_v, a_o, b_u, b_v, b_o, gamma):
    """The oracle's restated reference backend, in the dtype of x (the reference's behaviour).

    Always evaluated on the CPU (its batched einsums never run on the GPU); the result is
    returned on x's device.
    """
    from oracle.bigemm import bigemm_delta_reference

    dt = x.dtype
    cpu = {k: v.detach().cpu().to(dt) for k, v in
           dict(a_u=a_u, a_v=a_v, a_o=a_o, b_u=b_u, b_v=b_v, b_o=b_o, gamma=gamma).items()}
    out = bigemm_delta_reference(x=x.detach().cpu(), plan=plan, **cpu)
    return out.to(x.device)


@pytest.fixture
def oracle_backend():
    """Registers the oracle as omniwave_amd's ``"reference"`` backend for one test."""
    from omniwave_amd.bigemm import register_backend

    register_backend("reference", oracle_reference_backend)
    yield oracle_reference_backend
    register_backend("reference", None)
