"""Backend dispatch: mirrors the reference's tests/test_dispatch.py:13-66 with the hip backend
in place of triton, plus the package's refusal to run unregistered backends."""

from __future__ import annotations

import logging

import pytest
import torch

import omniwave_amd
from omniwave_amd.dispatch import select_backend


def test_auto_falls_back_on_cpu(caplog: pytest.LogCaptureFixture) -> None:
    with caplog.at_level(logging.INFO):
        backend, reason = select_backend(torch.randn(1), "auto", lambda _: (False, "CUDA is unavailable"))
    assert backend == "reference"
    assert reason == "CUDA is unavailable"
    assert "CUDA is unavailable" in caplog.text


def test_forced_hip_fails() -> None:
    with pytest.raises(RuntimeError, match="CUDA is unavailable"):
        select_backend(torch.randn(1), "hip", lambda _: (False, "CUDA is unavailable"))


def test_reference_passthrough() -> None:
    assert select_backend(torch.randn(1), "reference", lambda _: (True, None)) == ("reference", None)


def test_compile_passthrough() -> None:
    assert select_backend(torch.randn(1), "compile", lambda _: (True, None)) == ("compile", None)


def test_auto_selects_hip_when_supported() -> None:
    assert select_backend(torch.randn(1), "auto", lambda _: (True, None)) == ("hip", None)


def test_unknown_backend_rejected() -> None:
    with pytest.raises(ValueError, match="unknown backend"):
        select_backend(torch.randn(1), "cuda_graphs", lambda _: (True, None))


def _op_inputs(device="cpu"):
    plan = omniwave_amd.build_route_plan(8, 8, 128, 16, 64, "local")
    return dict(
        x=torch.randn(1, 8, 8, 128, device=device), plan=plan,
        a_u=torch.eye(16), a_v=torch.eye(16), a_o=torch.eye(16),
        b_u=torch.randn(2, 64, 128), b_v=torch.randn(2, 64, 128), b_o=torch.randn(2, 128, 64),
        gamma=torch.ones(128),
    )


def test_bigemm_unknown_backend() -> None:
    with pytest.raises(ValueError, match="unknown backend"):
        omniwave_amd.bigemm(backend="triton", **_op_inputs())


def test_bigemm_forced_hip_on_cpu_raises() -> None:
    with pytest.raises(RuntimeError, match="CUDA is unavailable"):
        omniwave_amd.bigemm(backend="hip", **_op_inputs())


def test_unregistered_reference_raises() -> None:
    """No silent CPU/eager path: without a registered reference backend, 'auto' on CPU fails."""
    with pytest.raises(RuntimeError, match="no reference backend is registered"):
        omniwave_amd.bigemm(backend="auto", **_op_inputs())
    with pytest.raises(RuntimeError, match="not registered"):
        omniwave_amd.bigemm(backend="reference", **_op_inputs())


def test_auto_uses_registered_reference_on_cpu(oracle_backend, caplog) -> None:
    kwargs = _op_inputs()
    with caplog.at_level(logging.INFO):
        out = omniwave_amd.bigemm(backend="auto", **kwargs)
    assert out.shape == kwargs["x"].shape
    assert "falling back to reference backend" in caplog.text


def test_register_backend_validates_name() -> None:
    with pytest.raises(ValueError):
        omniwave_amd.register_backend("hip", lambda **_: None)
