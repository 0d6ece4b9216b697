"""The benchmark harness on the GPU (``-m gpu``): hip rows beside the oracle's reference rows,
with the reference harness's numerical gate (forward and all-gradient max-abs errors within
5e-3 for 16-bit dtypes, 1e-4 for fp32) met on every route."""

from __future__ import annotations

import sys

import pytest
import torch

from omniwave_amd import harness
from omniwave_amd.bigemm import register_backend
from oracle.bigemm import bigemm_delta_reference

pytestmark = pytest.mark.gpu


def differentiable_oracle(*, x, plan, a_u, a_v, a_o, b_u, b_v, b_o, gamma):
    """The oracle as the reference backend, in x's dtype on the CPU, differentiable."""
    dt = x.dtype
    w = {k: v.cpu().to(dt) for k, v in dict(a_u=a_u, a_v=a_v, a_o=a_o, b_u=b_u, b_v=b_v, b_o=b_o, gamma=gamma).items()}
    return bigemm_delta_reference(x=x.cpu(), plan=plan, **w).to(x.device)


@pytest.fixture
def reference_backend():
    register_backend("reference", differentiable_oracle)
    yield
    register_backend("reference", None)


def test_operator_harness_hip_rows_meet_the_numerical_gate(reference_backend) -> None:
    print("\n[gpu-case] harness operator rows 56x56x128 / 14x14x512, bf16 + fp32", file=sys.stderr, flush=True)
    config = {"warmup": 2, "iterations": 5, "batch_sizes": [1], "dtypes": ["bfloat16", "float32"],
              "shapes": [{"height": 56, "width": 56, "channels": 128, "channel_tile": 64},
                         {"height": 14, "width": 14, "channels": 512, "channel_tile": 128}],
              "backends": ["reference", "hip"]}
    rows = harness.run_benchmark(config, torch.device("cuda", 0))
    hip = [r for r in rows if r["backend"] == "hip"]
    assert len(hip) == 2 * 3 * 2
    for r in hip:
        assert "error" not in r, r
        print(f"{r['shape']} {r['route']} {r['dtype']}: fwd {r['forward_max_abs_error']:.2e} "
              f"bwd {r['backward_max_abs_error']:.2e} mean {r['mean_ms']:.3f} ms", flush=True)
        assert r["forward_max_abs_error"] <= r["numerical_tolerance"]
        assert r["backward_max_abs_error"] <= r["numerical_tolerance"]
    paired = harness.pair_operator_rows(rows, "hip")
    assert len(paired) == len(hip)
    gate = harness.evaluate_operator_gates(paired)
    assert all(d["numerical_ok"] for d in gate["details"])
