"""Benchmark harness and gates (CPU): the reference's own harness tests
(tests/test_benchmark.py there) against omniwave_amd.harness, plus hip-row pairing and the
CLI."""

from __future__ import annotations

import json
import time

import pytest
import torch

from omniwave_amd import harness
from omniwave_amd.harness import BenchmarkResult, benchmark_fn, evaluate_operator_gates, pair_operator_rows


def test_percentile_ordering() -> None:
    result = benchmark_fn(lambda: time.sleep(0.0001), warmup=5, iterations=20, cuda_sync=False)
    assert result.p50_seconds <= result.p90_seconds <= result.p99_seconds


def test_mean_positive_and_fields() -> None:
    result = benchmark_fn(lambda: sum(range(100)), warmup=2, iterations=10, cuda_sync=False)
    assert isinstance(result, BenchmarkResult)
    assert result.mean_seconds > 0 and result.throughput_per_second > 0
    assert result.warmup == 2 and result.iterations == 10
    assert result.peak_allocated_bytes >= 0 and result.peak_reserved_bytes >= 0
    with pytest.raises(ValueError):
        benchmark_fn(lambda: None, warmup=-1)
    with pytest.raises(ValueError):
        benchmark_fn(lambda: None, iterations=0)


def _row(shape, **kw):
    row = {"shape": shape, "baseline_ms": 2.0, "triton_ms": 1.0, "baseline_memory": 100, "triton_memory": 90}
    row.update(kw)
    return row


def test_gate_rejects_missing_numerical_evidence() -> None:
    assert evaluate_operator_gates([_row(f"s{i}") for i in range(2)])["passed"] is False


def test_gate_requires_numerical_and_performance_pass() -> None:
    ok = dict(forward_max_abs_error=1e-3, backward_max_abs_error=2e-3, numerical_tolerance=5e-3)
    assert evaluate_operator_gates([_row(f"s{i}", **ok) for i in range(2)])["passed"] is True
    slow = [_row(f"s{i}", triton_ms=1.9, **ok) for i in range(2)]
    assert evaluate_operator_gates(slow)["passed"] is False
    fat = [_row(f"s{i}", triton_memory=101, **ok) for i in range(2)]
    assert evaluate_operator_gates(fat)["passed"] is False
    bad = [_row(f"s{i}", forward_max_abs_error=1.0, backward_max_abs_error=1.0) for i in range(2)]
    assert evaluate_operator_gates(bad)["passed"] is False


def test_gate_requires_distinct_passing_shapes() -> None:
    row = _row("56x56x128", forward_max_abs_error=1e-3, backward_max_abs_error=2e-3, numerical_tolerance=5e-3)
    result = evaluate_operator_gates([row, dict(row)])
    assert result["passed"] is False and result["passing_shapes"] == ["56x56x128"]


def _result(shape, backend, ms, mem, route="local", dtype="bfloat16", **kw):
    return {"shape": shape, "route": route, "batch_size": 8, "dtype": dtype, "backend": backend, "mean_ms": ms,
            "peak_allocated_mb": mem, **kw}


def test_hip_rows_pair_with_the_fastest_baseline_per_route() -> None:
    errs = dict(forward_max_abs_error=1e-4, backward_max_abs_error=1e-4, numerical_tolerance=5e-3)
    results = [
        _result("56x56x128", "reference", 3.0, 100), _result("56x56x128", "compile", 2.0, 120),
        _result("56x56x128", "hip", 0.5, 50, **errs),
        _result("56x56x128", "reference", 9.0, 100, route="shifted"),
        _result("56x56x128", "hip", 0.6, 50, route="shifted", **errs),
        _result("14x14x512", "reference", 1.0, 10), _result("14x14x512", "hip", 0.9, 5, **errs),
        _result("7x7x1024", "hip", 0.1, 5, **errs),             # no baseline: not paired
        {"shape": "28x28x256", "backend": "hip", "error": "boom"},  # error rows are skipped
    ]
    paired = pair_operator_rows(results, "hip")
    assert len(paired) == 3
    first = next(p for p in paired if p["shape"] == "56x56x128" and p["baseline_ms"] == 2.0)
    assert first["candidate_ms"] == 0.5 and first["baseline_memory"] == 120 and first["candidate_backend"] == "hip"
    gate = evaluate_operator_gates(paired)
    assert gate["passing_shapes"] == ["56x56x128"]  # 14x14x512 is only 1.11x faster
    assert gate["passed"] is False
    assert evaluate_operator_gates(paired, speedup_threshold=1.1)["passed"] is True


def test_check_gates_cli(tmp_path) -> None:
    errs = dict(forward_max_abs_error=1e-4, backward_max_abs_error=1e-4, numerical_tolerance=5e-3)
    results = [_result(s, "reference", 2.0, 10) for s in ("a", "b")] + \
              [_result(s, "hip", 1.0, 5, **errs) for s in ("a", "b")]
    src, out = tmp_path / "ops.json", tmp_path / "gates.json"
    src.write_text(json.dumps(results))
    assert harness.main(["check-gates", "--operator-results", str(src), "--output", str(out)]) == 0
    gate = json.loads(out.read_text())
    assert gate["passed"] and gate["passing_shapes"] == ["a", "b"]


def test_operator_tensors_follow_block_initialisation() -> None:
    t = harness.make_operator_tensors(batch_size=1, height=8, width=8, channels=16, spatial_tile=4, channel_tile=8,
                                      expansion=2, dtype=torch.float32, device=torch.device("cpu"))
    assert torch.equal(t["gamma"], torch.full((16,), 1e-5))
    assert torch.equal(t["a_o"], torch.eye(4))
    assert torch.allclose(t["a_u"] @ t["a_u"].T, torch.eye(4), atol=1e-5)
    assert t["b_u"].shape == (2, 8, 16) and t["b_o"].shape == (2, 16, 8)


def test_operator_benchmark_rows_on_cpu(oracle_backend) -> None:
    """Row schema of the operator section with the oracle as the reference backend, on the CPU,
    every route; the hip backend on the CPU reports its reason as an error row."""
    config = {"warmup": 1, "iterations": 2, "batch_sizes": [1], "dtypes": ["float32"],
              "shapes": [{"height": 8, "width": 8, "channels": 128, "channel_tile": 64}],
              "backends": ["reference", "hip"]}
    rows = harness.run_benchmark(config, torch.device("cpu"))
    assert {r["route"] for r in rows} == {"local", "shifted", "radix1"}
    ref = [r for r in rows if r["backend"] == "reference"]
    assert len(ref) == 3
    for r in ref:
        for key in ("shape", "batch_size", "dtype", "p50_ms", "p90_ms", "p99_ms", "mean_ms", "throughput",
                    "peak_allocated_mb", "peak_reserved_mb", "forward_max_abs_error", "backward_max_abs_error",
                    "numerical_tolerance"):
            assert key in r
        assert r["shape"] == "8x8x128" and r["numerical_tolerance"] == 1e-4
    hip = [r for r in rows if r["backend"] == "hip"]
    assert len(hip) == 3 and all("error" in r for r in hip)
