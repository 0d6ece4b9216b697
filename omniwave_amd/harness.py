"""Operator / model benchmark harness and gate check with ``backend="hip"`` rows.

Mirrors the reference's harness so its result files and gates read the same:

* ``BenchmarkResult`` / ``benchmark_fn`` — omniweave/evaluation/benchmark.py:14-89 (per-call
  synchronised timing, p50/p90/p99/mean, peak memory);
* ``make_operator_tensors`` / ``run_bigemm`` / ``numerical_errors`` — scripts/benchmark.py:17-117
  (block-scale initialisation, gamma 1e-5; max-abs forward and all-gradient errors of
  ``output.float().sum()`` against the ``"reference"`` backend);
* ``run_benchmark`` — scripts/benchmark.py:120-320 with the same row schema
  (scripts/benchmark.py:194-217, 288-310), every route of the block schedule rather than only
  ``local``, plus ``"route"`` in each row;
* ``evaluate_operator_gates`` / ``pair_operator_rows`` — scripts/check_gates.py:12-132, with
  ``hip`` rows paired against the fastest ``reference`` / ``compile`` row of the same shape,
  batch, dtype and route (``triton`` rows pair as before).

``python -m omniwave_amd.harness benchmark --config C --output O`` and
``python -m omniwave_amd.harness check-gates --operator-results O --output G`` are the two
command lines.  The ``"reference"`` and ``"compile"`` backends are whatever the caller
registered with ``omniwave_amd.register_backend`` (this package ships only the HIP
implementation); rows of an unregistered backend carry the error, as the reference's do.
"""

from __future__ import annotations

import argparse
import json
import math
import sys
import time
from collections.abc import Callable
from dataclasses import dataclass
from functools import partial
from pathlib import Path
from typing import Any

import numpy as np
import torch
import torch.nn as nn
import yaml

ROUTES = (("local", 0), ("shifted", 0), ("radix", 1))
CANDIDATES = ("hip", "triton")
BASELINES = ("reference", "compile")


@dataclass(frozen=True)
class BenchmarkResult:
    """One timing measurement (omniweave/evaluation/benchmark.py:14-26)."""

    p50_seconds: float
    p90_seconds: float
    p99_seconds: float
    mean_seconds: float
    throughput_per_second: float
    peak_allocated_bytes: int
    peak_reserved_bytes: int
    warmup: int
    iterations: int


def benchmark_fn(fn: Callable[[], Any], warmup: int = 100, iterations: int = 1000,
                 cuda_sync: bool = True) -> BenchmarkResult:
    """Time ``fn`` per call with a device synchronisation around each call
    (omniweave/evaluation/benchmark.py:29-89)."""
    if warmup < 0:
        raise ValueError("warmup must be non-negative")
    if iterations < 1:
        raise ValueError("iterations must be at least 1")
    gpu = torch.cuda.is_available()
    for _ in range(warmup):
        fn()
    if gpu:
        torch.cuda.reset_peak_memory_stats()
        if cuda_sync:
            torch.cuda.synchronize()
    times = np.empty(iterations)
    for i in range(iterations):
        if cuda_sync and gpu:
            torch.cuda.synchronize()
        t0 = time.perf_counter()
        fn()
        if cuda_sync and gpu:
            torch.cuda.synchronize()
        times[i] = time.perf_counter() - t0
    mean = float(times.mean())
    return BenchmarkResult(
        p50_seconds=float(np.percentile(times, 50)),
        p90_seconds=float(np.percentile(times, 90)),
        p99_seconds=float(np.percentile(times, 99)),
        mean_seconds=mean,
        throughput_per_second=1.0 / max(mean, 1e-12),
        peak_allocated_bytes=int(torch.cuda.max_memory_allocated()) if gpu else 0,
        peak_reserved_bytes=int(torch.cuda.max_memory_reserved()) if gpu else 0,
        warmup=warmup,
        iterations=iterations,
    )


_NAMES = ("x", "a_u", "a_v", "a_o", "b_u", "b_v", "b_o", "gamma")


def make_operator_tensors(*, batch_size: int, height: int, width: int, channels: int, spatial_tile: int,
                          channel_tile: int, expansion: int, dtype: torch.dtype,
                          device: torch.device) -> dict[str, torch.Tensor]:
    """Operator inputs at the block's initialisation scales (scripts/benchmark.py:56-110):
    x ~ N(0, 1); A_u, A_v orthogonal, A_o identity, B xavier-uniform (drawn in fp32, then cast);
    gamma = 1e-5."""
    rd = channel_tile * expansion
    q_c = math.ceil(channels / channel_tile)

    def init(shape, initializer):
        t = torch.empty(shape, dtype=torch.float32, device=device)
        initializer(t)
        return t.to(dtype)

    return {
        "x": torch.randn(batch_size, height, width, channels, dtype=dtype, device=device),
        "a_u": init((spatial_tile, spatial_tile), nn.init.orthogonal_),
        "a_v": init((spatial_tile, spatial_tile), nn.init.orthogonal_),
        "a_o": init((spatial_tile, spatial_tile), nn.init.eye_),
        "b_u": init((q_c, channel_tile, rd), nn.init.xavier_uniform_),
        "b_v": init((q_c, channel_tile, rd), nn.init.xavier_uniform_),
        "b_o": init((q_c, rd, channel_tile), nn.init.xavier_uniform_),
        "gamma": torch.full((channels,), 1e-5, dtype=dtype, device=device),
    }


@torch.inference_mode()
def run_bigemm(plan, backend: str, tensors: dict[str, torch.Tensor]) -> torch.Tensor:
    """scripts/benchmark.py:113-117."""
    from omniwave_amd.bigemm import bigemm

    return bigemm(plan=plan, backend=backend, **tensors)


def bigemm_with_gradients(backend: str, plan, tensors: dict[str, torch.Tensor]):
    """Output and the gradients of ``output.float().sum()`` w.r.t. all eight inputs
    (scripts/benchmark.py:17-33)."""
    from omniwave_amd.bigemm import bigemm

    values = [tensors[n].detach().clone().requires_grad_(True) for n in _NAMES]
    out = bigemm(plan=plan, backend=backend, **dict(zip(_NAMES, values)))
    grads = torch.autograd.grad(out.float().sum(), values)
    return out.detach(), [g.detach() for g in grads]


def numerical_errors(backend: str, plan, tensors: dict[str, torch.Tensor]) -> tuple[float, float]:
    """(forward, backward) max-abs errors against ``"reference"`` (scripts/benchmark.py:36-53)."""
    if backend == "reference":
        return 0.0, 0.0
    ref_out, ref_grads = bigemm_with_gradients("reference", plan, tensors)
    out, grads = bigemm_with_gradients(backend, plan, tensors)
    forward = (out.float() - ref_out.float()).abs().max().item()
    backward = max((g.float() - r.float()).abs().max().item() for g, r in zip(grads, ref_grads))
    return forward, backward


def _routes(config: dict[str, Any]) -> list[tuple[str, int]]:
    out = []
    for entry in config.get("routes", [f"{r}{lv}" if r == "radix" else r for r, lv in ROUTES]):
        name = str(entry)
        if name.startswith("radix"):
            out.append(("radix", int(name[5:] or 0)))
        else:
            out.append((name, 0))
    return out


def run_operator_benchmark(config: dict[str, Any], device: torch.device) -> list[dict[str, Any]]:
    """The ``shapes`` section of scripts/benchmark.py:150-228, over every configured route."""
    from omniwave_amd.routing import build_route_plan

    rows: list[dict[str, Any]] = []
    for shape in config.get("shapes", []):
        h, w, c, d = shape["height"], shape["width"], shape["channels"], shape["channel_tile"]
        g = int(shape.get("spatial_tile", 16))
        for route, level in _routes(config):
            for batch in config.get("batch_sizes", [1]):
                for dtype_name in config.get("dtypes", ["float32"]):
                    dtype = getattr(torch, dtype_name)
                    for backend in config.get("backends", ["reference"]):
                        base = {"shape": f"{h}x{w}x{c}", "route": f"{route}{level}" if route == "radix" else route,
                                "batch_size": batch, "dtype": dtype_name, "backend": backend}
                        try:
                            plan = build_route_plan(h, w, c, g, d, route, level)
                            tensors = make_operator_tensors(
                                batch_size=batch, height=h, width=w, channels=c, spatial_tile=g, channel_tile=d,
                                expansion=int(shape.get("expansion", 2)), dtype=dtype, device=device)
                            probe = run_bigemm(plan, backend, tensors)
                            if not torch.isfinite(probe).all():
                                raise RuntimeError("operator produced non-finite output")
                            fwd_err, bwd_err = numerical_errors(backend, plan, tensors)
                            res = benchmark_fn(partial(run_bigemm, plan, backend, tensors),
                                               warmup=config.get("warmup", 100),
                                               iterations=config.get("iterations", 1000))
                            rows.append({
                                **base,
                                "p50_ms": res.p50_seconds * 1000, "p90_ms": res.p90_seconds * 1000,
                                "p99_ms": res.p99_seconds * 1000, "mean_ms": res.mean_seconds * 1000,
                                "throughput": batch * res.throughput_per_second,
                                "peak_allocated_mb": res.peak_allocated_bytes / 2 ** 20,
                                "peak_reserved_mb": res.peak_reserved_bytes / 2 ** 20,
                                "forward_max_abs_error": fwd_err, "backward_max_abs_error": bwd_err,
                                "numerical_tolerance": 1e-4 if dtype == torch.float32 else 5e-3,
                            })
                        except (ValueError, RuntimeError) as exc:
                            rows.append({**base, "error": str(exc)})
    return rows


def run_model_benchmark(config: dict[str, Any], device: torch.device) -> list[dict[str, Any]]:
    """The ``resolutions`` section of scripts/benchmark.py:230-312."""
    from omniwave_amd.registry import create_model

    rows: list[dict[str, Any]] = []
    batches = [("latency", b) for b in config.get("latency_batch_sizes", [1, 8])] + \
              [("throughput", b) for b in config.get("throughput_batch_sizes", [32, 64])]
    for model_name in config.get("models", ["omniweave_t"]):
        for resolution in config["resolutions"]:
            for backend in config.get("backends", ["reference"]):
                for mode, batch in batches:
                    base = {"kind": "model", "model": model_name, "resolution": resolution, "mode": mode,
                            "batch_size": batch, "backend": backend}
                    try:
                        model = create_model(model_name, backend=backend, input_size=resolution).to(device).eval()
                        inputs = torch.randn(batch, 3, resolution, resolution, device=device)

                        def run(model=model, inputs=inputs):
                            with torch.inference_mode():
                                return model(inputs)

                        res = benchmark_fn(run, warmup=config.get("warmup", 100),
                                           iterations=config.get("iterations", 1000))
                        rows.append({
                            **base, "performance_only": resolution != 224,
                            "p50_ms": res.p50_seconds * 1000, "p90_ms": res.p90_seconds * 1000,
                            "p99_ms": res.p99_seconds * 1000, "mean_ms": res.mean_seconds * 1000,
                            "images_per_second": batch * res.throughput_per_second,
                            "peak_allocated_mb": res.peak_allocated_bytes / 2 ** 20,
                            "peak_reserved_mb": res.peak_reserved_bytes / 2 ** 20,
                        })
                    except (ValueError, RuntimeError) as exc:
                        rows.append({**base, "error": str(exc)})
    return rows


def run_benchmark(config: dict[str, Any], device: torch.device) -> list[dict[str, Any]]:
    rows = run_operator_benchmark(config, device) if "shapes" in config else []
    if "resolutions" in config:
        rows += run_model_benchmark(config, device)
    return rows


def evaluate_operator_gates(rows: list[dict[str, Any]], speedup_threshold: float = 1.3,
                            min_passing_shapes: int = 2) -> dict[str, Any]:
    """Gate A (forward and backward max-abs errors within tolerance) and gate B (speedup and no
    peak-memory regression on >= ``min_passing_shapes`` distinct shapes), scripts/check_gates.py:12-83.
    A row's candidate time / memory is ``candidate_ms`` / ``candidate_memory`` (hip) or
    ``triton_ms`` / ``triton_memory``."""
    passing: set[str] = set()
    details = []
    for row in rows:
        cand_ms = row.get("candidate_ms", row.get("triton_ms"))
        cand_mem = row.get("candidate_memory", row.get("triton_memory"))
        speedup = row["baseline_ms"] / max(cand_ms, 1e-12)
        memory_ok = cand_mem <= row["baseline_memory"]
        tol = float(row.get("numerical_tolerance", 5e-3))
        fe, be = row.get("forward_max_abs_error"), row.get("backward_max_abs_error")
        numerical_ok = fe is not None and be is not None and float(fe) <= tol and float(be) <= tol
        ok = numerical_ok and speedup >= speedup_threshold and memory_ok
        details.append({"shape": row["shape"], "speedup": round(speedup, 3), "memory_ok": memory_ok,
                        "numerical_ok": numerical_ok, "forward_max_abs_error": fe, "backward_max_abs_error": be,
                        "numerical_tolerance": tol, "passed": ok})
        if ok:
            passing.add(row["shape"])
    return {"passed": len(passing) >= min_passing_shapes, "passing_shapes": sorted(passing),
            "total_shapes": len({r["shape"] for r in rows}), "speedup_threshold": speedup_threshold,
            "min_passing_shapes": min_passing_shapes, "details": details}


def pair_operator_rows(results: list[dict[str, Any]], candidate: str = "hip") -> list[dict[str, Any]]:
    """Pairs each ``candidate`` row with the fastest baseline (``reference`` / ``compile``) row of
    the same shape, batch, dtype and route (scripts/check_gates.py:97-132)."""
    by_key: dict[str, dict[str, Any]] = {}
    for row in results:
        if "error" in row or "shape" not in row:
            continue
        key = f"{row['shape']}_{row.get('batch_size')}_{row.get('dtype')}_{row.get('route', 'local')}"
        slot = by_key.setdefault(key, {"shape": row["shape"]})
        ms = row.get("mean_ms", row.get("p50_ms", 0))
        if row.get("backend") in BASELINES:
            if "baseline_ms" not in slot or ms < slot["baseline_ms"]:
                slot["baseline_ms"] = ms
                slot["baseline_memory"] = row.get("peak_allocated_mb", float("inf"))
        elif row.get("backend") == candidate:
            slot["candidate_ms"] = ms
            slot["candidate_memory"] = row.get("peak_allocated_mb", float("inf"))
            slot["candidate_backend"] = candidate
            for k in ("forward_max_abs_error", "backward_max_abs_error"):
                slot[k] = row.get(k)
            slot["numerical_tolerance"] = row.get("numerical_tolerance", 5e-3)
    return [v for v in by_key.values() if "baseline_ms" in v and "candidate_ms" in v]


def main(argv: list[str] | None = None) -> int:
    ap = argparse.ArgumentParser(description="OmniWeave benchmark harness and gates (hip backend)")
    sub = ap.add_subparsers(dest="cmd", required=True)
    b = sub.add_parser("benchmark", help="run a benchmark config (scripts/benchmark.py)")
    b.add_argument("--config", required=True)
    b.add_argument("--output", required=True)
    b.add_argument("--device", default="cuda")
    g = sub.add_parser("check-gates", help="operator gates A/B (scripts/check_gates.py)")
    g.add_argument("--operator-results", required=True)
    g.add_argument("--output", required=True)
    g.add_argument("--candidate", default="hip", choices=CANDIDATES)
    g.add_argument("--speedup-threshold", type=float, default=1.3)
    g.add_argument("--min-passing-shapes", type=int, default=2)
    args = ap.parse_args(argv)

    if args.cmd == "benchmark":
        with open(args.config, encoding="utf-8") as fh:
            config = yaml.safe_load(fh)
        device = torch.device(args.device)
        if device.type == "cuda" and not torch.cuda.is_available():
            raise RuntimeError("CUDA benchmark requested but CUDA is unavailable")
        rows = run_benchmark(config, device)
        out = Path(args.output)
        out.parent.mkdir(parents=True, exist_ok=True)
        out.write_text(json.dumps(rows, indent=2), encoding="utf-8")
        print(f"Results written to {out}")
        return 0

    results = json.loads(Path(args.operator_results).read_text(encoding="utf-8"))
    gate = evaluate_operator_gates(pair_operator_rows(results, args.candidate), args.speedup_threshold,
                                   args.min_passing_shapes)
    out = Path(args.output)
    out.parent.mkdir(parents=True, exist_ok=True)
    out.write_text(json.dumps(gate, indent=2), encoding="utf-8")
    n = len(gate["passing_shapes"])
    print(f"Gate B {'PASSED' if gate['passed'] else 'FAILED'}: {n} shapes meet threshold")
    return 0 if gate["passed"] else 2


if __name__ == "__main__":
    sys.exit(main())
