"""GPU parity of the HIP backward against the oracle's fp32 autograd (``-m gpu``).

The oracle (CPU, fp32) is differentiated by torch.autograd on the same inputs, with the
weights rounded to the compute dtype as the kernels see them.  Every gradient of the block —
dx, d norm_weight, d gamma, dA_u/v/o, dB_u/v/o — must be within rel-L2 1e-2 (bf16) or 5e-3
(fp16) or 1e-4 (fp32) of it.  With the residual fused, dx - dy (the part that goes through the operator) is
compared, so the identity path cannot hide an error.
"""

from __future__ import annotations

import sys

import pytest
import torch

from oracle.bigemm import bigemm_delta_reference, block_reference, rel_l2
from oracle.routing import build_route_plan as oracle_plan
import omniwave_amd
from omniwave_amd.hip import bigemm_block_hip, bigemm_delta_hip

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda", 0)
TOL = {torch.bfloat16: 1e-2, torch.float16: 5e-3, torch.float32: 1e-4}
NAMES = ["a_u", "a_v", "a_o", "b_u", "b_v", "b_o", "gamma"]


def announce(msg: str) -> None:
    print(f"\n[gpu-case] {msg}", file=sys.stderr, flush=True)


def make_case(b, h, w, c, d, route, level, dtype, seed=0, rd=None):
    """Seeded inputs (x, A ~ N(0, 1/16), B ~ N(0, 1/fan_in), norm_w, gamma in [0.5, 1.5), dy)."""
    rd = rd or 2 * d
    gen = torch.Generator().manual_seed(seed)
    plan = omniwave_amd.build_route_plan(h, w, c, 16, d, route, level)
    q_c = plan.channel_indices.shape[0]
    x = torch.randn(b, h, w, c, generator=gen).to(dtype)
    params = {
        "a_u": torch.randn(16, 16, generator=gen) / 4.0,
        "a_v": torch.randn(16, 16, generator=gen) / 4.0,
        "a_o": torch.randn(16, 16, generator=gen) / 4.0,
        "b_u": (torch.randn(q_c, d, rd, generator=gen) / d ** 0.5).to(dtype).float(),
        "b_v": (torch.randn(q_c, d, rd, generator=gen) / d ** 0.5).to(dtype).float(),
        "b_o": (torch.randn(q_c, rd, d, generator=gen) / rd ** 0.5).to(dtype).float(),
        "gamma": torch.rand(c, generator=gen) + 0.5,
        "norm_weight": torch.rand(c, generator=gen) + 0.5,
    }
    for k in ("a_u", "a_v", "a_o"):
        params[k] = params[k].to(dtype).float()
    dy = torch.randn(b, h, w, c, generator=gen).to(dtype)
    return plan, x, params, dy


def oracle_grads(x, plan, params, dy, fused: bool, residual: bool):
    """fp32 CPU autograd of the oracle block (fused) or delta (not fused)."""
    oplan = oracle_plan(plan.height, plan.width, plan.channels, 16, int(plan.channel_indices.shape[1]),
                        plan.route, plan.radix_level)
    xs = x.float().clone().requires_grad_(True)
    ps = {k: v.clone().requires_grad_(True) for k, v in params.items()}
    if fused:
        out = block_reference(xs, oplan, ps, eps=1e-6, residual=residual)
    else:
        out = bigemm_delta_reference(x=xs, plan=oplan, **{k: ps[k] for k in NAMES})
    out.backward(dy.float())
    grads = {k: ps[k].grad for k in NAMES}
    if fused:
        grads["norm_weight"] = ps["norm_weight"].grad
    grads["x"] = xs.grad
    return grads


def hip_grads(x, plan, params, dy, fused: bool, residual: bool):
    xs = x.to(DEV).requires_grad_(True)
    ps = {k: v.to(DEV).requires_grad_(True) for k, v in params.items()}
    if fused:
        out = bigemm_block_hip(xs, ps["norm_weight"], plan, *[ps[k] for k in NAMES], eps=1e-6, residual=residual)
    else:
        out = bigemm_delta_hip(x=xs, plan=plan, **{k: ps[k] for k in NAMES})
    out.backward(dy.to(DEV))
    torch.cuda.synchronize()
    grads = {k: ps[k].grad.cpu() for k in NAMES}
    if fused:
        grads["norm_weight"] = ps["norm_weight"].grad.cpu()
    grads["x"] = xs.grad.cpu()
    return grads


def check(got, want, dy, residual: bool, dtype, label: str) -> None:
    tol = TOL[dtype]
    errs = {}
    for k in want:
        g, w = got[k].float(), want[k]
        if k == "x" and residual:
            g, w = g - dy.float(), w - dy.float()
        errs[k] = rel_l2(g, w)
    print(f"[{label}] rel-L2 " + " ".join(f"{k}={v:.2e}" for k, v in errs.items()), flush=True)
    bad = {k: v for k, v in errs.items() if not v <= tol}
    assert not bad, f"{label}: gradients beyond rel-L2 {tol}: {bad}"


CASES = [  # (B, H, W, C, d, route, level)
    ("s1-shifted", (2, 56, 56, 128, 64, "shifted", 0)),
    ("s3-shifted", (2, 14, 14, 512, 128, "shifted", 0)),
    ("s2-local", (2, 28, 28, 256, 64, "local", 0)),
    ("s4-radix1", (2, 7, 7, 1024, 128, "radix", 1)),
    ("ragged-radix2", (3, 7, 9, 96, 64, "radix", 2)),
    ("s2-radix1", (2, 28, 28, 256, 64, "radix", 1)),  # d = 64, strided channel groups
]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32], ids=["bf16", "f16", "f32"])
@pytest.mark.parametrize("name,case", CASES, ids=[n for n, _ in CASES])
def test_block_backward_matches_oracle(name, case, dtype) -> None:
    b, h, w, c, d, route, level = case
    announce(f"block backward {name} dtype={dtype} B={b}")
    plan, x, params, dy = make_case(b, h, w, c, d, route, level, dtype)
    want = oracle_grads(x, plan, params, dy, fused=True, residual=True)
    got = hip_grads(x, plan, params, dy, fused=True, residual=True)
    check(got, want, dy, True, dtype, f"block {name} {dtype}")


@pytest.mark.parametrize("name,case", CASES[:3], ids=[n for n, _ in CASES[:3]])
def test_delta_backward_matches_oracle(name, case) -> None:
    b, h, w, c, d, route, level = case
    announce(f"delta backward {name} bf16 B={b}")
    plan, x, params, dy = make_case(b, h, w, c, d, route, level, torch.bfloat16, seed=1)
    want = oracle_grads(x, plan, params, dy, fused=False, residual=False)
    got = hip_grads(x, plan, params, dy, fused=False, residual=False)
    check(got, want, dy, False, torch.bfloat16, f"delta {name}")


@pytest.mark.parametrize("b,h,w,c,d,rd", [(2, 8, 8, 128, 64, 256), (1, 14, 14, 128, 64, 128),
                                          (2, 8, 8, 256, 128, 128)], ids=["d64-rd256", "odd-pairs", "d128-rd128"])
def test_backward_rd_variants_and_odd_pair_counts(b, h, w, c, d, rd) -> None:
    """rd = 4d and rd = d, and a slot count that is not a multiple of 32 (B * Q_s odd: the
    batched-GEMM channel side instead of the fused d = 64 kernel)."""
    announce(f"block backward variant B={b} {h}x{w}x{c} d={d} rd={rd}")
    plan, x, params, dy = make_case(b, h, w, c, d, "shifted", 0, torch.bfloat16, seed=4, rd=rd)
    want = oracle_grads(x, plan, params, dy, fused=True, residual=True)
    got = hip_grads(x, plan, params, dy, fused=True, residual=True)
    check(got, want, dy, True, torch.bfloat16, f"variant d={d} rd={rd}")


def test_block_backward_without_residual() -> None:
    announce("block backward without residual s2-local bf16 B=2")
    plan, x, params, dy = make_case(2, 28, 28, 256, 64, "local", 0, torch.bfloat16, seed=2)
    want = oracle_grads(x, plan, params, dy, fused=True, residual=False)
    got = hip_grads(x, plan, params, dy, fused=True, residual=False)
    check(got, want, dy, False, torch.bfloat16, "block no-residual")


@pytest.mark.parametrize("stage", ["s1", "s3"])
def test_full_batch_backward_is_per_sample(stage) -> None:
    """At the full B=128 shape: dx of a sample depends on that sample only, and the parameter
    gradients are the sum over samples — checked on three samples against the oracle and on
    the batch sum against the sum of per-chunk HIP gradients."""
    h, w, c, d = {"s1": (56, 56, 128, 64), "s3": (14, 14, 512, 128)}[stage]
    announce(f"full-batch backward {stage} shifted bf16 B=128")
    plan, x, params, dy = make_case(128, h, w, c, d, "shifted", 0, torch.bfloat16, seed=3)
    full = hip_grads(x, plan, params, dy, fused=True, residual=True)
    for i in (0, 77, 127):
        want = oracle_grads(x[i:i + 1], plan, params, dy[i:i + 1], fused=True, residual=True)
        got = {"x": full["x"][i:i + 1]}
        check(got, {"x": want["x"]}, dy[i:i + 1], True, torch.bfloat16, f"{stage} sample {i}")
    halves = [hip_grads(x[s], plan, params, dy[s], fused=True, residual=True)
              for s in (slice(0, 64), slice(64, 128))]
    for k in NAMES + ["norm_weight"]:
        err = rel_l2(full[k], halves[0][k] + halves[1][k])
        assert err <= 5e-3, f"{stage} {k}: batch gradient != sum of halves (rel-L2 {err:.2e})"


def test_backward_beyond_the_addressing_limit_runs_in_chunks() -> None:
    """S1 at B = 1400: one pass's intermediates would reach 2 GiB (32-bit buffer offsets), so the
    backward runs as two chunks of 700 images.  Three sampled images' dx (one on each side of the
    chunk boundary) match the oracle, and the parameter gradients equal the sum of two separate
    700-image backward passes."""
    from omniwave_amd.backward import batch_chunks, native_batch_limit

    h, w, c, d = 56, 56, 128, 64
    announce("backward past the 2 GiB addressing limit s1 shifted bf16 B=1400")
    plan, x, params, dy = make_case(1400, h, w, c, d, "shifted", 0, torch.bfloat16, seed=6)
    assert batch_chunks(1400, native_batch_limit(torch.bfloat16, plan, 2, d, 2 * d), 196) == [(0, 700), (700, 1400)]
    full = hip_grads(x, plan, params, dy, fused=True, residual=True)
    for i in (0, 700, 1399):
        want = oracle_grads(x[i:i + 1], plan, params, dy[i:i + 1], fused=True, residual=True)
        check({"x": full["x"][i:i + 1]}, {"x": want["x"]}, dy[i:i + 1], True, torch.bfloat16, f"B=1400 sample {i}")
    halves = [hip_grads(x[s], plan, params, dy[s], fused=True, residual=True)
              for s in (slice(0, 700), slice(700, 1400))]
    assert torch.equal(full["x"], torch.cat([halves[0]["x"], halves[1]["x"]]))
    for k in NAMES + ["norm_weight"]:
        err = rel_l2(full[k], halves[0][k] + halves[1][k])
        assert err <= 1e-6, f"{k}: chunked gradient != sum of the chunks (rel-L2 {err:.2e})"


SCALE_CASES = [  # (B, H, W, C, d, route, level): the 16-token kernel, the statistics pass, neither
    ("wave16", (2, 56, 56, 128, 64, "shifted", 0)),
    ("wave16-q4-interleaved", (2, 28, 28, 256, 64, "radix", 1)),
    ("statistics-pass", (2, 14, 14, 512, 128, "shifted", 0)),
    ("resident-fallback", (2, 16, 16, 64, 64, "shifted", 0)),
]


@pytest.mark.parametrize("name,case", SCALE_CASES, ids=[n for n, _ in SCALE_CASES])
def test_forward_hands_its_row_scales_to_the_backward(name, case) -> None:
    """bigemm_fwd with want_scales returns every row's RMSNorm scale (the forward's own values,
    or ow_rms_scale's where the kernel does not form them in one place), equal to a separate
    ow_rms_scale pass to within the fp32 summation order, and the same output bits as without."""
    import ctypes
    from omniwave_amd import _native
    from omniwave_amd.hip import _plan_desc

    b, h, w, c, d, route, level = case
    announce(f"forward row scales {name} B={b} {h}x{w}x{c}")
    plan, x, params, _ = make_case(b, h, w, c, d, route, level, torch.bfloat16, seed=6)
    xs = x.to(DEV)
    ps = {k: v.to(DEV) for k, v in params.items()}
    args = (xs, ps["norm_weight"], ps["gamma"], ps["a_u"], ps["a_v"], ps["a_o"], ps["b_u"], ps["b_v"], ps["b_o"],
            _plan_desc(plan), _native.OW_FUSE_NORM | _native.OW_FUSE_RESIDUAL, 1e-6, None)
    with torch.no_grad():
        out_s, scales = torch.ops.omniwave_amd.bigemm_fwd(*args, True)
        out, none = torch.ops.omniwave_amd.bigemm_fwd(*args, False)
    rows = b * h * w
    want = torch.empty(rows, dtype=torch.float32, device=DEV)
    lib = _native.lib()
    _native.check(lib.ow_rms_scale(xs.data_ptr(), want.data_ptr(), rows, c, ctypes.c_float(1e-6), _native.OW_DTYPE_BF16,
                                   torch.cuda.current_stream(DEV).cuda_stream), "ow_rms_scale")
    torch.cuda.synchronize()
    assert none.numel() == 0 and scales.shape == (rows,)
    err = float(((scales - want).abs() / want.abs()).max())
    assert err <= 2e-6, f"{name}: row scales differ from the statistics pass by {err:.2e} (relative)"
    assert torch.equal(out_s, out), f"{name}: output changed when the scales were requested"
