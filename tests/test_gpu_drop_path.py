"""Training-mode drop-path on the hip backend (``-m gpu``).

The reference (omniweave/models/block.py:99-107) draws a per-image keep mask
``torch.empty([B, 1, 1, 1], dtype=delta.dtype).bernoulli_(keep_probability)`` and returns
``x + delta * keep_mask / keep_probability``.  With the hip backend the block draws the same
mask from the same generator state and the fused kernel applies ``keep_mask / keep_probability``
to each image's rounded delta before the residual (``ow_bigemm_fwd_drop``); the backward scales
the delta branch's upstream gradient the same way (``ow_scale_samples``).

Checks, with a fixed seed:
* forward: bitwise equal to that composition evaluated with PyTorch ops on the GPU around the
  unfused hip delta (``residual=False``), and within the parity gate of the oracle (CPU, fp32)
  given the same mask;
* backward: every parameter gradient bitwise equal to autograd through the same composition,
  dx within rounding of it (the composition rounds dy + dx_delta once more), and every gradient
  within the gate of the oracle's fp32 autograd with the same mask.
"""

from __future__ import annotations

import sys

import pytest
import torch

import omniwave_amd
from omniwave_amd.block import OmniWeaveBlock
from omniwave_amd.hip import bigemm_block_hip, drop_path_scale
from oracle.bigemm import block_reference, rel_l2
from oracle.routing import build_route_plan as oracle_plan

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda", 0)
NAMES = ["a_u", "a_v", "a_o", "b_u", "b_v", "b_o", "gamma"]
TOL = {torch.bfloat16: 1e-2, torch.float16: 5e-3, torch.float32: 1e-4}
CASES = [  # (H, W, C, d, route, level, dtype): 16-token kernel (contiguous q_c = 4, interleaved
    # q_c = 2 and 4), resident kernel (q_c = 1), persistent / streamed kernels, fp32 kernel
    (28, 28, 256, 64, "shifted", 0, torch.bfloat16),
    (56, 56, 128, 64, "radix", 1, torch.bfloat16),
    (28, 28, 256, 64, "radix", 1, torch.bfloat16),
    (16, 16, 64, 64, "shifted", 0, torch.bfloat16),
    (14, 14, 512, 128, "radix", 1, torch.bfloat16),
    (7, 7, 1024, 128, "local", 0, torch.float16),
    (14, 14, 512, 128, "local", 0, torch.float32),
]
RATE = 0.4
SEED = 3


def announce(msg: str) -> None:
    print(f"\n[gpu-case] {msg}", file=sys.stderr, flush=True)


def make_block(h, w, c, d, route, level, dtype) -> OmniWeaveBlock:
    torch.manual_seed(0)
    blk = OmniWeaveBlock(h, w, c, d, route, level, backend="hip", drop_path_rate=RATE)
    with torch.no_grad():
        # LayerScale 1, a non-trivial RMSNorm weight and N(0, 1/fan_in) channel matrices (the
        # xavier init over [Q_c, d, rd] is ~10x smaller): delta, and the part of dx that goes
        # through the operator, are then comparable to x and dy, so comparing dx - dy is not
        # dominated by the bf16 rounding of dx.
        blk.gamma.fill_(1.0)
        blk.norm_weight.uniform_(0.5, 1.5)
        blk.b_u.normal_(0.0, d ** -0.5)
        blk.b_v.normal_(0.0, d ** -0.5)
        blk.b_o.normal_(0.0, (2 * d) ** -0.5)
    return blk.to(device=DEV, dtype=dtype).train()


def draw_mask(batch, dtype) -> torch.Tensor:
    """The reference's keep mask under the test's seed (block.py:100-106)."""
    torch.manual_seed(SEED)
    return torch.empty((batch, 1, 1, 1), dtype=dtype, device=DEV).bernoulli_(1.0 - RATE)


def composed(blk: OmniWeaveBlock, x: torch.Tensor, mask: torch.Tensor) -> torch.Tensor:
    """The reference's block tail as PyTorch GPU ops around the unfused hip delta."""
    params = [getattr(blk, k) for k in NAMES]
    delta = bigemm_block_hip(x, blk.norm_weight, blk.plan, *params, eps=1e-6, residual=False)
    return x + delta * mask / (1.0 - RATE)


@pytest.mark.parametrize("h,w,c,d,route,level,dtype", CASES,
                         ids=[f"{h}x{w}x{c}-{r}{l}-{str(t)[6:]}" for h, w, c, _, r, l, t in CASES])
def test_fused_drop_path_matches_reference_composition(h, w, c, d, route, level, dtype) -> None:
    announce(f"drop-path h={h} w={w} c={c} route={route}{level} dtype={dtype} B=8 rate={RATE}")
    blk = make_block(h, w, c, d, route, level, dtype)
    gen = torch.Generator().manual_seed(1)
    x = torch.randn(8, h, w, c, generator=gen).to(dtype).to(DEV)
    dy = torch.randn(8, h, w, c, generator=gen).to(dtype).to(DEV)
    mask = draw_mask(8, dtype)
    kept = int(mask.sum().item())
    assert 0 < kept < 8, "the seed must keep some images and drop others"

    # Forward: the block under the same seed draws the same mask.
    torch.manual_seed(SEED)
    xf = x.clone().requires_grad_(True)
    out = blk(xf)
    xc = x.clone().requires_grad_(True)
    ref = composed(blk, xc, mask)
    torch.cuda.synchronize()
    assert torch.equal(out, ref), f"fused drop-path differs from the composition in {(out != ref).sum().item()} elements"
    dropped = (mask.reshape(-1) == 0).nonzero().reshape(-1)
    assert torch.equal(out[dropped], x[dropped]), "dropped images must pass through unchanged"

    # Backward: parameter gradients bitwise, dx to the gate.
    out.backward(dy)
    g_fused = {k: getattr(blk, k).grad.clone() for k in NAMES + ["norm_weight"]}
    dx_fused = xf.grad.clone()
    blk.zero_grad(set_to_none=True)
    ref.backward(dy)
    for k in NAMES + ["norm_weight"]:
        assert torch.equal(g_fused[k], getattr(blk, k).grad), f"d{k} differs from the composition's"
    # The composition rounds dx_delta to the activation dtype before autograd adds dy; the fused
    # backward adds dy in fp32 and rounds once.  The two roundings of the composition and the one
    # of the fused sum bound the gap by eps (|dx| + |dy|).
    eps = torch.finfo(dtype).eps
    gap = (dx_fused.float() - xc.grad.float()).abs()
    bound = eps * (dx_fused.float().abs() + xc.grad.float().abs() + dy.float().abs())
    assert bool((gap <= bound).all()), f"dx differs from the composition beyond rounding: {gap.max().item():.3e}"
    err = rel_l2((dx_fused - dy).float().cpu(), (xc.grad - dy).float().cpu())
    assert err <= 1e-2, f"dx - dy rel-L2 {err:.3e} vs the composition"

    # The oracle (CPU, fp32) with the same mask and the kernel's rounded weights.
    oplan = oracle_plan(h, w, c, 16, d, route, level)
    ps = {k: getattr(blk, k).detach().float().cpu().clone().requires_grad_(True) for k in NAMES + ["norm_weight"]}
    xo = x.float().cpu().requires_grad_(True)
    s = drop_path_scale_cpu(mask)
    delta_o = block_reference(xo, oplan, ps, eps=1e-6, residual=False)
    out_o = xo + delta_o * s
    tol = TOL[dtype]
    err = rel_l2((out - x).float().cpu(), (out_o - xo).detach())
    print(f"forward (out - x) rel-L2 vs oracle {err:.3e}", file=sys.stderr)
    assert err <= tol
    out_o.backward(dy.float().cpu())
    for k in NAMES + ["norm_weight"]:
        e = rel_l2(g_fused[k].float().cpu(), ps[k].grad)
        print(f"d{k} rel-L2 vs oracle {e:.3e}", file=sys.stderr)
        assert e <= tol, f"d{k} rel-L2 {e:.3e} > {tol}"
    e = rel_l2((dx_fused - dy).float().cpu(), xo.grad - dy.float().cpu())
    assert e <= tol, f"dx - dy rel-L2 {e:.3e} > {tol}"


def drop_path_scale_cpu(mask: torch.Tensor) -> torch.Tensor:
    return mask.float().cpu() / (1.0 - RATE)


def test_drop_path_scale_draws_like_the_reference() -> None:
    announce("drop_path_scale random stream")
    for dtype in (torch.bfloat16, torch.float32):
        mask = draw_mask(64, dtype)
        torch.manual_seed(SEED)
        scale = drop_path_scale(64, RATE, dtype, DEV)
        inv = torch.tensor(1.0, dtype=torch.float32) / torch.tensor(1.0 - RATE, dtype=torch.float32)
        assert torch.equal(scale.cpu(), mask.reshape(64).float().cpu() * inv)


def test_eval_mode_ignores_drop_path() -> None:
    announce("drop-path block in eval mode")
    blk = make_block(14, 14, 512, 128, "shifted", 0, torch.bfloat16).eval()
    x = torch.randn(2, 14, 14, 512, device=DEV).to(torch.bfloat16)
    params = [getattr(blk, k) for k in NAMES]
    with torch.no_grad():
        out = blk(x)
        plain = bigemm_block_hip(x, blk.norm_weight, blk.plan, *params, eps=1e-6)
    torch.cuda.synchronize()
    assert torch.equal(out, plain)


def test_drop_scale_shape_is_checked() -> None:
    announce("drop_scale argument check")
    blk = make_block(14, 14, 512, 128, "shifted", 0, torch.bfloat16)
    x = torch.randn(2, 14, 14, 512, device=DEV).to(torch.bfloat16)
    params = [getattr(blk, k) for k in NAMES]
    with pytest.raises(ValueError, match="drop_scale"):
        bigemm_block_hip(x, blk.norm_weight, blk.plan, *params, drop_scale=torch.ones(3, device=DEV))
    _ = omniwave_amd  # the package import registers the custom ops
