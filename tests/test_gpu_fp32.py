"""fp32 path on the GPU (``-m gpu``): rel-L2 <= 1e-4 against the fp32 oracle.

The fp32 kernel evaluates the operator in fp32 throughout, so it meets the reference's fp32
tolerance (rel-L2 1e-4 and the max-abs 1e-4 of its benchmark harness) on the same inputs.
"""

from __future__ import annotations

import sys

import pytest
import torch

import omniwave_amd
from omniwave_amd.hip import bigemm_block_hip, bigemm_delta_hip
from oracle.bigemm import bigemm_delta_reference, block_reference, rel_l2
from oracle.routing import build_route_plan as oracle_plan

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda", 0)
STAGES = {"s1": (56, 56, 128, 64), "s2": (28, 28, 256, 64), "s3": (14, 14, 512, 128), "s4": (7, 7, 1024, 128)}
ROUTES = [("local", 0), ("shifted", 0), ("radix", 1), ("radix", 2)]


def announce(msg: str) -> None:
    print(f"\n[gpu-case] {msg}", file=sys.stderr, flush=True)


def test_config1_fp32_matches_oracle() -> None:
    """x [8,14,14,512] ~ N(0,1), local route, d=128, A ~ N(0,1/16), B ~ N(0,1/fan_in), seed 0,
    LayerScale 1: rel-L2 <= 1e-4 and max-abs <= 1e-4 on delta."""
    announce("config1 x[8,14,14,512] local fp32 seed=0")
    torch.manual_seed(0)
    x = torch.randn(8, 14, 14, 512)
    a = [torch.randn(16, 16) / 4.0 for _ in range(3)]
    b_u, b_v = torch.randn(4, 128, 256) / 128 ** 0.5, torch.randn(4, 128, 256) / 128 ** 0.5
    b_o = torch.randn(4, 256, 128) / 256 ** 0.5
    params = dict(a_u=a[0], a_v=a[1], a_o=a[2], b_u=b_u, b_v=b_v, b_o=b_o, gamma=torch.ones(512))
    plan = omniwave_amd.build_route_plan(14, 14, 512, 16, 128, "local")
    got = bigemm_delta_hip(x=x.to(DEV), plan=plan, **{k: v.to(DEV) for k, v in params.items()}).cpu()
    ref = bigemm_delta_reference(x=x, plan=oracle_plan(14, 14, 512, 16, 128, "local"), **params)
    err, mx = rel_l2(got, ref), (got - ref).abs().max().item()
    print(f"config1 fp32 rel-L2 {err:.2e} max-abs {mx:.2e}", flush=True)
    assert err <= 1e-4 and mx <= 1e-4


@pytest.mark.parametrize("route,level", ROUTES, ids=[f"{r}{l}" for r, l in ROUTES])
@pytest.mark.parametrize("stage", list(STAGES))
def test_fp32_block_matches_oracle(stage, route, level) -> None:
    """Fused RMSNorm + BiGEMM + residual in fp32, random norm weight and LayerScale."""
    h, w, c, d = STAGES[stage]
    announce(f"fp32 block stage={stage} route={route}{level} B=2")
    gen = torch.Generator().manual_seed(3)
    plan = omniwave_amd.build_route_plan(h, w, c, 16, d, route, level)
    q_c, rd = plan.channel_indices.shape[0], 2 * d
    x = torch.randn(2, h, w, c, generator=gen)
    params = dict(
        a_u=torch.randn(16, 16, generator=gen) / 4, a_v=torch.randn(16, 16, generator=gen) / 4,
        a_o=torch.randn(16, 16, generator=gen) / 4,
        b_u=torch.randn(q_c, d, rd, generator=gen) / d ** 0.5, b_v=torch.randn(q_c, d, rd, generator=gen) / d ** 0.5,
        b_o=torch.randn(q_c, rd, d, generator=gen) / rd ** 0.5,
        gamma=torch.rand(c, generator=gen) + 0.5, norm_weight=torch.rand(c, generator=gen) + 0.5,
    )
    dp = {k: v.to(DEV) for k, v in params.items()}
    nw = dp.pop("norm_weight")
    delta = bigemm_block_hip(x.to(DEV), nw, plan, **dp, residual=False).cpu()
    out = bigemm_block_hip(x.to(DEV), nw, plan, **dp).cpu()
    oplan = oracle_plan(h, w, c, 16, d, route, level)
    ref = block_reference(x, oplan, params, residual=False)
    assert rel_l2(delta, ref) <= 1e-4
    assert rel_l2(out - x, ref) <= 1e-4


def test_fp32_ragged_and_rd_variants() -> None:
    """Pad tokens (7x9) and pad channels (C=96, d=64) with rd = d and rd = 4d."""
    for (h, w, c, d, rd, route, level) in [(7, 9, 96, 64, 256, "radix", 2), (8, 8, 256, 128, 128, "shifted", 0)]:
        announce(f"fp32 ragged {h}x{w}x{c} d={d} rd={rd} {route}{level}")
        gen = torch.Generator().manual_seed(4)
        plan = omniwave_amd.build_route_plan(h, w, c, 16, d, route, level)
        q_c = plan.channel_indices.shape[0]
        x = torch.randn(3, h, w, c, generator=gen)
        params = dict(
            a_u=torch.randn(16, 16, generator=gen) / 4, a_v=torch.randn(16, 16, generator=gen) / 4,
            a_o=torch.randn(16, 16, generator=gen) / 4,
            b_u=torch.randn(q_c, d, rd, generator=gen) / d ** 0.5,
            b_v=torch.randn(q_c, d, rd, generator=gen) / d ** 0.5,
            b_o=torch.randn(q_c, rd, d, generator=gen) / rd ** 0.5, gamma=torch.rand(c, generator=gen) + 0.5,
        )
        got = bigemm_delta_hip(x=x.to(DEV), plan=plan, **{k: v.to(DEV) for k, v in params.items()}).cpu()
        ref = bigemm_delta_reference(x=x, plan=oracle_plan(h, w, c, 16, d, route, level), **params)
        assert rel_l2(got, ref) <= 1e-4
