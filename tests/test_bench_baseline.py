"""The PyTorch-eager baseline of bench.py computes the reference operator (CPU, fp32)."""

from __future__ import annotations

import pytest
import torch

import bench
import omniwave_amd
from oracle.bigemm import bigemm_delta_reference, rel_l2
from oracle.routing import build_route_plan as oracle_plan


@pytest.mark.parametrize("h,w,c,d,route,level", [
    (8, 8, 128, 64, "shifted", 0),
    (7, 9, 96, 64, "radix", 2),
    (8, 8, 256, 128, "local", 0),
])
def test_eager_baseline_matches_oracle(h, w, c, d, route, level) -> None:
    gen = torch.Generator().manual_seed(0)
    plan = omniwave_amd.build_route_plan(h, w, c, 16, d, route, level)
    q_c, rd = plan.channel_indices.shape[0], 2 * d
    x = torch.randn(2, h, w, c, generator=gen)
    p = dict(
        a_u=torch.randn(16, 16, generator=gen) / 4, a_v=torch.randn(16, 16, generator=gen) / 4,
        a_o=torch.randn(16, 16, generator=gen) / 4,
        b_u=torch.randn(q_c, d, rd, generator=gen) / d ** 0.5,
        b_v=torch.randn(q_c, d, rd, generator=gen) / d ** 0.5,
        b_o=torch.randn(q_c, rd, d, generator=gen) / rd ** 0.5,
        gamma=torch.rand(c, generator=gen) + 0.5,
    )
    got = bench.eager_reference_delta(x=x, plan=plan, **p)
    want = bigemm_delta_reference(x=x, plan=oracle_plan(h, w, c, 16, d, route, level), **p)
    assert rel_l2(got, want) < 1e-6
