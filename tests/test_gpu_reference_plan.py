"""The hip entry points with the reference's own plan type (``-m gpu``).

``oracle.routing.OracleRoutePlan`` has exactly the fields of the reference's frozen ``RoutePlan``
(omniweave/models/routing.py:17-33) and nothing else, so it stands in for a plan that the
reference's ``build_route_plan`` returned and its ``OmniWeaveBlock`` passes to ``bigemm``
(omniweave/ops/bigemm.py:50-68, omniweave/models/block.py:87-98).  Every entry point must run
with it and give the same bytes as with this package's plan: the drop-in delta, the fused
block, its backward, the space_to_depth output and the chained statistics.
"""

from __future__ import annotations

import sys

import pytest
import torch

import omniwave_amd
from omniwave_amd.hip import bigemm_block_chain_hip, bigemm_block_hip, bigemm_block_s2d_hip, bigemm_delta_hip
from oracle.routing import OracleRoutePlan, build_route_plan as oracle_plan

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda", 0)
NAMES = ["a_u", "a_v", "a_o", "b_u", "b_v", "b_o", "gamma"]
CASES = [(56, 56, 128, 64, "local", 0), (28, 28, 256, 64, "radix", 1), (14, 14, 512, 128, "shifted", 0),
         (7, 7, 1024, 128, "radix", 2)]


def announce(msg: str) -> None:
    print(f"\n[gpu-case] {msg}", file=sys.stderr, flush=True)


def inputs(h, w, c, d, seed=0):
    gen = torch.Generator().manual_seed(seed)
    q_c = c // d
    x = torch.randn(2, h, w, c, generator=gen).to(torch.bfloat16)
    p = {
        "a_u": torch.randn(16, 16, generator=gen) / 4, "a_v": torch.randn(16, 16, generator=gen) / 4,
        "a_o": torch.randn(16, 16, generator=gen) / 4,
        "b_u": torch.randn(q_c, d, 2 * d, generator=gen) / d ** 0.5,
        "b_v": torch.randn(q_c, d, 2 * d, generator=gen) / d ** 0.5,
        "b_o": torch.randn(q_c, 2 * d, d, generator=gen) / (2 * d) ** 0.5,
        "gamma": torch.rand(c, generator=gen) + 0.5, "norm_weight": torch.rand(c, generator=gen) + 0.5,
    }
    dy = torch.randn(2, h, w, c, generator=gen).to(torch.bfloat16)
    return x.to(DEV), {k: v.to(DEV) for k, v in p.items()}, dy.to(DEV)


@pytest.mark.parametrize("h,w,c,d,route,level", CASES, ids=[f"{h}x{w}x{c}-{r}{l}" for h, w, c, _, r, l in CASES])
def test_reference_plan_gives_the_same_bytes(h, w, c, d, route, level) -> None:
    announce(f"reference plan h={h} w={w} c={c} route={route}{level} B=2 bf16")
    ref_plan = oracle_plan(h, w, c, 16, d, route, level)
    own_plan = omniwave_amd.build_route_plan(h, w, c, 16, d, route, level)
    assert isinstance(ref_plan, OracleRoutePlan)
    x, p, dy = inputs(h, w, c, d)
    w_args = [p[k] for k in NAMES]

    # Drop-in delta (the INTEGRATION stub's bigemm(backend="hip") branch passes the plan through).
    a = bigemm_delta_hip(x=x, plan=ref_plan, **{k: p[k] for k in NAMES})
    b = bigemm_delta_hip(x=x, plan=own_plan, **{k: p[k] for k in NAMES})
    assert torch.equal(a, b)

    # Fused block and its backward (the stub's OmniWeaveBlock.forward branch).
    grads = []
    for plan in (ref_plan, own_plan):
        xs = x.clone().requires_grad_(True)
        ps = [t.clone().requires_grad_(True) for t in w_args]
        nw = p["norm_weight"].clone().requires_grad_(True)
        out = bigemm_block_hip(xs, nw, plan, *ps, eps=1e-6)
        out.backward(dy)
        grads.append([out.detach(), xs.grad, nw.grad] + [t.grad for t in ps])
    for ga, gb in zip(*grads):
        assert torch.equal(ga, gb)

    with torch.no_grad():
        if h % 2 == 0 and w % 2 == 0:
            a = bigemm_block_s2d_hip(x, p["norm_weight"], ref_plan, *w_args, factor=2)
            b = bigemm_block_s2d_hip(x, p["norm_weight"], own_plan, *w_args, factor=2)
            assert torch.equal(a, b)
        ya, sa = bigemm_block_chain_hip(x, None, p["norm_weight"], ref_plan, *w_args)
        yb, sb = bigemm_block_chain_hip(x, None, p["norm_weight"], own_plan, *w_args)
        assert torch.equal(ya, yb)
        assert (sa is None) == (sb is None)
        if sa is not None:
            assert torch.equal(sa, sb)
    torch.cuda.synchronize()


def test_reference_side_bigemm_stub_runs_verbatim(oracle_backend) -> None:
    """The `bigemm` branches a maintainer adds to the reference,
    run with a reference-typed plan: "hip" calls bigemm_delta_hip(**kwargs) unchanged, "auto"
    asks hip_is_supported with the same plan."""
    announce("reference-side bigemm stub")
    from omniwave_amd.dispatch import select_backend
    from omniwave_amd.hip import hip_is_supported

    def reference_bigemm(*, x, plan, a_u, a_v, a_o, b_u, b_v, b_o, gamma, backend="reference"):
        kwargs = dict(x=x, plan=plan, a_u=a_u, a_v=a_v, a_o=a_o, b_u=b_u, b_v=b_v, b_o=b_o, gamma=gamma)
        if backend == "hip":
            return bigemm_delta_hip(**kwargs)
        if backend == "reference":
            return oracle_backend(**kwargs)
        if backend == "auto":
            chosen, reason = select_backend(x, "auto", lambda t: hip_is_supported(t, plan, b_u))
            return reference_bigemm(backend=chosen, **kwargs)
        raise ValueError(backend)

    ref_plan = oracle_plan(14, 14, 512, 16, 128, "shifted", 0)
    x, p, _ = inputs(14, 14, 512, 128)
    got_hip = reference_bigemm(x=x, plan=ref_plan, **{k: p[k] for k in NAMES}, backend="hip")
    got_auto = reference_bigemm(x=x, plan=ref_plan, **{k: p[k] for k in NAMES}, backend="auto")
    torch.cuda.synchronize()
    assert torch.equal(got_hip, got_auto)
