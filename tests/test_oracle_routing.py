"""Route plans: the oracle and the native route builder against the golden vectors, plus the
reference's own routing tests (tests/test_routing.py of the reference) run on both."""

from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest
import torch

import omniwave_amd.routing as prod
import oracle.routing as orc

GOLDEN = np.load(Path(__file__).parent / "golden" / "routes.npz")
CASES = sorted({k.rsplit("/", 1)[0] for k in GOLDEN.files if not k.startswith("schedule/")})
ROUTE_NAMES = ("local", "shifted", "radix")


def _case(key: str):
    h, w, c, g, d, level, q_s, q_c = (int(v) for v in GOLDEN[key + "/meta"])
    route = next(r for r in ROUTE_NAMES if key.split("_")[-1].startswith(r))
    return (h, w, c, g, d, route, level), q_s, q_c


@pytest.mark.parametrize("key", CASES)
def test_oracle_matches_golden(key: str) -> None:
    args, q_s, q_c = _case(key)
    plan = orc.build_route_plan(*args)
    assert plan.token_indices.shape == (q_s, args[3])
    assert plan.channel_indices.shape == (q_c, args[4])
    np.testing.assert_array_equal(plan.token_indices.reshape(-1).numpy(), GOLDEN[key + "/tok"])
    np.testing.assert_array_equal(plan.channel_indices.reshape(-1).numpy(), GOLDEN[key + "/ch"])


@pytest.mark.parametrize("key", CASES)
def test_native_builder_matches_golden(key: str) -> None:
    args, q_s, q_c = _case(key)
    plan = prod.build_route_plan(*args)
    np.testing.assert_array_equal(plan.token_indices.reshape(-1).numpy(), GOLDEN[key + "/tok"])
    np.testing.assert_array_equal(plan.channel_indices.reshape(-1).numpy(), GOLDEN[key + "/ch"])
    assert plan.token_indices.dtype == torch.int64 and plan.channel_indices.dtype == torch.int64
    n, c = args[0] * args[1], args[2]
    assert torch.equal(plan.token_mask, plan.token_indices < n)
    assert torch.equal(plan.channel_mask, plan.channel_indices < c)


@pytest.mark.parametrize("depth", range(1, 12))
def test_stage_schedule_matches_golden(depth: int) -> None:
    names = {0: "local", 1: "shifted", 2: "radix"}
    expected = [(names[int(r)], int(lvl)) for r, lvl in GOLDEN[f"schedule/{depth}"]]
    assert orc.build_stage_schedule(depth) == expected
    assert prod.build_stage_schedule(depth) == expected


def test_shifted_row_sets_at_14() -> None:
    """Closed form of the shifted route at 14x14: row windows {12,13,0,1},{2..5},{6..9},{10,11}."""
    plan = prod.build_route_plan(14, 14, 512, 16, 128, "shifted")
    order = plan.token_indices[plan.token_mask].tolist()
    rows = [t // 14 for t in order]
    firsts = [rows[0]]
    for r in rows[1:]:
        if r not in firsts:
            firsts.append(r)
    assert firsts == [12, 13, 0, 1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11]
    # First window: rows {12,13,0,1} x cols {12,13,0,1} in raster order.
    assert order[:16] == [r * 14 + c for r in (12, 13, 0, 1) for c in (12, 13, 0, 1)]


def test_radix_identity_cases() -> None:
    """Level 0 is the identity; a level whose stride reaches N is the identity too."""
    for n in (49, 196, 784):
        assert prod.radix_order(n, 16, 0) == list(range(n))
        assert orc.radix_order(n, 16, 0) == list(range(n))
    assert prod.radix_order(196, 16, 2) == list(range(196))
    assert prod.radix_order(196, 16, 1)[:13] == [16 * i for i in range(13)]


def test_channel_rotation_closed_form() -> None:
    """Level L with n groups: tile q holds channels {(q+L) mod n + k*n}."""
    for level in (1, 2, 3, 5):
        plan = prod.build_route_plan(14, 14, 512, 16, 128, "radix", level)
        for q in range(4):
            expected = [((q + level) % 4) + 4 * k for k in range(128)]
            assert plan.channel_indices[q].tolist() == expected


# Mirrors of the reference's tests/test_routing.py:10-74, run on both implementations.
@pytest.mark.parametrize("mod", [prod, orc], ids=["native", "oracle"])
def test_local_route_covers_tokens_once(mod) -> None:
    plan = mod.build_route_plan(8, 8, 128, 16, 64, "local")
    valid = plan.token_indices[plan.token_mask]
    assert torch.equal(torch.sort(valid).values, torch.arange(64))
    assert plan.token_indices.shape == (4, 16)
    assert plan.channel_indices.shape == (2, 64)


@pytest.mark.parametrize("mod", [prod, orc], ids=["native", "oracle"])
def test_shifted_route_is_a_permutation(mod) -> None:
    local = mod.build_route_plan(8, 8, 128, 16, 64, "local")
    shifted = mod.build_route_plan(8, 8, 128, 16, 64, "shifted")
    assert not torch.equal(local.token_indices, shifted.token_indices)
    assert torch.equal(torch.sort(shifted.token_indices[shifted.token_mask]).values, torch.arange(64))


@pytest.mark.parametrize("mod", [prod, orc], ids=["native", "oracle"])
def test_padding_masks_non_divisible_shapes(mod) -> None:
    plan = mod.build_route_plan(7, 7, 70, 16, 64, "radix", radix_level=1)
    assert plan.token_mask.sum().item() == 49
    assert plan.channel_mask.sum().item() == 70
    assert plan.token_indices.max().item() == 49
    assert plan.channel_indices.max().item() == 70


@pytest.mark.parametrize("mod", [prod, orc], ids=["native", "oracle"])
def test_radix_route_covers_tokens(mod) -> None:
    plan = mod.build_route_plan(8, 8, 128, 16, 64, "radix", radix_level=0)
    assert torch.equal(torch.sort(plan.token_indices[plan.token_mask]).values, torch.arange(64))


@pytest.mark.parametrize("mod", [prod, orc], ids=["native", "oracle"])
def test_local_route_small_spatial(mod) -> None:
    plan = mod.build_route_plan(4, 4, 32, 16, 32, "local")
    assert torch.equal(torch.sort(plan.token_indices[plan.token_mask]).values, torch.arange(16))
    assert plan.token_indices.shape == (1, 16)


@pytest.mark.parametrize("mod", [prod, orc], ids=["native", "oracle"])
def test_unknown_route_rejected(mod) -> None:
    with pytest.raises(ValueError, match="unknown route type"):
        mod.build_route_plan(8, 8, 16, 16, 8, "diagonal")


def test_route_plan_is_cached() -> None:
    assert prod.build_route_plan(8, 8, 16, 16, 8, "local") is prod.build_route_plan(8, 8, 16, 16, 8, "local")


def test_native_builder_rejects_bad_shapes() -> None:
    with pytest.raises(ValueError, match="height/width"):
        prod.build_route_plan(0, 8, 16, 16, 8, "local", 0)
    with pytest.raises(ValueError, match="radix_level"):
        prod.build_route_plan(8, 8, 16, 16, 8, "radix", -1)
