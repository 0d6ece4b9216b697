"""Pins the oracle's BiGEMM: the reference's own known-answer tests (tests/test_ops.py of the
reference), an fp64 per-tile brute force that shares no code with pack/einsum/unpack, and the
RMSNorm dtype sequence."""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle.bigemm import (
    bigemm_delta_bruteforce,
    bigemm_delta_reference,
    block_reference,
    pack_tiles,
    rel_l2,
    rmsnorm_reference,
    unpack_tiles,
)
from oracle.routing import build_route_plan


# --- mirrors of the reference's tests/test_ops.py:12-133 ---------------------------------

def test_pack_unpack_identity() -> None:
    x = torch.arange(2 * 7 * 7 * 70, dtype=torch.float32).reshape(2, 7, 7, 70)
    plan = build_route_plan(7, 7, 70, 16, 64, "radix", radix_level=1)
    tiles, mask = pack_tiles(x, plan)
    assert tiles.shape == (2, 4, 2, 16, 64)
    assert mask.shape == (1, 4, 2, 16, 64)
    torch.testing.assert_close(unpack_tiles(tiles, plan, 2), x)


def test_padding_values_are_zero() -> None:
    x = torch.ones(1, 7, 7, 70)
    plan = build_route_plan(7, 7, 70, 16, 64, "local")
    tiles, mask = pack_tiles(x, plan)
    assert torch.count_nonzero(tiles.masked_select(~mask)) == 0


def test_pack_unpack_exact_shapes() -> None:
    x = torch.randn(3, 8, 8, 128)
    plan = build_route_plan(8, 8, 128, 16, 64, "local")
    tiles, mask = pack_tiles(x, plan)
    assert tiles.shape == (3, 4, 2, 16, 64)
    assert mask.all()
    torch.testing.assert_close(unpack_tiles(tiles, plan, 3), x)


def test_pack_unpack_shifted() -> None:
    x = torch.randn(2, 8, 8, 128)
    plan = build_route_plan(8, 8, 128, 16, 64, "shifted")
    tiles, _ = pack_tiles(x, plan)
    torch.testing.assert_close(unpack_tiles(tiles, plan, 2), x)


def test_single_tile_matches_equation() -> None:
    torch.manual_seed(7)
    g, d, rd = 16, 4, 8
    x = torch.randn(1, 4, 4, 4, dtype=torch.float64)
    plan = build_route_plan(4, 4, 4, g, d, "local")
    a_u, a_v, a_o = (torch.randn(g, g, dtype=torch.float64) for _ in range(3))
    b_u = torch.randn(1, d, rd, dtype=torch.float64)
    b_v = torch.randn(1, d, rd, dtype=torch.float64)
    b_o = torch.randn(1, rd, d, dtype=torch.float64)
    gamma = torch.ones(d, dtype=torch.float64)
    actual = bigemm_delta_reference(x=x, plan=plan, a_u=a_u, a_v=a_v, a_o=a_o, b_u=b_u, b_v=b_v, b_o=b_o, gamma=gamma)
    tile = x.reshape(g, d)
    expected = (a_o @ (F.silu(a_u @ tile @ b_u[0]) * (a_v @ tile @ b_v[0])) @ b_o[0]).reshape_as(x)
    torch.testing.assert_close(actual, expected)


def test_bigemm_gradcheck() -> None:
    torch.manual_seed(42)
    g, d, rd = 16, 4, 8
    plan = build_route_plan(4, 4, 4, g, d, "local")
    args = (
        torch.randn(1, 4, 4, 4, dtype=torch.float64, requires_grad=True),
        *(torch.randn(g, g, dtype=torch.float64, requires_grad=True) for _ in range(3)),
        torch.randn(1, d, rd, dtype=torch.float64, requires_grad=True),
        torch.randn(1, d, rd, dtype=torch.float64, requires_grad=True),
        torch.randn(1, rd, d, dtype=torch.float64, requires_grad=True),
        torch.randn(d, dtype=torch.float64, requires_grad=True),
    )

    def func(x_, a_u_, a_v_, a_o_, b_u_, b_v_, b_o_, gamma_):
        return bigemm_delta_reference(x=x_, plan=plan, a_u=a_u_, a_v=a_v_, a_o=a_o_, b_u=b_u_, b_v=b_v_,
                                      b_o=b_o_, gamma=gamma_)

    torch.autograd.gradcheck(func, args, eps=1e-6, atol=1e-4, rtol=1e-3)


def test_bigemm_multi_channel_groups() -> None:
    torch.manual_seed(17)
    h, w, c, g, d, rd = 8, 8, 128, 16, 64, 128
    x = torch.randn(2, h, w, c, dtype=torch.float64)
    plan = build_route_plan(h, w, c, g, d, "radix", radix_level=0)
    a_u, a_v = torch.randn(g, g, dtype=torch.float64), torch.randn(g, g, dtype=torch.float64)
    a_o = torch.eye(g, dtype=torch.float64)
    b_u, b_v = torch.randn(2, d, rd, dtype=torch.float64), torch.randn(2, d, rd, dtype=torch.float64)
    b_o = torch.randn(2, rd, d, dtype=torch.float64)
    gamma = torch.ones(c, dtype=torch.float64) * 1e-5
    delta = bigemm_delta_reference(x=x, plan=plan, a_u=a_u, a_v=a_v, a_o=a_o, b_u=b_u, b_v=b_v, b_o=b_o, gamma=gamma)
    assert delta.shape == x.shape
    assert delta.abs().max().item() < 1.0


# --- brute force: every route, pad rows, pad channels, rotated channel groups ------------

def _weights(g, d, rd, q_c, seed, dtype=torch.float64):
    gen = torch.Generator().manual_seed(seed)
    a = [torch.randn(g, g, generator=gen, dtype=dtype) / 4 for _ in range(3)]
    b_u = torch.randn(q_c, d, rd, generator=gen, dtype=dtype) / d ** 0.5
    b_v = torch.randn(q_c, d, rd, generator=gen, dtype=dtype) / d ** 0.5
    b_o = torch.randn(q_c, rd, d, generator=gen, dtype=dtype) / rd ** 0.5
    return a, b_u, b_v, b_o


@pytest.mark.parametrize(
    "shape,route,level",
    [
        ((7, 7, 70, 64, 128), "radix", 1),     # pad rows + pad channels + rotated groups
        ((7, 7, 64, 16, 32), "shifted", 0),    # wrap-around windows, 4 groups
        ((6, 5, 48, 16, 32), "local", 0),      # partial windows
        ((9, 9, 64, 32, 64), "radix", 2),      # level 2 channel rotation
        ((4, 12, 32, 16, 48), "radix", 1),     # rd not a multiple of d
    ],
)
def test_oracle_matches_bruteforce(shape, route, level) -> None:
    h, w, c, d, rd = shape
    g = 16
    plan = build_route_plan(h, w, c, g, d, route, level)
    q_c = plan.channel_indices.shape[0]
    x = torch.randn(2, h, w, c, dtype=torch.float64, generator=torch.Generator().manual_seed(3))
    (a_u, a_v, a_o), b_u, b_v, b_o = _weights(g, d, rd, q_c, seed=5)
    gamma = torch.rand(c, dtype=torch.float64, generator=torch.Generator().manual_seed(9)) + 0.5
    got = bigemm_delta_reference(x=x, plan=plan, a_u=a_u, a_v=a_v, a_o=a_o, b_u=b_u, b_v=b_v, b_o=b_o, gamma=gamma)
    ref = bigemm_delta_bruteforce(x.numpy(), plan.token_indices.numpy(), plan.channel_indices.numpy(),
                                  a_u.numpy(), a_v.numpy(), a_o.numpy(), b_u.numpy(), b_v.numpy(), b_o.numpy(),
                                  gamma.numpy())
    np.testing.assert_allclose(got.numpy(), ref, rtol=1e-10, atol=1e-12)


def test_bruteforce_catches_transposed_operand() -> None:
    """Planted mistake: A_u^T instead of A_u must change the result."""
    h, w, c, d, rd = 4, 4, 16, 16, 32
    plan = build_route_plan(h, w, c, 16, d, "local")
    x = torch.randn(1, h, w, c, dtype=torch.float64)
    (a_u, a_v, a_o), b_u, b_v, b_o = _weights(16, d, rd, 1, seed=1)
    gamma = torch.ones(c, dtype=torch.float64)
    good = bigemm_delta_bruteforce(x.numpy(), plan.token_indices.numpy(), plan.channel_indices.numpy(),
                                   a_u.numpy(), a_v.numpy(), a_o.numpy(), b_u.numpy(), b_v.numpy(), b_o.numpy(),
                                   gamma.numpy())
    bad = bigemm_delta_reference(x=x, plan=plan, a_u=a_u.T, a_v=a_v, a_o=a_o, b_u=b_u, b_v=b_v, b_o=b_o, gamma=gamma)
    assert np.abs(bad.numpy() - good).max() > 1e-3


def test_identity_weights_closed_form() -> None:
    """A = I, B_u = B_v = [I 0], B_o = [I; 0]: delta = gamma * SiLU(x) * x, any route."""
    for route, level in (("local", 0), ("shifted", 0), ("radix", 1)):
        h, w, c, d, rd = 7, 7, 32, 16, 32
        plan = build_route_plan(h, w, c, 16, d, route, level)
        q_c = plan.channel_indices.shape[0]
        eye = torch.eye(16, dtype=torch.float64)
        b_in = torch.zeros(q_c, d, rd, dtype=torch.float64)
        b_in[:, :, :d] = torch.eye(d, dtype=torch.float64)
        b_out = b_in.transpose(1, 2).contiguous()
        x = torch.randn(2, h, w, c, dtype=torch.float64)
        gamma = torch.linspace(0.5, 1.5, c, dtype=torch.float64)
        got = bigemm_delta_reference(x=x, plan=plan, a_u=eye, a_v=eye, a_o=eye, b_u=b_in, b_v=b_in, b_o=b_out,
                                     gamma=gamma)
        torch.testing.assert_close(got, F.silu(x) * x * gamma)


# --- RMSNorm ---------------------------------------------------------------------------------

def test_rmsnorm_fp64_textbook() -> None:
    x = torch.randn(3, 5, 5, 64, dtype=torch.float64)
    w = torch.rand(64, dtype=torch.float64) + 0.5
    expected = x / torch.sqrt((x * x).mean(-1, keepdim=True) + 1e-6) * w
    torch.testing.assert_close(rmsnorm_reference(x, w), expected.to(torch.float64), rtol=1e-6, atol=1e-7)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_rmsnorm_dtype_sequence(dtype) -> None:
    """Element-wise restatement of block.py:83-85's rounding points in the low dtype."""
    x = torch.randn(2, 4, 4, 96).to(dtype)
    w = torch.rand(96) + 0.5
    var = (x.float() ** 2).mean(-1, keepdim=True).to(dtype)
    r = torch.rsqrt((var.float() + 1e-6).to(dtype).float()).to(dtype)
    expected = ((x.float() * r.float()).to(dtype).float() * w).to(dtype)
    assert torch.equal(rmsnorm_reference(x, w), expected)
    assert rel_l2(rmsnorm_reference(x, w), rmsnorm_reference(x.double(), w.double())) < 1e-2


def test_block_reference_is_residual_plus_delta() -> None:
    h, w, c, d = 7, 7, 32, 16
    plan = build_route_plan(h, w, c, 16, d, "shifted")
    (a_u, a_v, a_o), b_u, b_v, b_o = _weights(16, d, 2 * d, 2, seed=2, dtype=torch.float32)
    params = dict(norm_weight=torch.rand(c) + 0.5, a_u=a_u, a_v=a_v, a_o=a_o, b_u=b_u, b_v=b_v, b_o=b_o,
                  gamma=torch.ones(c))
    x = torch.randn(2, h, w, c)
    delta = block_reference(x, plan, params, residual=False)
    torch.testing.assert_close(block_reference(x, plan, params), x + delta)
    assert delta.abs().mean() > 1e-3
