"""Backbone glue on the CPU: the oracle's space_to_depth and stem pinned against element
loops, the product's space_to_depth against the oracle, and the native output-row table
(``ow_route_s2d_rows``) against the oracle's layout applied to an index image."""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

import omniwave_amd
from omniwave_amd import _native
from omniwave_amd.backbone import space_to_depth_nhwc
from omniwave_amd.hip import stem_is_supported
from omniwave_amd.routing import native_plan, s2d_rows_table
from oracle.backbone import space_to_depth_loops, space_to_depth_nhwc as oracle_s2d, stem_reference


@pytest.mark.parametrize("factor", [2, 4])
def test_oracle_space_to_depth_matches_element_loop(factor) -> None:
    x = torch.randn(2, 8, 12, 5, generator=torch.Generator().manual_seed(0))
    assert torch.equal(oracle_s2d(x, factor), space_to_depth_loops(x, factor))
    assert torch.equal(space_to_depth_nhwc(x, factor), oracle_s2d(x, factor))
    with pytest.raises(ValueError):
        oracle_s2d(x[:, :7], 2)


def test_oracle_stem_matches_patch_dot_products() -> None:
    gen = torch.Generator().manual_seed(1)
    img = torch.randn(2, 3, 8, 12, generator=gen)
    w = torch.randn(5, 48, generator=gen)
    got = stem_reference(img, w)
    assert got.shape == (2, 2, 3, 5)
    img64, w64 = img.double(), w.double()
    for b in range(2):
        for i in range(2):
            for j in range(3):
                for n in range(5):
                    acc = 0.0
                    for dr in range(4):
                        for dc in range(4):
                            for c in range(3):
                                acc += float(img64[b, c, 4 * i + dr, 4 * j + dc]) * float(w64[n, dr * 12 + dc * 3 + c])
                    assert abs(float(got[b, i, j, n]) - acc) <= 1e-4 * (1 + abs(acc))


@pytest.mark.parametrize("shape,route,level", [
    ((56, 56, 128, 64), "local", 0), ((56, 56, 128, 64), "shifted", 0), ((28, 28, 256, 64), "radix", 2),
    ((14, 14, 512, 128), "radix", 1), ((14, 14, 512, 128), "shifted", 0), ((6, 10, 96, 64), "local", 0),
])
@pytest.mark.parametrize("factor", [2])
def test_s2d_rows_table_places_tokens_like_space_to_depth(shape, route, level, factor) -> None:
    h, w, c, d = shape
    plan = omniwave_amd.build_route_plan(h, w, c, 16, d, route, level)
    rows = s2d_rows_table(plan, factor, torch.device("cpu")).numpy()
    tok = plan.token_indices.reshape(-1).numpy()
    n = h * w
    # Index image: the value at pixel t is t; after space_to_depth, row r of the [H*W, 1] view
    # holds the pixel that lands there.
    idx = torch.arange(n, dtype=torch.float64).reshape(1, h, w, 1)
    landed = oracle_s2d(idx, factor).reshape(-1).long().numpy()  # landed[row] = pixel
    where = np.empty(n, dtype=np.int64)
    where[landed] = np.arange(n)
    valid = tok < n
    assert np.array_equal(rows[valid], where[tok[valid]])
    assert np.all(rows[~valid] == n)
    assert sorted(rows[valid].tolist()) == list(range(n))


def test_s2d_rows_rejects_indivisible_sizes() -> None:
    plan = omniwave_amd.build_route_plan(7, 7, 128, 16, 64, "local", 0)
    tok = np.ascontiguousarray(plan.token_indices.reshape(-1).numpy(), dtype=np.int32)
    out = np.empty_like(tok)
    native = native_plan(plan)
    rc = _native.lib().ow_route_s2d_rows(ctypes.byref(native), 2, tok.ctypes.data_as(_native._c_int32_p),
                                         out.ctypes.data_as(_native._c_int32_p))
    assert rc != 0
    assert b"divisible" in _native.lib().ow_last_error()


def test_stem_support_reasons_on_cpu() -> None:
    ok, reason = stem_is_supported(torch.zeros(1, 3, 8, 8, dtype=torch.bfloat16), torch.zeros(128, 48, dtype=torch.bfloat16))
    assert not ok and reason


def test_model_forward_on_cpu_keeps_the_reference_composition(oracle_backend) -> None:
    torch.manual_seed(0)
    model = omniwave_amd.create_model("omniweave_t", input_size=64).eval()
    for stage in model.stages:
        for blk in stage.blocks:
            blk.backend = "reference"
    x = torch.randn(1, 3, 64, 64)
    with torch.no_grad():
        feats = model.forward_features(x)
        want = model.head(feats["stage4"].mean(dim=(1, 2)))
        got = model(x)
    assert torch.equal(got, want)
