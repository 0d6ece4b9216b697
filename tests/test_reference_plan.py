"""The boundary takes the reference's own plan type.

The reference's ``RoutePlan`` (omniweave/models/routing.py:17-33) is a frozen dataclass with
nine fields and no methods.  ``oracle.routing.OracleRoutePlan`` has exactly those fields, so a
plan built by the oracle stands in for one built by the reference: every helper of the package
that reads a plan (descriptor, cache key, device tables, output-row tables, the support probe)
must accept it and give what it gives for the package's own plan.
"""

from __future__ import annotations

import ctypes
import dataclasses

import pytest
import torch

import omniwave_amd
from omniwave_amd import _native
from omniwave_amd.hip import _plan_desc, hip_is_supported
from omniwave_amd.routing import RoutePlan, device_tables, native_plan, plan_key, plan_tiles, s2d_rows_table
from oracle.routing import OracleRoutePlan, build_route_plan as oracle_plan

CASES = [(14, 14, 512, 128, "shifted", 0), (56, 56, 128, 64, "local", 0), (7, 7, 1024, 128, "radix", 1),
         (28, 28, 256, 64, "radix", 2)]


def test_package_plan_has_exactly_the_reference_fields() -> None:
    assert [f.name for f in dataclasses.fields(RoutePlan)] == [f.name for f in dataclasses.fields(OracleRoutePlan)]
    assert [f.name for f in dataclasses.fields(RoutePlan)] == [
        "token_indices", "channel_indices", "token_mask", "channel_mask", "height", "width", "channels", "route",
        "radix_level"]


@pytest.mark.parametrize("h,w,c,d,route,level", CASES)
def test_descriptor_key_and_tables_match(h, w, c, d, route, level) -> None:
    ours = omniwave_amd.build_route_plan(h, w, c, 16, d, route, level)
    ref = oracle_plan(h, w, c, 16, d, route, level)
    assert not isinstance(ref, RoutePlan)
    assert plan_tiles(ref) == plan_tiles(ours) == (16, d)
    assert plan_key(ref) == plan_key(ours) == (h, w, c, 16, d, route, level)
    assert _plan_desc(ref) == _plan_desc(ours) == [h, w, c, 16, d, _native.OW_ROUTE[route], level]
    a, b = native_plan(ref), native_plan(ours)
    assert [getattr(a, f) for f, _ in _native.OwPlan._fields_] == [getattr(b, f) for f, _ in _native.OwPlan._fields_]
    q_s, q_c = ctypes.c_int32(), ctypes.c_int32()
    assert _native.lib().ow_plan_dims(ctypes.byref(a), ctypes.byref(q_s), ctypes.byref(q_c)) == 0
    assert (q_s.value, q_c.value) == tuple(ref.token_indices.shape[:1]) + tuple(ref.channel_indices.shape[:1])
    cpu = torch.device("cpu")
    for t_ref, t_ours in zip(device_tables(ref, cpu), device_tables(ours, cpu)):
        assert torch.equal(t_ref, t_ours)
    if h % 2 == 0 and w % 2 == 0:
        assert torch.equal(s2d_rows_table(ref, 2, cpu), s2d_rows_table(ours, 2, cpu))


def test_support_probe_accepts_reference_plan_on_the_cpu() -> None:
    ref = oracle_plan(14, 14, 512, 16, 128, "shifted", 0)
    x = torch.zeros(1, 14, 14, 512, dtype=torch.bfloat16)
    ok, reason = hip_is_supported(x, ref, torch.zeros(4, 128, 256))
    assert not ok and reason == "CUDA is unavailable"


def test_unknown_route_in_a_reference_plan_is_a_value_error() -> None:
    ref = dataclasses.replace(oracle_plan(7, 7, 128, 16, 64, "local", 0), route="diagonal")
    with pytest.raises(ValueError, match="unknown route"):
        _plan_desc(ref)
    with pytest.raises(ValueError, match="unknown route"):
        native_plan(ref)
