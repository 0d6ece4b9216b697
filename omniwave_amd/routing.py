"""Route plans for the BiGEMM operator.

Same API as the reference (``omniweave/models/routing.py:17-198``): ``RoutePlan``,
``build_route_plan`` (cached), ``build_stage_schedule`` and ``radix_order``.  The index maps
are computed by the native route builder (``ow_route_build`` in libomniwave_amd.so) and
returned as CPU int64 tensors with pad index ``N`` for tokens and ``C`` for channels, exactly
like the reference's plans.  ``device_tables`` keeps an int32 copy of each plan's tables on
each device for the HIP kernels.
"""

from __future__ import annotations

import functools
from dataclasses import dataclass

import numpy as np
import torch

from omniwave_amd import _native

WINDOW = 4  # omniweave/models/routing.py:57,71
SHIFT = 2   # omniweave/models/routing.py:72


@dataclass(frozen=True)
class RoutePlan:
    """Immutable routing specification for one block (omniweave/models/routing.py:17-33).

    Exactly the reference's fields.  Everything this package derives from a plan goes through
    the free functions below (``plan_tiles``, ``plan_key``, ``native_plan``), which read only
    these fields, so the reference's own ``RoutePlan`` objects are accepted wherever a plan is.
    """

    token_indices: torch.Tensor    # [Q_s, g] int64, pad index = N
    channel_indices: torch.Tensor  # [Q_c, d] int64, pad index = C
    token_mask: torch.Tensor       # [Q_s, g] bool
    channel_mask: torch.Tensor     # [Q_c, d] bool
    height: int
    width: int
    channels: int
    route: str
    radix_level: int


def plan_tiles(plan) -> tuple[int, int]:
    """(g, d): the spatial and channel tile of any plan with the reference's fields."""
    return int(plan.token_indices.shape[1]), int(plan.channel_indices.shape[1])


def plan_key(plan) -> tuple:
    """Hashable descriptor of a plan (its tensors make the dataclass itself unsuitable as a
    key): the arguments of build_route_plan, which determine the tables."""
    g, d = plan_tiles(plan)
    return (int(plan.height), int(plan.width), int(plan.channels), g, d, str(plan.route), int(plan.radix_level))


def native_plan(plan) -> _native.OwPlan:
    """The C-ABI descriptor (OwPlan) of a plan."""
    g, d = plan_tiles(plan)
    if plan.route not in _native.OW_ROUTE:
        raise ValueError(f"unknown route type: {plan.route!r}")
    return _native.make_plan(int(plan.height), int(plan.width), int(plan.channels), g, d, plan.route,
                             int(plan.radix_level), WINDOW, SHIFT)


def _route_tables(height, width, channels, spatial_tile, channel_tile, route, radix_level):
    if route not in _native.OW_ROUTE:
        raise ValueError(f"unknown route type: {route!r}")
    lib = _native.lib()
    plan = _native.make_plan(height, width, channels, spatial_tile, channel_tile, route, radix_level,
                             WINDOW, SHIFT)
    q_s = _native.ctypes.c_int32()
    q_c = _native.ctypes.c_int32()
    _native.check(lib.ow_plan_dims(_native.ctypes.byref(plan), _native.ctypes.byref(q_s),
                                   _native.ctypes.byref(q_c)), "ow_plan_dims")
    tok = np.empty(q_s.value * spatial_tile, dtype=np.int32)
    ch = np.empty(q_c.value * channel_tile, dtype=np.int32)
    ptr = _native._c_int32_p
    _native.check(lib.ow_route_build(_native.ctypes.byref(plan), tok.ctypes.data_as(ptr),
                                     ch.ctypes.data_as(ptr)), "ow_route_build")
    return tok.reshape(q_s.value, spatial_tile), ch.reshape(q_c.value, channel_tile)


@functools.lru_cache(maxsize=256)
def build_route_plan(
    height: int,
    width: int,
    channels: int,
    spatial_tile: int,
    channel_tile: int,
    route: str,
    radix_level: int = 0,
) -> RoutePlan:
    """Deterministic, cached route plan (omniweave/models/routing.py:128-179).

    ``route`` is ``"local"``, ``"shifted"`` or ``"radix"``; unknown routes raise ValueError.
    """
    tok, ch = _route_tables(height, width, channels, spatial_tile, channel_tile, route, radix_level)
    token_indices = torch.from_numpy(tok.astype(np.int64))
    channel_indices = torch.from_numpy(ch.astype(np.int64))
    return RoutePlan(
        token_indices=token_indices,
        channel_indices=channel_indices,
        token_mask=token_indices < height * width,
        channel_mask=channel_indices < channels,
        height=height,
        width=width,
        channels=channels,
        route=route,
        radix_level=radix_level,
    )


def radix_order(token_count: int, group_size: int, level: int) -> list[int]:
    """Mixed-radix token order at ``level`` (omniweave/models/routing.py:93-104)."""
    tok, _ = _route_tables(1, token_count, 1, group_size, 1, "radix", level)
    flat = tok.reshape(-1)
    return [int(v) for v in flat[flat < token_count]]


def build_stage_schedule(depth: int) -> list[tuple[str, int]]:
    """Route schedule of a stage: local, shifted, radix-0, radix-1, radix-2, repeated
    (omniweave/models/routing.py:182-198)."""
    cycle = (("local", 0), ("shifted", 0), ("radix", 0), ("radix", 1), ("radix", 2))
    return [cycle[i % len(cycle)] for i in range(depth)]


_DEVICE_TABLES: dict[tuple, tuple[torch.Tensor, torch.Tensor]] = {}


def device_tables(plan, device: torch.device) -> tuple[torch.Tensor, torch.Tensor]:
    """int32 token/channel tables of ``plan`` resident on ``device`` (uploaded once)."""
    dev = torch.device(device)
    key = plan_key(plan) + (dev.type, dev.index)
    hit = _DEVICE_TABLES.get(key)
    if hit is None:
        tok = plan.token_indices.reshape(-1).to(torch.int32).to(dev)
        ch = plan.channel_indices.reshape(-1).to(torch.int32).to(dev)
        hit = (tok, ch)
        _DEVICE_TABLES[key] = hit
    return hit


_S2D_ROWS: dict[tuple, torch.Tensor] = {}


def s2d_rows_table(plan, factor: int, device: torch.device) -> torch.Tensor:
    """int32 ``[Q_s * g]`` output-row table on ``device`` (``ow_route_s2d_rows``): the row each
    token slot occupies in ``space_to_depth(out, factor)`` viewed as ``[H*W, C]`` rows per image
    (omniweave/models/backbone.py:14-27); pad slots hold H*W."""
    dev = torch.device(device)
    key = plan_key(plan) + (int(factor), dev.type, dev.index)
    hit = _S2D_ROWS.get(key)
    if hit is None:
        lib = _native.lib()
        tok = np.ascontiguousarray(plan.token_indices.reshape(-1).numpy(), dtype=np.int32)
        rows = np.empty_like(tok)
        ptr = _native._c_int32_p
        native = native_plan(plan)
        _native.check(lib.ow_route_s2d_rows(_native.ctypes.byref(native), int(factor), tok.ctypes.data_as(ptr),
                                            rows.ctypes.data_as(ptr)), "ow_route_s2d_rows")
        hit = torch.from_numpy(rows).to(dev)
        _S2D_ROWS[key] = hit
    return hit

