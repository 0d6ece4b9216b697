"""Oracle route plans: literal restatement of the reference's routing (test infrastructure).

Follows ``omniweave/models/routing.py`` line by line, with Python lists and loops, so that
the product's native route builder can be compared against it.  Every function cites the
reference lines it restates.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch


@dataclass(frozen=True)
class OracleRoutePlan:
    """Same fields as ``RoutePlan`` (omniweave/models/routing.py:17-33)."""

    token_indices: torch.Tensor    # [Q_s, g] int64, pad = N
    channel_indices: torch.Tensor  # [Q_c, d] int64, pad = C
    token_mask: torch.Tensor       # [Q_s, g] bool
    channel_mask: torch.Tensor     # [Q_c, d] bool
    height: int
    width: int
    channels: int
    route: str
    radix_level: int


def pad_and_mask(indices: list[int], group_size: int, pad_value: int):
    """omniweave/models/routing.py:40-54."""
    n = len(indices)
    n_groups = math.ceil(n / group_size)
    total = n_groups * group_size
    padded = indices + [pad_value] * (total - n)
    idx = torch.tensor(padded, dtype=torch.long).reshape(n_groups, group_size)
    mask = torch.ones(n_groups, group_size, dtype=torch.bool)
    if total > n:
        mask.reshape(-1)[n:] = False
    return idx, mask


def local_token_order(height: int, width: int, window: int = 4) -> list[int]:
    """omniweave/models/routing.py:57-65."""
    order: list[int] = []
    for row_base in range(0, height, window):
        for col_base in range(0, width, window):
            for r in range(row_base, min(row_base + window, height)):
                for c in range(col_base, min(col_base + window, width)):
                    order.append(r * width + c)
    return order


def shifted_token_order(height: int, width: int, window: int = 4, shift: int = 2) -> list[int]:
    """omniweave/models/routing.py:68-90 (wrap-around windows, first occurrence wins)."""
    order: list[int] = []
    for row_base in range(-shift, height - shift, window):
        for col_base in range(-shift, width - shift, window):
            for r in range(row_base, row_base + window):
                for c in range(col_base, col_base + window):
                    order.append((r % height) * width + (c % width))
    seen: set[int] = set()
    deduped: list[int] = []
    for idx in order:
        if idx not in seen:
            seen.add(idx)
            deduped.append(idx)
    return deduped


def radix_order(token_count: int, group_size: int, level: int) -> list[int]:
    """omniweave/models/routing.py:93-104."""
    stride = group_size ** level
    block = stride * group_size
    order: list[int] = []
    for base in range(0, token_count, block):
        for offset in range(stride):
            for digit in range(group_size):
                index = base + digit * stride + offset
                if index < token_count:
                    order.append(index)
    return order


def channel_order(channels: int, channel_tile: int, radix_level: int) -> list[int]:
    """omniweave/models/routing.py:107-121."""
    n_groups = math.ceil(channels / channel_tile)
    indices = list(range(channels))
    if radix_level == 0 or n_groups <= 1:
        return indices
    groups: list[list[int]] = [[] for _ in range(n_groups)]
    for i, idx in enumerate(indices):
        groups[i % n_groups].append(idx)
    rotation = radix_level % n_groups
    rotated = groups[rotation:] + groups[:rotation]
    return [idx for group in rotated for idx in group]


def build_route_plan(
    height: int,
    width: int,
    channels: int,
    spatial_tile: int,
    channel_tile: int,
    route: str,
    radix_level: int = 0,
) -> OracleRoutePlan:
    """omniweave/models/routing.py:128-179."""
    n_tokens = height * width
    if route == "local":
        token_order = local_token_order(height, width)
    elif route == "shifted":
        token_order = shifted_token_order(height, width)
    elif route == "radix":
        token_order = radix_order(n_tokens, spatial_tile, radix_level)
    else:
        raise ValueError(f"unknown route type: {route!r}")
    token_indices, token_mask = pad_and_mask(token_order, spatial_tile, n_tokens)
    ch_order = channel_order(channels, channel_tile, radix_level)
    channel_indices, channel_mask = pad_and_mask(ch_order, channel_tile, channels)
    return OracleRoutePlan(
        token_indices=token_indices,
        channel_indices=channel_indices,
        token_mask=token_mask,
        channel_mask=channel_mask,
        height=height,
        width=width,
        channels=channels,
        route=route,
        radix_level=radix_level,
    )


def build_stage_schedule(depth: int) -> list[tuple[str, int]]:
    """omniweave/models/routing.py:182-198."""
    cycle = [("local", 0), ("shifted", 0), ("radix", 0), ("radix", 1), ("radix", 2)]
    return [cycle[i % len(cycle)] for i in range(depth)]
