"""Oracle backbone glue: CPU restatement of the OmniWeave-T stem and downsample layout (test
infrastructure only).

``space_to_depth_nhwc`` restates ``omniweave/models/backbone.py:14-27`` (packing order: row
offset, column offset, channel); ``stem_reference`` restates the stem of
``forward_features`` (``backbone.py:173-176``: NCHW -> NHWC permute, space_to_depth(4),
bias-free Linear) in fp32; ``space_to_depth_loops`` is an element-by-element loop over the
definition that shares no code with the reshape form, used to pin it.
"""

from __future__ import annotations

import torch
from torch import Tensor


def space_to_depth_nhwc(x: Tensor, factor: int) -> Tensor:
    """``[B, H, W, C] -> [B, H/f, W/f, f*f*C]`` (omniweave/models/backbone.py:14-27)."""
    b, h, w, c = x.shape
    if h % factor or w % factor:
        raise ValueError(f"H={h}, W={w} must be divisible by factor {factor}")
    x = x.reshape(b, h // factor, factor, w // factor, factor, c)
    x = x.permute(0, 1, 3, 2, 4, 5)
    return x.reshape(b, h // factor, w // factor, factor * factor * c)


def space_to_depth_loops(x: Tensor, factor: int) -> Tensor:
    """Element loop: out[b, i, j, (dr*f + dc)*C + ch] = x[b, i*f + dr, j*f + dc, ch]."""
    b, h, w, c = x.shape
    out = torch.empty(b, h // factor, w // factor, factor * factor * c, dtype=x.dtype)
    for i in range(h // factor):
        for j in range(w // factor):
            for dr in range(factor):
                for dc in range(factor):
                    k = (dr * factor + dc) * c
                    out[:, i, j, k:k + c] = x[:, i * factor + dr, j * factor + dc, :]
    return out


def stem_reference(image: Tensor, weight: Tensor) -> Tensor:
    """NCHW image ``[B, 3, H, W]``, weight ``[N, 48]`` -> NHWC ``[B, H/4, W/4, N]`` in fp32
    (omniweave/models/backbone.py:121,173-176)."""
    x = space_to_depth_nhwc(image.float().permute(0, 2, 3, 1), 4)
    return x @ weight.float().t()
