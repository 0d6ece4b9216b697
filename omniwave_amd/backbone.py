"""OmniWeave-T hierarchical backbone (omniweave/models/backbone.py:14-197).

Stem space-to-depth(4) -> Linear(48, C1); four stages of OmniWeaveBlocks (with a Linear
anchor at the start of stages 3 and 4); space-to-depth(2) -> Linear(4C, 2C) between stages;
global average pool -> Linear(C4, num_classes).  Module and parameter names match the
reference.
"""

from __future__ import annotations

from collections import OrderedDict

import torch
import torch.nn as nn
import torch.nn.functional as F
from torch import Tensor

from omniwave_amd.block import OmniWeaveBlock
from omniwave_amd.hip import stem_hip, stem_is_supported
from omniwave_amd.routing import build_stage_schedule


def space_to_depth_nhwc(x: Tensor, factor: int) -> Tensor:
    """``[B, H, W, C] -> [B, H/f, W/f, C*f*f]`` with (row offset, col offset, channel) packing
    (omniweave/models/backbone.py:14-27)."""
    b, h, w, c = x.shape
    if h % factor or w % factor:
        raise ValueError(f"height {h} and width {w} must be divisible by factor {factor}")
    x = x.reshape(b, h // factor, factor, w // factor, factor, c)
    return x.permute(0, 1, 3, 2, 4, 5).reshape(b, h // factor, w // factor, c * factor * factor)


class _Stage(nn.Module):
    """Optional anchor Linear, then blocks on the stage schedule (backbone.py:30-80)."""

    def __init__(self, height, width, dim, depth, channel_tile, expansion, layer_scale_init, spatial_tile,
                 use_anchor, backend, drop_path_rates) -> None:
        super().__init__()
        self.anchor: nn.Linear | None = nn.Linear(dim, dim, bias=False) if use_anchor else None
        self.blocks = nn.ModuleList()
        for (route, radix_level), rate in zip(build_stage_schedule(depth), drop_path_rates, strict=True):
            self.blocks.append(OmniWeaveBlock(
                height=height, width=width, dim=dim, channel_tile=channel_tile, route=route,
                radix_level=radix_level, expansion=expansion, layer_scale_init=layer_scale_init,
                spatial_tile=spatial_tile, backend=backend, drop_path_rate=rate,
            ))

    def forward(self, x: Tensor) -> Tensor:
        if self.anchor is not None:
            x = self.anchor(x)
        for block in self.blocks:
            x = block(x)
        return x

    def forward_blocks_s2d(self, x: Tensor, factor: int) -> Tensor:
        """``space_to_depth`` of the blocks' output (the anchor is the caller's); the last block
        writes that layout itself when it can, and each block hands the next its RMSNorm
        statistics when it can (``OmniWeaveBlock.forward_chain``)."""
        x, stats = self._chain(self.blocks[:-1], x)
        r = self.blocks[-1].forward_chain(x, stats, factor)
        if r is not None:
            return r[0]
        y = self.blocks[-1].forward_s2d(x, factor)
        return y if y is not None else space_to_depth_nhwc(self.blocks[-1](x), factor)

    def forward_blocks(self, x: Tensor) -> Tensor:
        """The blocks (the anchor is the caller's), chained as in ``forward_blocks_s2d``."""
        return self._chain(self.blocks, x)[0]

    @staticmethod
    def _chain(blocks, x: Tensor) -> tuple[Tensor, Tensor | None]:
        stats = None
        for block in blocks:
            r = block.forward_chain(x, stats)
            if r is None:
                x, stats = block(x), None
            else:
                x, stats = r
        return x, stats


class OmniWeaveBackbone(nn.Module):
    """Input ``[B, 3, H, W]`` (NCHW) -> logits ``[B, num_classes]``."""

    def __init__(
        self,
        widths: list[int] | None = None,
        depths: list[int] | None = None,
        channel_tiles: list[int] | None = None,
        num_classes: int = 1000,
        expansion: int = 2,
        layer_scale_init: float = 1e-5,
        anchor_stages: list[int] | None = None,
        spatial_tile: int = 16,
        backend: str = "auto",
        input_size: int = 224,
        drop_path_rate: float = 0.0,
    ) -> None:
        super().__init__()
        widths = widths or [128, 256, 512, 1024]
        depths = depths or [2, 3, 8, 2]
        channel_tiles = channel_tiles or [64, 64, 128, 128]
        if anchor_stages is None:
            anchor_stages = [3, 4]
        if not (len(widths) == len(depths) == len(channel_tiles) == 4):
            raise ValueError("widths, depths, and channel_tiles must each have length 4")
        if not 0.0 <= drop_path_rate < 1.0:
            raise ValueError("drop_path_rate must be in [0, 1)")
        self.stem_proj = nn.Linear(3 * 4 * 4, widths[0], bias=False)
        res0 = input_size // 4
        resolutions = [res0 // (2 ** i) for i in range(4)]
        self.downsamples = nn.ModuleList(
            nn.Linear(widths[i] * 4, widths[i + 1], bias=False) for i in range(3)
        )
        total = sum(depths)
        rates = [drop_path_rate * i / max(total - 1, 1) for i in range(total)]
        self.stages = nn.ModuleList()
        offset = 0
        for i in range(4):
            self.stages.append(_Stage(
                height=resolutions[i], width=resolutions[i], dim=widths[i], depth=depths[i],
                channel_tile=channel_tiles[i], expansion=expansion, layer_scale_init=layer_scale_init,
                spatial_tile=spatial_tile, use_anchor=(i + 1) in anchor_stages, backend=backend,
                drop_path_rates=rates[offset:offset + depths[i]],
            ))
            offset += depths[i]
        self.head = nn.Linear(widths[-1], num_classes)
        self._widths = widths
        self._entry_cache: dict[int, tuple[tuple, Tensor]] = {}

    def _entry_weight(self, i: int) -> Tensor:
        """Weight of the Linear that enters stage ``i`` (> 0) from the previous stage's
        space_to_depth output: the downsample, with the stage's anchor folded in when it has
        one — both are bias-free, so ``anchor(downsample(x)) = x (W_a W_ds)^T``; the product is
        formed in fp32 and rounded once.  Cached while both weights are unchanged."""
        w_ds = self.downsamples[i - 1].weight
        anchor = self.stages[i].anchor
        if anchor is None:
            return w_ds
        w_a = anchor.weight
        key = tuple((t.data_ptr(), t.dtype, t.device, t._version) for t in (w_ds, w_a))
        hit = self._entry_cache.get(i)
        if hit is None or hit[0] != key:
            with torch.no_grad():
                fused = (w_a.float() @ w_ds.float()).to(w_ds.dtype)
            hit = (key, fused)
            self._entry_cache[i] = hit
        return hit[1]

    def _hip_glue(self, x: Tensor) -> bool:
        """Inference with every block on the hip backend: run the stem and the block before each
        downsample as the fused kernels (``stem_hip``, ``OmniWeaveBlock.forward_s2d``)."""
        if torch.is_grad_enabled() or not x.is_cuda:
            return False
        return all(blk.backend in ("hip", "auto") for stage in self.stages for blk in stage.blocks)

    def _stem(self, x: Tensor) -> Tensor:
        """NCHW image -> NHWC stem features (backbone.py:173-176)."""
        if self._hip_glue(x) and stem_is_supported(x, self.stem_proj.weight)[0]:
            return stem_hip(x, self.stem_proj.weight)
        return self.stem_proj(space_to_depth_nhwc(x.permute(0, 2, 3, 1), 4))

    def forward_features(self, x: Tensor) -> OrderedDict[str, Tensor]:
        """NCHW image -> OrderedDict ``stage1..stage4`` of NHWC feature maps (backbone.py:165-189)."""
        x = self._stem(x)
        features: OrderedDict[str, Tensor] = OrderedDict()
        for i, stage in enumerate(self.stages):
            x = stage(x)
            features[f"stage{i + 1}"] = x
            if i < 3:
                x = space_to_depth_nhwc(x, 2)
                x = self.downsamples[i](x)
        return features

    def forward(self, x: Tensor) -> Tensor:
        """NCHW image -> logits (backbone.py:191-197).  Under ``torch.no_grad`` /
        ``inference_mode`` with the blocks on the hip backend, the stem and each stage's last
        block write the layout the next Linear reads, so no space_to_depth copy is made, and a
        stage's anchor Linear is folded into the downsample before it (``_entry_weight``)."""
        if not self._hip_glue(x):
            stage4 = self.forward_features(x)["stage4"]
            return self.head(stage4.mean(dim=(1, 2)))
        x = self._stem(x)
        for i, stage in enumerate(self.stages):
            if i > 0:  # downsample (+ anchor) on the previous stage's space_to_depth output
                x = F.linear(x, self._entry_weight(i))
            elif stage.anchor is not None:
                x = stage.anchor(x)
            if i < 3:
                x = stage.forward_blocks_s2d(x, 2)
            else:
                x = stage.forward_blocks(x)
        return self.head(x.mean(dim=(1, 2)))
