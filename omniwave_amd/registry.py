"""Model registry: ``create_model('omniweave_t')`` (omniweave/models/registry.py:12-81).

The backbone's ``backend`` defaults to ``"auto"``, which resolves to the fused HIP kernels on
a gfx950 GPU.
"""

from __future__ import annotations

from pathlib import Path
from typing import Any

import torch.nn as nn
import yaml

from omniwave_amd.backbone import OmniWeaveBackbone

_REGISTRY: dict[str, dict[str, Any]] = {
    "omniweave_t": {
        "widths": [128, 256, 512, 1024],
        "depths": [2, 3, 8, 2],
        "channel_tiles": [64, 64, 128, 128],
        "expansion": 2,
        "layer_scale_init": 1e-5,
        "anchor_stages": [3, 4],
    },
}

_REQUIRED_MODEL_KEYS = frozenset({"name", "widths", "depths", "spatial_tile", "channel_tiles", "expansion",
                                  "layer_scale_init", "num_classes"})
_VALID_SPATIAL_TILES = frozenset({8, 16, 32})


def create_model(name: str, pretrained: bool = False, **kwargs: Any) -> nn.Module:
    """Create a registered model; kwargs override the registry defaults (registry.py:30-61)."""
    if pretrained:
        raise NotImplementedError(
            "pretrained weights are not yet available; supply an explicit checkpoint path instead"
        )
    if name not in _REGISTRY:
        raise ValueError(f"unknown model: {name!r}; available: {sorted(_REGISTRY)}")
    defaults = _REGISTRY[name].copy()
    defaults.update(kwargs)
    return OmniWeaveBackbone(**defaults)


def omniweave_t(pretrained: bool = False, **kwargs: Any) -> nn.Module:
    for key in ("cache_dir", "pretrained_cfg", "pretrained_cfg_overlay"):
        kwargs.pop(key, None)
    return create_model("omniweave_t", pretrained=pretrained, **kwargs)


def validate_model_config(cfg: dict[str, Any]) -> None:
    """Model-section checks of omniweave/utils/config.py:42-66."""
    model = cfg.get("model")
    if not isinstance(model, dict):
        raise ValueError("configuration must contain a model mapping")
    missing = sorted(_REQUIRED_MODEL_KEYS - set(model))
    if missing:
        raise ValueError(f"missing model keys: {missing}")
    widths, depths, tiles = list(model["widths"]), list(model["depths"]), list(model["channel_tiles"])
    if not (len(widths) == len(depths) == len(tiles) == 4):
        raise ValueError("widths, depths, and channel_tiles must have the same length of four")
    if int(model["spatial_tile"]) not in _VALID_SPATIAL_TILES:
        raise ValueError("spatial_tile must be one of 8, 16, or 32")
    for width, tile in zip(widths, tiles, strict=True):
        if int(width) % int(tile) != 0:
            raise ValueError(f"stage width {width} is not divisible by channel tile {tile}")


def create_model_from_config(config_path: str | Path, **kwargs: Any) -> nn.Module:
    """Build a backbone from a YAML file's ``model`` section (registry.py:71-81)."""
    with Path(config_path).open("r", encoding="utf-8") as handle:
        cfg = yaml.safe_load(handle)
    if not isinstance(cfg, dict):
        raise ValueError("configuration root must be a mapping")
    validate_model_config(cfg)
    model_cfg = dict(cfg["model"])
    model_cfg.pop("name")
    model_cfg.update(kwargs)
    return OmniWeaveBackbone(**model_cfg)
