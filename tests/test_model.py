"""Block and backbone structure on CPU (mirrors the reference's tests/test_model.py), with the
oracle registered as the ``"reference"`` backend."""

from __future__ import annotations

import pytest
import torch

from omniwave_amd import create_model, create_model_from_config
from omniwave_amd.backbone import OmniWeaveBackbone, space_to_depth_nhwc
from omniwave_amd.block import OmniWeaveBlock

SMALL = dict(widths=[32, 64, 128, 256], depths=[1, 1, 1, 1], channel_tiles=[32, 32, 64, 64], input_size=32)


@pytest.mark.parametrize("route,level", [("shifted", 0), ("local", 0), ("radix", 1)])
def test_block_preserves_shape(oracle_backend, route, level) -> None:
    block = OmniWeaveBlock(height=8, width=8, dim=128, channel_tile=64, route=route, radix_level=level,
                           expansion=2, backend="reference")
    x = torch.randn(2, 8, 8, 128)
    out = block(x)
    assert out.shape == x.shape
    assert not torch.equal(out, x)


def test_backbone_feature_shapes(oracle_backend) -> None:
    model = OmniWeaveBackbone(backend="reference")
    outputs = model.forward_features(torch.randn(1, 3, 224, 224))
    assert [tuple(x.shape) for x in outputs.values()] == [
        (1, 56, 56, 128), (1, 28, 28, 256), (1, 14, 14, 512), (1, 7, 7, 1024),
    ]


def test_backbone_classification_auto_on_cpu(oracle_backend) -> None:
    model = create_model("omniweave_t", **SMALL)
    assert model(torch.randn(2, 3, 32, 32)).shape == (2, 1000)


def test_parameter_count_target() -> None:
    count = sum(p.numel() for p in OmniWeaveBackbone().parameters())
    assert count == 10_232_040  # derived for the OmniWeave-T defaults; reference target 10M-20M
    assert 10_000_000 <= count <= 20_000_000


def test_state_dict_names_match_reference_layout() -> None:
    names = set(OmniWeaveBackbone(**SMALL).state_dict())
    for key in ("stem_proj.weight", "downsamples.0.weight", "stages.2.anchor.weight", "head.bias",
                "stages.0.blocks.0.norm_weight", "stages.0.blocks.0.a_u", "stages.0.blocks.0.b_o",
                "stages.3.blocks.0.gamma"):
        assert key in names


def test_anchor_stages_can_be_disabled() -> None:
    model = OmniWeaveBackbone(**{**SMALL, "anchor_stages": []})
    assert all(stage.anchor is None for stage in model.stages)


def test_backbone_gradient_flows(oracle_backend) -> None:
    model = OmniWeaveBackbone(**SMALL, num_classes=10, backend="reference")
    x = torch.randn(1, 3, 32, 32, requires_grad=True)
    model(x).sum().backward()
    assert x.grad is not None and x.grad.abs().sum() > 0


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_block_preserves_amp_input_dtype(dtype, monkeypatch) -> None:
    observed = {}

    def capture(*, x, **_):
        observed["dtype"] = x.dtype
        return torch.zeros_like(x)

    monkeypatch.setattr("omniwave_amd.block.bigemm", capture)
    block = OmniWeaveBlock(height=8, width=8, dim=16, channel_tile=8, route="local", radix_level=0)
    x = torch.randn(1, 8, 8, 16, dtype=dtype)
    assert block(x).dtype == dtype
    assert observed["dtype"] == dtype


def test_drop_path_schedule_is_linear() -> None:
    model = OmniWeaveBackbone(widths=[16, 32, 64, 128], depths=[1, 2, 1, 1], channel_tiles=[8, 8, 16, 16],
                              input_size=32, drop_path_rate=0.2)
    rates = [b.drop_path_rate for s in model.stages for b in s.blocks]
    torch.testing.assert_close(torch.tensor(rates), torch.linspace(0.0, 0.2, len(rates)))


def test_space_to_depth_layout() -> None:
    x = torch.arange(2 * 4 * 4 * 3).reshape(2, 4, 4, 3)
    y = space_to_depth_nhwc(x, 2)
    assert y.shape == (2, 2, 2, 12)
    # output channel (i*f + j)*C + c holds x[b, 2r+i, 2s+j, c]
    assert y[1, 1, 0, (1 * 2 + 0) * 3 + 2] == x[1, 3, 0, 2]
    with pytest.raises(ValueError):
        space_to_depth_nhwc(torch.zeros(1, 5, 4, 3), 2)


def test_create_model_errors() -> None:
    with pytest.raises(ValueError, match="unknown model"):
        create_model("resnet50")
    with pytest.raises(NotImplementedError):
        create_model("omniweave_t", pretrained=True)


def test_create_model_from_config(tmp_path) -> None:
    cfg = tmp_path / "m.yaml"
    cfg.write_text(
        "model:\n  name: omniweave_t\n  widths: [32, 64, 128, 256]\n  depths: [1, 1, 1, 1]\n"
        "  spatial_tile: 16\n  channel_tiles: [32, 32, 64, 64]\n  expansion: 2\n"
        "  layer_scale_init: 1.0e-5\n  num_classes: 10\n  input_size: 32\n"
    )
    model = create_model_from_config(cfg)
    assert model.head.out_features == 10
    bad = tmp_path / "bad.yaml"
    bad.write_text(cfg.read_text().replace("spatial_tile: 16", "spatial_tile: 12"))
    with pytest.raises(ValueError, match="spatial_tile"):
        create_model_from_config(bad)
