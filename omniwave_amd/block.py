"""OmniWeave block: RMSNorm -> BiGEMM -> residual (omniweave/models/block.py:15-108).

Parameter names, shapes and initialisation match the reference so state_dicts interchange.
When the resolved backend is ``hip`` the whole block runs as one fused kernel
(``bigemm_block_hip``); otherwise RMSNorm runs here and ``bigemm`` (a module-level import, so
callers can patch ``omniwave_amd.block.bigemm``) computes the delta.
"""

from __future__ import annotations

import math

import torch
import torch.nn as nn
from torch import Tensor

from omniwave_amd.bigemm import bigemm
from omniwave_amd.hip import (bigemm_block_chain_hip, bigemm_block_hip, bigemm_block_s2d_hip, drop_path_scale,
                              hip_is_supported)
from omniwave_amd.routing import RoutePlan, build_route_plan

RMS_EPS = 1e-6  # omniweave/models/block.py:84


class OmniWeaveBlock(nn.Module):
    """One OmniWeave block; owns one route plan and returns ``x + delta``."""

    def __init__(
        self,
        height: int,
        width: int,
        dim: int,
        channel_tile: int,
        route: str,
        radix_level: int,
        expansion: int = 2,
        layer_scale_init: float = 1e-5,
        spatial_tile: int = 16,
        backend: str = "auto",
        drop_path_rate: float = 0.0,
    ) -> None:
        super().__init__()
        if not 0.0 <= drop_path_rate < 1.0:
            raise ValueError("drop_path_rate must be in [0, 1)")
        self.height = height
        self.width = width
        self.dim = dim
        self.backend = backend
        self.drop_path_rate = drop_path_rate
        g = spatial_tile
        d = channel_tile
        rd = d * expansion
        q_c = math.ceil(dim / d)
        self.plan: RoutePlan = build_route_plan(height, width, dim, g, d, route, radix_level)
        self.norm_weight = nn.Parameter(torch.ones(dim))
        self.a_u = nn.Parameter(torch.empty(g, g))
        self.a_v = nn.Parameter(torch.empty(g, g))
        self.a_o = nn.Parameter(torch.empty(g, g))
        self.b_u = nn.Parameter(torch.empty(q_c, d, rd))
        self.b_v = nn.Parameter(torch.empty(q_c, d, rd))
        self.b_o = nn.Parameter(torch.empty(q_c, rd, d))
        self.gamma = nn.Parameter(torch.full((dim,), layer_scale_init))
        self.fp8 = False  # e4m3fn channel side (inference with the hip backend); see enable_fp8
        self._init_weights()

    def _init_weights(self) -> None:
        """omniweave/models/block.py:72-78."""
        nn.init.orthogonal_(self.a_u)
        nn.init.orthogonal_(self.a_v)
        nn.init.eye_(self.a_o)
        nn.init.xavier_uniform_(self.b_u)
        nn.init.xavier_uniform_(self.b_v)
        nn.init.xavier_uniform_(self.b_o)

    def _fused(self, x: Tensor) -> bool:
        if self.backend not in ("hip", "auto"):
            return False
        ok, reason = hip_is_supported(x, self.plan, self.b_u)
        if not ok and self.backend == "hip":
            raise RuntimeError(reason)
        return ok

    def _drop_path(self, delta: Tensor) -> Tensor:
        """Per-sample stochastic depth in training (omniweave/models/block.py:99-107)."""
        keep = 1.0 - self.drop_path_rate
        shape = (delta.shape[0],) + (1,) * (delta.ndim - 1)
        mask = torch.empty(shape, dtype=delta.dtype, device=delta.device).bernoulli_(keep)
        return delta * mask / keep

    def forward_s2d(self, x: Tensor, factor: int = 2) -> Tensor | None:
        """``space_to_depth(self(x), factor)`` as one kernel — the block writes its output rows
        straight into the ``[B, H/f, W/f, C f^2]`` layout (omniweave/models/backbone.py:14-27,
        183-186) — when nothing needs a gradient and the fused hip path takes ``x`` (bf16 /
        fp16); ``None`` otherwise, and the caller composes the two."""
        if torch.is_grad_enabled() or (self.training and (self.drop_path_rate > 0 or self.fp8)):
            return None
        if x.dtype not in (torch.bfloat16, torch.float16) or not self._fused(x):
            return None
        if x.shape[1] % factor or x.shape[2] % factor:
            return None
        params = (self.a_u, self.a_v, self.a_o, self.b_u, self.b_v, self.b_o, self.gamma)
        return bigemm_block_s2d_hip(x, self.norm_weight, self.plan, *params, factor=factor, eps=RMS_EPS,
                                    fp8=self.fp8)

    def forward_chain(self, x: Tensor, stats: Tensor | None, factor: int = 0) -> tuple[Tensor, Tensor | None] | None:
        """``self(x)`` (factor 0) or ``forward_s2d(x, factor)`` for a block of a stage's chain
        (inference): returns ``(y, stats)``, ``stats`` being the RMSNorm statistics of ``y`` for
        the next block (or None), given ``stats`` of ``x`` from the previous block; ``None``
        when the chained hip path does not apply and the caller uses the plain calls."""
        if torch.is_grad_enabled() or (self.training and (self.drop_path_rate > 0 or self.fp8)):
            return None
        if x.dtype not in (torch.bfloat16, torch.float16) or not self._fused(x):
            return None
        if factor and (x.shape[1] % factor or x.shape[2] % factor):
            return None
        params = (self.a_u, self.a_v, self.a_o, self.b_u, self.b_v, self.b_o, self.gamma)
        return bigemm_block_chain_hip(x, stats, self.norm_weight, self.plan, *params, factor=factor, eps=RMS_EPS,
                                      fp8=self.fp8)

    def forward(self, x: Tensor) -> Tensor:
        """``x``: ``[B, H, W, C]`` -> ``[B, H, W, C]``."""
        params = (self.a_u, self.a_v, self.a_o, self.b_u, self.b_v, self.b_o, self.gamma)
        dropping = self.training and self.drop_path_rate > 0
        fused = self._fused(x)
        if self.fp8:
            if self.training:
                raise RuntimeError("the fp8 BiGEMM variant is inference-only; call model.eval()")
            if not fused:
                raise RuntimeError("the fp8 BiGEMM variant needs the hip backend on a gfx950 GPU")
            return bigemm_block_hip(x, self.norm_weight, self.plan, *params, eps=RMS_EPS, fp8=True)
        if fused:
            # Drop-path (block.py:99-107) fused: the kernel scales each image's rounded delta
            # before the residual; the keep mask is drawn as the reference draws it.
            scale = drop_path_scale(x.shape[0], self.drop_path_rate, x.dtype, x.device) if dropping else None
            return bigemm_block_hip(x, self.norm_weight, self.plan, *params, eps=RMS_EPS, drop_scale=scale)
        variance = x.float().square().mean(dim=-1, keepdim=True)
        normalized = x * torch.rsqrt(variance.to(x.dtype) + RMS_EPS)
        normalized = (normalized * self.norm_weight).to(x.dtype)
        delta = bigemm(
            x=normalized, plan=self.plan,
            a_u=self.a_u, a_v=self.a_v, a_o=self.a_o,
            b_u=self.b_u, b_v=self.b_v, b_o=self.b_o,
            gamma=self.gamma, backend=self.backend,
        )
        if dropping:
            delta = self._drop_path(delta)
        return x + delta


def enable_fp8(model: nn.Module, enabled: bool = True, min_channel_tile: int = 128) -> nn.Module:
    """Switch the OmniWeaveBlocks of ``model`` whose channel tile is at least
    ``min_channel_tile`` to the fp8-e4m3 channel side (inference with bf16 / fp16 activations on
    the hip backend), or every block back (``enabled=False``); returns ``model``.

    The default leaves d = 64 blocks (OmniWeave-T's stages 1-2) in bf16: their resident-weight
    kernel is bound by VALU work, which fp8 MFMAs do not reduce, and the fp8 variant of those
    shapes runs on the slower streamed kernel.  ``min_channel_tile=64`` switches every block.
    """
    for module in model.modules():
        if isinstance(module, OmniWeaveBlock):
            module.fp8 = enabled and int(module.b_u.shape[1]) >= min_channel_tile
    return model
