"""Oracle BiGEMM: CPU restatement of the reference backend (test infrastructure only).

``pack_tiles``, ``unpack_tiles`` and ``bigemm_delta_reference`` restate
``omniweave/ops/reference.py:16-173``; ``rmsnorm_reference`` and ``block_reference`` restate
``omniweave/models/block.py:80-108``.  ``bigemm_delta_bruteforce`` is an fp64 per-tile loop
that shares no code with the pack/einsum path; tests use it to pin the oracle.
"""

from __future__ import annotations

import numpy as np
import torch
import torch.nn.functional as F
from torch import Tensor


def pack_tiles(x: Tensor, plan) -> tuple[Tensor, Tensor]:
    """omniweave/ops/reference.py:16-64: NHWC -> tiles [B,Q_s,Q_c,g,d] and mask [1,Q_s,Q_c,g,d]."""
    b, h, w, c = x.shape
    n = h * w
    flat = x.reshape(b, n, c)
    flat = torch.cat([flat, flat.new_zeros(b, 1, c)], dim=1)
    flat = torch.cat([flat, flat.new_zeros(b, n + 1, 1)], dim=2)
    tok_idx = plan.token_indices
    q_s, g = tok_idx.shape
    tok = tok_idx.reshape(1, q_s * g, 1).expand(b, -1, c + 1).to(flat.device)
    gathered = torch.gather(flat, 1, tok).reshape(b, q_s, g, c + 1)
    ch_idx = plan.channel_indices
    q_c, d = ch_idx.shape
    ch = ch_idx.reshape(1, 1, 1, q_c * d).expand(b, q_s, g, -1).to(gathered.device)
    tiles = torch.gather(gathered, 3, ch)
    tiles = tiles.reshape(b, q_s, g, q_c, d).permute(0, 1, 3, 2, 4)
    tok_mask = plan.token_mask.to(x.device)
    ch_mask = plan.channel_mask.to(x.device)
    mask = (tok_mask.unsqueeze(1).unsqueeze(-1) & ch_mask.unsqueeze(0).unsqueeze(2)).unsqueeze(0)
    return tiles * mask.to(tiles.dtype), mask


def unpack_tiles(tiles: Tensor, plan, batch_size: int) -> Tensor:
    """omniweave/ops/reference.py:67-117: tiles -> NHWC (scatter; maps are permutations)."""
    b = batch_size
    h, w, c = plan.height, plan.width, plan.channels
    n = h * w
    q_s, g = plan.token_indices.shape
    q_c, d = plan.channel_indices.shape
    output = tiles.new_zeros(b, n + 1, c + 1)
    spatial = tiles.permute(0, 1, 3, 2, 4).reshape(b, q_s, g, q_c * d)
    ch_flat = plan.channel_indices.to(tiles.device).reshape(q_c * d)
    inter = tiles.new_zeros(b, q_s, g, c + 1)
    inter.scatter_add_(3, ch_flat.reshape(1, 1, 1, q_c * d).expand(b, q_s, g, -1), spatial)
    tok_flat = plan.token_indices.to(tiles.device).reshape(q_s * g)
    output.scatter_add_(
        1, tok_flat.reshape(1, q_s * g, 1).expand(b, -1, c + 1), inter.reshape(b, q_s * g, c + 1)
    )
    return output[:, :n, :c].reshape(b, h, w, c)


def bigemm_delta_reference(*, x, plan, a_u, a_v, a_o, b_u, b_v, b_o, gamma) -> Tensor:
    """omniweave/ops/reference.py:120-173: delta = gamma * mask * A_o (SiLU(A_u T B_u) * (A_v T B_v)) B_o.

    The einsums contract left to right (no opt_einsum), as in the reference, so in bf16 the
    rounding points are (A T), (A T) B, SiLU, the gate product, (A_o Z), (A_o Z) B_o, mask
    and LayerScale.
    """
    tiles, mask = pack_tiles(x, plan)
    b, q_s, q_c, g, d = tiles.shape
    flat = tiles.reshape(b * q_s, q_c, g, d)
    u = torch.einsum("ij,bqjk,qke->bqie", a_u, flat, b_u)
    v = torch.einsum("ij,bqjk,qke->bqie", a_v, flat, b_v)
    z = F.silu(u) * v
    delta = torch.einsum("ij,bqje,qed->bqid", a_o, z, b_o)
    delta = delta.reshape(b, q_s, q_c, g, d) * mask.to(delta.dtype)
    ch_idx = plan.channel_indices.clamp_max(plan.channels - 1).to(gamma.device)
    ch_mask = plan.channel_mask.to(gamma.device, gamma.dtype)
    grouped_gamma = gamma[ch_idx] * ch_mask
    delta = delta * grouped_gamma[None, None, :, None, :]
    return unpack_tiles(delta, plan, b)


def rmsnorm_reference(x: Tensor, norm_weight: Tensor, eps: float = 1e-6) -> Tensor:
    """omniweave/models/block.py:83-85, including its dtype sequence.

    ``var`` is accumulated in fp32, rounded to ``x.dtype`` before ``+ eps`` and ``rsqrt``;
    the scaled value is rounded to ``x.dtype`` before and after the weight multiply.
    """
    variance = x.float().square().mean(dim=-1, keepdim=True)
    normalized = x * torch.rsqrt(variance.to(x.dtype) + eps)
    return (normalized * norm_weight).to(x.dtype)


def block_reference(x, plan, params: dict, eps: float = 1e-6, residual: bool = True) -> Tensor:
    """omniweave/models/block.py:80-108 in eval mode (no drop-path): x + bigemm(RMSNorm(x))."""
    normalized = rmsnorm_reference(x, params["norm_weight"], eps)
    delta = bigemm_delta_reference(
        x=normalized, plan=plan,
        a_u=params["a_u"], a_v=params["a_v"], a_o=params["a_o"],
        b_u=params["b_u"], b_v=params["b_v"], b_o=params["b_o"],
        gamma=params["gamma"],
    )
    return x + delta if residual else delta


def bigemm_delta_bruteforce(x, token_indices, channel_indices, a_u, a_v, a_o, b_u, b_v, b_o, gamma):
    """fp64 per-tile brute force (numpy), independent of pack/einsum/unpack.

    For every tile (b, q_s, q_c): gather T[i, k] = x[b, tok[q_s, i], ch[q_c, k]] (zero for pad
    indices), evaluate A_o (SiLU(A_u T B_u) * (A_v T B_v)) B_o with explicit matrix products,
    scale column k by gamma[ch[q_c, k]] and write valid rows/columns back.  Small inputs only.
    """
    x = np.asarray(x, dtype=np.float64)
    b, h, w, c = x.shape
    n = h * w
    flat = x.reshape(b, n, c)
    tok = np.asarray(token_indices)
    ch = np.asarray(channel_indices)
    a_u, a_v, a_o = (np.asarray(t, dtype=np.float64) for t in (a_u, a_v, a_o))
    b_u, b_v, b_o = (np.asarray(t, dtype=np.float64) for t in (b_u, b_v, b_o))
    gamma = np.asarray(gamma, dtype=np.float64)
    out = np.zeros((b, n, c), dtype=np.float64)
    q_s, g = tok.shape
    q_c, d = ch.shape
    for bi in range(b):
        for s in range(q_s):
            for qc in range(q_c):
                t = np.zeros((g, d))
                for i in range(g):
                    if tok[s, i] >= n:
                        continue
                    for k in range(d):
                        if ch[qc, k] < c:
                            t[i, k] = flat[bi, tok[s, i], ch[qc, k]]
                u = a_u @ t @ b_u[qc]
                v = a_v @ t @ b_v[qc]
                z = (u / (1.0 + np.exp(-u))) * v
                y = a_o @ z @ b_o[qc]
                for i in range(g):
                    if tok[s, i] >= n:
                        continue
                    for k in range(d):
                        if ch[qc, k] < c:
                            out[bi, tok[s, i], ch[qc, k]] = y[i, k] * gamma[ch[qc, k]]
    return out.reshape(b, h, w, c)


def rel_l2(actual: Tensor, expected: Tensor) -> float:
    """||actual - expected||_2 / ||expected||_2 in fp64."""
    a = actual.detach().double().cpu()
    e = expected.detach().double().cpu()
    den = e.norm().item()
    return (a - e).norm().item() / (den if den > 0 else 1.0)
