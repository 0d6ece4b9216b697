"""CPU check of the backward decomposition the HIP kernels implement.

The HIP backward forms gradients for folded operands (B_u'' = -log2(e) w B_u,
B_v'' = -ln(2) w B_v, B_o'' = B_o diag(gamma), gate U'V' / (1 + 2^U')) and maps them back to
the parameters.  Here the same steps run in fp64 with torch on the CPU, per 16-row tile, and
are compared with torch.autograd of the oracle block: a wrong folding constant, gate
derivative or RMSNorm term fails this before any GPU run.
"""

from __future__ import annotations

import math

import pytest
import torch

from oracle.bigemm import block_reference, rel_l2
from oracle.routing import build_route_plan

LOG2E = 1.0 / math.log(2.0)
LN2 = math.log(2.0)


def decomposed_backward(x, plan, p, dy, eps):
    """Every gradient of x + bigemm(RMSNorm(x)) by the folded decomposition (fp64)."""
    b, h, w, c = x.shape
    n = h * w
    tok, ch = plan.token_indices, plan.channel_indices
    q_s, q_c, d = tok.shape[0], ch.shape[0], ch.shape[1]
    xf = x.reshape(b, n, c)
    r = torch.rsqrt(xf.square().mean(-1) + eps)  # [b, n]
    valid_ch = ch < c
    chc = ch.clamp_max(c - 1)
    wv = p["norm_weight"][chc] * valid_ch            # [q_c, d]
    gv = p["gamma"][chc] * valid_ch
    bu = -LOG2E * wv[:, :, None] * p["b_u"]
    bv = -LN2 * wv[:, :, None] * p["b_v"]
    bo = p["b_o"] * gv[:, None, :]
    # Gather X' = x r and dY into tiles [b, q_s, q_c, 16, d].
    xt = torch.zeros(b, q_s, q_c, 16, d, dtype=x.dtype)
    dyt = torch.zeros_like(xt)
    dyf = dy.reshape(b, n, c)
    for s in range(q_s):
        for i in range(16):
            t = int(tok[s, i])
            if t >= n:
                continue
            for q in range(q_c):
                m = valid_ch[q]
                xt[:, s, q, i, m] = xf[:, t, ch[q, m]] * r[:, t, None]
                dyt[:, s, q, i, m] = dyf[:, t, ch[q, m]]
    a_u, a_v, a_o = p["a_u"], p["a_v"], p["a_o"]
    pu = torch.einsum("ij,bsqjk->bsqik", a_u, xt)
    pv = torch.einsum("ij,bsqjk->bsqik", a_v, xt)
    u = torch.einsum("bsqik,qke->bsqie", pu, bu)
    v = torch.einsum("bsqik,qke->bsqie", pv, bv)
    sg = 1.0 / (1.0 + torch.exp2(u))
    z = u * v * sg
    dw = torch.einsum("ji,bsqjk->bsqik", a_o, dyt)
    dz = torch.einsum("bsqik,qek->bsqie", dw, bo)
    du = dz * v * sg * (1.0 - LN2 * u * (1.0 - sg))
    dv = dz * u * sg
    d_bu = torch.einsum("bsqik,bsqie->qke", pu, du)
    d_bv = torch.einsum("bsqik,bsqie->qke", pv, dv)
    d_bo = torch.einsum("bsqie,bsqik->qek", z, dw)
    wp = torch.einsum("bsqie,qek->bsqik", z, bo)
    dpu = torch.einsum("bsqie,qke->bsqik", du, bu)
    dpv = torch.einsum("bsqie,qke->bsqik", dv, bv)
    g_au = torch.einsum("bsqik,bsqjk->ij", dpu, xt)
    g_av = torch.einsum("bsqik,bsqjk->ij", dpv, xt)
    g_ao = torch.einsum("bsqik,bsqjk->ij", dyt, wp)
    dxt = torch.einsum("ji,bsqjk->bsqik", a_u, dpu) + torch.einsum("ji,bsqjk->bsqik", a_v, dpv)
    g = torch.zeros(b, n, c, dtype=x.dtype)
    for s in range(q_s):
        for i in range(16):
            t = int(tok[s, i])
            if t >= n:
                continue
            for q in range(q_c):
                m = valid_ch[q]
                g[:, t, ch[q, m]] = dxt[:, s, q, i, m]
    coef = (g * xf).sum(-1) * r ** 3 / c
    dx = dyf + r[..., None] * g - coef[..., None] * xf
    g_bu = d_bu * (-LOG2E) * wv[:, :, None]
    g_bv = d_bv * (-LN2) * wv[:, :, None]
    g_bo = d_bo * gv[:, None, :]
    per_gamma = (d_bo * p["b_o"]).sum(1)                                    # [q_c, d]
    per_w = (-LOG2E * d_bu * p["b_u"] - LN2 * d_bv * p["b_v"]).sum(2)      # [q_c, d]
    g_gamma = torch.zeros(c, dtype=x.dtype)
    g_nw = torch.zeros(c, dtype=x.dtype)
    g_gamma[ch[valid_ch]] = per_gamma[valid_ch]
    g_nw[ch[valid_ch]] = per_w[valid_ch]
    return {"x": dx.reshape(b, h, w, c), "a_u": g_au, "a_v": g_av, "a_o": g_ao, "b_u": g_bu, "b_v": g_bv,
            "b_o": g_bo, "gamma": g_gamma, "norm_weight": g_nw}


@pytest.mark.parametrize("h,w,c,d,route,level", [
    (8, 8, 128, 64, "shifted", 0),
    (7, 9, 96, 64, "radix", 2),
    (8, 8, 256, 128, "local", 0),
])
def test_decomposition_matches_autograd(h, w, c, d, route, level) -> None:
    gen = torch.Generator().manual_seed(0)
    plan = build_route_plan(h, w, c, 16, d, route, level)
    q_c, rd, b = plan.channel_indices.shape[0], 2 * d, 2
    dt = torch.float64
    x = torch.randn(b, h, w, c, generator=gen, dtype=dt)
    p = {
        "a_u": torch.randn(16, 16, generator=gen, dtype=dt) / 4,
        "a_v": torch.randn(16, 16, generator=gen, dtype=dt) / 4,
        "a_o": torch.randn(16, 16, generator=gen, dtype=dt) / 4,
        "b_u": torch.randn(q_c, d, rd, generator=gen, dtype=dt) / d ** 0.5,
        "b_v": torch.randn(q_c, d, rd, generator=gen, dtype=dt) / d ** 0.5,
        "b_o": torch.randn(q_c, rd, d, generator=gen, dtype=dt) / rd ** 0.5,
        "gamma": torch.rand(c, generator=gen, dtype=dt) + 0.5,
        "norm_weight": torch.rand(c, generator=gen, dtype=dt) + 0.5,
    }
    dy = torch.randn(b, h, w, c, generator=gen, dtype=dt)
    xs = x.clone().requires_grad_(True)
    ps = {k: v.clone().requires_grad_(True) for k, v in p.items()}
    block_reference(xs, plan, ps, eps=1e-6, residual=True).backward(dy)
    want = {k: v.grad for k, v in ps.items()}
    want["x"] = xs.grad
    got = decomposed_backward(x, plan, p, dy, 1e-6)
    for k in want:
        # 1e-6, not fp64 round-off: the oracle RMSNorm accumulates its variance in fp32.
        assert rel_l2(got[k], want[k]) < 1e-6, k


def test_cast_group_one_buffer_and_fallback() -> None:
    """The parameter gradients are cast per dtype group: views of one buffer with one cast, or
    tensor by tensor (separate storages, mixed dtypes); values and shapes as a plain .to()."""
    from omniwave_amd.backward import _cast_group

    buf = torch.randn(3, 256)
    views = tuple(buf[m].view(16, 16) for m in range(3))
    out = _cast_group(views, (torch.bfloat16,) * 3)
    assert all(o.shape == (16, 16) and o.dtype == torch.bfloat16 for o in out)
    assert all(torch.equal(o, v.to(torch.bfloat16)) for o, v in zip(out, views))
    assert out[0].untyped_storage().data_ptr() == out[2].untyped_storage().data_ptr()
    sep = tuple(torch.randn(4, 5) for _ in range(3))
    out = _cast_group(sep, (torch.bfloat16, torch.float16, torch.float32))
    assert [o.dtype for o in out] == [torch.bfloat16, torch.float16, torch.float32]
    assert all(torch.equal(o, s.to(o.dtype)) for o, s in zip(out, sep))


def test_native_batch_limit_and_chunks() -> None:
    """The 16-bit backward kernels address every buffer with 32-bit byte offsets: the largest
    batch of one pass keeps x / dy / g and each [q_c, slots, rd] intermediate below 2 GiB, and
    larger batches are cut into chunks no larger than that."""
    from omniwave_amd.backward import batch_chunks, native_batch_limit
    from omniwave_amd.routing import build_route_plan

    s1 = build_route_plan(56, 56, 128, 16, 64, "shifted", 0)
    s3 = build_route_plan(14, 14, 512, 16, 128, "shifted", 0)
    lim1 = native_batch_limit(torch.bfloat16, s1, 2, 64, 128)
    lim3 = native_batch_limit(torch.float16, s3, 4, 128, 256)
    assert lim1 == 1337 and 2 * 196 * 16 * 128 * 2 * lim1 < 2 ** 31 <= 2 * 196 * 16 * 128 * 2 * (lim1 + 1)
    assert lim3 == 5041 and 4 * 13 * 16 * 256 * 2 * lim3 < 2 ** 31 <= 4 * 13 * 16 * 256 * 2 * (lim3 + 1)
    assert native_batch_limit(torch.float32, s1, 2, 64, 128) is None
    assert batch_chunks(128, lim1, 196) == [(0, 128)]
    assert batch_chunks(1400, lim1, 196) == [(0, 700), (700, 1400)]
    chunks = batch_chunks(4000, lim1, 196)
    assert chunks[0][0] == 0 and chunks[-1][1] == 4000 and all(e - s <= lim1 for s, e in chunks)
    assert all(chunks[i][1] == chunks[i + 1][0] for i in range(len(chunks) - 1))
    # odd Q_s (13 at 14x14): even chunk sizes keep each chunk's slot count a multiple of 32
    assert batch_chunks(11, 5, 13) == [(0, 4), (4, 8), (8, 11)]
    assert batch_chunks(7, None, 13) == [(0, 7)]
