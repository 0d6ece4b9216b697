"""Backward of the fused BiGEMM block (dX, dA_u/v/o, dB_u/v/o, dgamma, dnorm_weight).

Replaces the fp32 autograd recompute of the accelerated backend
(omniweave/ops/triton.py:256-292).  The pass runs in the forward's compute dtype with fp32
accumulation, entirely on the HIP stream of the gradient:

* routing, RMSNorm, gate and parameter fold-back are the libomniwave_amd.so kernels
  (``ow_bwd_gather``, ``ow_bwd_gate``, ``ow_bwd_scatter``, ``ow_bwd_rmsnorm``,
  ``ow_bwd_params``, ``ow_fold_weights``);
* for d = 64 one fused MFMA kernel (``ow_bwd_fused``) does the token side (P_u, P_v, dW', the
  only intermediates it stores), the channel side and gate (U', V', dZ, Z, dU', dV', W', dP_u,
  dP_v), dX' and the token-matrix gradients (per-workgroup partials); for d = 128 two kernels share that work
  (``ow_bwd_channel``: token side, U', V', dZ and the gate; ``ow_bwd_channel2``: dP_u, dP_v,
  dX', W' and the token-matrix gradients; with the identity channel order their ``_routed``
  forms read x / dy and write dX' straight to the NHWC gradient, so neither the gather nor the
  scatter pass runs);
  otherwise (fp32) the 16x16 token-side products are
  ``ow_tile_mix`` / ``ow_tile_outer`` (16x16x16 MFMA) around plain batched GEMMs over all slots
  of a channel group (``torch.bmm`` -> hipBLASLt, every right operand contiguous) and
  ``ow_bwd_gate``;
* the parameter-gradient reductions over slots: ``ow_bwd_param_reduce64`` from the d = 64 fused
  kernel's P_u, P_v, dW' (recomputing U', V', dZ and the gate), ``ow_bwd_param_reduce128`` over the d = 128 channel
  kernels' slot-major ones (fp32 batched GEMMs for the fp32 path), and every per-workgroup fp32
  partial summed by ``ow_sum_rows`` in a fixed order.

Gradients are formed for the folded operands the forward evaluates (B_u'' = -log2(e) w B_u,
B_v'' = -ln(2) w B_v, B_o'' = B_o diag(gamma), SiLU(U) V = U'V' / (1 + 2^U')) and mapped back
to the parameters by ``ow_bwd_params``.
"""

from __future__ import annotations

import ctypes

import torch
from torch import Tensor

from omniwave_amd import _native
from omniwave_amd.routing import RoutePlan, device_tables, native_plan

_DTYPE_CODE = {torch.float32: _native.OW_DTYPE_F32, torch.bfloat16: _native.OW_DTYPE_BF16,
               torch.float16: _native.OW_DTYPE_F16}
# Waves of ow_tile_outer: each sums a strided share of the tiles into one [16][16] partial;
# about 8 tiles per wave (two in flight per loop step), between 256 and 8192 waves.
_OUTER_TILES_PER_WAVE = 8
_OUTER_WAVES_MIN, _OUTER_WAVES_MAX = 256, 8192


def _outer_waves(n_tiles: int) -> int:
    waves = -(-n_tiles // _OUTER_TILES_PER_WAVE)
    waves = -(-waves // 4) * 4
    return max(_OUTER_WAVES_MIN, min(_OUTER_WAVES_MAX, waves))
# Most slot chunks of a parameter-gradient GEMM (see _slot_reduce).
_SPLITS = 64


def _stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _tile_mix(lib, in1: Tensor, m1: Tensor, in2: Tensor | None, m2: Tensor | None, d: int, code: int,
              stream: int) -> Tensor:
    out = torch.empty_like(in1)
    n_tiles = in1.numel() // (16 * d)
    _native.check(lib.ow_tile_mix(in1.data_ptr(), m1.data_ptr(), in2.data_ptr() if in2 is not None else None,
                                  m2.data_ptr() if m2 is not None else None, out.data_ptr(), n_tiles, d, code,
                                  stream), "ow_tile_mix")
    return out


def _tile_outer(lib, in1: Tensor, in2: Tensor, d: int, code: int, stream: int) -> Tensor:
    n_tiles = in1.numel() // (16 * d)
    n_waves = _outer_waves(n_tiles)
    partial = torch.empty(16, 16, n_waves, dtype=torch.float32, device=in1.device)
    _native.check(lib.ow_tile_outer(in1.data_ptr(), in2.data_ptr(), partial.data_ptr(), n_waves, n_tiles, d,
                                    code, stream), "ow_tile_outer")
    return partial.sum(dim=2)


def _sum_rows(lib, partial: Tensor, rows: int, out: Tensor, stream: int) -> None:
    """out = the sum of the ``rows`` equal-sized row blocks of the fp32 buffer ``partial``
    (``ow_sum_rows``: a fixed summation order, so replays and reruns give identical bits).
    Both buffers are contiguous fp32 and start 16-byte aligned."""
    cols = out.numel()
    assert partial.is_contiguous() and out.is_contiguous() and partial.numel() == rows * cols
    _native.check(lib.ow_sum_rows(partial.data_ptr(), rows, cols, out.data_ptr(), stream), "ow_sum_rows")


def _slot_reduce(a: Tensor, b: Tensor) -> Tensor:
    """sum over slots of a^T b per channel group ([q_c, S, m] x [q_c, S, n] -> fp32 [q_c, m, n]).

    The slot axis (hundreds of thousands long) is split into up to _SPLITS chunks of whole
    tiles that run as separate batch entries of one GEMM, so the launch has q_c * splits
    output blocks instead of q_c; the chunk results leave the GEMM in fp32 (its accumulator
    type: rounding them to bf16 put the sum 1.7e-3 rel-L2 from the exact one, fp32 1e-6) and are
    summed in fp32.  The split count also keeps those fp32 partials within an eighth of the
    operand bytes (16 splits at 14x14x512, 64 at 56x56x128, B = 128).
    """
    q_c, slots, m = a.shape
    n = b.shape[2]
    tiles = slots // 16
    cap = max(1, min(_SPLITS, slots * (m + n) * a.element_size() // (8 * m * n * 4)))
    splits = max(s for s in range(1, min(cap, tiles) + 1) if tiles % s == 0) if tiles else 1
    chunk = slots // splits
    lhs, rhs = a.view(q_c * splits, chunk, m).transpose(1, 2), b.view(q_c * splits, chunk, n)
    if a.dtype == torch.float32:
        part = torch.bmm(lhs, rhs)
    else:
        part = torch.bmm(lhs, rhs, out_dtype=torch.float32)
    return part.view(q_c, splits, m, n).sum(dim=1)


def _fp32(t: Tensor, device) -> Tensor:
    return t.detach().to(device=device, dtype=torch.float32).contiguous()


# The bf16 / fp16 backward kernels address x, dy, g and the [q_c, slots, rd] intermediates with
# 32-bit byte offsets (buffer descriptors): each of those buffers must stay below 2 GiB.
_ADDR_LIMIT = 1 << 31


def native_batch_limit(dtype: torch.dtype, plan: RoutePlan, q_c: int, d: int, rd: int) -> int | None:
    """Largest batch one pass of the 16-bit backward kernels can address (None: no limit).

    Per image, x / dy / g hold H*W*C values and each intermediate (P_u, P_v, dW', Z, dU', dV',
    the gathered tiles) q_c * Q_s * 16 * max(d, rd); the kernels need every buffer below 2 GiB.
    The reference backward (omniweave/ops/reference.py:120-173 through autograd) has no batch
    ceiling, so ``bigemm_backward`` runs larger batches in chunks of at most this many images.
    """
    if dtype == torch.float32:
        return None
    elt = torch.empty((), dtype=dtype).element_size()
    q_s = int(plan.token_indices.shape[0])
    per_image = max(plan.height * plan.width * plan.channels, q_c * q_s * 16 * max(d, rd)) * elt
    return max(1, (_ADDR_LIMIT - 1) // per_image)


def batch_chunks(batch: int, limit: int | None, q_s: int) -> list[tuple[int, int]]:
    """[start, end) image ranges of at most ``limit`` images covering ``batch``, as even in size
    as possible; with an odd Q_s the chunk size is kept even where it can be, so each chunk's
    slot count stays a multiple of 32 (the fused d = 64 kernel)."""
    if limit is None or batch <= limit:
        return [(0, batch)]
    n = -(-batch // limit)
    size = -(-batch // n)
    if q_s % 2 and size % 2 and size > 1:
        size -= 1
    out, s = [], 0
    while s < batch:
        out.append((s, min(batch, s + size)))
        s += size
    return out


def bigemm_backward(grad: Tensor, x: Tensor, norm_weight: Tensor | None, gamma: Tensor, a_u: Tensor, a_v: Tensor,
                    a_o: Tensor, b_u: Tensor, b_v: Tensor, b_o: Tensor, plan: RoutePlan, flags: int, eps: float,
                    drop_scale: Tensor | None = None, row_scale: Tensor | None = None):
    """Gradients of ``bigemm_fwd(x, norm_weight, gamma, a_u, .., b_o, plan, flags, eps, drop_scale)``.

    Returns ``(dx, d_norm_weight, d_gamma, d_a_u, d_a_v, d_a_o, d_b_u, d_b_v, d_b_o)``, each in
    its input's dtype (``d_norm_weight`` is None without OW_FUSE_NORM).  With ``drop_scale``
    (per-image drop-path factors of the forward) the delta branch receives the upstream
    gradient scaled per image and rounded (``ow_scale_samples``), the residual the plain one.
    Batches beyond ``native_batch_limit`` run in chunks: dx per chunk, the parameter gradients
    summed over chunks in fp32 before the cast.  ``row_scale`` ([B * H * W] fp32, or None): the
    RMSNorm row scales the forward applied (``ow_bigemm_fwd_scales``), else formed here.
    """
    fuse_norm = bool(flags & _native.OW_FUSE_NORM)
    q_c, d, rd = b_u.shape
    chunks = batch_chunks(x.shape[0], native_batch_limit(x.dtype, plan, q_c, d, rd),
                          int(plan.token_indices.shape[0]))
    n_tok = plan.height * plan.width
    if row_scale is not None and row_scale.numel() != x.shape[0] * n_tok:
        row_scale = None
    if len(chunks) == 1:
        dx, g_all = _backward_once(grad, x, norm_weight, gamma, a_u, a_v, a_o, b_u, b_v, b_o, plan, flags, eps,
                                   drop_scale, row_scale)
    else:
        dxs, g_all = [], None
        for s, e in chunks:
            dx_c, g_c = _backward_once(grad[s:e], x[s:e], norm_weight, gamma, a_u, a_v, a_o, b_u, b_v, b_o, plan,
                                       flags, eps, drop_scale[s:e] if drop_scale is not None else None,
                                       row_scale[s * n_tok:e * n_tok] if row_scale is not None else None)
            dxs.append(dx_c)
            g_all = g_c if g_all is None else g_all.add_(g_c)
        dx = torch.cat(dxs)
    return _cast_grads(dx, g_all, fuse_norm, plan.channels, q_c, d, rd,
                       norm_weight, gamma, a_u, a_v, a_o, b_u, b_v, b_o)


def _cast_grads(dx, g_all, fuse_norm, channels, q_c, d, rd, norm_weight, gamma, a_u, a_v, a_o, b_u, b_v, b_o):
    """Parameter gradients as views of the fp32 buffer ``g_all`` (the token matrices, B_u, B_v,
    B_o, then gamma and the norm weight), cast to each parameter's dtype: one cast of the whole
    buffer when they share a dtype."""
    nb = q_c * d * rd
    params = ([norm_weight] if fuse_norm else []) + [gamma, a_u, a_v, a_o, b_u, b_v, b_o]

    def views(buf):
        o_a = buf[:768].view(3, 16, 16)
        o_b = buf[768:768 + 3 * nb]
        o_c = buf[768 + 3 * nb:].view(-1, channels)
        return (o_c[1] if fuse_norm else None, o_c[0], o_a[0], o_a[1], o_a[2],
                o_b[:nb].view(q_c, d, rd), o_b[nb:2 * nb].view(q_c, d, rd), o_b[2 * nb:].view(q_c, rd, d))

    if len({t.dtype for t in params}) == 1:
        return (dx, *views(g_all.to(params[0].dtype)))
    g_nw, g_gamma, g_au, g_av, g_ao, g_bu, g_bv, g_bo = views(g_all)
    return (
        dx,
        g_nw.to(norm_weight.dtype) if g_nw is not None else None,
        *_cast_group((g_gamma,), (gamma.dtype,)),
        *_cast_group((g_au, g_av, g_ao), (a_u.dtype, a_v.dtype, a_o.dtype)),
        *_cast_group((g_bu, g_bv, g_bo), (b_u.dtype, b_v.dtype, b_o.dtype)),
    )


def _backward_once(grad: Tensor, x: Tensor, norm_weight: Tensor | None, gamma: Tensor, a_u: Tensor, a_v: Tensor,
                   a_o: Tensor, b_u: Tensor, b_v: Tensor, b_o: Tensor, plan: RoutePlan, flags: int, eps: float,
                   drop_scale: Tensor | None, row_scale: Tensor | None = None):
    """One pass of the kernels over the whole batch: dx and the fp32 parameter-gradient buffer
    (layout of ``_cast_grads``)."""
    lib = _native.lib()
    dev = x.device
    dtype = x.dtype
    code = _DTYPE_CODE[dtype]
    fuse_norm = bool(flags & _native.OW_FUSE_NORM)
    residual = bool(flags & _native.OW_FUSE_RESIDUAL)
    x = x.contiguous()
    grad = grad.to(dtype).contiguous()
    batch = x.shape[0]
    q_c, d, rd = b_u.shape
    q_s = plan.token_indices.shape[0]
    slots = batch * q_s * 16
    n_rows = batch * plan.height * plan.width
    tok, ch = device_tables(plan, dev)
    oplan = native_plan(plan)
    stream = _stream(dev)
    grad_delta = grad  # upstream gradient of the delta branch (drop-path scaled below)

    ws = [w.detach().contiguous() for w in (b_u, b_v, b_o)]
    wdtype = ws[0].dtype
    if any(w.dtype != wdtype for w in ws) or wdtype not in _DTYPE_CODE:
        wdtype = torch.float32
        ws = [w.float() for w in ws]
    # The small fp32 operands (norm weight, gamma, token matrices): one conversion kernel into
    # one buffer (ow_small_to_f32).
    small = ([norm_weight] if fuse_norm else []) + [gamma, a_u, a_v, a_o]
    if all(t.device == dev and t.dtype in _DTYPE_CODE for t in small):
        srcs = [t.detach().contiguous() for t in small]
        counts = [t.numel() for t in srcs]
        flat = torch.empty(sum(counts), dtype=torch.float32, device=dev)
        n = len(srcs)
        _native.check(lib.ow_small_to_f32((ctypes.c_void_p * n)(*[t.data_ptr() for t in srcs]),
                                          (ctypes.c_int32 * n)(*[_DTYPE_CODE[t.dtype] for t in srcs]),
                                          (ctypes.c_int64 * n)(*counts), n, flat.data_ptr(), _stream(dev)),
                      "ow_small_to_f32")
        parts = list(torch.split(flat, counts))
        nw = parts.pop(0) if fuse_norm else None
        gm, au, av, ao = parts[0], parts[1].view(16, 16), parts[2].view(16, 16), parts[3].view(16, 16)
    else:
        nw = _fp32(norm_weight, dev) if fuse_norm else None
        gm = _fp32(gamma, dev)
        au, av, ao = (_fp32(a, dev) for a in (a_u, a_v, a_o))
    # The fp32 parameter gradients in one buffer (the token matrices, B_u, B_v, B_o, then gamma
    # and the norm weight: every block that a kernel sums into starts 16-byte aligned), so that
    # parameters of one dtype are cast back with one kernel.
    n_c = (2 if fuse_norm else 1) * plan.channels
    nb = q_c * d * rd
    g_all = torch.empty(768 + 3 * nb + n_c, dtype=torch.float32, device=dev)
    g_a = g_all[:768].view(3, 256)

    with torch.cuda.device(dev):
        if drop_scale is not None:
            scale = drop_scale.to(device=dev, dtype=torch.float32).contiguous()
            grad_delta = torch.empty_like(grad)
            _native.check(lib.ow_scale_samples(grad.data_ptr(), scale.data_ptr(), grad_delta.data_ptr(), batch,
                                               grad.numel() // max(batch, 1), code, stream), "ow_scale_samples")
        rscale = None
        if fuse_norm and row_scale is not None:
            rscale = row_scale.to(device=dev, dtype=torch.float32).contiguous()  # the forward's own scales
        elif fuse_norm:
            rscale = torch.empty(n_rows, dtype=torch.float32, device=dev)
            _native.check(lib.ow_rms_scale(x.data_ptr(), rscale.data_ptr(), n_rows, plan.channels, eps, code,
                                           stream), "ow_rms_scale")

        fused = d == 64 and slots % 32 == 0 and dtype != torch.float32
        chan128 = d == 128 and dtype != torch.float32
        # The d = 64 fused kernel and the d = 128 channel kernels read x / dy and write g
        # themselves when group q is channels [d q, d q + d) (routing.py:107-121: radix level 0
        # or a single group): no gather and no scatter pass.
        identity = plan.channels == q_c * d and (plan.radix_level == 0 or q_c == 1)
        routed = (fused or chan128) and identity
        g = torch.empty(n_rows, plan.channels, dtype=dtype, device=dev)  # fully written: no clearing
        rs_ptr = rscale.data_ptr() if rscale is not None else None
        if not routed:
            # Routed tiles of X' = x r and of dY.
            xt = torch.empty(q_c, slots, d, dtype=dtype, device=dev)
            dyt = torch.empty_like(xt)
            _native.check(lib.ow_bwd_gather(x.data_ptr(), grad_delta.data_ptr(), rscale.data_ptr() if rscale is not None
                                            else None, tok.data_ptr(), ch.data_ptr(), ctypes.byref(oplan),
                                            batch, code, xt.data_ptr(), dyt.data_ptr(), stream), "ow_bwd_gather")

        if fused:
            # One fused kernel: token side, channel side and gate, dX', and the token-matrix
            # gradients as per-workgroup partials.
            nbytes = lib.ow_bwd_packed_bytes(q_c, d, rd)
            wpk = torch.empty(nbytes, dtype=torch.uint8, device=dev)
            _native.check(lib.ow_pack_bwd_weights(*[w.data_ptr() for w in ws], _DTYPE_CODE[wdtype],
                                                  nw.data_ptr() if nw is not None else None, gm.data_ptr(),
                                                  ch.data_ptr(), plan.channels, q_c, d, rd, code, wpk.data_ptr(),
                                                  stream), "ow_pack_bwd_weights")
            pu = torch.empty(q_c, slots, d, dtype=dtype, device=dev)
            pv, dw = torch.empty_like(pu), torch.empty_like(pu)
            n_part = lib.ow_bwd_fused_partials(slots, q_c, rd)
            partial = torch.empty(n_part, 3, 256, dtype=torch.float32, device=dev)
            if routed:
                _native.check(lib.ow_bwd_fused_routed(x.data_ptr(), grad_delta.data_ptr(), rscale.data_ptr() if rscale
                                                      is not None else None, tok.data_ptr(),
                                                      ctypes.byref(oplan), batch, au.data_ptr(),
                                                      av.data_ptr(), ao.data_ptr(), wpk.data_ptr(), nbytes,
                                                      pu.data_ptr(), pv.data_ptr(), dw.data_ptr(), g.data_ptr(),
                                                      partial.data_ptr(), n_part, rd, code, stream),
                              "ow_bwd_fused_routed")
            else:
                dxt = torch.empty_like(xt)
                _native.check(lib.ow_bwd_fused(xt.data_ptr(), dyt.data_ptr(), au.data_ptr(), av.data_ptr(),
                                               ao.data_ptr(), wpk.data_ptr(), nbytes, pu.data_ptr(), pv.data_ptr(),
                                               dw.data_ptr(), dxt.data_ptr(), partial.data_ptr(), n_part, slots, q_c,
                                               d, rd, code, stream), "ow_bwd_fused")
                del xt, dyt
            _sum_rows(lib, partial, n_part, g_a, stream)  # [3, 256]: dA_u, dA_v, dA_o
            g_au, g_av, g_ao = (g_a[m].view(16, 16) for m in range(3))
            # dB_u'', dB_v'', dB_o'' from P_u, P_v, dW' (the gate recomputed): per slot range one
            # [3, q_c, d * rd] block, summed over the ranges.
            n_red = lib.ow_bwd_param_reduce64_partials(slots, q_c, rd)
            red = torch.empty(n_red, 3 * d * rd, dtype=torch.float32, device=dev)
            _native.check(lib.ow_bwd_param_reduce64(pu.data_ptr(), pv.data_ptr(), dw.data_ptr(), wpk.data_ptr(), nbytes,
                                                    red.data_ptr(), n_red, slots, q_c, rd, code, stream),
                          "ow_bwd_param_reduce64")
            g_b3 = torch.empty(3, q_c, d * rd, dtype=torch.float32, device=dev)
            _sum_rows(lib, red, n_red // q_c, g_b3, stream)
            d_bu = g_b3[0].view(q_c, d, rd)
            d_bv = g_b3[1].view(q_c, d, rd)
            d_bo = g_b3[2].view(q_c, rd, d)
            del pu, pv, dw
        elif d == 128 and dtype != torch.float32:
            # Two kernels over 256-slot units: (1) token side P_u, P_v, dW', then U', V', dZ per
            # 32-row chunk and the gate backward (Z, dU', dV'); (2) dP_u, dP_v, dX', W' and the
            # token-matrix gradients (per-workgroup partials).
            nbytes = lib.ow_bwd_packed_bytes(q_c, d, rd)
            wpk = torch.empty(nbytes, dtype=torch.uint8, device=dev)
            _native.check(lib.ow_pack_bwd_weights(*[w.data_ptr() for w in ws], _DTYPE_CODE[wdtype],
                                                  nw.data_ptr() if nw is not None else None, gm.data_ptr(),
                                                  ch.data_ptr(), plan.channels, q_c, d, rd, code, wpk.data_ptr(),
                                                  stream), "ow_pack_bwd_weights")
            pu = torch.empty(q_c, slots, d, dtype=dtype, device=dev)
            pv, dw = torch.empty_like(pu), torch.empty_like(pu)
            z = torch.empty(q_c, slots, rd, dtype=dtype, device=dev)
            du, dv = torch.empty_like(z), torch.empty_like(z)
            n_part = lib.ow_bwd_channel_partials(slots, q_c)
            partial = torch.empty(n_part, 3, 256, dtype=torch.float32, device=dev)
            if routed:
                _native.check(lib.ow_bwd_channel_routed(x.data_ptr(), grad_delta.data_ptr(), rs_ptr, tok.data_ptr(),
                                                        ctypes.byref(oplan), batch, au.data_ptr(), av.data_ptr(),
                                                        ao.data_ptr(), wpk.data_ptr(), nbytes, pu.data_ptr(),
                                                        pv.data_ptr(), dw.data_ptr(), z.data_ptr(), du.data_ptr(),
                                                        dv.data_ptr(), rd, code, stream), "ow_bwd_channel_routed")
                _native.check(lib.ow_bwd_channel2_routed(x.data_ptr(), grad_delta.data_ptr(), rs_ptr, z.data_ptr(),
                                                         du.data_ptr(), dv.data_ptr(), au.data_ptr(), av.data_ptr(),
                                                         wpk.data_ptr(), nbytes, tok.data_ptr(), ctypes.byref(oplan),
                                                         batch, g.data_ptr(), partial.data_ptr(), n_part, rd, code,
                                                         stream), "ow_bwd_channel2_routed")
            else:
                _native.check(lib.ow_bwd_channel(xt.data_ptr(), dyt.data_ptr(), au.data_ptr(), av.data_ptr(),
                                                 ao.data_ptr(), wpk.data_ptr(), nbytes, pu.data_ptr(), pv.data_ptr(),
                                                 dw.data_ptr(), z.data_ptr(), du.data_ptr(), dv.data_ptr(), slots,
                                                 q_c, d, rd, code, stream), "ow_bwd_channel")
                dxt = torch.empty_like(xt)
                _native.check(lib.ow_bwd_channel2(xt.data_ptr(), dyt.data_ptr(), z.data_ptr(), du.data_ptr(),
                                                  dv.data_ptr(), au.data_ptr(), av.data_ptr(), wpk.data_ptr(), nbytes,
                                                  dxt.data_ptr(), partial.data_ptr(), n_part, slots, q_c, d, rd, code,
                                                  stream), "ow_bwd_channel2")
            _sum_rows(lib, partial, n_part, g_a, stream)  # [3, 256]: dA_u, dA_v, dA_o
            g_au, g_av, g_ao = (g_a[m].view(16, 16) for m in range(3))
            # dB_u'', dB_v'', dB_o'' from the slot-major intermediates, as for d = 64.
            n_red = lib.ow_bwd_param_reduce128_partials(slots, q_c, rd)
            red = torch.empty(n_red, 3 * d * rd, dtype=torch.float32, device=dev)
            _native.check(lib.ow_bwd_param_reduce128(pu.data_ptr(), pv.data_ptr(), dw.data_ptr(), z.data_ptr(),
                                                     du.data_ptr(), dv.data_ptr(), red.data_ptr(), n_red, slots, q_c,
                                                     rd, code, stream), "ow_bwd_param_reduce128")
            g_b3 = torch.empty(3, q_c, d * rd, dtype=torch.float32, device=dev)
            _sum_rows(lib, red, n_red // q_c, g_b3, stream)
            d_bu = g_b3[0].view(q_c, d, rd)
            d_bv = g_b3[1].view(q_c, d, rd)
            d_bo = g_b3[2].view(q_c, rd, d)
            del wpk, z, du, dv, pu, pv, dw
            if not routed:
                del xt, dyt
        else:
            # Folded weights in the compute dtype, plain and transposed (both contiguous).
            bu = torch.empty(q_c, d, rd, dtype=dtype, device=dev)
            bv, bo_t = torch.empty_like(bu), torch.empty_like(bu)
            bu_t = torch.empty(q_c, rd, d, dtype=dtype, device=dev)
            bv_t, bo = torch.empty_like(bu_t), torch.empty_like(bu_t)
            _native.check(lib.ow_fold_weights(*[w.data_ptr() for w in ws], _DTYPE_CODE[wdtype],
                                              nw.data_ptr() if nw is not None else None, gm.data_ptr(), ch.data_ptr(),
                                              plan.channels, q_c, d, rd, code, bu.data_ptr(), bu_t.data_ptr(),
                                              bv.data_ptr(), bv_t.data_ptr(), bo.data_ptr(), bo_t.data_ptr(), stream),
                          "ow_fold_weights")
            au_t, av_t, ao_t = (a.t().contiguous() for a in (au, av, ao))
            # Token side: P_u = A_u X', P_v = A_v X', dW' = A_o^T dY (per 16-slot tile).
            pu = _tile_mix(lib, xt, au, None, None, d, code, stream)
            pv = _tile_mix(lib, xt, av, None, None, d, code, stream)
            dw = _tile_mix(lib, dyt, ao_t, None, None, d, code, stream)
            # Channel side: batched GEMMs + the gate kernel.
            u = torch.bmm(pu, bu)
            v = torch.bmm(pv, bv)
            dz = torch.bmm(dw, bo_t)
            z, du, dv = torch.empty_like(u), torch.empty_like(u), torch.empty_like(u)
            _native.check(lib.ow_bwd_gate(u.data_ptr(), v.data_ptr(), dz.data_ptr(), z.data_ptr(), du.data_ptr(),
                                          dv.data_ptr(), u.numel(), code, stream), "ow_bwd_gate")
            del u, v, dz
            wp = torch.bmm(z, bo)
            dpu = torch.bmm(du, bu_t)
            dpv = torch.bmm(dv, bv_t)
            d_bu = _slot_reduce(pu, du)   # [q_c, d, rd]
            d_bv = _slot_reduce(pv, dv)
            d_bo = _slot_reduce(z, dw)    # [q_c, rd, d]
            del z, du, dv, pu, pv, dw

            # Token-matrix gradients and dX'.
            g_au = _tile_outer(lib, dpu, xt, d, code, stream)
            g_av = _tile_outer(lib, dpv, xt, d, code, stream)
            g_ao = _tile_outer(lib, dyt, wp, d, code, stream)
            dxt = _tile_mix(lib, dpu, au_t, dpv, av_t, d, code, stream)
            del dpu, dpv, wp, xt, dyt

        # dX' back to NHWC (unless a kernel wrote g), then through the RMSNorm (+ the residual's
        # identity).
        if not routed:
            _native.check(lib.ow_bwd_scatter(dxt.data_ptr(), tok.data_ptr(), ch.data_ptr(),
                                             ctypes.byref(oplan), batch, code, g.data_ptr(), stream),
                          "ow_bwd_scatter")
            del dxt
        dx = torch.empty_like(x)
        _native.check(lib.ow_bwd_rmsnorm(x.data_ptr(), g.data_ptr(), rscale.data_ptr() if rscale is not None
                                         else None, grad.data_ptr(), dx.data_ptr(), n_rows, plan.channels,
                                         int(residual), code, stream), "ow_bwd_rmsnorm")

        # Parameter gradients from the folded ones, into g_all (every element is written: each
        # channel of the permutation exactly once).
        g_b = g_all[768:768 + 3 * nb]
        g_bu, g_bv = g_b[:nb].view(q_c, d, rd), g_b[nb:2 * nb].view(q_c, d, rd)
        g_bo = g_b[2 * nb:].view(q_c, rd, d)
        g_c = g_all[768 + 3 * nb:].view(-1, plan.channels)
        g_gamma = g_c[0]
        g_nw = g_c[1] if fuse_norm else None
        _native.check(lib.ow_bwd_params(*[w.data_ptr() for w in ws], _DTYPE_CODE[wdtype],
                                        nw.data_ptr() if nw is not None else None, gm.data_ptr(), ch.data_ptr(),
                                        plan.channels, q_c, d, rd, d_bu.data_ptr(), d_bv.data_ptr(), d_bo.data_ptr(),
                                        g_bu.data_ptr(), g_bv.data_ptr(), g_bo.data_ptr(), g_gamma.data_ptr(),
                                        g_nw.data_ptr() if g_nw is not None else None, stream), "ow_bwd_params")

    # The token-matrix gradients of the batched-GEMM path are separate tensors: into g_all too.
    if not all(t.untyped_storage().data_ptr() == g_all.untyped_storage().data_ptr() for t in (g_au, g_av, g_ao)):
        g_a.copy_(torch.stack([g_au.reshape(256), g_av.reshape(256), g_ao.reshape(256)]))
    return dx, g_all


def _cast_group(ts: tuple[Tensor, ...], dtypes: tuple[torch.dtype, ...]) -> tuple[Tensor, ...]:
    """Casts each tensor to its dtype; when all share one dtype and one contiguous storage run,
    with a single kernel (the views of the cast buffer keep their shapes)."""
    if len(set(dtypes)) == 1 and len(ts) > 1:
        base = ts[0]
        flat = [t.reshape(-1) for t in ts]
        storage = base.untyped_storage().data_ptr()
        contiguous_run = all(t.is_contiguous() and t.untyped_storage().data_ptr() == storage for t in ts) and all(
            flat[i + 1].data_ptr() == flat[i].data_ptr() + flat[i].numel() * flat[i].element_size()
            for i in range(len(ts) - 1))
        if contiguous_run:
            n = sum(t.numel() for t in ts)
            whole = torch.as_strided(base, (n,), (1,)).to(dtypes[0])
            out, o = [], 0
            for t in ts:
                out.append(whole[o:o + t.numel()].view(t.shape))
                o += t.numel()
            return tuple(out)
    return tuple(t.to(dt) for t, dt in zip(ts, dtypes))
