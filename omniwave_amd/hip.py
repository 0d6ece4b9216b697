"""HIP backend of the BiGEMM operator (replaces omniweave/ops/triton.py).

* ``hip_is_supported(x, plan, b_u) -> (bool, reason)`` — same tuple contract as
  ``triton_is_supported`` (omniweave/ops/triton.py:26-55).
* ``bigemm_delta_hip`` — drop-in for ``bigemm_delta_triton`` (triton.py:58-85): pre-normalised
  x in, delta out.
* ``bigemm_block_hip`` — the fused RMSNorm -> BiGEMM -> residual of OmniWeaveBlock.forward
  (omniweave/models/block.py:80-108) in one kernel.
* ``bigemm_block_s2d_hip`` — the same block with its output written directly in
  ``space_to_depth`` layout (inference; the block before a downsample).
* ``stem_hip`` — the backbone stem (NCHW image -> space_to_depth(4) -> Linear) in one kernel.

Both go through the ``omniwave_amd::bigemm_fwd`` torch.library custom op, whose implementation
calls ``ow_bigemm_fwd`` of libomniwave_amd.so on the current HIP stream.  Weights are packed
into MFMA operand order by ``ow_pack_weights`` and cached while the parameter tensors are
unchanged (same object, same version counter).
"""

from __future__ import annotations

import ctypes
import functools
import weakref
from collections import OrderedDict

import torch
from torch import Tensor

from omniwave_amd import _native
from omniwave_amd.routing import (RoutePlan, build_route_plan, device_tables, native_plan, plan_key, plan_tiles,
                                  s2d_rows_table)

SPATIAL_TILE = 16
CHANNEL_TILES = (64, 128)
EXPANDED_TILES = (128, 256)
SUPPORTED_DTYPES = (torch.bfloat16, torch.float16, torch.float32)
_DTYPE_CODE = {torch.float32: _native.OW_DTYPE_F32, torch.bfloat16: _native.OW_DTYPE_BF16,
               torch.float16: _native.OW_DTYPE_F16}
_ROUTE_NAME = {v: k for k, v in _native.OW_ROUTE.items()}


@functools.lru_cache(maxsize=16)
def _device_arch(index: int) -> str:
    return str(torch.cuda.get_device_properties(index).gcnArchName)


def hip_is_supported(x: Tensor, plan: RoutePlan, b_u: Tensor) -> tuple[bool, str | None]:
    """Whether the HIP kernels can run these inputs; ``(False, reason)`` otherwise."""
    err = _native.load_error()
    if err is not None:
        return False, f"native library unavailable: {err}"
    if not x.is_cuda:
        return False, "CUDA is unavailable"
    arch = _device_arch(x.device.index if x.device.index is not None else torch.cuda.current_device())
    if not arch.startswith("gfx950"):
        return False, f"device architecture {arch} is not gfx950"
    if x.dtype not in SUPPORTED_DTYPES:
        return False, f"unsupported dtype {x.dtype}; expected float16, bfloat16 or float32"
    g = plan.token_indices.shape[1]
    if g != SPATIAL_TILE:
        return False, f"unsupported spatial tile g={g}; expected 16"
    if b_u.dim() != 3:
        return False, f"b_u must be [Q_c, d, rd], got shape {tuple(b_u.shape)}"
    q_c, d, rd = b_u.shape
    if d not in CHANNEL_TILES:
        return False, f"unsupported channel tile d={d}; expected 64 or 128"
    if rd not in EXPANDED_TILES:
        return False, f"unsupported expanded dim rd={rd}; expected 128 or 256"
    if x.dim() != 4 or tuple(x.shape[1:]) != (plan.height, plan.width, plan.channels):
        return False, f"input shape {tuple(x.shape)} does not match the plan ({plan.height}, {plan.width}, {plan.channels})"
    if plan.channel_indices.shape != (q_c, d):
        return False, f"plan channel tiles {tuple(plan.channel_indices.shape)} do not match b_u {tuple(b_u.shape)}"
    return True, None


# ---------------------------------------------------------------------------------------
# Packed weights


class _PackEntry:
    __slots__ = ("refs", "versions", "packed")


_PACK_CACHE: OrderedDict[tuple, _PackEntry] = OrderedDict()
_PACK_CACHE_SIZE = 64


def _version(t: Tensor) -> int | None:
    try:
        return int(t._version)
    except RuntimeError:  # inference tensors carry no version counter
        return None


def _stream_ptr(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def pack_weights(a_u, a_v, a_o, b_u, b_v, b_o, compute_dtype: torch.dtype, norm_weight: Tensor | None = None,
                 plan: RoutePlan | None = None, gamma: Tensor | None = None, fp8: bool = False) -> Tensor:
    """Pack the six BiGEMM weights into the kernel's MFMA operand order (uint8 buffer).

    With the block's ``plan`` (whose channel table routes per-channel vectors), the LayerScale
    ``gamma`` is folded into the B_o columns and ``norm_weight`` (the RMSNorm weight) into the
    B_u / B_v rows, as OW_FUSE_NORM expects; pad channels are packed as zero.  ``fp8`` packs
    B_u'' / B_v'' as e4m3fn with per-tensor scales (``ow_pack_weights_fp8``) for OW_FUSE_FP8.
    """
    lib = _native.lib()
    ws = [a_u, a_v, a_o, b_u, b_v, b_o]
    wdtype = ws[0].dtype
    if any(w.dtype != wdtype for w in ws) or wdtype not in _DTYPE_CODE:
        wdtype = torch.float32
    ws = [w.detach().to(wdtype).contiguous() for w in ws]
    q_c, d, rd = b_u.shape
    if tuple(a_u.shape) != (SPATIAL_TILE, SPATIAL_TILE) or tuple(b_o.shape) != (q_c, rd, d) \
            or tuple(b_v.shape) != (q_c, d, rd) or a_v.shape != a_u.shape or a_o.shape != a_u.shape:
        raise ValueError("inconsistent BiGEMM weight shapes: "
                         f"a_u {tuple(a_u.shape)}, b_u {tuple(b_u.shape)}, b_v {tuple(b_v.shape)}, b_o {tuple(b_o.shape)}")
    cdt = _DTYPE_CODE[compute_dtype]
    nbytes = lib.ow_packed_weight_bytes_fp8(q_c, d, rd) if fp8 else lib.ow_packed_weight_bytes(q_c, d, rd, cdt)
    if nbytes == 0:
        raise ValueError(f"unsupported packing shape q_c={q_c}, d={d}, rd={rd}")
    packed = torch.empty(nbytes, dtype=torch.uint8, device=b_u.device)
    nw_ptr = gm_ptr = ch_ptr = 0
    channels = q_c * d
    keep = []  # fp32 copies alive until the pack kernel is queued
    if norm_weight is not None or gamma is not None:
        if plan is None:
            raise ValueError("folding norm_weight / gamma needs the block's route plan")
        ch = device_tables(plan, b_u.device)[1]
        ch_ptr, channels = ch.data_ptr(), plan.channels
        if norm_weight is not None:
            keep.append(norm_weight.detach().to(device=b_u.device, dtype=torch.float32).contiguous())
            nw_ptr = keep[-1].data_ptr()
        if gamma is not None:
            keep.append(gamma.detach().to(device=b_u.device, dtype=torch.float32).contiguous())
            gm_ptr = keep[-1].data_ptr()
    pack = lib.ow_pack_weights_fp8 if fp8 else lib.ow_pack_weights
    with torch.cuda.device(b_u.device):
        _native.check(
            pack(*[w.data_ptr() for w in ws], _DTYPE_CODE[wdtype], nw_ptr, gm_ptr, ch_ptr, channels,
                 SPATIAL_TILE, q_c, d, rd, cdt, packed.data_ptr(), _stream_ptr(b_u.device)),
            "ow_pack_weights_fp8" if fp8 else "ow_pack_weights",
        )
    return packed


def _cached_operands(norm_weight, gamma, a_u, a_v, a_o, b_u, b_v, b_o, compute_dtype, plan: RoutePlan,
                     fp8: bool = False):
    srcs = (a_u, a_v, a_o, b_u, b_v, b_o, gamma) + ((norm_weight,) if norm_weight is not None else ())
    versions = tuple(_version(t) for t in srcs)
    key = tuple((t.data_ptr(), t.dtype, tuple(t.shape)) for t in srcs) + (compute_dtype, plan_key(plan), fp8)
    entry = _PACK_CACHE.get(key)
    if (entry is not None and None not in versions and entry.versions == versions
            and all(r() is t for r, t in zip(entry.refs, srcs))):
        _PACK_CACHE.move_to_end(key)
        return entry.packed
    entry = _PackEntry()
    entry.refs = tuple(weakref.ref(t) for t in srcs)
    entry.versions = versions
    entry.packed = pack_weights(a_u, a_v, a_o, b_u, b_v, b_o, compute_dtype, norm_weight, plan, gamma, fp8)
    if None not in versions:
        _PACK_CACHE[key] = entry
        while len(_PACK_CACHE) > _PACK_CACHE_SIZE:
            _PACK_CACHE.popitem(last=False)
    return entry.packed


def clear_pack_cache() -> None:
    _PACK_CACHE.clear()


# ---------------------------------------------------------------------------------------
# Custom op


def _plan_desc(plan) -> list[int]:
    """The custom ops' plan argument: build_route_plan's arguments as integers, read from the
    plan's fields (this package's RoutePlan or the reference's, omniweave/models/routing.py:17-33)."""
    h, w, c, g, d, route, level = plan_key(plan)
    if route not in _native.OW_ROUTE:
        raise ValueError(f"unknown route type: {route!r}")
    return [h, w, c, g, d, _native.OW_ROUTE[route], level]


def _plan_from_desc(desc: list[int]) -> RoutePlan:
    h, w, c, g, d, route, level = desc
    return build_route_plan(h, w, c, g, d, _ROUTE_NAME[route], level)


@torch.library.custom_op("omniwave_amd::bigemm_fwd", mutates_args=())
def bigemm_fwd(
    x: Tensor,
    norm_weight: Tensor | None,
    gamma: Tensor,
    a_u: Tensor,
    a_v: Tensor,
    a_o: Tensor,
    b_u: Tensor,
    b_v: Tensor,
    b_o: Tensor,
    plan_desc: list[int],
    flags: int,
    eps: float,
    drop_scale: Tensor | None,
    want_scales: bool,
) -> tuple[Tensor, Tensor]:
    """(out, row_scale): out = delta (flags=0) or x + delta with the block's RMSNorm fused
    (flags=3), NHWC; flag OW_FUSE_FP8 selects the fp8 channel side.  ``drop_scale`` ([B] fp32 or
    None): per-image multiplier of the rounded delta, the drop-path of training.  With
    ``want_scales`` and the RMSNorm fused, row_scale is [B * H * W] fp32, the RMSNorm scale of
    every row of x, which the backward needs (``ow_bigemm_fwd_scales``: the forward's own values
    where its kernel forms them in one place, else ``ow_rms_scale``); otherwise it is empty."""
    plan = _plan_from_desc(plan_desc)
    x = x.contiguous()
    fuse_norm = bool(flags & _native.OW_FUSE_NORM)
    if fuse_norm and norm_weight is None:
        raise ValueError("OW_FUSE_NORM needs norm_weight")
    fp8 = bool(flags & _native.OW_FUSE_FP8)
    packed = _cached_operands(norm_weight if fuse_norm else None, gamma, a_u, a_v, a_o, b_u, b_v, b_o, x.dtype, plan,
                              fp8)
    tok, ch = device_tables(plan, x.device)
    out = torch.empty_like(x, memory_format=torch.contiguous_format)
    oplan = native_plan(plan)
    lib = _native.lib()
    ws_bytes = lib.ow_fwd_workspace_bytes(ctypes.byref(oplan), x.shape[0], flags)
    workspace = torch.empty(max(ws_bytes // 4, 1), dtype=torch.float32, device=x.device)
    common = (x.data_ptr(), out.data_ptr(), eps, packed.data_ptr(), packed.numel(), tok.data_ptr(), ch.data_ptr(),
              ctypes.byref(oplan), x.shape[0], b_u.shape[2], _DTYPE_CODE[x.dtype], flags)
    n_rows = x.shape[0] * plan.height * plan.width
    scales = torch.empty(n_rows if (want_scales and fuse_norm) else 0, dtype=torch.float32, device=x.device)
    with torch.cuda.device(x.device):
        if scales.numel():
            written = ctypes.c_int32(0)
            scale = _drop_scale_arg(drop_scale, x) if drop_scale is not None else None
            _native.check(lib.ow_bigemm_fwd_scales(*common, scale.data_ptr() if scale is not None else None,
                                                   scales.data_ptr(), ctypes.byref(written), workspace.data_ptr(),
                                                   ws_bytes, _stream_ptr(x.device)), "ow_bigemm_fwd_scales")
            if not written.value:
                _native.check(lib.ow_rms_scale(x.data_ptr(), scales.data_ptr(), n_rows, plan.channels, eps,
                                               _DTYPE_CODE[x.dtype], _stream_ptr(x.device)), "ow_rms_scale")
        elif drop_scale is None:
            _native.check(lib.ow_bigemm_fwd(*common, workspace.data_ptr(), ws_bytes, _stream_ptr(x.device)),
                          "ow_bigemm_fwd")
        else:
            scale = _drop_scale_arg(drop_scale, x)
            _native.check(lib.ow_bigemm_fwd_drop(*common, scale.data_ptr(), workspace.data_ptr(), ws_bytes,
                                                 _stream_ptr(x.device)), "ow_bigemm_fwd_drop")
    return out, scales


def _drop_scale_arg(drop_scale: Tensor, x: Tensor) -> Tensor:
    if drop_scale.shape != (x.shape[0],) or drop_scale.device != x.device:
        raise ValueError(f"drop_scale must be [{x.shape[0]}] on {x.device}, got {tuple(drop_scale.shape)} on "
                         f"{drop_scale.device}")
    return drop_scale.to(torch.float32).contiguous()


@bigemm_fwd.register_fake
def _bigemm_fwd_fake(x, norm_weight, gamma, a_u, a_v, a_o, b_u, b_v, b_o, plan_desc, flags, eps, drop_scale,
                     want_scales):
    h, w = plan_desc[0], plan_desc[1]
    n = x.shape[0] * h * w if (want_scales and flags & _native.OW_FUSE_NORM) else 0
    return (torch.empty_like(x, memory_format=torch.contiguous_format),
            torch.empty(n, dtype=torch.float32, device=x.device))


def _bigemm_fwd_setup_context(ctx, inputs, output):
    x, norm_weight, gamma, a_u, a_v, a_o, b_u, b_v, b_o, plan_desc, flags, eps, drop_scale, want_scales = inputs
    _, scales = output
    ctx.mark_non_differentiable(scales)
    ctx.set_materialize_grads(False)  # no zero-filled gradient for the scales output
    ctx.save_for_backward(x, norm_weight, gamma, a_u, a_v, a_o, b_u, b_v, b_o, drop_scale, scales)
    ctx.plan_desc, ctx.flags, ctx.eps = list(plan_desc), int(flags), float(eps)


def _bigemm_fwd_backward(ctx, grad, grad_scales):
    from omniwave_amd.backward import bigemm_backward

    if ctx.flags & _native.OW_FUSE_FP8:
        raise NotImplementedError("the fp8 BiGEMM variant is inference-only (no backward)")
    if grad is None:
        return (None,) * 14
    x, norm_weight, gamma, a_u, a_v, a_o, b_u, b_v, b_o, drop_scale, scales = ctx.saved_tensors
    grads = bigemm_backward(grad, x, norm_weight, gamma, a_u, a_v, a_o, b_u, b_v, b_o,
                            _plan_from_desc(ctx.plan_desc), ctx.flags, ctx.eps, drop_scale=drop_scale,
                            row_scale=scales if scales.numel() else None)
    grads = tuple(g if need else None for g, need in zip(grads, ctx.needs_input_grad))
    return grads + (None, None, None, None, None)


bigemm_fwd.register_autograd(_bigemm_fwd_backward, setup_context=_bigemm_fwd_setup_context)


def _require(x, plan, b_u) -> None:
    ok, reason = hip_is_supported(x, plan, b_u)
    if not ok:
        raise RuntimeError(f"hip backend not supported: {reason}")


def bigemm_delta_hip(*, x, plan, a_u, a_v, a_o, b_u, b_v, b_o, gamma) -> Tensor:
    """delta for pre-normalised x (omniweave/ops/reference.py:120-173 semantics)."""
    _require(x, plan, b_u)
    return bigemm_fwd(x, None, gamma, a_u, a_v, a_o, b_u, b_v, b_o, _plan_desc(plan), 0, 0.0, None, False)[0]


def bigemm_block_hip(x, norm_weight, plan, a_u, a_v, a_o, b_u, b_v, b_o, gamma, eps: float = 1e-6,
                     residual: bool = True, fp8: bool = False, drop_scale: Tensor | None = None) -> Tensor:
    """RMSNorm(x) -> BiGEMM -> (+ x) fused (omniweave/models/block.py:83-108).

    ``drop_scale`` ([B] float32 on x's device, or None): the per-sample drop-path of training
    (block.py:99-107), ``keep_mask / keep_probability`` per image, applied to the rounded delta
    inside the kernel, with a matching backward (see ``drop_path_scale``).  ``fp8=True`` runs
    the channel-side products on e4m3fn MFMAs (inference only; bf16 / fp16 activations).
    """
    _require(x, plan, b_u)
    if fp8 and x.dtype not in (torch.bfloat16, torch.float16):
        raise RuntimeError(f"hip backend not supported: the fp8 variant takes bf16 or fp16 activations, not {x.dtype}")
    flags = _native.OW_FUSE_NORM | (_native.OW_FUSE_RESIDUAL if residual else 0) | (_native.OW_FUSE_FP8 if fp8 else 0)
    # The RMSNorm row scales are kept for the backward when one will run.
    want_scales = (not fp8 and torch.is_grad_enabled()
                   and any(t.requires_grad for t in (x, norm_weight, gamma, a_u, a_v, a_o, b_u, b_v, b_o)))
    return bigemm_fwd(x, norm_weight, gamma, a_u, a_v, a_o, b_u, b_v, b_o, _plan_desc(plan), flags, float(eps),
                      drop_scale, want_scales)[0]


def drop_path_scale(batch: int, drop_path_rate: float, dtype: torch.dtype, device) -> Tensor:
    """Per-image drop-path factors for ``bigemm_block_hip(..., drop_scale=...)``.

    Draws the keep mask exactly as the reference does (omniweave/models/block.py:100-106: a
    ``[B, 1, 1, 1]`` tensor of the activation dtype, ``bernoulli_(keep_probability)``), so the
    random stream is consumed identically, and returns ``keep_mask * (1 / keep_probability)``
    in float32 ([B]): the reference's ``delta * keep_mask / keep_probability`` on the GPU
    multiplies by that fp32 reciprocal.
    """
    keep = 1.0 - drop_path_rate
    mask = torch.empty((batch, 1, 1, 1), dtype=dtype, device=device).bernoulli_(keep)
    inv = torch.tensor(1.0, dtype=torch.float32) / torch.tensor(keep, dtype=torch.float32)
    return mask.reshape(batch).to(torch.float32) * inv.to(device)


# ---------------------------------------------------------------------------------------
# Backbone glue (inference): a block whose output feeds space_to_depth, and the stem.


@torch.library.custom_op("omniwave_amd::bigemm_fwd_s2d", mutates_args=())
def bigemm_fwd_s2d(
    x: Tensor,
    norm_weight: Tensor,
    gamma: Tensor,
    a_u: Tensor,
    a_v: Tensor,
    a_o: Tensor,
    b_u: Tensor,
    b_v: Tensor,
    b_o: Tensor,
    plan_desc: list[int],
    flags: int,
    eps: float,
    factor: int,
) -> Tensor:
    """``space_to_depth(x + delta, factor)`` ([B, H/f, W/f, C f^2]) with the block's RMSNorm
    fused: ``ow_bigemm_fwd_rows`` with the ``ow_route_s2d_rows`` table, one pass over HBM.
    Inference only (no autograd)."""
    plan = _plan_from_desc(plan_desc)
    x = x.contiguous()
    b, h, w, c = x.shape
    if h % factor or w % factor:
        raise ValueError(f"height {h} and width {w} must be divisible by factor {factor}")
    fp8 = bool(flags & _native.OW_FUSE_FP8)
    packed = _cached_operands(norm_weight, gamma, a_u, a_v, a_o, b_u, b_v, b_o, x.dtype, plan, fp8)
    tok, ch = device_tables(plan, x.device)
    rows = s2d_rows_table(plan, factor, x.device)
    out = torch.empty((b, h // factor, w // factor, c * factor * factor), dtype=x.dtype, device=x.device)
    oplan = native_plan(plan)
    lib = _native.lib()
    ws_bytes = lib.ow_fwd_workspace_bytes(ctypes.byref(oplan), b, flags)
    workspace = torch.empty(max(ws_bytes // 4, 1), dtype=torch.float32, device=x.device)
    with torch.cuda.device(x.device):
        _native.check(
            lib.ow_bigemm_fwd_rows(
                x.data_ptr(), out.data_ptr(), eps, packed.data_ptr(), packed.numel(),
                tok.data_ptr(), ch.data_ptr(), rows.data_ptr(), ctypes.byref(oplan), b, b_u.shape[2],
                _DTYPE_CODE[x.dtype], flags, workspace.data_ptr(), ws_bytes, _stream_ptr(x.device),
            ),
            "ow_bigemm_fwd_rows",
        )
    return out


@bigemm_fwd_s2d.register_fake
def _bigemm_fwd_s2d_fake(x, norm_weight, gamma, a_u, a_v, a_o, b_u, b_v, b_o, plan_desc, flags, eps, factor):
    b, h, w, c = x.shape
    return x.new_empty((b, h // factor, w // factor, c * factor * factor))


def bigemm_block_s2d_hip(x, norm_weight, plan, a_u, a_v, a_o, b_u, b_v, b_o, gamma, factor: int = 2,
                         eps: float = 1e-6, fp8: bool = False) -> Tensor:
    """``space_to_depth(bigemm_block_hip(x, ...), factor)`` as one kernel (omniweave/models/
    block.py:80-108 then backbone.py:14-27,183-186); bf16 / fp16 activations, inference only."""
    _require(x, plan, b_u)
    if x.dtype not in (torch.bfloat16, torch.float16):
        raise RuntimeError(f"hip backend not supported: the space_to_depth output takes bf16 or fp16, not {x.dtype}")
    if torch.is_grad_enabled() and any(t.requires_grad for t in (x, norm_weight, gamma, a_u, b_u)):
        raise RuntimeError("bigemm_block_s2d_hip is inference-only (no backward); run it under torch.no_grad()")
    flags = _native.OW_FUSE_NORM | _native.OW_FUSE_RESIDUAL | (_native.OW_FUSE_FP8 if fp8 else 0)
    return bigemm_fwd_s2d(x, norm_weight, gamma, a_u, a_v, a_o, b_u, b_v, b_o, _plan_desc(plan), flags, float(eps),
                          int(factor))


@torch.library.custom_op("omniwave_amd::bigemm_fwd_chain", mutates_args=())
def bigemm_fwd_chain(
    x: Tensor,
    norm_weight: Tensor,
    gamma: Tensor,
    a_u: Tensor,
    a_v: Tensor,
    a_o: Tensor,
    b_u: Tensor,
    b_v: Tensor,
    b_o: Tensor,
    plan_desc: list[int],
    flags: int,
    eps: float,
    stats_in: Tensor | None,
    factor: int,
) -> tuple[Tensor, Tensor, Tensor]:
    """One block of a stage's chain (``ow_bigemm_fwd_chain``), inference only: ``out`` as
    ``bigemm_fwd`` (factor 0) or ``bigemm_fwd_s2d`` (factor > 0); ``stats`` ([B*H*W, Q_c] fp32,
    [0, Q_c] with factor > 0): per output row and channel group, the sum of squares of the
    stored values, valid when ``written`` (a CPU int32 [1]) is 1; ``stats_in``: the previous
    block's ``stats`` (its RMSNorm statistics, so the launch reads only its groups' columns)."""
    plan = _plan_from_desc(plan_desc)
    x = x.contiguous()
    b, h, w, c = x.shape
    fp8 = bool(flags & _native.OW_FUSE_FP8)
    packed = _cached_operands(norm_weight, gamma, a_u, a_v, a_o, b_u, b_v, b_o, x.dtype, plan, fp8)
    tok, ch = device_tables(plan, x.device)
    q_c = ch.numel() // plan_tiles(plan)[1]
    if factor > 0:
        if h % factor or w % factor:
            raise ValueError(f"height {h} and width {w} must be divisible by factor {factor}")
        rows = s2d_rows_table(plan, factor, x.device).data_ptr()
        out = torch.empty((b, h // factor, w // factor, c * factor * factor), dtype=x.dtype, device=x.device)
        stats = torch.empty((0, q_c), dtype=torch.float32, device=x.device)
    else:
        rows = None
        out = torch.empty_like(x)
        stats = torch.empty((b * h * w, q_c), dtype=torch.float32, device=x.device)
    parts = 0
    if stats_in is not None:
        if stats_in.dtype != torch.float32 or stats_in.dim() != 2 or stats_in.shape[0] != b * h * w:
            raise ValueError(f"stats_in must be float32 [{b * h * w}, parts], got {stats_in.dtype} "
                             f"{tuple(stats_in.shape)}")
        stats_in = stats_in.contiguous()
        parts = stats_in.shape[1]
    oplan = native_plan(plan)
    lib = _native.lib()
    ws_bytes = lib.ow_fwd_workspace_bytes(ctypes.byref(oplan), b, flags)
    workspace = torch.empty(max(ws_bytes // 4, 1), dtype=torch.float32, device=x.device)
    written = ctypes.c_int32(0)
    with torch.cuda.device(x.device):
        _native.check(
            lib.ow_bigemm_fwd_chain(
                x.data_ptr(), out.data_ptr(), eps, packed.data_ptr(), packed.numel(),
                tok.data_ptr(), ch.data_ptr(), rows, ctypes.byref(oplan), b, b_u.shape[2],
                _DTYPE_CODE[x.dtype], flags, None if stats_in is None else stats_in.data_ptr(), parts,
                stats.data_ptr() if stats.numel() else None, ctypes.byref(written),
                workspace.data_ptr(), ws_bytes, _stream_ptr(x.device),
            ),
            "ow_bigemm_fwd_chain",
        )
    return out, stats, torch.tensor([written.value], dtype=torch.int32)


@bigemm_fwd_chain.register_fake
def _bigemm_fwd_chain_fake(x, norm_weight, gamma, a_u, a_v, a_o, b_u, b_v, b_o, plan_desc, flags, eps, stats_in,
                           factor):
    b, h, w, c = x.shape
    q_c = -(-plan_desc[2] // plan_desc[4])
    if factor > 0:
        out = x.new_empty((b, h // factor, w // factor, c * factor * factor))
        stats = x.new_empty((0, q_c), dtype=torch.float32)
    else:
        out = x.new_empty(x.shape)
        stats = x.new_empty((b * h * w, q_c), dtype=torch.float32)
    return out, stats, torch.empty((1,), dtype=torch.int32)


def bigemm_block_chain_hip(x, stats_in, norm_weight, plan, a_u, a_v, a_o, b_u, b_v, b_o, gamma, factor: int = 0,
                           eps: float = 1e-6, fp8: bool = False) -> tuple[Tensor, Tensor | None]:
    """``bigemm_block_hip`` (factor 0) or ``bigemm_block_s2d_hip`` (factor > 0) for consecutive
    blocks of a stage (omniweave/models/backbone.py:75-80): returns ``(out, stats)``, where
    ``stats`` is the next block's ``stats_in`` (its RMSNorm statistics) or None when this
    launch wrote none.  The output equals the unchained call's up to the summation order of the
    RMSNorm mean of squares.  bf16 / fp16 activations, inference only."""
    _require(x, plan, b_u)
    if x.dtype not in (torch.bfloat16, torch.float16):
        raise RuntimeError(f"hip backend not supported: chained blocks take bf16 or fp16, not {x.dtype}")
    if torch.is_grad_enabled() and any(t.requires_grad for t in (x, norm_weight, gamma, a_u, b_u)):
        raise RuntimeError("bigemm_block_chain_hip is inference-only (no backward); run it under torch.no_grad()")
    flags = _native.OW_FUSE_NORM | _native.OW_FUSE_RESIDUAL | (_native.OW_FUSE_FP8 if fp8 else 0)
    out, stats, written = bigemm_fwd_chain(x, norm_weight, gamma, a_u, a_v, a_o, b_u, b_v, b_o, _plan_desc(plan),
                                           flags, float(eps), stats_in, int(factor))
    return out, (stats if int(written[0]) else None)


STEM_CHANNELS = (32, 64, 96, 128, 192, 256)


def stem_is_supported(image: Tensor, weight: Tensor) -> tuple[bool, str | None]:
    """Whether ``stem_hip`` can run these inputs; ``(False, reason)`` otherwise."""
    err = _native.load_error()
    if err is not None:
        return False, f"native library unavailable: {err}"
    if not image.is_cuda:
        return False, "CUDA is unavailable"
    arch = _device_arch(image.device.index if image.device.index is not None else torch.cuda.current_device())
    if not arch.startswith("gfx950"):
        return False, f"device architecture {arch} is not gfx950"
    if image.dtype not in (torch.bfloat16, torch.float16) or weight.dtype != image.dtype:
        return False, f"stem takes bf16 or fp16 image and weight of one dtype, not {image.dtype} / {weight.dtype}"
    if image.dim() != 4 or image.shape[1] != 3 or image.shape[2] % 4 or image.shape[3] % 4:
        return False, f"image must be [B, 3, H, W] with H, W divisible by 4, got {tuple(image.shape)}"
    if weight.dim() != 2 or weight.shape[1] != 48 or weight.shape[0] not in STEM_CHANNELS:
        return False, f"weight must be [N, 48] with N in {STEM_CHANNELS}, got {tuple(weight.shape)}"
    return True, None


@torch.library.custom_op("omniwave_amd::stem_fwd", mutates_args=())
def stem_fwd(image: Tensor, weight: Tensor) -> Tensor:
    """``Linear(space_to_depth(image.permute(0, 2, 3, 1), 4))`` ([B, H/4, W/4, N]) in one kernel
    (``ow_stem_fwd``).  Inference only (no autograd)."""
    image = image.contiguous()
    weight = weight.contiguous()
    b, _, h, w = image.shape
    n = weight.shape[0]
    out = torch.empty((b, h // 4, w // 4, n), dtype=image.dtype, device=image.device)
    with torch.cuda.device(image.device):
        _native.check(
            _native.lib().ow_stem_fwd(image.data_ptr(), weight.data_ptr(), out.data_ptr(), b, h, w, n,
                                      _DTYPE_CODE[image.dtype], _stream_ptr(image.device)),
            "ow_stem_fwd",
        )
    return out


@stem_fwd.register_fake
def _stem_fwd_fake(image, weight):
    b, _, h, w = image.shape
    return image.new_empty((b, h // 4, w // 4, weight.shape[0]))


def stem_hip(image: Tensor, weight: Tensor) -> Tensor:
    """Backbone stem (omniweave/models/backbone.py:121,173-176) on the HIP kernel; raises if
    unsupported or if a gradient is needed."""
    ok, reason = stem_is_supported(image, weight)
    if not ok:
        raise RuntimeError(f"hip stem not supported: {reason}")
    if torch.is_grad_enabled() and (image.requires_grad or weight.requires_grad):
        raise RuntimeError("stem_hip is inference-only (no backward); run it under torch.no_grad()")
    return stem_fwd(image, weight)

