"""ctypes binding of libomniwave_amd.so (the C ABI declared in include/omniwave_amd.h)."""

from __future__ import annotations

import ctypes
import threading
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libomniwave_amd.so"

OW_OK = 0
OW_ROUTE = {"local": 0, "shifted": 1, "radix": 2}
OW_DTYPE_F32, OW_DTYPE_BF16, OW_DTYPE_F16 = 0, 1, 2
OW_FUSE_NORM, OW_FUSE_RESIDUAL, OW_FUSE_FP8 = 1, 2, 4

_c_int32_p = ctypes.POINTER(ctypes.c_int32)


class OwPlan(ctypes.Structure):
    _fields_ = [
        ("height", ctypes.c_int32),
        ("width", ctypes.c_int32),
        ("channels", ctypes.c_int32),
        ("spatial_tile", ctypes.c_int32),
        ("channel_tile", ctypes.c_int32),
        ("route", ctypes.c_int32),
        ("radix_level", ctypes.c_int32),
        ("window", ctypes.c_int32),
        ("shift", ctypes.c_int32),
    ]


_SIGNATURES = {
    "ow_version": (ctypes.c_int, []),
    "ow_last_error": (ctypes.c_char_p, []),
    "ow_plan_dims": (ctypes.c_int, [ctypes.POINTER(OwPlan), _c_int32_p, _c_int32_p]),
    "ow_route_build": (ctypes.c_int, [ctypes.POINTER(OwPlan), _c_int32_p, _c_int32_p]),
    "ow_packed_weight_bytes": (ctypes.c_size_t, [ctypes.c_int32] * 4),
    "ow_pack_weights": (
        ctypes.c_int,
        [ctypes.c_void_p] * 6 + [ctypes.c_int32, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int32]
        + [ctypes.c_int32] * 5 + [ctypes.c_void_p, ctypes.c_void_p],
    ),
    "ow_packed_weight_bytes_fp8": (ctypes.c_size_t, [ctypes.c_int32] * 3),
    "ow_pack_weights_fp8": (
        ctypes.c_int,
        [ctypes.c_void_p] * 6 + [ctypes.c_int32, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int32]
        + [ctypes.c_int32] * 5 + [ctypes.c_void_p, ctypes.c_void_p],
    ),
    "ow_rms_scale": (
        ctypes.c_int,
        [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64, ctypes.c_int32, ctypes.c_float, ctypes.c_int32,
         ctypes.c_void_p],
    ),
    "ow_fwd_workspace_bytes": (ctypes.c_size_t, [ctypes.POINTER(OwPlan), ctypes.c_int32, ctypes.c_int32]),
    "ow_bigemm_fwd": (
        ctypes.c_int,
        [
            ctypes.c_void_p, ctypes.c_void_p, ctypes.c_float,
            ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p, ctypes.c_void_p,
            ctypes.POINTER(OwPlan), ctypes.c_int32, ctypes.c_int32, ctypes.c_int32,
            ctypes.c_int32, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p,
        ],
    ),
    "ow_bigemm_fwd_rows": (
        ctypes.c_int,
        [
            ctypes.c_void_p, ctypes.c_void_p, ctypes.c_float,
            ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
            ctypes.POINTER(OwPlan), ctypes.c_int32, ctypes.c_int32, ctypes.c_int32,
            ctypes.c_int32, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p,
        ],
    ),
    "ow_bigemm_fwd_chain": (
        ctypes.c_int,
        [
            ctypes.c_void_p, ctypes.c_void_p, ctypes.c_float,
            ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
            ctypes.POINTER(OwPlan), ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32,
            ctypes.c_void_p, ctypes.c_int32, ctypes.c_void_p, ctypes.POINTER(ctypes.c_int32),
            ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p,
        ],
    ),
    "ow_bigemm_fwd_scales": (
        ctypes.c_int,
        [
            ctypes.c_void_p, ctypes.c_void_p, ctypes.c_float,
            ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p, ctypes.c_void_p,
            ctypes.POINTER(OwPlan), ctypes.c_int32, ctypes.c_int32, ctypes.c_int32,
            ctypes.c_int32, ctypes.c_void_p, ctypes.c_void_p, ctypes.POINTER(ctypes.c_int32), ctypes.c_void_p,
            ctypes.c_size_t, ctypes.c_void_p,
        ],
    ),
    "ow_bigemm_fwd_drop": (
        ctypes.c_int,
        [
            ctypes.c_void_p, ctypes.c_void_p, ctypes.c_float,
            ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p, ctypes.c_void_p,
            ctypes.POINTER(OwPlan), ctypes.c_int32, ctypes.c_int32, ctypes.c_int32,
            ctypes.c_int32, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p,
        ],
    ),
    "ow_bigemm_fwd_noalloc": (
        ctypes.c_int,
        [
            ctypes.c_void_p, ctypes.c_void_p, ctypes.c_float,
            ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p, ctypes.c_void_p,
            ctypes.POINTER(OwPlan), ctypes.c_int32, ctypes.c_int32, ctypes.c_int32,
            ctypes.c_int32, ctypes.c_void_p,
        ],
    ),
    "ow_scale_samples": (
        ctypes.c_int,
        [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64, ctypes.c_int32,
         ctypes.c_void_p],
    ),
    "ow_route_s2d_rows": (ctypes.c_int, [ctypes.POINTER(OwPlan), ctypes.c_int32, _c_int32_p, _c_int32_p]),
    "ow_stem_fwd": (
        ctypes.c_int,
        [ctypes.c_void_p] * 3 + [ctypes.c_int32] * 5 + [ctypes.c_void_p],
    ),
    "ow_fold_weights": (
        ctypes.c_int,
        [ctypes.c_void_p] * 3 + [ctypes.c_int32, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p]
        + [ctypes.c_int32] * 5 + [ctypes.c_void_p] * 7,
    ),
    "ow_bwd_gather": (
        ctypes.c_int,
        [ctypes.c_void_p] * 5 + [ctypes.POINTER(OwPlan), ctypes.c_int32, ctypes.c_int32] + [ctypes.c_void_p] * 3,
    ),
    "ow_bwd_gate": (ctypes.c_int, [ctypes.c_void_p] * 6 + [ctypes.c_int64, ctypes.c_int32, ctypes.c_void_p]),
    "ow_bwd_scatter": (
        ctypes.c_int,
        [ctypes.c_void_p] * 3 + [ctypes.POINTER(OwPlan), ctypes.c_int32, ctypes.c_int32, ctypes.c_void_p,
                                 ctypes.c_void_p],
    ),
    "ow_bwd_rmsnorm": (
        ctypes.c_int,
        [ctypes.c_void_p] * 5 + [ctypes.c_int64, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, ctypes.c_void_p],
    ),
    "ow_tile_mix": (
        ctypes.c_int, [ctypes.c_void_p] * 5 + [ctypes.c_int64, ctypes.c_int32, ctypes.c_int32, ctypes.c_void_p],
    ),
    "ow_tile_outer": (
        ctypes.c_int,
        [ctypes.c_void_p] * 3 + [ctypes.c_int32, ctypes.c_int64, ctypes.c_int32, ctypes.c_int32, ctypes.c_void_p],
    ),
    "ow_bwd_packed_bytes": (ctypes.c_size_t, [ctypes.c_int32] * 3),
    "ow_pack_bwd_weights": (
        ctypes.c_int,
        [ctypes.c_void_p] * 3 + [ctypes.c_int32, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p]
        + [ctypes.c_int32] * 5 + [ctypes.c_void_p, ctypes.c_void_p],
    ),
    "ow_bwd_fused_partials": (ctypes.c_int64, [ctypes.c_int64, ctypes.c_int32, ctypes.c_int32]),
    "ow_bwd_fused": (
        ctypes.c_int,
        [ctypes.c_void_p] * 6 + [ctypes.c_size_t] + [ctypes.c_void_p] * 5
        + [ctypes.c_int64, ctypes.c_int64, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32,
           ctypes.c_void_p],
    ),
    "ow_bwd_channel": (
        ctypes.c_int,
        [ctypes.c_void_p] * 6 + [ctypes.c_size_t] + [ctypes.c_void_p] * 6
        + [ctypes.c_int64, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, ctypes.c_void_p],
    ),
    "ow_bwd_channel_partials": (ctypes.c_int64, [ctypes.c_int64, ctypes.c_int32]),
    "ow_bwd_channel2": (
        ctypes.c_int,
        [ctypes.c_void_p] * 8 + [ctypes.c_size_t] + [ctypes.c_void_p] * 2
        + [ctypes.c_int64, ctypes.c_int64, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32,
           ctypes.c_void_p],
    ),
    "ow_bwd_channel_routed": (
        ctypes.c_int,
        [ctypes.c_void_p] * 5 + [ctypes.c_int32] + [ctypes.c_void_p] * 4 + [ctypes.c_size_t] + [ctypes.c_void_p] * 6
        + [ctypes.c_int32, ctypes.c_int32, ctypes.c_void_p],
    ),
    "ow_bwd_channel2_routed": (
        ctypes.c_int,
        [ctypes.c_void_p] * 9 + [ctypes.c_size_t] + [ctypes.c_void_p] * 2 + [ctypes.c_int32]
        + [ctypes.c_void_p] * 2 + [ctypes.c_int64, ctypes.c_int32, ctypes.c_int32, ctypes.c_void_p],
    ),
    "ow_bwd_param_reduce64_partials": (ctypes.c_int64, [ctypes.c_int64, ctypes.c_int32, ctypes.c_int32]),
    "ow_bwd_param_reduce64": (
        ctypes.c_int,
        [ctypes.c_void_p] * 4 + [ctypes.c_size_t, ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64, ctypes.c_int32,
                                 ctypes.c_int32, ctypes.c_int32, ctypes.c_void_p],
    ),
    "ow_bwd_param_reduce128_partials": (ctypes.c_int64, [ctypes.c_int64, ctypes.c_int32, ctypes.c_int32]),
    "ow_bwd_param_reduce128": (
        ctypes.c_int,
        [ctypes.c_void_p] * 7 + [ctypes.c_int64, ctypes.c_int64, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32,
                                 ctypes.c_void_p],
    ),
    "ow_small_to_f32": (ctypes.c_int, [ctypes.c_void_p] * 3 + [ctypes.c_int32, ctypes.c_void_p, ctypes.c_void_p]),
    "ow_sum_rows": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64, ctypes.c_void_p, ctypes.c_void_p]),
    "ow_bwd_fused_routed": (
        ctypes.c_int,
        [ctypes.c_void_p] * 5 + [ctypes.c_int32] + [ctypes.c_void_p] * 4 + [ctypes.c_size_t] + [ctypes.c_void_p] * 5
        + [ctypes.c_int64, ctypes.c_int32, ctypes.c_int32, ctypes.c_void_p],
    ),
    "ow_bwd_params": (
        ctypes.c_int,
        [ctypes.c_void_p] * 3 + [ctypes.c_int32, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p]
        + [ctypes.c_int32] * 4 + [ctypes.c_void_p] * 9,
    ),
}

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None
_load_error: str | None = None


class NativeLibraryError(RuntimeError):
    """libomniwave_amd.so is missing or does not load."""


def _load() -> ctypes.CDLL | None:
    global _lib, _load_error
    with _lock:
        if _lib is not None or _load_error is not None:
            return _lib
        if not LIB_PATH.exists():
            _load_error = f"{LIB_PATH.name} is not built (run omniwave_amd._build.build())"
            return None
        try:
            lib = ctypes.CDLL(str(LIB_PATH))
            for name, (restype, argtypes) in _SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype = restype
                fn.argtypes = argtypes
        except (OSError, AttributeError) as exc:
            _load_error = f"cannot load {LIB_PATH}: {exc}"
            return None
        _lib = lib
        return _lib


def load_error() -> str | None:
    """Why the library is unusable, or None when it loaded."""
    _load()
    return _load_error


def lib() -> ctypes.CDLL:
    handle = _load()
    if handle is None:
        raise NativeLibraryError(_load_error or "libomniwave_amd.so unavailable")
    return handle


def check(rc: int, what: str) -> None:
    """Raise the library's error text for a non-zero status."""
    if rc != OW_OK:
        msg = lib().ow_last_error().decode(errors="replace")
        exc = ValueError if rc == 1 else RuntimeError
        raise exc(f"{what} failed (status {rc}): {msg}")


def make_plan(height, width, channels, spatial_tile, channel_tile, route, radix_level, window=4, shift=2) -> OwPlan:
    return OwPlan(height, width, channels, spatial_tile, channel_tile, OW_ROUTE[route], radix_level, window, shift)


def exported_symbols() -> list[str]:
    return sorted(_SIGNATURES)
