"""The C-ABI library loads on a machine without a GPU and exports every symbol the header
declares; host-only entry points validate their arguments; the HIP path refuses CPU inputs."""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest
import torch

from omniwave_amd import _native
from omniwave_amd.hip import hip_is_supported
from omniwave_amd.routing import build_route_plan

HEADER = Path(__file__).resolve().parent.parent / "include" / "omniwave_amd.h"


def declared_symbols() -> list[str]:
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(ow_[a-z0-9_]+)\s*\(", text)))


def test_library_loads() -> None:
    assert _native.load_error() is None
    assert _native.lib().ow_version() >= 100


def test_every_declared_symbol_is_exported() -> None:
    names = declared_symbols()
    assert len(names) >= 7
    raw = ctypes.CDLL(str(_native.LIB_PATH))
    for name in names:
        assert hasattr(raw, name), f"{name} declared in include/omniwave_amd.h but not exported"
    assert set(names) == set(_native.exported_symbols())


def test_plan_dims_and_errors() -> None:
    lib = _native.lib()
    q_s, q_c = ctypes.c_int32(), ctypes.c_int32()
    plan = _native.make_plan(14, 14, 512, 16, 128, "shifted", 0)
    assert lib.ow_plan_dims(ctypes.byref(plan), ctypes.byref(q_s), ctypes.byref(q_c)) == 0
    assert (q_s.value, q_c.value) == (13, 4)
    bad = _native.make_plan(14, 14, 512, 16, 128, "local", 0)
    bad.route = 7
    assert lib.ow_plan_dims(ctypes.byref(bad), ctypes.byref(q_s), ctypes.byref(q_c)) == 1
    assert b"unknown route" in lib.ow_last_error()
    assert lib.ow_plan_dims(None, ctypes.byref(q_s), ctypes.byref(q_c)) == 1


def test_packed_weight_bytes() -> None:
    lib = _native.lib()
    # head (3 x 256 elements) + q_c * 3*d*rd elements, 2 bytes each
    assert lib.ow_packed_weight_bytes(4, 128, 256, _native.OW_DTYPE_BF16) == 2 * (768 + 4 * 3 * 128 * 256)
    assert lib.ow_packed_weight_bytes(2, 64, 128, _native.OW_DTYPE_F16) == 2 * (768 + 2 * 3 * 64 * 128)
    assert lib.ow_packed_weight_bytes(0, 64, 128, _native.OW_DTYPE_F16) == 0


def test_fwd_rejects_bad_arguments_without_touching_the_gpu() -> None:
    lib = _native.lib()
    plan = _native.make_plan(14, 14, 512, 16, 128, "local", 0)
    rc = lib.ow_bigemm_fwd(None, None, None, 1e-6, None, None, 0, None, None, ctypes.byref(plan), 1, 256,
                           _native.OW_DTYPE_BF16, 0, None)
    assert rc == 1 and b"NULL" in lib.ow_last_error()
    p = ctypes.c_void_p(16)
    NB = lib.ow_packed_weight_bytes(4, 128, 256, _native.OW_DTYPE_BF16)
    rc = lib.ow_bigemm_fwd(p, ctypes.c_void_p(32), None, 1e-6, p, p, NB, p, p, ctypes.byref(plan), 1, 256,
                           _native.OW_DTYPE_BF16, _native.OW_FUSE_NORM, None)
    assert rc == 1 and b"norm_weight" in lib.ow_last_error()
    bad = _native.make_plan(14, 14, 512, 8, 128, "local", 0)
    rc = lib.ow_bigemm_fwd(p, ctypes.c_void_p(32), None, 1e-6, p, p, NB, p, p, ctypes.byref(bad), 1, 256,
                           _native.OW_DTYPE_BF16, 0, None)
    assert rc == 2 and b"spatial tile" in lib.ow_last_error()
    rc = lib.ow_bigemm_fwd(p, ctypes.c_void_p(32), None, 1e-6, p, p, NB, p, p, ctypes.byref(plan), 1, 192,
                           _native.OW_DTYPE_BF16, 0, None)
    assert rc == 1 and b"rd=192" in lib.ow_last_error()  # packed size cannot match an unsupported rd
    rc = lib.ow_bigemm_fwd(p, ctypes.c_void_p(32), None, 1e-6, p, p, NB - 2, p, p, ctypes.byref(plan), 1, 256,
                           _native.OW_DTYPE_BF16, 0, None)
    assert rc == 1 and b"packed weights" in lib.ow_last_error()


def test_hip_is_supported_reasons_on_cpu() -> None:
    plan = build_route_plan(14, 14, 512, 16, 128, "local")
    ok, reason = hip_is_supported(torch.randn(1, 14, 14, 512), plan, torch.randn(4, 128, 256))
    assert not ok and reason == "CUDA is unavailable"


def test_check_raises_with_library_message() -> None:
    lib = _native.lib()
    plan = _native.make_plan(0, 14, 512, 16, 128, "local", 0)
    q = ctypes.c_int32()
    with pytest.raises(ValueError, match="height/width"):
        _native.check(lib.ow_plan_dims(ctypes.byref(plan), ctypes.byref(q), ctypes.byref(q)), "ow_plan_dims")
