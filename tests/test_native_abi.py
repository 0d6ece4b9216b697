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
    # head (3 token-operand rows of 64 lanes x 8) + q_c * 3*d*rd elements, 2 bytes each
    assert lib.ow_packed_weight_bytes(4, 128, 256, _native.OW_DTYPE_BF16) == 2 * (1536 + 4 * 3 * 128 * 256)
    # d = 64, rd = 128: a second section of 16x16x32 fragments, the same element count again
    assert lib.ow_packed_weight_bytes(2, 64, 128, _native.OW_DTYPE_F16) == 2 * (1536 + 2 * 2 * 3 * 64 * 128)
    assert lib.ow_packed_weight_bytes(2, 64, 256, _native.OW_DTYPE_F16) == 2 * (1536 + 2 * 3 * 64 * 256)
    assert lib.ow_packed_weight_bytes(2, 64, 128, _native.OW_DTYPE_F32) == 4 * (1536 + 2 * 3 * 64 * 128)
    assert lib.ow_packed_weight_bytes(0, 64, 128, _native.OW_DTYPE_F16) == 0


def test_fwd_rejects_bad_arguments_without_touching_the_gpu() -> None:
    lib = _native.lib()
    plan = _native.make_plan(14, 14, 512, 16, 128, "local", 0)
    bf16 = _native.OW_DTYPE_BF16

    def fwd(x, out, packed_bytes, p, rd=256, flags=0, ws=None, ws_bytes=0):
        return lib.ow_bigemm_fwd(x, out, 1e-6, P, packed_bytes, P, P, ctypes.byref(p), 1, rd, bf16, flags,
                                 ws, ws_bytes, None)

    P = None
    assert fwd(None, None, 0, plan) == 1 and b"NULL" in lib.ow_last_error()
    P = ctypes.c_void_p(16)
    NB = lib.ow_packed_weight_bytes(4, 128, 256, bf16)
    out = ctypes.c_void_p(32)
    # An unaligned x takes element access, whose RMSNorm statistics come from a pass into the
    # workspace: without one the call is refused before any launch.
    x_unaligned = ctypes.c_void_p(18)
    assert fwd(x_unaligned, out, NB, plan, flags=_native.OW_FUSE_NORM) == 1 and b"workspace" in lib.ow_last_error()
    assert lib.ow_fwd_workspace_bytes(ctypes.byref(plan), 3, _native.OW_FUSE_NORM) == 3 * 196 * 4
    assert lib.ow_fwd_workspace_bytes(ctypes.byref(plan), 3, 0) == 0
    bad = _native.make_plan(14, 14, 512, 8, 128, "local", 0)
    assert fwd(P, out, NB, bad) == 2 and b"spatial tile" in lib.ow_last_error()
    assert fwd(P, out, NB, plan, rd=192) == 1 and b"rd=192" in lib.ow_last_error()
    assert fwd(P, out, NB - 2, plan) == 1 and b"packed weights" in lib.ow_last_error()
    assert fwd(P, P, NB, plan) == 1 and b"alias" in lib.ow_last_error()
    assert lib.ow_rms_scale(None, None, 4, 512, 1e-6, bf16, None) == 1
    assert lib.ow_rms_scale(None, None, 0, 512, 1e-6, bf16, None) == 0  # empty: nothing launched


def test_fwd_chain_rejects_bad_arguments_without_touching_the_gpu() -> None:
    lib = _native.lib()
    plan = _native.make_plan(14, 14, 512, 16, 128, "local", 0)
    bf16, f32 = _native.OW_DTYPE_BF16, _native.OW_DTYPE_F32
    P, out = ctypes.c_void_p(16), ctypes.c_void_p(32)
    NB = lib.ow_packed_weight_bytes(4, 128, 256, bf16)
    written = ctypes.c_int32(7)

    def chain(dtype=bf16, flags=_native.OW_FUSE_NORM, stats_in=None, parts=0, w=ctypes.byref(written), x=P,
              stats_out=None):
        return lib.ow_bigemm_fwd_chain(x, out, 1e-6, P, NB, P, P, None, ctypes.byref(plan), 1, 256, dtype, flags,
                                       stats_in, parts, stats_out, w, None, 0, None)

    assert chain(w=None) == 1 and b"stats_written" in lib.ow_last_error()
    assert chain(dtype=f32) == 2 and written.value == 0
    assert chain(stats_in=P, parts=0) == 1 and b"stats_in_parts" in lib.ow_last_error()
    assert chain(stats_in=P, parts=65) == 1 and b"stats_in_parts" in lib.ow_last_error()
    assert chain(stats_in=P, parts=4, flags=0) == 1 and b"OW_FUSE_NORM" in lib.ow_last_error()
    written.value = 7
    # Unaligned x: element access, RMSNorm statistics from a workspace pass; none is given.
    assert chain(x=ctypes.c_void_p(18)) == 1 and b"workspace" in lib.ow_last_error() and written.value == 0
    # stats_in ([196, 4] floats) and stats_out ([196, 4]) must not share memory.
    base = 1 << 20
    for s_in, s_out in ((base, base), (base, base + 4 * 196 * 4 - 4), (base + 4, base)):
        assert chain(stats_in=ctypes.c_void_p(s_in), parts=4, stats_out=ctypes.c_void_p(s_out)) == 1
        assert b"overlap" in lib.ow_last_error()


def test_bwd_channel_entries_reject_bad_arguments_without_touching_the_gpu() -> None:
    """The d = 128 backward entry points (tiles and routed forms) refuse unsupported plans, bad
    sizes and NULL or unaligned buffers before any launch."""
    lib = _native.lib()
    bf16 = _native.OW_DTYPE_BF16
    P = ctypes.c_void_p(16)
    NB = lib.ow_bwd_packed_bytes(4, 128, 256)
    assert NB == 4 * (256 // 32) * (3 * 128 // 16 + 6 * 128 // 32) * 1024
    plan = _native.make_plan(14, 14, 512, 16, 128, "shifted", 0)
    radix = _native.make_plan(14, 14, 512, 16, 128, "radix", 1)
    d64 = _native.make_plan(28, 28, 256, 16, 64, "local", 0)
    slots = 2 * 13 * 16
    n_part = lib.ow_bwd_channel_partials(slots, 4)
    assert n_part > 0 and lib.ow_bwd_channel_partials(slots + 8, 4) == 0

    def chan(x=P, nb=NB, rd=256, dtype=bf16, s=slots):
        return lib.ow_bwd_channel(x, P, P, P, P, P, nb, P, P, P, P, P, P, s, 4, 128, rd, dtype, None)

    def chan_routed(p=plan, x=P, nb=NB, batch=2):
        return lib.ow_bwd_channel_routed(x, P, None, P, ctypes.byref(p), batch, P, P, P, P, nb, P, P, P, P, P, P,
                                         256, bf16, None)

    def chan2_routed(p=plan, g=P, npart=n_part, batch=2):
        return lib.ow_bwd_channel2_routed(P, P, None, P, P, P, P, P, P, NB, P, ctypes.byref(p), batch, g, P, npart,
                                          256, bf16, None)

    assert chan(rd=192) == 2 and b"rd in {128, 256}" in lib.ow_last_error()
    assert chan(dtype=_native.OW_DTYPE_F32) == 2
    assert chan(s=slots + 8) == 1 and b"multiple of 16" in lib.ow_last_error()
    assert chan(nb=NB - 2) == 1 and b"packed backward weights" in lib.ow_last_error()
    assert chan(x=None) == 1 and b"NULL" in lib.ow_last_error()
    assert chan(x=ctypes.c_void_p(18)) == 1 and b"aligned" in lib.ow_last_error()
    assert chan(s=0) == 0  # empty: nothing launched
    assert chan_routed(p=radix) == 2 and b"identity channel order" in lib.ow_last_error()
    assert chan_routed(p=d64) == 2
    assert chan_routed(x=None) == 1 and b"NULL" in lib.ow_last_error()
    assert chan_routed(batch=-1) == 1 and b"bad batch" in lib.ow_last_error()
    assert chan_routed(batch=1 << 22) == 1 and b"2 GiB" in lib.ow_last_error()
    assert chan2_routed(p=radix) == 2 and b"identity channel order" in lib.ow_last_error()
    assert chan2_routed(g=None) == 1 and b"NULL" in lib.ow_last_error()
    assert chan2_routed(npart=n_part + 1) == 1 and b"ow_bwd_channel_partials" in lib.ow_last_error()
    assert chan2_routed(g=ctypes.c_void_p(18)) == 1 and b"aligned" in lib.ow_last_error()

    # The d = 64 parameter-gradient reduction over the fused kernel's fragment-ordered tiles.
    n_red = lib.ow_bwd_param_reduce64_partials(64 * 32, 2, 128)
    assert n_red > 0 and n_red % 2 == 0
    assert lib.ow_bwd_param_reduce64_partials(64 * 32 + 16, 2, 128) == 0
    assert lib.ow_bwd_param_reduce64_partials(64 * 32, 2, 192) == 0

    NB64 = lib.ow_bwd_packed_bytes(2, 64, 128)

    def reduce64(n=n_red, s=64 * 32, rd=128, pu=P, nb=NB64):
        return lib.ow_bwd_param_reduce64(pu, P, P, P, nb, P, n, s, 2, rd, bf16, None)

    assert reduce64(rd=192) == 2 and b"rd in {128, 256}" in lib.ow_last_error()
    assert reduce64(s=64 * 32 + 16) == 1 and b"multiple of 32" in lib.ow_last_error()
    assert reduce64(nb=NB64 - 2) == 1 and b"packed backward weights" in lib.ow_last_error()
    assert reduce64(n=n_red + 2) == 1 and b"ow_bwd_param_reduce64_partials" in lib.ow_last_error()
    assert reduce64(pu=None) == 1 and b"NULL" in lib.ow_last_error()
    assert reduce64(pu=ctypes.c_void_p(18)) == 1 and b"aligned" in lib.ow_last_error()
    assert reduce64(s=1 << 24, n=lib.ow_bwd_param_reduce64_partials(1 << 24, 2, 128)) == 1
    assert b"2 GiB" in lib.ow_last_error()
    assert reduce64(s=0, n=0) == 0  # empty: nothing launched

    # The d = 128 reduction over the channel kernels' slot-major intermediates.
    n128 = lib.ow_bwd_param_reduce128_partials(13 * 16, 3, 256)
    assert n128 > 0 and n128 % 3 == 0
    assert lib.ow_bwd_param_reduce128_partials(13 * 16 + 8, 3, 256) == 0
    assert lib.ow_bwd_param_reduce128_partials(13 * 16, 3, 192) == 0

    def reduce128(n=n128, s=13 * 16, rd=256, pu=P, q_c=3):
        return lib.ow_bwd_param_reduce128(pu, P, P, P, P, P, P, n, s, q_c, rd, bf16, None)

    assert reduce128(rd=192) == 2 and b"rd in {128, 256}" in lib.ow_last_error()
    assert reduce128(s=13 * 16 + 8) == 1 and b"multiple of 16" in lib.ow_last_error()
    assert reduce128(n=n128 + 3) == 1 and b"ow_bwd_param_reduce128_partials" in lib.ow_last_error()
    assert reduce128(pu=None) == 1 and b"NULL" in lib.ow_last_error()
    assert reduce128(pu=ctypes.c_void_p(18)) == 1 and b"aligned" in lib.ow_last_error()
    assert reduce128(s=1 << 22, n=lib.ow_bwd_param_reduce128_partials(1 << 22, 3, 256)) == 1
    assert b"2 GiB" in lib.ow_last_error()
    assert reduce128(s=0, n=0) == 0  # empty: nothing launched

    # The fixed-order row sum.
    assert lib.ow_sum_rows(P, 4, 6, P, None) == 1 and b"multiple of 4" in lib.ow_last_error()
    assert lib.ow_sum_rows(P, 0, 8, P, None) == 1 and b"bad shape" in lib.ow_last_error()
    assert lib.ow_sum_rows(None, 4, 8, P, None) == 1 and b"NULL" in lib.ow_last_error()
    assert lib.ow_sum_rows(P, 4, 8, ctypes.c_void_p(20), None) == 1 and b"aligned" in lib.ow_last_error()
    assert lib.ow_sum_rows(P, 4, 0, P, None) == 0  # no columns: nothing launched

    # The small-parameter conversion.
    srcs = (ctypes.c_void_p * 2)(16, 32)
    dts = (ctypes.c_int32 * 2)(bf16, _native.OW_DTYPE_F32)
    cnt = (ctypes.c_int64 * 2)(4, 8)
    assert lib.ow_small_to_f32(srcs, dts, cnt, 0, P, None) == 1 and b"between 1 and 8" in lib.ow_last_error()
    assert lib.ow_small_to_f32(srcs, dts, cnt, 9, P, None) == 1
    assert lib.ow_small_to_f32(srcs, (ctypes.c_int32 * 2)(bf16, 7), cnt, 2, P, None) == 1
    assert b"unknown dtype" in lib.ow_last_error()
    assert lib.ow_small_to_f32(srcs, dts, (ctypes.c_int64 * 2)(4, -1), 2, P, None) == 1
    assert lib.ow_small_to_f32((ctypes.c_void_p * 2)(None, 32), dts, cnt, 2, P, None) == 1
    assert b"source 0 is NULL" in lib.ow_last_error()
    assert lib.ow_small_to_f32(srcs, dts, cnt, 2, None, None) == 1 and b"NULL" in lib.ow_last_error()
    assert lib.ow_small_to_f32((ctypes.c_void_p * 2)(None, None), dts, (ctypes.c_int64 * 2)(0, 0), 2, P, None) == 0


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


def test_noalloc_rejects_more_rows_than_the_scratch() -> None:
    """The size check of ow_bigemm_fwd_noalloc runs on the host before any device call, so it is
    exercised here without a GPU: the pointers are never dereferenced (a regression fails at the
    device lookup, not in a kernel)."""
    from omniwave_amd.routing import native_plan

    h, w, c, d = 56, 56, 128, 64
    plan = build_route_plan(h, w, c, 16, d, "local", 0)
    b = (1 << 20) // (h * w) + 1
    lib = _native.lib()
    oplan = native_plan(plan)
    nbytes = lib.ow_packed_weight_bytes(c // d, d, 2 * d, _native.OW_DTYPE_BF16)
    flags = _native.OW_FUSE_NORM | _native.OW_FUSE_RESIDUAL
    fake = ctypes.c_void_p(18)  # unaligned: element access, which needs the row scales
    rc = lib.ow_bigemm_fwd_noalloc(fake, ctypes.c_void_p(1 << 20), 1e-6, ctypes.c_void_p(1 << 24), nbytes, fake, fake,
                                   ctypes.byref(oplan), b, 2 * d, _native.OW_DTYPE_BF16, flags, None)
    assert rc == 2 and b"scratch" in lib.ow_last_error()
