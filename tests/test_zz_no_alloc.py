"""ow_bigemm_fwd_noalloc: the forward with the library's own scratch instead of a workspace.

The entry point has no counterpart in the reference; it is for callers that cannot allocate.
Through the C ABI (ctypes), on two calls in a row — the second with a smaller input, so the
scratch holds the first call's row scales when the second starts — its output must equal
ow_bigemm_fwd's bit for bit on paths that use the scratch (element access of unaligned rows,
fp32 activations) and on one that does not (aligned rows, statistics read with the tile).
"""

from __future__ import annotations

import ctypes
import sys

import pytest
import torch

import omniwave_amd
from omniwave_amd import _native
from omniwave_amd.hip import _DTYPE_CODE, pack_weights
from omniwave_amd.routing import device_tables, native_plan

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda", 0)
FLAGS = _native.OW_FUSE_NORM | _native.OW_FUSE_RESIDUAL
SCRATCH_ROWS = 1 << 20


def announce(msg: str) -> None:
    print(f"\n[gpu-case] {msg}", file=sys.stderr, flush=True)


def weights(c, d, dtype, plan, seed=0):
    gen = torch.Generator().manual_seed(seed)
    q_c, rd = c // d, 2 * d
    p = [torch.randn(16, 16, generator=gen) / 4 for _ in range(3)]
    p += [torch.randn(q_c, d, rd, generator=gen) / d ** 0.5, torch.randn(q_c, d, rd, generator=gen) / d ** 0.5,
          torch.randn(q_c, rd, d, generator=gen) / rd ** 0.5]
    gamma = torch.rand(c, generator=gen) + 0.5
    norm_w = torch.rand(c, generator=gen) + 0.5
    p = [t.to(DEV) for t in p]
    return pack_weights(*p, dtype, norm_weight=norm_w.to(DEV), plan=plan, gamma=gamma.to(DEV))


def activations(b, h, w, c, dtype, aligned, seed):
    """x on the device; unaligned: a view starting one element into its storage."""
    gen = torch.Generator().manual_seed(seed)
    src = torch.randn(b, h, w, c, generator=gen).to(dtype)
    if aligned:
        return src.to(DEV)
    buf = torch.empty(src.numel() + 1, dtype=dtype, device=DEV)
    x = buf[1:].view(b, h, w, c)
    x.copy_(src.to(DEV))
    return x


def run_both(x, packed, plan, dtype):
    lib = _native.lib()
    tok, ch = device_tables(plan, DEV)
    oplan = native_plan(plan)
    b = x.shape[0]
    d = int(plan.channel_indices.shape[1])
    out_ref = torch.empty(x.shape, dtype=dtype, device=DEV)
    out_new = torch.empty(x.shape, dtype=dtype, device=DEV)
    ws_bytes = lib.ow_fwd_workspace_bytes(ctypes.byref(oplan), b, FLAGS)
    ws = torch.empty(max(ws_bytes // 4, 1), dtype=torch.float32, device=DEV)
    stream = torch.cuda.current_stream(DEV).cuda_stream
    code = _DTYPE_CODE[dtype]
    _native.check(lib.ow_bigemm_fwd(x.data_ptr(), out_ref.data_ptr(), 1e-6, packed.data_ptr(), packed.numel(),
                                    tok.data_ptr(), ch.data_ptr(), ctypes.byref(oplan), b, 2 * d, code, FLAGS,
                                    ws.data_ptr(), ws_bytes, stream), "ow_bigemm_fwd")
    _native.check(lib.ow_bigemm_fwd_noalloc(x.data_ptr(), out_new.data_ptr(), 1e-6, packed.data_ptr(),
                                            packed.numel(), tok.data_ptr(), ch.data_ptr(), ctypes.byref(oplan), b,
                                            2 * d, code, FLAGS, stream), "ow_bigemm_fwd_noalloc")
    torch.cuda.synchronize()
    return out_ref, out_new


CASES = [  # (H, W, C, d, dtype, aligned, batches): scratch paths first, then the in-kernel one
    (14, 14, 512, 128, torch.bfloat16, False, (6, 2)),
    (28, 28, 256, 64, torch.float16, False, (3, 1)),
    (7, 7, 1024, 128, torch.float32, True, (5, 2)),
    (14, 14, 512, 128, torch.bfloat16, True, (4, 1)),
]


@pytest.mark.parametrize("h,w,c,d,dtype,aligned,batches", CASES,
                         ids=[f"{h}x{w}x{c}-{str(t)[6:]}-{'al' if a else 'unal'}" for h, w, c, _, t, a, _ in CASES])
def test_noalloc_matches_fwd_on_two_calls(h, w, c, d, dtype, aligned, batches) -> None:
    plan = omniwave_amd.build_route_plan(h, w, c, 16, d, "shifted", 0)
    packed = weights(c, d, dtype, plan)
    for i, b in enumerate(batches):
        announce(f"noalloc {h}x{w}x{c} {dtype} aligned={aligned} call {i + 1} B={b}")
        x = activations(b, h, w, c, dtype, aligned, seed=10 + i)
        ref, new = run_both(x, packed, plan, dtype)
        assert torch.equal(ref, new), f"call {i + 1} (B={b}): {(ref != new).sum().item()} elements differ"


def test_noalloc_rejects_more_rows_than_the_scratch() -> None:
    announce("noalloc size limit")
    h, w, c, d = 56, 56, 128, 64
    plan = omniwave_amd.build_route_plan(h, w, c, 16, d, "local", 0)
    b = SCRATCH_ROWS // (h * w) + 1
    lib = _native.lib()
    oplan = native_plan(plan)
    nbytes = lib.ow_packed_weight_bytes(c // d, d, 2 * d, _native.OW_DTYPE_BF16)
    fake = ctypes.c_void_p(18)  # unaligned: element access, which needs the row scales
    rc = lib.ow_bigemm_fwd_noalloc(fake, ctypes.c_void_p(1 << 20), 1e-6, ctypes.c_void_p(1 << 24), nbytes, fake, fake,
                                   ctypes.byref(oplan), b, 2 * d, _native.OW_DTYPE_BF16, FLAGS, None)
    assert rc == 2 and b"scratch" in lib.ow_last_error()
