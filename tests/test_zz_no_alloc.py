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


def run_fwd(x, packed, plan, dtype):
    """ow_bigemm_fwd with a workspace of its own (the entry the no-allocation one must equal)."""
    lib = _native.lib()
    tok, ch = device_tables(plan, DEV)
    oplan = native_plan(plan)
    b = x.shape[0]
    d = int(plan.channel_indices.shape[1])
    out_ref = torch.empty(x.shape, dtype=dtype, device=DEV)
    ws_bytes = lib.ow_fwd_workspace_bytes(ctypes.byref(oplan), b, FLAGS)
    ws = torch.empty(max(ws_bytes // 4, 1), dtype=torch.float32, device=DEV)
    stream = torch.cuda.current_stream(DEV).cuda_stream
    _native.check(lib.ow_bigemm_fwd(x.data_ptr(), out_ref.data_ptr(), 1e-6, packed.data_ptr(), packed.numel(),
                                    tok.data_ptr(), ch.data_ptr(), ctypes.byref(oplan), b, 2 * d, _DTYPE_CODE[dtype],
                                    FLAGS, ws.data_ptr(), ws_bytes, stream), "ow_bigemm_fwd")
    return out_ref


def run_both(x, packed, plan, dtype):
    lib = _native.lib()
    tok, ch = device_tables(plan, DEV)
    oplan = native_plan(plan)
    b = x.shape[0]
    d = int(plan.channel_indices.shape[1])
    out_ref = run_fwd(x, packed, plan, dtype)
    out_new = torch.empty(x.shape, dtype=dtype, device=DEV)
    stream = torch.cuda.current_stream(DEV).cuda_stream
    code = _DTYPE_CODE[dtype]
    _native.check(lib.ow_bigemm_fwd_noalloc(x.data_ptr(), out_new.data_ptr(), 1e-6, packed.data_ptr(),
                                            packed.numel(), tok.data_ptr(), ch.data_ptr(), ctypes.byref(oplan), b,
                                            2 * d, code, FLAGS, stream), "ow_bigemm_fwd_noalloc")
    torch.cuda.synchronize()
    return out_ref, out_new


def test_noalloc_inside_graph_capture() -> None:
    """The entry called first inside a torch.cuda.graph capture (in a process that has not called
    it before, this is where the per-device scratch lookup happens): every replay of the graph
    equals ow_bigemm_fwd's eager output bit for bit, with eager work between the replays."""
    h, w, c, d, dtype = 14, 14, 512, 128, torch.bfloat16
    announce(f"noalloc inside graph capture {h}x{w}x{c} {dtype} unaligned B=3")
    plan = omniwave_amd.build_route_plan(h, w, c, 16, d, "shifted", 0)
    packed = weights(c, d, dtype, plan, seed=5)
    x = activations(3, h, w, c, dtype, aligned=False, seed=21)  # element access: uses the scratch
    lib = _native.lib()
    tok, ch = device_tables(plan, DEV)
    oplan = native_plan(plan)
    ref = run_fwd(x, packed, plan, dtype)
    torch.cuda.synchronize()
    out = torch.empty(x.shape, dtype=dtype, device=DEV)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        stream = torch.cuda.current_stream(DEV).cuda_stream
        _native.check(lib.ow_bigemm_fwd_noalloc(x.data_ptr(), out.data_ptr(), 1e-6, packed.data_ptr(),
                                                packed.numel(), tok.data_ptr(), ch.data_ptr(), ctypes.byref(oplan),
                                                3, 2 * d, _DTYPE_CODE[dtype], FLAGS, stream),
                      "ow_bigemm_fwd_noalloc (captured)")
    for i in range(3):
        out.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ref), f"replay {i}: {(out != ref).sum().item()} elements differ"
        run_both(activations(1, h, w, c, dtype, aligned=False, seed=30 + i), packed, plan, dtype)


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
