"""GPU checks of the backward's slot reductions and partial sums (``-m gpu``).

``ow_bwd_param_reduce128`` (dB_u'' = P_u^T dU', dB_v'' = P_v^T dV', dB_o'' = Z^T dW' per channel
group, the sums over slots that the reference's autograd forms inside its GEMMs,
omniweave/ops/triton.py:256-292) is compared with float64 products of the same 16-bit
intermediates: the products of 16-bit values are exact in fp32, so only the fp32 summation
order differs (rel-L2 <= 1e-5).  ``ow_sum_rows`` is compared with a float64 sum and must give
identical bits on a second call; ``ow_small_to_f32`` equals torch's (exact) widening conversion.
"""

from __future__ import annotations

import ctypes
import sys

import pytest
import torch

from omniwave_amd import _native

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda", 0)
CODE = {torch.bfloat16: _native.OW_DTYPE_BF16, torch.float16: _native.OW_DTYPE_F16}


def announce(msg: str) -> None:
    print(f"\n[gpu-case] {msg}", file=sys.stderr, flush=True)


def rel_l2(a: torch.Tensor, b: torch.Tensor) -> float:
    a, b = a.double(), b.double()
    return float((a - b).norm() / b.norm().clamp_min(1e-30))


def sum_rows(partial: torch.Tensor, rows: int, out: torch.Tensor) -> None:
    lib = _native.lib()
    stream = torch.cuda.current_stream(DEV).cuda_stream
    _native.check(lib.ow_sum_rows(partial.data_ptr(), rows, out.numel(), out.data_ptr(), stream), "ow_sum_rows")


def reduce128(pu, pv, dw, z, du, dv, q_c: int, slots: int, rd: int, dtype) -> torch.Tensor:
    """[3, q_c, 128 * rd] fp32: dB_u'', dB_v'', dB_o'' of every group, via the partial rows."""
    lib = _native.lib()
    stream = torch.cuda.current_stream(DEV).cuda_stream
    n = lib.ow_bwd_param_reduce128_partials(slots, q_c, rd)
    assert n > 0 and n % q_c == 0
    red = torch.empty(n, 3 * 128 * rd, dtype=torch.float32, device=DEV)
    _native.check(lib.ow_bwd_param_reduce128(pu.data_ptr(), pv.data_ptr(), dw.data_ptr(), z.data_ptr(),
                                             du.data_ptr(), dv.data_ptr(), red.data_ptr(), n, slots, q_c, rd,
                                             CODE[dtype], stream), "ow_bwd_param_reduce128")
    out = torch.empty(3, q_c, 128 * rd, dtype=torch.float32, device=DEV)
    sum_rows(red, n // q_c, out)
    torch.cuda.synchronize()
    return out


REDUCE_CASES = [  # (q_c, slots, rd, dtype)
    (3, 13 * 16, 256, torch.bfloat16),        # one image of 14x14: slots % 32 == 16
    (2, 2 * 4 * 16, 128, torch.float16),      # rd = d
    (4, 128 * 13 * 16, 256, torch.bfloat16),  # 14x14x512, B = 128: many steps per range
    (8, 128 * 4 * 16, 256, torch.bfloat16),   # 7x7x1024, B = 128
]


@pytest.mark.parametrize("q_c,slots,rd,dtype", REDUCE_CASES,
                         ids=[f"qc{c[0]}-s{c[1]}-rd{c[2]}-{str(c[3])[6:]}" for c in REDUCE_CASES])
def test_param_reduce128_matches_float64(q_c, slots, rd, dtype) -> None:
    announce(f"param_reduce128 q_c={q_c} slots={slots} rd={rd} {dtype}")
    gen = torch.Generator().manual_seed(slots + rd)
    t = lambda w: torch.randn(q_c, slots, w, generator=gen).to(dtype)  # noqa: E731
    pu, pv, dw = t(128), t(128), t(128)
    z, du, dv = t(rd), t(rd), t(rd)
    got = reduce128(*[v.to(DEV) for v in (pu, pv, dw, z, du, dv)], q_c, slots, rd, dtype).cpu()
    want = torch.stack([
        torch.bmm(pu.double().transpose(1, 2), du.double()).reshape(q_c, -1),
        torch.bmm(pv.double().transpose(1, 2), dv.double()).reshape(q_c, -1),
        torch.bmm(z.double().transpose(1, 2), dw.double()).reshape(q_c, -1),
    ])
    for k, name in enumerate(("dB_u", "dB_v", "dB_o")):
        err = rel_l2(got[k], want[k])
        print(f"[reduce128 q_c={q_c} slots={slots} rd={rd}] {name} rel-L2 {err:.2e}", flush=True)
        assert err <= 1e-5, f"{name}: rel-L2 {err:.2e}"


@pytest.mark.parametrize("rows,cols", [(1, 768), (5, 280), (21, 3 * 4 * 128 * 256), (300, 768), (64, 1024)])
def test_sum_rows_matches_float64_and_repeats_bitwise(rows, cols) -> None:
    announce(f"sum_rows rows={rows} cols={cols}")
    gen = torch.Generator().manual_seed(rows * 7 + cols)
    partial = torch.randn(rows, cols, generator=gen)
    p = partial.to(DEV)
    outs = []
    for _ in range(2):
        out = torch.full((cols,), float("nan"), device=DEV)
        sum_rows(p, rows, out)
        torch.cuda.synchronize()
        outs.append(out.cpu())
    want = partial.double().sum(dim=0)
    err = rel_l2(outs[0], want)
    assert err <= 1e-6, f"rel-L2 {err:.2e}"
    assert torch.equal(outs[0], outs[1]), "two calls on the same input differ"


def test_small_to_f32_converts_each_source_exactly() -> None:
    """ow_small_to_f32: bf16, fp16 and fp32 sources of ragged lengths into one fp32 buffer,
    equal to torch's conversion of each (a widening conversion: exact)."""
    announce("small_to_f32 bf16 / fp16 / fp32 sources")
    gen = torch.Generator().manual_seed(5)
    srcs = [torch.randn(n, generator=gen).to(dt).to(DEV)
            for n, dt in ((7, torch.bfloat16), (256, torch.float16), (33, torch.float32), (1, torch.bfloat16))]
    lib = _native.lib()
    n = len(srcs)
    out = torch.full((sum(t.numel() for t in srcs),), float("nan"), device=DEV)
    code = {torch.bfloat16: _native.OW_DTYPE_BF16, torch.float16: _native.OW_DTYPE_F16,
            torch.float32: _native.OW_DTYPE_F32}
    _native.check(lib.ow_small_to_f32((ctypes.c_void_p * n)(*[t.data_ptr() for t in srcs]),
                                      (ctypes.c_int32 * n)(*[code[t.dtype] for t in srcs]),
                                      (ctypes.c_int64 * n)(*[t.numel() for t in srcs]), n, out.data_ptr(),
                                      torch.cuda.current_stream(DEV).cuda_stream), "ow_small_to_f32")
    torch.cuda.synchronize()
    assert torch.equal(out.cpu(), torch.cat([t.float() for t in srcs]).cpu())
