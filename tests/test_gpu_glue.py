"""Backbone glue on the GPU (``-m gpu``): the stem kernel against the oracle stem, the block
output written in space_to_depth layout against space_to_depth of the fused block's output
(bit-exact: the same kernel math, only the output rows move), and the model's fused-glue
forward against its forward_features composition (bit-exact)."""

from __future__ import annotations

import sys

import pytest
import torch

import omniwave_amd
from omniwave_amd.backbone import space_to_depth_nhwc
from omniwave_amd.block import OmniWeaveBlock
from omniwave_amd.hip import (bigemm_block_chain_hip, bigemm_block_hip, bigemm_block_s2d_hip, stem_hip,
                              stem_is_supported)
from oracle.backbone import stem_reference

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda", 0)
# Relative rounding bound of one conversion to the dtype (half an ulp), doubled for the
# fp32 accumulation-order difference.
ULP = {torch.bfloat16: 2.0 ** -8, torch.float16: 2.0 ** -11}


def announce(msg: str) -> None:
    print(f"\n[gpu-case] {msg}", file=sys.stderr, flush=True)


STEM_CASES = [(2, 224, 224, 128), (3, 36, 44, 96), (1, 288, 272, 64), (2, 16, 8, 256), (1, 8, 8, 32), (2, 12, 20, 192)]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "f16"])
@pytest.mark.parametrize("case", STEM_CASES, ids=[f"b{b}_{h}x{w}_n{n}" for b, h, w, n in STEM_CASES])
def test_stem_matches_oracle(case, dtype) -> None:
    b, h, w, n = case
    announce(f"stem B={b} {h}x{w} N={n} dtype={dtype}")
    gen = torch.Generator().manual_seed(h * w + n)
    img = torch.randn(b, 3, h, w, generator=gen).to(dtype)
    wt = (torch.randn(n, 48, generator=gen) / 48 ** 0.5).to(dtype)
    with torch.no_grad():
        got = stem_hip(img.to(DEV), wt.to(DEV))
    torch.cuda.synchronize()
    want = stem_reference(img, wt)
    assert got.shape == want.shape and got.dtype == dtype
    err = (got.float().cpu() - want).abs()
    bound = want.abs() * ULP[dtype] + 1e-5
    assert bool((err <= bound).all()), f"max excess {(err - bound).max().item():.3e}"


def test_stem_rejects_unsupported_inputs() -> None:
    announce("stem argument checks")
    img = torch.zeros(1, 3, 8, 8, dtype=torch.bfloat16, device=DEV)
    w = torch.zeros(128, 48, dtype=torch.bfloat16, device=DEV)
    assert stem_is_supported(img, w)[0]
    assert not stem_is_supported(img[:, :, :6], w)[0]
    assert not stem_is_supported(img, w[:, :47])[0]
    assert not stem_is_supported(img, w[:100])[0]
    assert not stem_is_supported(img.float(), w.float())[0]
    with pytest.raises(RuntimeError):
        stem_hip(img.float(), w.float())
    with pytest.raises(RuntimeError, match="inference-only"):
        stem_hip(img, w.clone().requires_grad_(True))


STAGES = {"s1": (56, 56, 128, 64), "s2": (28, 28, 256, 64), "s3": (14, 14, 512, 128), "pad": (6, 10, 96, 64)}
S2D_CASES = [("s1", "local", 0), ("s1", "shifted", 0), ("s1", "radix", 1), ("s2", "local", 0), ("s2", "radix", 2),
             ("s3", "local", 0), ("s3", "shifted", 0), ("s3", "radix", 1), ("s3", "radix", 2), ("pad", "local", 0)]


def make_case(b, h, w, c, d, route, level, dtype, seed=0):
    gen = torch.Generator().manual_seed(seed)
    plan = omniwave_amd.build_route_plan(h, w, c, 16, d, route, level)
    q_c, rd = plan.channel_indices.shape[0], 2 * d
    x = torch.randn(b, h, w, c, generator=gen).to(dtype).to(DEV)
    p = dict(a_u=torch.randn(16, 16, generator=gen) / 4.0, a_v=torch.randn(16, 16, generator=gen) / 4.0,
             a_o=torch.randn(16, 16, generator=gen) / 4.0, b_u=torch.randn(q_c, d, rd, generator=gen) / d ** 0.5,
             b_v=torch.randn(q_c, d, rd, generator=gen) / d ** 0.5, b_o=torch.randn(q_c, rd, d, generator=gen) / rd ** 0.5,
             gamma=torch.full((c,), 1.0))
    nw = (torch.rand(c, generator=gen) + 0.5).to(DEV)
    return plan, x, {k: v.to(DEV) for k, v in p.items()}, nw


@pytest.mark.parametrize("variant", ["bf16", "f16", "fp8"])
@pytest.mark.parametrize("stage,route,level", S2D_CASES, ids=[f"{s}-{r}{l}" for s, r, l in S2D_CASES])
def test_block_s2d_equals_space_to_depth_of_block(stage, route, level, variant) -> None:
    h, w, c, d = STAGES[stage]
    dtype = torch.float16 if variant == "f16" else torch.bfloat16
    fp8 = variant == "fp8"
    announce(f"block s2d stage={stage} route={route}{level} variant={variant} B=3")
    plan, x, p, nw = make_case(3, h, w, c, d, route, level, dtype)
    with torch.no_grad():
        want = space_to_depth_nhwc(bigemm_block_hip(x, nw, plan, **p, fp8=fp8), 2)
        got = bigemm_block_s2d_hip(x, nw, plan, **p, factor=2, fp8=fp8)
    torch.cuda.synchronize()
    assert got.shape == want.shape
    assert torch.equal(got, want)


def test_block_s2d_is_inference_only() -> None:
    announce("block s2d under autograd")
    plan, x, p, nw = make_case(1, 14, 14, 512, 128, "local", 0, torch.bfloat16)
    p["b_u"].requires_grad_(True)
    with pytest.raises(RuntimeError, match="inference-only"):
        bigemm_block_s2d_hip(x, nw, plan, **p)


@pytest.mark.parametrize("fp8", [False, True], ids=["bf16", "fp8"])
def test_model_fused_glue_matches_forward_features(fp8) -> None:
    announce(f"omniweave_t fused glue vs forward_features B=2 fp8={fp8}")
    torch.manual_seed(0)
    model = omniwave_amd.create_model("omniweave_t").eval()
    with torch.no_grad():
        for stage in model.stages:
            for blk in stage.blocks:
                blk.gamma.fill_(1.0)
    model = model.to(device=DEV, dtype=torch.bfloat16)
    if fp8:
        omniwave_amd.enable_fp8(model, min_channel_tile=64)
    x = torch.randn(2, 3, 224, 224, generator=torch.Generator().manual_seed(1)).to(DEV, torch.bfloat16)
    with torch.no_grad():
        got = model(x)
        feats = model.forward_features(x)
        want = model.head(feats["stage4"].mean(dim=(1, 2)))
        # The same composition with the anchors unfolded: downsample, then anchor.
        h = model._stem(x)
        for i, stage in enumerate(model.stages):
            if i > 0:
                h = model.downsamples[i - 1](h)
            if stage.anchor is not None:
                h = stage.anchor(h)
            h = stage.forward_blocks_s2d(h, 2) if i < 3 else stage.blocks[1](stage.blocks[0](h))
        unfolded = model.head(h.mean(dim=(1, 2)))
    torch.cuda.synchronize()
    # Stages 1-2 and the space_to_depth layout are exact (checked per block above); in stages
    # 3-4 each block after the first takes its RMSNorm statistics from its predecessor's
    # launch (another summation order of the mean of squares: rare one-ulp differences), and
    # folding the anchor into the downsample changes one bf16 rounding of the stage-3/4 entry.
    rel = ((got.float() - want.float()).norm() / want.float().norm()).item()
    rel_unfolded = ((unfolded.float() - want.float()).norm() / want.float().norm()).item()
    print(f"fused glue vs forward_features rel-L2 {rel:.2e}; unfolded anchors {rel_unfolded:.2e}", flush=True)
    assert rel <= 1e-2, rel
    assert rel_unfolded <= 2e-3, rel_unfolded
    if not fp8:  # with autograd on, the reference composition runs (no fused glue, no stem kernel)
        eager = model(x)
        rel_eager = ((eager.float() - want.float()).norm() / want.float().norm()).item()
        assert rel_eager <= 1e-2, rel_eager


def test_model_fused_glue_graph_replays_match_eager() -> None:
    """The inference path (stem kernel, s2d-layout blocks, folded entry GEMMs) captured in one
    HIP graph: every replay, with eager work and synchronisation in between, reproduces the
    eager logits exactly."""
    announce("omniweave_t fused glue under HIP graph capture, B=4")
    torch.manual_seed(0)
    model = omniwave_amd.create_model("omniweave_t").to(device=DEV, dtype=torch.bfloat16).eval()
    x = torch.randn(4, 3, 224, 224, generator=torch.Generator().manual_seed(3)).to(DEV, torch.bfloat16)
    with torch.inference_mode():
        eager = model(x).clone()
        stream = torch.cuda.Stream()
        stream.wait_stream(torch.cuda.current_stream())
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.stream(stream):
            model(x)
            torch.cuda.current_stream().synchronize()
            with torch.cuda.graph(graph, stream=stream):
                logits = model(x)
        torch.cuda.current_stream().wait_stream(stream)
        for k in range(3):
            graph.replay()
            torch.cuda.synchronize()
            assert torch.equal(logits, eager), f"replay {k}"
            model(x[:2])  # eager work between replays
            torch.cuda.synchronize()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "f16"])
@pytest.mark.parametrize("size", [64, 160])
def test_model_fused_glue_other_sizes_and_dtypes(size, dtype) -> None:
    """Other input resolutions (stage grids 16/8/4/2 and 40/20/10/5) and fp16: the inference
    path against the reference composition on the same GPU (forward_features with autograd
    on, which uses neither the stem kernel nor the space_to_depth output)."""
    announce(f"omniweave_t fused glue input {size} dtype={dtype} B=2")
    torch.manual_seed(0)
    model = omniwave_amd.create_model("omniweave_t", input_size=size).eval()
    with torch.no_grad():
        for stage in model.stages:
            for blk in stage.blocks:
                blk.gamma.fill_(0.5)
    model = model.to(device=DEV, dtype=dtype)
    x = torch.randn(2, 3, size, size, generator=torch.Generator().manual_seed(5)).to(DEV, dtype)
    with torch.no_grad():
        got = model(x)
    want = model.head(model.forward_features(x)["stage4"].mean(dim=(1, 2)))  # autograd on: reference glue
    torch.cuda.synchronize()
    rel = ((got.float() - want.float()).norm() / want.float().norm()).item()
    print(f"input {size} {dtype}: rel-L2 {rel:.2e}", flush=True)
    assert rel <= 1e-2, rel


def test_block_s2d_falls_back_when_unsupported() -> None:
    """fp32 activations and odd grids: forward_s2d returns None (the caller composes
    space_to_depth); the backbone path then matches the reference composition."""
    announce("block forward_s2d fallbacks")
    blk = OmniWeaveBlock(height=14, width=14, dim=512, channel_tile=128, route="local", radix_level=0).to(DEV).eval()
    x32 = torch.randn(1, 14, 14, 512, device=DEV)
    with torch.no_grad():
        assert blk.forward_s2d(x32, 2) is None
        assert blk.to(torch.bfloat16).forward_s2d(x32.to(torch.bfloat16), 3) is None  # 14 % 3 != 0
        y = blk.forward_s2d(x32.to(torch.bfloat16), 2)
    assert y is not None and y.shape == (1, 7, 7, 2048)


def _rel(a, b) -> float:
    return ((a.float() - b.float()).norm() / b.float().norm()).item()


# name, H, W, C, d, route, level, fp8: contiguous and strided (radix) d = 128 groups on the
# persistent kernel; d = 64 with the fp8 channel side runs the streamed kernel (8 lanes per
# 64-column group row).
CHAIN_CASES = [("s3", 14, 14, 512, 128, "shifted", 0, False), ("s4", 7, 7, 1024, 128, "shifted", 0, False),
               ("s3b", 14, 14, 256, 128, "shifted", 0, False), ("s3-radix1", 14, 14, 512, 128, "radix", 1, False),
               ("s3-radix2", 14, 14, 512, 128, "radix", 2, False), ("s4-radix1", 7, 7, 1024, 128, "radix", 1, False),
               ("s3-radix1-fp8", 14, 14, 512, 128, "radix", 1, True), ("s2-fp8", 28, 28, 256, 64, "local", 0, True)]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "f16"])
@pytest.mark.parametrize("name,h,w,c,d,route,level,fp8", CHAIN_CASES, ids=[k[0] for k in CHAIN_CASES])
def test_chain_stats_are_group_sums_of_squares(name, h, w, c, d, route, level, fp8, dtype) -> None:
    """A chained launch writes, per output row and channel group, the sum of squares of the
    stored values of the group's channels (the plan's channel table: contiguous or strided); its
    output is the unchained launch's, bit for bit."""
    announce(f"chain stats {name} {dtype} B=3")
    plan, x, p, nw = make_case(3, h, w, c, d, route, level, dtype)
    q_c = c // d
    with torch.no_grad():
        y, stats = bigemm_block_chain_hip(x, None, nw, plan, **p, fp8=fp8)
        want = bigemm_block_hip(x, nw, plan, **p, fp8=fp8)
    torch.cuda.synchronize()
    assert torch.equal(y, want)
    assert stats is not None and stats.shape == (3 * h * w, q_c)
    chan = plan.channel_indices.to(DEV)
    rows = want.float().reshape(3 * h * w, c)
    ref = torch.stack([rows[:, chan[q]].square().sum(-1) for q in range(q_c)], dim=1)
    torch.testing.assert_close(stats, ref, rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("route,level", [("local", 0), ("shifted", 0), ("radix", 1), ("radix", 2)])
@pytest.mark.parametrize("variant", ["bf16", "f16", "fp8"])
def test_chain_consumer_matches_unchained_block(route, level, variant) -> None:
    """A block given its predecessor's statistics (stats_in) reads only its groups' columns; the
    result equals the unchained block's up to the summation order of the mean of squares, and
    both are within the bf16 tolerance of the oracle."""
    from oracle.bigemm import block_reference
    from oracle.routing import build_route_plan as oracle_plan

    dtype = torch.float16 if variant == "f16" else torch.bfloat16
    fp8 = variant == "fp8"
    announce(f"chain consumer s3 {route}{level} {variant} B=4")
    plan0, x0, p0, nw0 = make_case(4, 14, 14, 512, 128, "local", 0, dtype, seed=1)
    plan, _, p, nw = make_case(4, 14, 14, 512, 128, route, level, dtype, seed=2)
    with torch.no_grad():
        x, stats = bigemm_block_chain_hip(x0, None, nw0, plan0, **p0)
        got, nxt = bigemm_block_chain_hip(x, stats, nw, plan, **p, fp8=fp8)
        want = bigemm_block_hip(x, nw, plan, **p, fp8=fp8)
    torch.cuda.synchronize()
    assert stats is not None and nxt is not None  # contiguous and strided d = 128 producers chain
    rel = _rel(got, want)
    equal = (got == want).float().mean().item()
    print(f"chained vs unchained rel-L2 {rel:.2e}, {equal:.4%} elements equal", flush=True)
    assert rel <= 2e-3, rel
    oplan = oracle_plan(14, 14, 512, 16, 128, route, level)
    params = {k: v.to(dtype).float().cpu() for k, v in p.items()}
    params["norm_weight"] = nw.to(dtype).float().cpu()
    ref = block_reference(x.float().cpu(), oplan, params)
    tol = 5e-2 if fp8 else 1e-2
    assert _rel(got.cpu(), ref) <= tol


@pytest.mark.parametrize("route,level", [("shifted", 0), ("radix", 1)])
def test_chain_and_drop_path_multi_round_match_small_batches(route, level) -> None:
    """14x14x512 at B = 256, the model's batch: 832 units on 256 CUs, so the persistent kernel
    runs its multi-round schedules (whole units round robin for contiguous groups, each group's
    pairs split evenly for strided ones).  The chained launch's output and per-group statistics,
    a consumer's output given them, and a block with per-image drop-path scales must equal, bit
    for bit, the same images run in batches of 64 (one unit per workgroup)."""
    b, hw = 256, 14 * 14
    announce(f"chain + drop path multi-round s3 {route}{level} bf16 B={b}")
    plan0, x0, p0, nw0 = make_case(b, 14, 14, 512, 128, route, level, torch.bfloat16, seed=6)
    plan, _, p, nw = make_case(1, 14, 14, 512, 128, route, level, torch.bfloat16, seed=7)
    ds = torch.rand(b, generator=torch.Generator().manual_seed(8)).add_(0.5).to(DEV)
    with torch.no_grad():
        y, st = bigemm_block_chain_hip(x0, None, nw0, plan0, **p0)
        z, st2 = bigemm_block_chain_hip(y, st, nw, plan, **p)
        dr = bigemm_block_hip(x0, nw0, plan0, **p0, drop_scale=ds)
        for i0 in range(0, b, 64):
            sl, rows = slice(i0, i0 + 64), slice(i0 * hw, (i0 + 64) * hw)
            ys, sts = bigemm_block_chain_hip(x0[sl].contiguous(), None, nw0, plan0, **p0)
            zs, st2s = bigemm_block_chain_hip(ys, sts, nw, plan, **p)
            drs = bigemm_block_hip(x0[sl].contiguous(), nw0, plan0, **p0, drop_scale=ds[sl].contiguous())
            assert torch.equal(y[sl], ys) and torch.equal(st[rows], sts), f"producer, images {sl}"
            assert torch.equal(z[sl], zs) and torch.equal(st2[rows], st2s), f"consumer, images {sl}"
            assert torch.equal(dr[sl], drs), f"drop path, images {sl}"
    torch.cuda.synchronize()


def test_chain_s2d_consumer_and_resident_producer() -> None:
    """factor 2: the chained launch writes the space_to_depth layout and no statistics; a d = 64
    block (the resident kernel) takes no statistics and writes none."""
    announce("chain s2d consumer + d=64 producer")
    plan0, x0, p0, nw0 = make_case(2, 14, 14, 512, 128, "local", 0, torch.bfloat16, seed=3)
    plan, _, p, nw = make_case(2, 14, 14, 512, 128, "shifted", 0, torch.bfloat16, seed=4)
    with torch.no_grad():
        x, stats = bigemm_block_chain_hip(x0, None, nw0, plan0, **p0)
        got, nxt = bigemm_block_chain_hip(x, stats, nw, plan, **p, factor=2)
        want = bigemm_block_s2d_hip(x, nw, plan, **p, factor=2)
        plan1, x1, p1, nw1 = make_case(2, 28, 28, 256, 64, "local", 0, torch.bfloat16, seed=5)
        y1, s1 = bigemm_block_chain_hip(x1, None, nw1, plan1, **p1)
        want1 = bigemm_block_hip(x1, nw1, plan1, **p1)
    torch.cuda.synchronize()
    assert nxt is None and got.shape == want.shape
    assert _rel(got, want) <= 2e-3
    assert s1 is None and torch.equal(y1, want1)


def test_chain_rejects_bad_stats() -> None:
    announce("chain rejects bad stats_in")
    plan, x, p, nw = make_case(1, 14, 14, 512, 128, "local", 0, torch.bfloat16)
    with torch.no_grad():
        with pytest.raises(ValueError, match="stats_in"):
            bigemm_block_chain_hip(x, torch.zeros(5, 4, device=DEV), nw, plan, **p)
        with pytest.raises(ValueError, match="stats_in"):
            bigemm_block_chain_hip(x, torch.zeros(196, 4, device=DEV, dtype=torch.float64), nw, plan, **p)
        with pytest.raises(ValueError, match="stats_in_parts"):
            bigemm_block_chain_hip(x, torch.zeros(196, 65, device=DEV), nw, plan, **p)
        with pytest.raises(RuntimeError):
            bigemm_block_chain_hip(x.float(), None, nw, plan, **p)
