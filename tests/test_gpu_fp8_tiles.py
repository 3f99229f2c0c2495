"""GPU parity of the large-M FP8 GEMM paths and the FP8-MFMA precision record.

* The 256 x 256 kernel (fp8_square.hip) at the shapes its dispatch rule takes:
  partial token tiles, a single scale block (K = 128), an odd block count, and
  zero scale blocks (a token's activation block and a whole 128-row weight
  block), each against the fp32 oracle, plus determinism.
* FERRET_FP8_MMA_E4M3 (the opt-in FP8-MFMA instance of the tiled kernels):
  its max relative error under the reference metric
  (examples/fp8-gemm/v002_dense_tp8_validated_065.cu:345-360) is measured on
  the dense DeepSeek-V3 shapes and the MoE prefill and printed.  The default
  (exact-widening) path must pass the 1e-2 gate with margin (< 5e-3); the
  FP8-MFMA instance is dispatched by default only where it also stays below
  5e-3, and the test fails if a shape it is not dispatched for starts to meet
  that margin (then the dispatch should take it).
"""
import sys

import numpy as np
import pytest
import torch

from oracle import gemm as G
from oracle import metrics as MT
from tests.gpu_helpers import assert_gemm_close, bf16_out, codes8, f32, moe_sample_pairs

pytestmark = pytest.mark.gpu

MARGIN = 5e-3   # FP8-MFMA dispatch bar: half the reference's 1e-2 gate


def _say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def ops(hip):
    from ferret_amd import ops as _ops
    return _ops


def _inputs(M, N, K, seed):
    from ferret_amd import workloads as W
    a, sa = W.quant_act_1x128(W.randn((M, K), seed, "cuda"))
    b, sb = W.quant_weight_128x128(W.randn((N, K), seed + 1, "cuda"))
    return a, sa, b, sb


def _rows(M):
    return np.unique(np.r_[0:24, M - 24:M, np.random.default_rng(1).integers(0, M, 48)])


@pytest.mark.parametrize("M,N,K", [(3000, 4096, 256), (4096, 4096, 128), (4000, 4096, 384), (2048, 7168, 512)])
def test_square_kernel_shapes(hip, ops, M, N, K):
    assert hip.ferret_workspace_bytes(1, M, N, K, 0) == 0
    _say(f"square kernel M={M} N={N} K={K}")
    a, sa, b, sb = _inputs(M, N, K, 70)
    y = ops.fp8_gemm_blockscale(a, sa, b, sb)
    y2 = ops.fp8_gemm_blockscale(a, sa, b, sb)
    torch.cuda.synchronize()
    rows = _rows(M)
    ref = G.fp8_blockscale_gemm(codes8(a)[rows], f32(sa)[rows], codes8(b), f32(sb))
    assert_gemm_close(bf16_out(y)[rows], ref, f"square M={M} N={N} K={K}")
    assert torch.equal(y.view(torch.int16), y2.view(torch.int16)), "non-deterministic output"


@pytest.mark.parametrize("path", ["square", "tiled"])
def test_zero_scale_blocks(ops, path):
    """A zero activation or weight block scale removes that block's products,
    whatever the e4m3 bytes hold (the oracle multiplies them by 0)."""
    M, N, K = (3000, 4096, 512) if path == "square" else (700, 512, 512)
    _say(f"zero-scale blocks, {path} path M={M} N={N} K={K}")
    a, sa, b, sb = _inputs(M, N, K, 80)
    sa[5:9, 1] = 0.0         # four tokens, K block 1
    sa[300:301, 0] = 0.0     # one token, the first block
    sb[3, 2] = 0.0           # weight rows 384..511, K block 2
    sa[40, 3] = 0.0          # a token's last block
    y = ops.fp8_gemm_blockscale(a, sa, b, sb)
    torch.cuda.synchronize()
    rows = np.unique(np.r_[0:48, 290:310, _rows(M)])
    ref = G.fp8_blockscale_gemm(codes8(a)[rows], f32(sa)[rows], codes8(b), f32(sb))
    assert_gemm_close(bf16_out(y)[rows], ref, f"zero scales ({path})")


FP8_MMA_DENSE = ["dsv3_fp8_M4096", "dsv3_fp8_M128", "dsv3_q_b_proj_M8192", "dsv3_kv_b_proj_M8192",
                 "dsv3_o_proj_M8192", "dsv3_o_proj_M2048"]


@pytest.mark.parametrize("key", FP8_MMA_DENSE)
def test_fp8_mma_precision_dense(ops, key):
    from ferret_amd import workloads as W
    wl = W.WORKLOADS[key]
    inp = W.make_inputs(wl, "cuda")
    rows = np.arange(wl.M) if wl.M <= 128 else np.sort(np.random.default_rng(0).choice(wl.M, 256, replace=False))
    ref = G.fp8_blockscale_gemm(codes8(inp["a"])[rows], f32(inp["sa"])[rows], codes8(inp["b"]), f32(inp["sb"]))
    errs = {}
    for mma in ("bf16", "e4m3"):
        y = ops.fp8_gemm_blockscale(inp["a"], inp["sa"], inp["b"], inp["sb"], mma=mma)
        torch.cuda.synchronize()
        err, nbad = MT.fp8_rel_err(bf16_out(y)[rows], ref)
        assert nbad == 0
        errs[mma] = err
    _say(f"FP8-MFMA precision {key}: exact-widening {errs['bf16']:.5f}, fp8 mfma {errs['e4m3']:.5f}")
    assert errs["bf16"] < MARGIN
    assert errs["e4m3"] >= MARGIN, f"{key}: the FP8 MFMA meets the {MARGIN} margin here; dispatch it"


def test_vendor_fp8_gemm_misses_the_gate_too(ops):
    """The vendor library's FP8 GEMM (hipBLASLt through torch._scaled_mm, unit
    scales, so only the matrix cores' summation differs from the fp32 oracle)
    misses the reference's 1e-2 gate on the headline operands, with the same
    error as this library's opt-in FP8-MFMA instance; the exact-widening path
    meets it.  Recorded evidence for dispatching the bf16 path: the limit is
    the FP8 MFMA, not this library's use of it."""
    from ferret_amd import workloads as W
    wl = W.WORKLOADS["dsv3_fp8_M4096"]
    inp = W.make_inputs(wl, "cuda")
    rows = np.sort(np.random.default_rng(0).choice(wl.M, 128, replace=False))
    ones_a, ones_b = torch.ones_like(inp["sa"]), torch.ones_like(inp["sb"])
    ref = G.fp8_blockscale_gemm(codes8(inp["a"])[rows], f32(ones_a)[rows], codes8(inp["b"]), f32(ones_b))
    one = torch.tensor(1.0, device="cuda")
    try:
        y = torch._scaled_mm(inp["a"], inp["b"].t(), scale_a=one, scale_b=one, out_dtype=torch.float32)
    except (RuntimeError, NotImplementedError) as ex:
        pytest.skip(f"torch._scaled_mm unavailable: {ex}")
    torch.cuda.synchronize()
    vendor, _ = MT.fp8_rel_err(y.cpu().numpy()[rows], ref)
    errs = {}
    for mma in ("bf16", "e4m3"):
        c = ops.fp8_gemm_blockscale(inp["a"], ones_a, inp["b"], ones_b, mma=mma)
        torch.cuda.synchronize()
        errs[mma], _ = MT.fp8_rel_err(bf16_out(c)[rows], ref)
    _say(f"FP8 GEMM precision at K=7168: hipBLASLt fp8 {vendor:.5f}, this library fp8 mfma {errs['e4m3']:.5f}, "
         f"exact widening {errs['bf16']:.5f}")
    assert errs["bf16"] < MARGIN
    assert vendor >= MARGIN and errs["e4m3"] >= MARGIN


@pytest.mark.parametrize("key", ["dsv3_moe_w13_prefill", "dsv3_moe_w2_prefill"])
def test_fp8_mma_precision_moe_prefill(ops, key):
    from ferret_amd import workloads as W
    wl = W.WORKLOADS[key]
    inp = W.make_inputs(wl, "cuda")
    ids, _ = ops.moe_route_topk(inp["logits"], wl.topk)
    rt = ops.moe_permute(ids, wl.E)
    ids_np = ids.cpu().numpy()
    pairs, experts = moe_sample_pairs(ids_np, wl.E, max_experts=6, max_rows=96)
    emap = {e: i for i, e in enumerate(experts)}
    sub = np.vectorize(lambda v: emap.get(int(v), -1))(ids_np).astype(np.int32)
    ex = torch.tensor(experts, device="cuda")
    errs = {}
    for mma in ("bf16", "e4m3"):
        if wl.kind == "moe_fp8":
            y = ops.moe_w13_fp8(inp["x"], inp["sx"], inp["w"], inp["sw"], rt, mma=mma)
            ref = G.moe_w13_fp8(codes8(inp["x"]), f32(inp["sx"]), codes8(inp["w"][ex]), f32(inp["sw"][ex]), sub,
                                pairs=pairs)
        else:
            y = ops.moe_w2_fp8(inp["h"], inp["sh"], inp["w"], inp["sw"], rt, mma=mma)
            ref = G.moe_w2_fp8(codes8(inp["h"]), f32(inp["sh"]), codes8(inp["w"][ex]), f32(inp["sw"][ex]), sub,
                               pairs=pairs)
        torch.cuda.synchronize()
        err, nbad = MT.fp8_rel_err(bf16_out(y)[pairs], ref)
        assert nbad == 0
        errs[mma] = err
    _say(f"FP8-MFMA precision {key}: exact-widening {errs['bf16']:.5f}, fp8 mfma {errs['e4m3']:.5f}")
    assert errs["bf16"] < MARGIN
    assert errs["e4m3"] >= MARGIN, f"{key}: the FP8 MFMA meets the {MARGIN} margin here; dispatch it"
