"""GPU parity of the MoE layer around the grouped GEMMs: the 1x128 activation
quantizer (bit-exact), the FP8 w2 down projection (GEMM tolerance), the top-k
combine, and the chained layer w13 -> quantize -> w2 -> combine.

Every case is named on stdout (flushed) before its GPU work starts.
"""
import sys

import numpy as np
import pytest
import torch

from oracle import formats as F
from oracle import gemm as G
from oracle import quant as Q
from tests.gpu_helpers import assert_gemm_close, bf16_out, bits16, codes8, f32

pytestmark = pytest.mark.gpu


def _say(msg):
    print(f"[case] {msg}", flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def ops():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from ferret_amd import ops as O
    return O


def _bf16(x: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(F.f32_to_bf16_bits(x).view(np.int16)).view(torch.bfloat16).cuda()


# ------------------------------------------------------------------ quantizer

@pytest.mark.parametrize("M,K,scale", [(1, 128, 1.0), (33, 2048, 0.01), (256, 7168, 3.0), (7, 384, 1e-3)])
def test_quant_act_matches_oracle_bit_exact(ops, M, K, scale):
    _say(f"quant_act M={M} K={K} scale={scale}")
    rng = np.random.default_rng(M + K)
    x = (rng.standard_normal((M, K)) * scale).astype(np.float32)
    x[0, :128] = 0.0                                      # all-zero block: the 1e-4 amax floor
    if M > 2:
        x[2, -128:] *= 1e-6                               # tiny block: e4m3 subnormals after scaling
    xt = _bf16(x)
    q, s = ops.quant_act_e4m3(xt)
    torch.cuda.synchronize()
    rq, rs = Q.quant_act_1x128(bf16_out(xt))
    assert np.array_equal(codes8(q), rq)
    assert np.array_equal(f32(s).view(np.uint32), rs.view(np.uint32))


def test_quant_act_rounds_every_e4m3_midpoint_to_nearest_even(ops):
    """A block whose max is 448 scales by exactly 1, so q = e4m3_RNE(x): every
    exact e4m3 value, every midpoint between neighbours (ties to even), and a
    bf16 step either side of each midpoint, both signs."""
    _say("quant_act e4m3 midpoints")
    vals = np.unique(F.e4m3_to_f32(np.arange(0, 0x7F, dtype=np.uint8)).astype(np.float64))
    mids = (vals[:-1] + vals[1:]) / 2
    cand = [vals, mids]
    for m in mids:
        b = F.f32_to_bf16_bits(np.array([m], np.float32)).astype(np.int64)
        cand.append(F.bf16_bits_to_f32((b + 1).astype(np.uint16)).astype(np.float64))
        cand.append(F.bf16_bits_to_f32((b - 1).astype(np.uint16)).astype(np.float64))
    pos = np.unique(np.concatenate([np.atleast_1d(c) for c in cand]))
    pos = pos[(pos >= 0) & (pos <= 448)]
    allv = np.concatenate([pos, -pos]).astype(np.float32)
    assert np.array_equal(F.bf16_round(allv), allv)       # inputs exactly representable in bf16
    nblk = (allv.size + 126) // 127
    x = np.zeros((nblk, 128), np.float32)
    x[:, 0] = 448.0
    flat = np.zeros(nblk * 127, np.float32)
    flat[:allv.size] = allv
    x[:, 1:] = flat.reshape(nblk, 127)
    xt = _bf16(x)
    q, s = ops.quant_act_e4m3(xt)
    torch.cuda.synchronize()
    assert np.all(f32(s) == np.float32(1.0))
    assert np.array_equal(codes8(q), F.f32_to_e4m3(x))


# ------------------------------------------------------------------ w2 (down)

def _w2_inputs(ops, P, E, N, K, seed):
    from ferret_amd import workloads as W
    h, sh = W.quant_act_1x128(W.randn((P, K), seed, "cuda"))
    w = torch.empty((E, N, K), dtype=torch.float8_e4m3fn, device="cuda")
    sw = torch.empty((E, N // 128, K // 128), dtype=torch.float32, device="cuda")
    for e in range(E):
        w[e], sw[e] = W.quant_weight_128x128(W.randn((N, K), seed + 10 + e, "cuda"))
    return h, sh, w, sw


@pytest.mark.parametrize("T,E,N,K,topk,tile_m", [(16, 8, 256, 256, 2, 16), (40, 6, 1024, 2048, 3, 16),
                                                 (24, 12, 7168, 2048, 8, 16), (9, 5, 384, 896, 2, 16),
                                                 (300, 4, 256, 512, 2, 128), (200, 6, 7168, 2048, 4, 128),
                                                 (64, 16, 640, 896, 4, 128)])
def test_moe_w2_fp8_small(ops, T, E, N, K, topk, tile_m):
    _say(f"moe_w2_fp8 T={T} E={E} N={N} K={K} topk={topk} tile_m={tile_m}")
    P = T * topk
    h, sh, w, sw = _w2_inputs(ops, P, E, N, K, seed=T + E + N + K)
    from ferret_amd import workloads as W
    logits = W.randn((T, E), T + 7, "cuda")
    ids, _ = ops.moe_route_topk(logits, topk)
    rt = ops.moe_permute(ids, E, tile_m)
    out = torch.full((P, N), float("nan"), dtype=torch.bfloat16, device="cuda")
    ops.moe_w2_fp8(h, sh, w, sw, rt, out=out)
    torch.cuda.synchronize()
    ref = G.moe_w2_fp8(codes8(h), f32(sh), codes8(w), f32(sw), ids.cpu().numpy())
    assert_gemm_close(bf16_out(out), ref, "moe_w2_fp8")


def test_moe_w2_fp8_padded_grid_and_empty_experts(ops):
    """N = 7168 has 28 row blocks per tile (not a multiple of the 8 XCDs); two of the
    eight experts receive no pair."""
    _say("moe_w2_fp8 padded grid")
    T, E, N, K, topk = 96, 8, 7168, 2048, 2
    P = T * topk
    h, sh, w, sw = _w2_inputs(ops, P, E, N, K, seed=77)
    ids = torch.randint(0, 6, (T, topk), device="cuda", dtype=torch.int32,
                        generator=torch.Generator(device="cuda").manual_seed(5))
    ids[:, 1] = (ids[:, 0] + 1) % 6
    rt = ops.moe_permute(ids, E, 128)
    out = ops.moe_w2_fp8(h, sh, w, sw, rt)
    torch.cuda.synchronize()
    ref = G.moe_w2_fp8(codes8(h), f32(sh), codes8(w), f32(sw), ids.cpu().numpy())
    assert_gemm_close(bf16_out(out), ref, "moe_w2_fp8 padded")


# ------------------------------------------------------------------ combine

@pytest.mark.parametrize("T,topk,N", [(1, 1, 8), (37, 8, 7168), (128, 4, 1024)])
def test_moe_combine_matches_oracle(ops, T, topk, N):
    _say(f"moe_combine T={T} topk={topk} N={N}")
    rng = np.random.default_rng(T * 31 + N)
    o = _bf16(rng.standard_normal((T * topk, N)).astype(np.float32))
    wts = torch.softmax(torch.from_numpy(rng.standard_normal((T, topk)).astype(np.float32)), dim=1).cuda()
    y = ops.moe_combine(o, wts)
    torch.cuda.synchronize()
    ref = G.moe_combine(bits16(o), f32(wts))
    got = bf16_out(y)
    # the fp32 fma chain and the oracle's multiply-add differ by fp32 roundings of
    # the partial sums (bounded by their magnitudes); then one bf16 rounding each
    mag = (np.abs(f32(wts))[:, :, None] * np.abs(bf16_out(o)).reshape(T, topk, N)).sum(axis=1)
    assert np.all(np.abs(got - ref) <= np.abs(ref) * 2.0 ** -8 + mag * 2.0 ** -20)


def test_tail_workloads_at_bench_size(ops):
    """The bench's prefill tail workloads at full size: the quantizer on bf16
    [32768, 2048] bit-exact over every row, the top-8 combine of [32768, 7168]
    on 512 sampled tokens within the combine bound."""
    from ferret_amd import workloads as W
    _say("moe_quant_act_prefill at full size")
    wl = W.WORKLOADS["moe_quant_act_prefill"]
    x = W.make_inputs(wl, "cuda")["x"]
    q, s = ops.quant_act_e4m3(x)
    torch.cuda.synchronize()
    rq, rs = Q.quant_act_1x128(bf16_out(x))
    assert np.array_equal(codes8(q), rq)
    assert np.array_equal(f32(s).view(np.uint32), rs.view(np.uint32))
    del x, q, s
    _say("moe_combine_prefill at full size")
    wl = W.WORKLOADS["moe_combine_prefill"]
    inp = W.make_inputs(wl, "cuda")
    y = ops.moe_combine(inp["o"], inp["w"])
    torch.cuda.synchronize()
    toks = np.sort(np.random.default_rng(0).choice(wl.T, 512, replace=False))
    rows = (toks[:, None] * wl.topk + np.arange(wl.topk)[None, :]).reshape(-1)
    ob, wts = bits16(inp["o"])[rows], f32(inp["w"])[toks]
    ref = G.moe_combine(ob, wts)
    got = bf16_out(y)[toks]
    mag = (np.abs(wts)[:, :, None] * np.abs(F.bf16_bits_to_f32(ob)).reshape(len(toks), wl.topk, wl.N)).sum(axis=1)
    assert np.all(np.abs(got - ref) <= np.abs(ref) * 2.0 ** -8 + mag * 2.0 ** -20)


def test_moe_combine_one_hot_weights_select_rows_exactly(ops):
    _say("moe_combine one-hot")
    T, topk, N = 50, 8, 256
    rng = np.random.default_rng(3)
    o = _bf16(rng.standard_normal((T * topk, N)).astype(np.float32))
    sel = rng.integers(0, topk, size=T)
    w = np.zeros((T, topk), np.float32)
    w[np.arange(T), sel] = 1.0
    y = ops.moe_combine(o, torch.from_numpy(w).cuda())
    torch.cuda.synchronize()
    assert np.array_equal(bits16(y), bits16(o)[np.arange(T) * topk + sel])


# ------------------------------------------------------------------ the layer

def test_moe_layer_chain_w13_quant_w2_combine(ops):
    """Each stage on the GPU, each checked against the oracle fed the previous
    GPU stage's output: quantizer bit-exact, GEMMs and combine to tolerance."""
    from ferret_amd import workloads as W
    T, E, topk, H, I2 = 24, 8, 4, 1024, 512          # hidden, w13 rows (gate + up)
    _say(f"moe layer chain T={T} E={E} topk={topk} hidden={H} inter={I2 // 2}")
    x, sx = W.quant_act_1x128(W.randn((T, H), 41, "cuda"))
    w13 = torch.empty((E, I2, H), dtype=torch.float8_e4m3fn, device="cuda")
    s13 = torch.empty((E, I2 // 128, H // 128), dtype=torch.float32, device="cuda")
    w2 = torch.empty((E, H, I2 // 2), dtype=torch.float8_e4m3fn, device="cuda")
    s2 = torch.empty((E, H // 128, I2 // 256), dtype=torch.float32, device="cuda")
    for e in range(E):
        w13[e], s13[e] = W.quant_weight_128x128(W.randn((I2, H), 50 + e, "cuda"))
        w2[e], s2[e] = W.quant_weight_128x128(W.randn((H, I2 // 2), 80 + e, "cuda"))
    ids, wts = ops.moe_route_topk(W.randn((T, E), 43, "cuda"), topk)
    rt = ops.moe_permute(ids, E, 16)
    h = ops.moe_w13_fp8(x, sx, w13, s13, rt)
    hq, hs = ops.quant_act_e4m3(h)
    o = ops.moe_w2_fp8(hq, hs, w2, s2, rt)
    y = ops.moe_combine(o, wts)
    torch.cuda.synchronize()
    idn = ids.cpu().numpy()
    assert_gemm_close(bf16_out(h), G.moe_w13_fp8(codes8(x), f32(sx), codes8(w13), f32(s13), idn), "chain w13")
    rq, rs = Q.quant_act_1x128(bf16_out(h))
    assert np.array_equal(codes8(hq), rq) and np.array_equal(f32(hs), rs)
    assert_gemm_close(bf16_out(o), G.moe_w2_fp8(rq, rs, codes8(w2), f32(s2), idn), "chain w2")
    ref_y = G.moe_combine(bits16(o), f32(wts))
    mag = (np.abs(f32(wts))[:, :, None] * np.abs(bf16_out(o)).reshape(T, topk, -1)).sum(axis=1)
    assert np.all(np.abs(bf16_out(y) - ref_y) <= np.abs(ref_y) * 2.0 ** -8 + mag * 2.0 ** -20)
