"""GPU parity: every C-ABI entry point against the CPU oracle on the same inputs.

Small shapes are compared in full; the full workload sizes are compared on
sampled rows / experts plus size-independent properties (determinism, routing
invariants).  Integer outputs (routing, permutation, tiles) must be bit-exact;
GEMM outputs must be within max relative error 1e-2 of the fp32 oracle.
"""
import os
import sys

import numpy as np
import pytest
import torch

from oracle import formats as F
from oracle import gemm as G
from oracle import routing as R
from oracle import metrics as MT

from tests.gpu_helpers import (assert_gemm_close, bf16_out, bits16, codes8, f32, moe_sample_pairs,
                               oracle_routing)

pytestmark = pytest.mark.gpu


def _say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def ops(hip):
    from ferret_amd import ops as _ops
    return _ops


def test_single_hip_runtime(hip):
    with open("/proc/self/maps") as fh:
        libs = {line.split()[-1] for line in fh if "libamdhip64" in line}
    assert len(libs) == 1, f"more than one HIP runtime mapped: {libs}"


# ------------------------------------------------------------------ bf16 linear

@pytest.mark.parametrize("M,N,K,res", [(1, 64, 128, False), (5, 256, 512, True), (16, 512, 4096, False),
                                       (16, 128, 12288, True), (20, 96, 1024, False), (3, 48, 896, True),
                                       (20, 256, 4096, False), (9, 1024, 7168, False), (33, 48, 4096, False),
                                       # >= 4 row units per CU: the 4-wave stream units (+ residual, K = 1024 / 3584)
                                       (3, 16384, 1024, True), (16, 20480, 3584, False), (1, 16384, 4096, True)])
def test_linear_bf16_small(ops, M, N, K, res):
    _say(f"linear_bf16 M={M} N={N} K={K} res={res}")
    g = torch.Generator(device="cuda").manual_seed(M * 1000 + N + K)
    x = torch.randn((M, K), generator=g, device="cuda").to(torch.bfloat16)
    w = (torch.randn((N, K), generator=g, device="cuda") * 0.05).to(torch.bfloat16)
    r = torch.randn((M, N), generator=g, device="cuda").to(torch.bfloat16) if res else None
    y = ops.linear_bf16(x, w, r)
    torch.cuda.synchronize()
    ref = G.linear_bf16(bits16(x), bits16(w), bits16(r) if res else None)
    got = bf16_out(y)
    assert_gemm_close(got, ref, "linear_bf16")
    e, nbad = MT.linear_rel_err(got, ref)
    assert nbad == 0 and e < 5e-3


@pytest.mark.parametrize("M,N,K,res", [(16, 6144, 4096, False), (16, 4096, 12288, True), (1, 4096, 12288, True),
                                       (16, 4096, 4096, True), (5, 6144, 4096, True), (13, 4096, 12288, False)])
def test_linear_bf16_split_k_and_residual_paths(hip, M, N, K, res):
    """QKV- and Down-shaped products split K over a workspace (partials summed
    in split order with the residual by a second kernel); O-shaped ones add the
    residual in the stream kernel.  With the workspace, without it (same
    product unsplit) and one byte short: all meet the oracle."""
    _say(f"linear_bf16 split/residual M={M} N={N} K={K} res={res}")
    g = torch.Generator(device="cuda").manual_seed(M * 7 + N + K)
    x = torch.randn((M, K), generator=g, device="cuda").to(torch.bfloat16)
    w = (torch.randn((N, K), generator=g, device="cuda") * 0.05).to(torch.bfloat16)
    r = torch.randn((M, N), generator=g, device="cuda").to(torch.bfloat16) if res else None
    ref = G.linear_bf16(bits16(x), bits16(w), bits16(r) if res else None)
    need = int(hip.ferret_workspace_bytes(0, M, N, K, 0))
    ws = torch.empty(max(need, 1), dtype=torch.uint8, device="cuda")
    for ws_ptr, ws_bytes, tag in ((ws.data_ptr(), need, "ws"), (None, 0, "null-ws"),
                                  (ws.data_ptr(), max(need - 1, 0), "short-ws")):
        y = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device="cuda")
        rc = hip.ferret_linear_bf16(x.data_ptr(), w.data_ptr(), r.data_ptr() if res else None, y.data_ptr(),
                                    M, N, K, ws_ptr, ws_bytes, torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        assert rc == 0, tag
        got = bf16_out(y)
        e, nbad = MT.linear_rel_err(got, ref)
        assert nbad == 0 and e < 5e-3, f"{tag}: {e}"


@pytest.mark.parametrize("M,N,K,res", [(16, 6144, 4096, False), (16, 4096, 12288, True), (1, 6144, 4096, True)])
def test_linear_bf16_split_k_fixup_workspace_contract(hip, M, N, K, res):
    """Split-K products over a caller workspace: it needs no initialisation
    (filled with random bits here), one workspace serves consecutive calls,
    and a HIP graph replays the call (GEMM + split reduce) with eager calls on
    the same workspace in between -- every result bit-identical to the first."""
    _say(f"linear_bf16 split-K fix-up M={M} N={N} K={K} res={res}")
    g = torch.Generator(device="cuda").manual_seed(M * 5 + N + K)
    x = torch.randn((M, K), generator=g, device="cuda").to(torch.bfloat16)
    w = (torch.randn((N, K), generator=g, device="cuda") * 0.05).to(torch.bfloat16)
    r = torch.randn((M, N), generator=g, device="cuda").to(torch.bfloat16) if res else None
    need = int(hip.ferret_workspace_bytes(0, M, N, K, 0))
    assert need > 0, "shape expected to split K"
    ws = torch.randint(0, 256, (need,), dtype=torch.uint8, device="cuda", generator=g)
    st = torch.cuda.current_stream().cuda_stream

    def call(y):
        return hip.ferret_linear_bf16(x.data_ptr(), w.data_ptr(), r.data_ptr() if res else None, y.data_ptr(),
                                      M, N, K, ws.data_ptr(), need, torch.cuda.current_stream().cuda_stream)

    ys = [torch.full((M, N), float("nan"), dtype=torch.bfloat16, device="cuda") for _ in range(3)]
    for y in ys:
        assert call(y) == 0
    torch.cuda.synchronize()
    ref = G.linear_bf16(bits16(x), bits16(w), bits16(r) if res else None)
    e, nbad = MT.linear_rel_err(bf16_out(ys[0]), ref)
    assert nbad == 0 and e < 5e-3
    for y in ys[1:]:
        assert torch.equal(y, ys[0])
    yg = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device="cuda")
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.graph(graph, stream=side):
        assert call(yg) == 0
    for i in range(4):
        yg.fill_(float("nan"))
        assert call(ys[1]) == 0            # eager work on the same workspace between the replays
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(yg, ys[0]) and torch.equal(ys[1], ys[0]), f"replay {i}"
    del st


def test_launch_gemv_compat(hip):
    """The reference ctypes ABI (M = 1) writes the same result as ferret_linear_bf16."""
    N, K = 256, 1024
    g = torch.Generator(device="cuda").manual_seed(11)
    x = torch.randn((1, K), generator=g, device="cuda").to(torch.bfloat16)
    w = (torch.randn((N, K), generator=g, device="cuda") * 0.05).to(torch.bfloat16)
    r = torch.randn((1, N), generator=g, device="cuda").to(torch.bfloat16)
    out = torch.empty((1, N), dtype=torch.bfloat16, device="cuda")
    hip.launch_gemv(x.data_ptr(), w.data_ptr(), r.data_ptr(), out.data_ptr(), N, K,
                    torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    ref = G.linear_bf16(bits16(x), bits16(w), bits16(r))
    assert_gemm_close(bf16_out(out), ref, "launch_gemv")


def test_linear_bf16_rejects_bad_shapes(ops):
    from ferret_amd.lib import FerretError
    x = torch.zeros((2, 100), dtype=torch.bfloat16, device="cuda")
    w = torch.zeros((64, 100), dtype=torch.bfloat16, device="cuda")
    with pytest.raises(FerretError):
        ops.linear_bf16(x, w)


def test_wrappers_reject_wrong_output_buffers(ops):
    """A caller-supplied output (or q/scale) of the wrong shape is refused on the
    host, before any launch could write past it."""
    from ferret_amd import workloads as W
    x = torch.zeros((4, 256), dtype=torch.bfloat16, device="cuda")
    w = torch.zeros((64, 256), dtype=torch.bfloat16, device="cuda")
    with pytest.raises(ValueError, match="out must have shape"):
        ops.linear_bf16(x, w, out=torch.empty((4, 32), dtype=torch.bfloat16, device="cuda"))
    with pytest.raises(ValueError, match="residual must have shape"):
        ops.linear_bf16(x, w, residual=torch.empty((2, 64), dtype=torch.bfloat16, device="cuda"))
    a, sa = W.quant_act_1x128(W.randn((32, 256), 1, "cuda"))
    b, sb = W.quant_weight_128x128(W.randn((128, 256), 2, "cuda"))
    with pytest.raises(ValueError, match="out must have shape"):
        ops.fp8_gemm_blockscale(a, sa, b, sb, out=torch.empty((32, 64), dtype=torch.bfloat16, device="cuda"))
    with pytest.raises(ValueError, match="q must have shape"):
        ops.quant_act_e4m3(x, q=torch.empty((4, 128), dtype=torch.float8_e4m3fn, device="cuda"))
    with pytest.raises(ValueError, match="scale must have shape"):
        ops.quant_act_e4m3(x, scale=torch.empty((4, 1), dtype=torch.float32, device="cuda"))
    ids = torch.zeros((4, 2), dtype=torch.int32, device="cuda")
    rt = ops.moe_permute(ids, 4)
    xq, sx = W.quant_act_1x128(W.randn((4, 256), 3, "cuda"))
    wq = torch.zeros((4, 256, 256), dtype=torch.float8_e4m3fn, device="cuda")
    sw = torch.ones((4, 2, 2), dtype=torch.float32, device="cuda")
    with pytest.raises(ValueError, match="out must have shape"):
        ops.moe_w13_fp8(xq, sx, wq, sw, rt, out=torch.empty((8, 64), dtype=torch.bfloat16, device="cuda"))
    h, sh = W.quant_act_1x128(W.randn((8, 256), 4, "cuda"))
    with pytest.raises(ValueError, match="out must have shape"):
        ops.moe_w2_fp8(h, sh, wq, sw, rt, out=torch.empty((8, 128), dtype=torch.bfloat16, device="cuda"))
    o = torch.zeros((8, 64), dtype=torch.bfloat16, device="cuda")
    wts = torch.ones((4, 2), dtype=torch.float32, device="cuda")
    with pytest.raises(ValueError, match="out must have shape"):
        ops.moe_combine(o, wts, out=torch.empty((4, 32), dtype=torch.bfloat16, device="cuda"))
    with pytest.raises(ValueError, match="one device"):
        ops.moe_combine(o, wts.cpu())


# ------------------------------------------------------------------ FP8 dense

def _fp8_inputs(M, N, K, seed):
    from ferret_amd import workloads as W
    a, sa = W.quant_act_1x128(W.randn((M, K), seed, "cuda"))
    b, sb = W.quant_weight_128x128(W.randn((N, K), seed + 1, "cuda"))
    return a, sa, b, sb


@pytest.mark.parametrize("M,N,K", [(1, 128, 128), (16, 256, 1024), (7, 4096, 7168), (17, 128, 512),
                                   (128, 256, 1024), (200, 384, 896), (256, 512, 7168),
                                   (3, 384, 2048), (16, 128, 2048), (16, 256, 3584)])
def test_fp8_gemm_small(ops, M, N, K):
    _say(f"fp8_gemm M={M} N={N} K={K}")
    a, sa, b, sb = _fp8_inputs(M, N, K, seed=M + N + K)
    c = ops.fp8_gemm_blockscale(a, sa, b, sb)
    torch.cuda.synchronize()
    ref = G.fp8_blockscale_gemm(codes8(a), f32(sa), codes8(b), f32(sb))
    assert_gemm_close(bf16_out(c), ref, f"fp8 M={M}")


@pytest.mark.parametrize("M,N,K", [(128, 256, 1024), (77, 1024, 2048), (256, 512, 1024)])
def test_fp8_gemm_workspace_and_plain_paths(hip, ops, M, N, K):
    """16 < M <= 256: the split-K path (workspace given) and the plain path
    (ws NULL, or one byte too small) both meet the oracle."""
    _say(f"fp8_gemm workspace/plain M={M} N={N} K={K}")
    a, sa, b, sb = _fp8_inputs(M, N, K, seed=3 * M + K)
    need = ops.fp8_workspace_bytes(M, N, K)
    assert need >= 2 * M * N * 4, "shape expected to take the split-K path"
    ref = G.fp8_blockscale_gemm(codes8(a), f32(sa), codes8(b), f32(sb))
    ws = torch.empty(need, dtype=torch.uint8, device="cuda")
    for ws_ptr, ws_bytes, tag in ((ws.data_ptr(), need, "split"), (None, 0, "null-ws"),
                                  (ws.data_ptr(), need - 1, "short-ws")):
        c = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device="cuda")
        rc = hip.ferret_fp8_gemm_blockscale(a.data_ptr(), sa.data_ptr(), b.data_ptr(), sb.data_ptr(), c.data_ptr(),
                                            M, N, K, ws_ptr, ws_bytes, torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        assert rc == 0, tag
        assert_gemm_close(bf16_out(c), ref, f"fp8 {tag} M={M}")


def _tile_config(M, N):
    """The tiled configuration of a shape run without a workspace, by the dispatch
    rule of ferret_fp8_gemm_tiled: 128 x 128 tiles where the 256 x 128 grid
    would fill at most half of 256 CUs and the 128 x 128 grid fits them."""
    mb = -(-M // 128)
    t256, t128 = -(-N // 256) * mb, (N // 128) * mb
    return "128x128" if 2 * t256 <= 256 and t128 <= 256 else "256x128"


@pytest.mark.parametrize("M,N,K,cfg", [
    (128, 256, 128, "128x128"), (256, 256, 256, "128x128"), (384, 512, 384, "128x128"), (512, 256, 640, "128x128"),
    (520, 3072, 1536, "128x128"), (1000, 1024, 512, "128x128"),
    (1152, 4096, 128, "256x128"), (1152, 4096, 256, "256x128"), (1100, 4096, 384, "256x128"),
    (1100, 4096, 640, "256x128")])
def test_fp8_gemm_staggered_short_k(hip, M, N, K, cfg):
    """Without a workspace both tiled configurations run the staggered
    two-half loop; K of 1, 2, 3 and 5 K-steps covers its prologue (three
    stages in flight for one half) and its last-stage waits, on full and
    partial last token tiles (M % 128 != 0), above M = 256 too."""
    assert _tile_config(M, N) == cfg
    _say(f"fp8_gemm staggered M={M} N={N} K={K} ({cfg} tiles)")
    a, sa, b, sb = _fp8_inputs(M, N, K, seed=11 * M + K)
    ref = G.fp8_blockscale_gemm(codes8(a), f32(sa), codes8(b), f32(sb))
    c = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device="cuda")
    rc = hip.ferret_fp8_gemm_blockscale(a.data_ptr(), sa.data_ptr(), b.data_ptr(), sb.data_ptr(), c.data_ptr(),
                                        M, N, K, None, 0, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert rc == 0
    assert_gemm_close(bf16_out(c), ref, f"fp8 staggered M={M} K={K}")


def test_fp8_gemm_power_of_two_scales_exactish(ops):
    """Small-integer e4m3 values with power-of-two scales: exact sums, only the bf16 rounding differs."""
    M, N, K = 32, 256, 512
    rng = np.random.default_rng(5)
    vals = np.array([0x38, 0x40, 0xB8, 0x30, 0x00], np.uint8)
    a = torch.from_numpy(rng.choice(vals, size=(M, K))).cuda()
    b = torch.from_numpy(rng.choice(vals, size=(N, K))).cuda()
    sa = torch.from_numpy((2.0 ** rng.integers(-2, 3, size=(M, K // 128))).astype(np.float32)).cuda()
    sb = torch.from_numpy((2.0 ** rng.integers(-2, 3, size=(N // 128, K // 128))).astype(np.float32)).cuda()
    for m in (M, 8):
        c = ops.fp8_gemm_blockscale(a[:m].contiguous(), sa[:m].contiguous(), b, sb)
        torch.cuda.synchronize()
        ref = G.fp8_blockscale_gemm(codes8(a[:m]), f32(sa[:m]), codes8(b), f32(sb))
        assert np.array_equal(bf16_out(c), F.bf16_round(ref)), f"M={m}"


# ------------------------------------------------------------------ routing

@pytest.mark.parametrize("T,E,k", [(128, 256, 8), (64, 384, 8), (7, 16, 3), (33, 1024, 16), (4, 8, 8)])
def test_route_topk_bit_exact(ops, T, E, k):
    g = torch.Generator(device="cuda").manual_seed(T * E + k)
    logits = torch.randn((T, E), generator=g, device="cuda")
    # ties and NaNs
    logits[0, : E // 2] = 0.5
    logits[min(1, T - 1), 3] = float("nan")
    logits = logits.round(decimals=1) if T % 2 else logits
    ids, w = ops.moe_route_topk(logits, k)
    torch.cuda.synchronize()
    ref_ids, ref_w = R.route_topk(f32(logits), k)
    assert np.array_equal(ids.cpu().numpy(), ref_ids)
    np.testing.assert_allclose(w.cpu().numpy(), ref_w, rtol=1e-5, atol=1e-7)


@pytest.mark.parametrize("E,k", [(256, 8), (384, 8), (64, 16), (1024, 16), (7, 7)])
def test_route_topk_ties_across_lanes(ops, E, k):
    """Rows whose top logits repeat in many lanes (the top-k's tie path: the
    expert decides among equal logits), signed zeros (-0 ties +0), -inf and NaN
    rows, against the stable argsort of the oracle."""
    T = 6
    lg = np.zeros((T, E), dtype=np.float32)
    lg[0] = 1.0                                                   # every logit equal
    lg[1] = np.where(np.arange(E) % 2 == 0, -0.0, 0.0)            # signed zeros only
    lg[2] = np.where(np.arange(E) % 3 == 0, 2.0, -1.0)            # a third tied at the top
    lg[3] = -np.inf
    lg[3, E - 1] = np.nan                                         # -inf and NaN: index order
    lg[4] = np.float32(np.nan)                                    # all NaN
    lg[5] = np.round(np.random.default_rng(E).standard_normal(E), 0)  # few distinct values
    logits = torch.from_numpy(lg).cuda()
    ids, w = ops.moe_route_topk(logits, k)
    torch.cuda.synchronize()
    ref_ids, ref_w = R.route_topk(lg, k)
    assert np.array_equal(ids.cpu().numpy(), ref_ids)
    np.testing.assert_allclose(w.cpu().numpy(), ref_w, rtol=1e-5, atol=1e-7)


@pytest.mark.parametrize("T,k,E,tile_m,invalid", [(128, 8, 256, 16, False), (4096, 8, 256, 128, False),
                                                  (64, 8, 384, 16, False), (50, 3, 7, 4, True),
                                                  (1500, 2, 1024, 16, True), (1, 1, 1, 16, False)])
def test_permute_bit_exact(ops, T, k, E, tile_m, invalid):
    rng = np.random.default_rng(T + k + E)
    if T >= 4096:   # skewed: a few hot experts
        p = 1.0 / np.arange(1, E + 1) ** 1.1
        ids_np = np.stack([rng.choice(E, size=k, replace=False, p=p / p.sum()) for _ in range(T)]).astype(np.int32)
    else:
        ids_np = rng.integers(0, E, size=(T, k)).astype(np.int32)
    if invalid:
        ids_np[0, 0] = -1
        ids_np[-1, -1] = E + 5
    ids = torch.from_numpy(ids_np).cuda()
    rt = ops.moe_permute(ids, E, tile_m)
    torch.cuda.synchronize()
    counts, offsets, sp, tiles = oracle_routing(ids_np, E, tile_m)
    assert np.array_equal(rt.counts.cpu().numpy(), counts)
    assert np.array_equal(rt.offsets.cpu().numpy(), offsets)
    assert np.array_equal(rt.sorted_pair.cpu().numpy()[: len(sp)], sp)
    nt = int(rt.ntiles.item())
    assert nt == len(tiles)
    assert np.array_equal(rt.tiles.cpu().numpy()[:nt], tiles)
    assert not rt.tiles.cpu().numpy()[nt:].any()        # the table's tail is (0, 0, 0)


@pytest.mark.parametrize("T,k,E,tile_m", [(3000, 8, 384, 16), (4096, 8, 256, 128), (2049, 1, 7, 128),
                                          (2500, 8, 1024, 16),     # one scan thread per expert, 20 chunks
                                          (3000, 1, 1, 128)])      # 1024 scan threads on one expert
def test_permute_multi_group_matches_single_group(hip, ops, T, k, E, tile_m):
    """The multi-work-group path (workspace given) and the one-group path (NULL) agree bit for bit."""
    rng = np.random.default_rng(T * k + E)
    ids_np = rng.integers(-1, E + 1, size=(T, k)).astype(np.int32)  # includes dropped ids
    ids = torch.from_numpy(ids_np).cuda()
    P = T * k
    need = int(hip.ferret_workspace_bytes(4, P, 0, 0, E))
    assert need > 0
    with_ws = ops.moe_permute(ids, E, tile_m)          # takes the multi-group path
    L = hip
    max_tiles = with_ws.max_tiles
    outs = [torch.full_like(t, -7) for t in (with_ws.counts, with_ws.offsets, with_ws.sorted_pair, with_ws.tiles,
                                             with_ws.ntiles)]
    rc = L.ferret_moe_permute(ids.data_ptr(), T, k, E, tile_m, outs[0].data_ptr(), outs[1].data_ptr(),
                              outs[2].data_ptr(), outs[3].data_ptr(), max_tiles, outs[4].data_ptr(), None, 0,
                              torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert rc == 0
    nt = int(with_ws.ntiles.item())
    assert torch.equal(outs[0], with_ws.counts) and torch.equal(outs[1], with_ws.offsets)
    n_valid = int(with_ws.offsets[E].item())
    assert torch.equal(outs[2][:n_valid], with_ws.sorted_pair[:n_valid])
    assert int(outs[4].item()) == nt and torch.equal(outs[3], with_ws.tiles)   # zero tails included
    counts, offsets, sp, tiles = oracle_routing(ids_np, E, tile_m)
    assert np.array_equal(with_ws.sorted_pair.cpu().numpy()[: len(sp)], sp)


# ------------------------------------------------------------------ MoE w13

def _moe_fp8_small(T, E, N, K, topk, seed):
    from ferret_amd import workloads as W
    x, sx = W.quant_act_1x128(W.randn((T, K), seed, "cuda"))
    w = torch.empty((E, N, K), dtype=torch.float8_e4m3fn, device="cuda")
    sw = torch.empty((E, N // 128, K // 128), dtype=torch.float32, device="cuda")
    for e in range(E):
        w[e], sw[e] = W.quant_weight_128x128(W.randn((N, K), seed + 10 + e, "cuda"))
    logits = W.randn((T, E), seed + 5, "cuda")
    return x, sx, w, sw, logits


@pytest.mark.parametrize("T,E,N,K,topk,tile_m", [(16, 8, 256, 256, 2, 16), (40, 6, 512, 1024, 3, 16),
                                                 (300, 4, 256, 512, 2, 128), (64, 16, 512, 896, 4, 128),
                                                 (3, 5, 256, 128, 5, 16), (24, 6, 512, 4096, 3, 16),
                                                 (40, 12, 256, 7168, 8, 16)])
def test_moe_w13_fp8_small(ops, T, E, N, K, topk, tile_m):
    _say(f"moe_w13_fp8 T={T} E={E} N={N} K={K} topk={topk} tile_m={tile_m}")
    x, sx, w, sw, logits = _moe_fp8_small(T, E, N, K, topk, seed=T + E + N)
    ids, _ = ops.moe_route_topk(logits, topk)
    rt = ops.moe_permute(ids, E, tile_m)
    out = ops.moe_w13_fp8(x, sx, w, sw, rt)
    torch.cuda.synchronize()
    ref = G.moe_w13_fp8(codes8(x), f32(sx), codes8(w), f32(sw), ids.cpu().numpy())
    assert_gemm_close(bf16_out(out), ref, "moe_w13_fp8")


@pytest.mark.parametrize("T,E,N,K,topk", [(8, 8, 64, 256, 2), (64, 12, 256, 1024, 8), (5, 3, 32, 128, 3),
                                          (32, 16, 128, 7168, 4), (24, 6, 512, 4096, 3)])
def test_moe_w13_w4a16_small(ops, T, E, N, K, topk):
    _say(f"moe_w13_w4a16 T={T} E={E} N={N} K={K} topk={topk}")
    g = torch.Generator(device="cuda").manual_seed(T + E + N + K)
    x = torch.randn((T, K), generator=g, device="cuda").to(torch.bfloat16)
    wq = torch.randint(-2 ** 31, 2 ** 31, (E, N, K // 8), generator=g, device="cuda", dtype=torch.int32)
    ws = (torch.randn((E, N, K // 32), generator=g, device="cuda") * 0.01).to(torch.bfloat16)
    logits = torch.randn((T, E), generator=g, device="cuda")
    ids, _ = ops.moe_route_topk(logits, topk)
    rt = ops.moe_permute(ids, E, 16)
    out = ops.moe_w13_w4a16(x, wq, ws, rt)
    torch.cuda.synchronize()
    ref = G.moe_w13_w4a16(bits16(x), wq.cpu().numpy(), bits16(ws), ids.cpu().numpy())
    assert_gemm_close(bf16_out(out), ref, "moe_w13_w4a16")


def test_int4_dequant_bit_exact_via_one_hot_activation(ops):
    """One-hot activations x[t, k_t] = 4096 turn the w13 output into single
    dequantized weights: gate = 4096*deq[e,n,k_t], up = 4096*deq[e,N/2+n,k_t], both
    exact in fp32.  Where gate > 20, silu(gate) == gate exactly in fp32, so
    out = bf16_RNE(gate * up) (an exact fp32 product) must match bit for bit:
    any nibble-order, sign, group-scale or rounding error in the in-register
    dequant changes it."""
    T, E, N, K = 64, 2, 256, 256
    g = torch.Generator(device="cuda").manual_seed(77)
    wq = torch.randint(-2 ** 31, 2 ** 31, (E, N, K // 8), generator=g, device="cuda", dtype=torch.int32)
    ws = (torch.randn((E, N, K // 32), generator=g, device="cuda") * 0.01).to(torch.bfloat16)
    x = torch.zeros((T, K), dtype=torch.bfloat16, device="cuda")
    ks = [(t * 37 + t // 7) % K for t in range(T)]
    for t in range(T):
        x[t, ks[t]] = 4096.0
    ids = torch.zeros((T, 1), dtype=torch.int32, device="cuda")
    ids[T // 2:] = 1
    rt = ops.moe_permute(ids, E, 16)
    out = ops.moe_w13_w4a16(x, wq, ws, rt)
    torch.cuda.synchronize()
    deq = F.int4_dequant(wq.cpu().numpy(), bits16(ws))           # [E, N, K] bf16-exact
    got_all = bf16_out(out)
    checked = 0
    for t in range(T):
        e = int(ids[t, 0])
        gate = np.float32(4096.0) * deq[e, : N // 2, ks[t]]
        up = np.float32(4096.0) * deq[e, N // 2:, ks[t]]
        sel = gate > 20.0
        expect = F.bf16_round((gate * up).astype(np.float32))
        assert np.array_equal(got_all[t][sel], expect[sel]), f"token {t}"
        checked += int(sel.sum())
    assert checked > 500


# ------------------------------------------------------------------ full sizes

_ATTN_TP8 = [f"dsv3_{p}_M{m}" for m in (1, 16, 512, 1024, 2048, 4096, 8192)
             for p in ("q_b_proj", "kv_b_proj", "o_proj")]


@pytest.mark.parametrize("key", ["qwen3_gateup_M16", "dsv3_fp8_M16", "dsv3_fp8_M128", "dsv3_fp8_M4096",
                                 "qwen3_lmhead_M16", "qwen3_lmhead_M1", "qwen3_qkv_M16", "qwen3_down_M16",
                                 "qwen3_o_M1"]
                         + _ATTN_TP8)
def test_dense_full_size(ops, key):
    from ferret_amd import workloads as W
    wl = W.WORKLOADS[key]
    _say(f"full-size {key}")
    inp = W.make_inputs(wl, "cuda")
    if wl.kind == "linear_bf16":
        r = inp.get("r")
        y = ops.linear_bf16(inp["x"], inp["w"], residual=r)
        y2 = ops.linear_bf16(inp["x"], inp["w"], residual=r)
        torch.cuda.synchronize()
        ref = G.linear_bf16(bits16(inp["x"]), bits16(inp["w"]), bits16(r) if r is not None else None)
        assert_gemm_close(bf16_out(y), ref, key)
    else:
        y = ops.fp8_gemm_blockscale(inp["a"], inp["sa"], inp["b"], inp["sb"])
        y2 = ops.fp8_gemm_blockscale(inp["a"], inp["sa"], inp["b"], inp["sb"])
        torch.cuda.synchronize()
        rows = np.arange(wl.M) if wl.M <= 128 else np.unique(np.r_[0:32, wl.M - 32:wl.M,
                                                              np.random.default_rng(0).integers(0, wl.M, 64)])
        ref = G.fp8_blockscale_gemm(codes8(inp["a"])[rows], f32(inp["sa"])[rows], codes8(inp["b"]), f32(inp["sb"]))
        assert_gemm_close(bf16_out(y)[rows], ref, key)
    assert torch.equal(y.view(torch.int16), y2.view(torch.int16)), "non-deterministic output"


@pytest.mark.parametrize("key", ["dsv3_moe_w13_decode", "kimi_w4a16_w13_decode", "dsv3_moe_w13_prefill",
                                 "kimi_w4a16_w13_T8_tp8", "kimi_w4a16_w13_T1_tp8", "dsv3_moe_w2_decode",
                                 "dsv3_moe_w2_prefill"]
                         + [f"dsv3_ep8_{p}_M{m}" for m in (1, 16, 64, 512) for p in ("gate_up", "down")])
def test_moe_full_size(ops, key):
    from ferret_amd import workloads as W
    wl = W.WORKLOADS[key]
    _say(f"full-size {key}")
    inp = W.make_inputs(wl, "cuda")
    ids, _ = ops.moe_route_topk(inp["logits"], wl.topk)
    rt = ops.moe_permute(ids, wl.E)
    torch.cuda.synchronize()
    ids_np = ids.cpu().numpy()
    ref_ids, _ = R.route_topk(f32(inp["logits"]), wl.topk)
    assert np.array_equal(ids_np, ref_ids)
    counts, offsets, sp, tiles = oracle_routing(ids_np, wl.E, rt.tile_m)
    assert np.array_equal(rt.sorted_pair.cpu().numpy(), sp)
    assert np.array_equal(rt.tiles.cpu().numpy()[: int(rt.ntiles.item())], tiles)
    if wl.kind == "moe_fp8":
        out = ops.moe_w13_fp8(inp["x"], inp["sx"], inp["w"], inp["sw"], rt)
        out2 = ops.moe_w13_fp8(inp["x"], inp["sx"], inp["w"], inp["sw"], rt)
    elif wl.kind == "moe_fp8_w2":
        out = ops.moe_w2_fp8(inp["h"], inp["sh"], inp["w"], inp["sw"], rt)
        out2 = ops.moe_w2_fp8(inp["h"], inp["sh"], inp["w"], inp["sw"], rt)
    else:
        out = ops.moe_w13_w4a16(inp["x"], inp["w"], inp["ws"], rt)
        out2 = ops.moe_w13_w4a16(inp["x"], inp["w"], inp["ws"], rt)
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), out2.view(torch.int16)), "non-deterministic output"
    pairs, experts = moe_sample_pairs(ids_np, wl.E)
    # Host copies of only the sampled experts' weights.
    x_host = bits16(inp["x"]) if wl.kind == "moe_w4a16" else codes8(inp["h" if wl.kind == "moe_fp8_w2" else "x"])
    sub = np.full_like(ids_np, -1)
    emap = {e: i for i, e in enumerate(experts)}
    for t in range(ids_np.shape[0]):
        for j in range(ids_np.shape[1]):
            if int(ids_np[t, j]) in emap:
                sub[t, j] = emap[int(ids_np[t, j])]
    ex_t = torch.tensor(experts, device="cuda")
    if wl.kind == "moe_fp8":
        ref = G.moe_w13_fp8(x_host, f32(inp["sx"]), codes8(inp["w"][ex_t]), f32(inp["sw"][ex_t]), sub, pairs=pairs)
    elif wl.kind == "moe_fp8_w2":
        ref = G.moe_w2_fp8(x_host, f32(inp["sh"]), codes8(inp["w"][ex_t]), f32(inp["sw"][ex_t]), sub, pairs=pairs)
    else:
        ref = G.moe_w13_w4a16(x_host, inp["w"][ex_t].cpu().numpy(), bits16(inp["ws"][ex_t]), sub, pairs=pairs)
    got = bf16_out(out)[pairs]
    assert_gemm_close(got, ref, key)
