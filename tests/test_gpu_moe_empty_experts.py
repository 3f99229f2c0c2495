"""GPU parity of the grouped MoE GEMMs when the routing leaves experts empty.

Crafted top-1 routings put 0 rows on every other expert and 1 .. 33 rows on
the rest (both sides of the 16-row decode tile and of the 128-row prefill
tile), so the tile tables skip empty experts between full and partial tiles.
Covered: FP8 w13 (SiLU) and w2 on the 16-row (stream kernel) and 128-row
(tiled kernel) tables, and INT4 W4A16 w13 on the checkpoint words and on
their tiles, against the oracle; every routed row is written (the output
starts as NaN) and both INT4 weight layouts give the same bits.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import gemm as G
from tests.gpu_helpers import assert_gemm_close, bf16_out, bits16, codes8, f32

pytestmark = pytest.mark.gpu

# rows per expert: empty experts between short, exact and just-past-a-tile ones
ROWS_DECODE = [0, 1, 0, 15, 16, 17, 0, 0, 31, 32, 33, 0, 5]
ROWS_PREFILL = [0, 127, 0, 128, 129, 0, 0, 1, 255, 0, 64]


def _say(msg):
    print(f"[case] {msg}", flush=True)


@pytest.fixture(scope="module")
def ops(hip):
    from ferret_amd import ops as O
    return O


def _ids(rows, seed):
    ids = np.concatenate([np.full(n, e, dtype=np.int32) for e, n in enumerate(rows)])
    np.random.default_rng(seed).shuffle(ids)
    return torch.from_numpy(ids.reshape(-1, 1)).cuda()


def _fp8_weights(E, N, K, seed):
    from ferret_amd import workloads as W
    w = torch.empty((E, N, K), dtype=torch.float8_e4m3fn, device="cuda")
    sw = torch.empty((E, N // 128, K // 128), dtype=torch.float32, device="cuda")
    for e in range(E):
        w[e], sw[e] = W.quant_weight_128x128(W.randn((N, K), seed + e, "cuda"))
    return w, sw


def _no_nan(out, what):
    assert not torch.isnan(out.float()).any().item(), f"{what}: a routed row was not written"


@pytest.mark.parametrize("rows,tile_m,N,K", [(ROWS_DECODE, 16, 512, 1024), (ROWS_DECODE, 16, 256, 7168),
                                             (ROWS_PREFILL, 128, 512, 1024)])
def test_w13_fp8_with_empty_experts(ops, rows, tile_m, N, K):
    from ferret_amd import workloads as W
    _say(f"w13 fp8 empty experts tile_m={tile_m} N={N} K={K}")
    ids = _ids(rows, N + K + tile_m)
    T, E = ids.shape[0], len(rows)
    x, sx = W.quant_act_1x128(W.randn((T, K), 11, "cuda"))
    w, sw = _fp8_weights(E, N, K, 300)
    rt = ops.moe_permute(ids, E, tile_m)
    assert int(rt.ntiles.item()) == sum((n + tile_m - 1) // tile_m for n in rows)
    out = torch.full((T, N // 2), float("nan"), dtype=torch.bfloat16, device="cuda")
    ops.moe_w13_fp8(x, sx, w, sw, rt, out=out)
    torch.cuda.synchronize()
    _no_nan(out, "w13")
    ref = G.moe_w13_fp8(codes8(x), f32(sx), codes8(w), f32(sw), ids.cpu().numpy())
    assert_gemm_close(bf16_out(out), ref, f"w13 tile_m={tile_m} N={N} K={K}")


@pytest.mark.parametrize("rows,tile_m,N,K", [(ROWS_DECODE, 16, 1024, 512), (ROWS_PREFILL, 128, 384, 768)])
def test_w2_fp8_with_empty_experts(ops, rows, tile_m, N, K):
    from ferret_amd import workloads as W
    _say(f"w2 fp8 empty experts tile_m={tile_m} N={N} K={K}")
    ids = _ids(rows, N + K + tile_m + 1)
    P, E = ids.shape[0], len(rows)
    h, sh = W.quant_act_1x128(W.randn((P, K), 13, "cuda"))
    w, sw = _fp8_weights(E, N, K, 500)
    rt = ops.moe_permute(ids, E, tile_m)
    out = torch.full((P, N), float("nan"), dtype=torch.bfloat16, device="cuda")
    ops.moe_w2_fp8(h, sh, w, sw, rt, out=out)
    torch.cuda.synchronize()
    _no_nan(out, "w2")
    ref = G.moe_w2_fp8(codes8(h), f32(sh), codes8(w), f32(sw), ids.cpu().numpy())
    assert_gemm_close(bf16_out(out), ref, f"w2 tile_m={tile_m} N={N} K={K}")


@pytest.mark.parametrize("N,K", [(256, 1024), (512, 7168)])
def test_w13_w4a16_with_empty_experts(ops, N, K):
    _say(f"w13 w4a16 empty experts N={N} K={K}")
    ids = _ids(ROWS_DECODE, N + K + 2)
    T, E = ids.shape[0], len(ROWS_DECODE)
    g = torch.Generator(device="cuda").manual_seed(N + K)
    x = torch.randn((T, K), generator=g, device="cuda").to(torch.bfloat16)
    wq = torch.randint(-2 ** 31, 2 ** 31, (E, N, K // 8), generator=g, device="cuda", dtype=torch.int32)
    ws = (torch.randn((E, N, K // 32), generator=g, device="cuda") * 0.01).to(torch.bfloat16)
    rt = ops.moe_permute(ids, E, 16)
    out = torch.full((T, N // 2), float("nan"), dtype=torch.bfloat16, device="cuda")
    ops.moe_w13_w4a16(x, wq, ws, rt, out=out)
    out_t = ops.moe_w13_w4a16(x, ops.int4_tile_weights(wq), ws, rt)
    torch.cuda.synchronize()
    _no_nan(out, "w4a16")
    assert torch.equal(out.view(torch.int16), out_t.view(torch.int16)), "the two INT4 layouts differ"
    ref = G.moe_w13_w4a16(bits16(x), wq.cpu().numpy(), bits16(ws), ids.cpu().numpy())
    assert_gemm_close(bf16_out(out), ref, f"w4a16 N={N} K={K}")
