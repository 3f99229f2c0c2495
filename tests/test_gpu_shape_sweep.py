"""GPU parity over a seeded sweep of shapes across the dispatch space of the
dense and decode-MoE entry points, against the oracle:

- FP8 block-scaled GEMM at M <= 16 (stream-kernel configurations by K-steps
  per wave, the 14-wave single-unit case, the per-unit kernel, N not a
  multiple of 128), 16 < M <= 256 (split-K tiles with a workspace) and M up to
  640 (256 x 128 tiles);
- bf16 linear at decode M, with and without residual, from a few row units per
  CU to many (the 4-wave units whose first unit interleaves its activations
  with its weight stages, across token-tile and K-split boundaries);
- every path at K/128 counts that no K-step count divides into at most 16
  waves (19, 23, 38, 45, ...): the per-unit kernel's ragged last wave;
- the FP8 and W4A16 MoE w13 decode at such K.

The shapes come from fixed seeds, so every run sees the same list; they are
sized so that the oracle finishes in seconds.
"""
import sys

import numpy as np
import pytest
import torch

from oracle import gemm as G
from tests.gpu_helpers import assert_gemm_close, bf16_out, bits16, codes8, f32

pytestmark = pytest.mark.gpu

# K/128 counts with no divisor in {1, 2, 4, 7, 8} giving 1..16 waves
RAGGED_NKB = [17, 19, 23, 25, 31, 33, 38, 45, 61, 67, 97, 125]


def _say(msg):
    print(f"[case] {msg}", flush=True)
    sys.stdout.flush()


def _fp8_shapes():
    rng = np.random.default_rng(20261202)
    out = []
    for _ in range(12):  # decode: N % 16, K up to 8192 (1..64 K-steps)
        out.append((int(rng.integers(1, 17)), 16 * int(rng.integers(1, 257)), 128 * int(rng.integers(1, 65))))
    out += [(16, 4096, 7168), (1, 4096, 1792), (9, 2048, 3584)]  # 14-wave / 8-wave K-step patterns
    for nkb in RAGGED_NKB[::2]:  # decode at ragged K
        out.append((int(rng.integers(1, 17)), 16 * int(rng.integers(1, 129)), 128 * nkb))
    for _ in range(8):  # 16 < M <= 256
        out.append((int(rng.integers(17, 257)), 128 * int(rng.integers(1, 17)), 128 * int(rng.integers(1, 41))))
    for _ in range(4):  # M up to 640
        out.append((int(rng.integers(257, 641)), 128 * int(rng.integers(1, 9)), 128 * int(rng.integers(1, 25))))
    return out


def _bf16_shapes():
    rng = np.random.default_rng(20261203)
    out = []
    for _ in range(10):
        out.append((int(rng.integers(1, 17)), 16 * int(rng.integers(1, 513)), 128 * int(rng.integers(1, 49)),
                    bool(rng.integers(0, 2))))
    for _ in range(4):  # >= 4 row units per CU, with token tiles past 16 rows
        out.append((int(rng.integers(1, 41)), 16384 + 16 * int(rng.integers(0, 257)), 128 * int(rng.integers(2, 17)),
                    bool(rng.integers(0, 2))))
    for nkb in RAGGED_NKB[1::2]:
        out.append((int(rng.integers(1, 17)), 16 * int(rng.integers(1, 257)), 128 * nkb, bool(rng.integers(0, 2))))
    return out


def _quant_weight(N, K, seed):
    """128 x 128 block-quantized e4m3 weights for any N % 16 == 0: the last
    scale block covers the remaining rows (zero padding adds nothing to amax)."""
    from ferret_amd import workloads as W
    n128 = (N + 127) // 128 * 128
    full = torch.zeros((n128, K), dtype=torch.float32, device="cuda")
    full[:N] = W.randn((N, K), seed, "cuda")
    b, sb = W.quant_weight_128x128(full)
    return b[:N].contiguous(), sb.contiguous()


@pytest.fixture(scope="module")
def ops(hip):
    from ferret_amd import ops as O
    return O


@pytest.mark.parametrize("M,N,K", _fp8_shapes())
def test_fp8_gemm_shape_sweep(ops, M, N, K):
    from ferret_amd import workloads as W
    _say(f"fp8 sweep M={M} N={N} K={K}")
    a, sa = W.quant_act_1x128(W.randn((M, K), M * 7 + K, "cuda"))
    b, sb = _quant_weight(N, K, N + K)
    ws = torch.empty(max(1, ops.fp8_workspace_bytes(M, N, K)), dtype=torch.uint8, device="cuda")
    c = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device="cuda")
    ops.fp8_gemm_blockscale(a, sa, b, sb, out=c, workspace=ws)
    torch.cuda.synchronize()
    ref = G.fp8_blockscale_gemm(codes8(a), f32(sa), codes8(b), f32(sb))
    assert_gemm_close(bf16_out(c), ref, f"fp8 sweep M={M} N={N} K={K}")


@pytest.mark.parametrize("M,N,K,res", _bf16_shapes())
def test_linear_bf16_shape_sweep(ops, M, N, K, res):
    _say(f"bf16 sweep M={M} N={N} K={K} res={res}")
    g = torch.Generator(device="cuda").manual_seed(M * 131 + N + K)
    x = torch.randn((M, K), generator=g, device="cuda").to(torch.bfloat16)
    w = (torch.randn((N, K), generator=g, device="cuda") * 0.05).to(torch.bfloat16)
    r = torch.randn((M, N), generator=g, device="cuda").to(torch.bfloat16) if res else None
    ws = torch.empty(max(1, ops.linear_workspace_bytes(M, N, K)), dtype=torch.uint8, device="cuda")
    y = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device="cuda")
    ops.linear_bf16(x, w, r, out=y, workspace=ws)
    torch.cuda.synchronize()
    ref = G.linear_bf16(bits16(x), bits16(w), bits16(r) if res else None)
    assert_gemm_close(bf16_out(y), ref, f"bf16 sweep M={M} N={N} K={K}")


@pytest.mark.parametrize("T,E,N,nkb,topk", [(24, 6, 256, 19, 3), (40, 5, 512, 45, 2), (9, 4, 256, 23, 4)])
def test_moe_w13_fp8_decode_ragged_k(ops, T, E, N, nkb, topk):
    from ferret_amd import workloads as W
    K = 128 * nkb
    _say(f"moe_w13_fp8 ragged T={T} E={E} N={N} K={K} topk={topk}")
    x, sx = W.quant_act_1x128(W.randn((T, K), T + K, "cuda"))
    w = torch.empty((E, N, K), dtype=torch.float8_e4m3fn, device="cuda")
    sw = torch.empty((E, N // 128, K // 128), dtype=torch.float32, device="cuda")
    for e in range(E):
        w[e], sw[e] = W.quant_weight_128x128(W.randn((N, K), 100 + e + K, "cuda"))
    ids, _ = ops.moe_route_topk(W.randn((T, E), T + 5, "cuda"), topk)
    rt = ops.moe_permute(ids, E, 16)
    out = ops.moe_w13_fp8(x, sx, w, sw, rt)
    torch.cuda.synchronize()
    ref = G.moe_w13_fp8(codes8(x), f32(sx), codes8(w), f32(sw), ids.cpu().numpy())
    assert_gemm_close(bf16_out(out), ref, f"moe_w13_fp8 ragged K={K}")


@pytest.mark.parametrize("T,E,N,nkb,topk", [(16, 6, 128, 19, 3), (33, 5, 256, 38, 2)])
def test_moe_w13_w4a16_decode_ragged_k(ops, T, E, N, nkb, topk):
    K = 128 * nkb
    _say(f"moe_w13_w4a16 ragged T={T} E={E} N={N} K={K} topk={topk}")
    g = torch.Generator(device="cuda").manual_seed(T + E + N + K)
    x = torch.randn((T, K), generator=g, device="cuda").to(torch.bfloat16)
    wq = torch.randint(-2 ** 31, 2 ** 31, (E, N, K // 8), generator=g, device="cuda", dtype=torch.int32)
    ws = (torch.randn((E, N, K // 32), generator=g, device="cuda") * 0.01).to(torch.bfloat16)
    ids, _ = ops.moe_route_topk(torch.randn((T, E), generator=g, device="cuda"), topk)
    rt = ops.moe_permute(ids, E, 16)
    out = ops.moe_w13_w4a16(x, wq, ws, rt)
    torch.cuda.synchronize()
    ref = G.moe_w13_w4a16(bits16(x), wq.cpu().numpy(), bits16(ws), ids.cpu().numpy())
    assert_gemm_close(bf16_out(out), ref, f"moe_w13_w4a16 ragged K={K}")
