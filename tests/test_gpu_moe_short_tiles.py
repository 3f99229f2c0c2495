"""GPU parity of the prefill MoE GEMMs (128-row tile table, fp8_tiled_kernel)
over experts whose row counts fall on both sides of 16, 64 and 128, so tiles
of every occupancy (one 16-row sub-tile up to full, and a full tile followed
by a one-row tile) meet, for w13 (SiLU epilogue) and w2 (routed store), on
shapes with one, four and eight scale blocks per row, against the oracle.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import gemm as G
from tests.gpu_helpers import assert_gemm_close, bf16_out, codes8, f32

pytestmark = pytest.mark.gpu

ROWS = [1, 15, 16, 17, 33, 63, 64, 65, 127, 128, 129, 200]


def _say(msg):
    print(f"[case] {msg}", flush=True)


@pytest.fixture(scope="module")
def ops(hip):
    from ferret_amd import ops as O
    return O


def _ids_for_rows(rows, seed):
    """topk = 1 routing with expert e receiving rows[e] tokens, tokens shuffled."""
    ids = np.concatenate([np.full(n, e, dtype=np.int32) for e, n in enumerate(rows)])
    np.random.default_rng(seed).shuffle(ids)
    return torch.from_numpy(ids.reshape(-1, 1)).cuda()


def _weights(E, N, K, seed):
    from ferret_amd import workloads as W
    w = torch.empty((E, N, K), dtype=torch.float8_e4m3fn, device="cuda")
    sw = torch.empty((E, N // 128, K // 128), dtype=torch.float32, device="cuda")
    for e in range(E):
        w[e], sw[e] = W.quant_weight_128x128(W.randn((N, K), seed + e, "cuda"))
    return w, sw


@pytest.mark.parametrize("N,K", [(256, 512), (512, 2048), (768, 256)])
def test_w13_prefill_short_and_long_tiles(ops, N, K):
    from ferret_amd import workloads as W
    _say(f"w13 short tiles N={N} K={K}")
    ids = _ids_for_rows(ROWS, N + K)
    T, E = ids.shape[0], len(ROWS)
    x, sx = W.quant_act_1x128(W.randn((T, K), 3, "cuda"))
    w, sw = _weights(E, N, K, 40)
    rt = ops.moe_permute(ids, E, 128)
    out = torch.full((T, N // 2), float("nan"), dtype=torch.bfloat16, device="cuda")
    ops.moe_w13_fp8(x, sx, w, sw, rt, out=out)
    out2 = ops.moe_w13_fp8(x, sx, w, sw, rt)
    torch.cuda.synchronize()
    ref = G.moe_w13_fp8(codes8(x), f32(sx), codes8(w), f32(sw), ids.cpu().numpy())
    assert_gemm_close(bf16_out(out), ref, f"w13 N={N} K={K}")
    assert torch.equal(out.view(torch.int16), out2.view(torch.int16)), "non-deterministic output"


@pytest.mark.parametrize("N,K", [(256, 512), (7168, 2048), (384, 768)])
def test_w2_prefill_short_and_long_tiles(ops, N, K):
    from ferret_amd import workloads as W
    _say(f"w2 short tiles N={N} K={K}")
    ids = _ids_for_rows(ROWS, N + K + 1)
    P, E = ids.shape[0], len(ROWS)
    h, sh = W.quant_act_1x128(W.randn((P, K), 5, "cuda"))
    w, sw = _weights(E, N, K, 70)
    rt = ops.moe_permute(ids, E, 128)
    out = torch.full((P, N), float("nan"), dtype=torch.bfloat16, device="cuda")
    ops.moe_w2_fp8(h, sh, w, sw, rt, out=out)
    torch.cuda.synchronize()
    ref = G.moe_w2_fp8(codes8(h), f32(sh), codes8(w), f32(sw), ids.cpu().numpy())
    assert_gemm_close(bf16_out(out), ref, f"w2 N={N} K={K}")
