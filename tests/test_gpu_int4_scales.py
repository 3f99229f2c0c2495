"""The INT4 W4A16 kernel's dequantized weights for every bf16 group scale and
every nibble, read out through the w13 GEMM, against the oracle.

One expert, N = 2048, K = 2048: the 1024 up rows carry the 65,536 bf16 scale
bit patterns, one per 32-wide group, and column k holds nibble k % 16, so
every (scale, nibble) pair occurs.  The gate rows hold nibble 12 (value 4)
under scale 8, a weight of exactly 32.  Token t has the one-hot activation
x[t, t] = 1, so gate = 32 and up = the dequantized weight u[n, t], both exact in
the fp32 accumulation; silu(32) is 32 in fp32 (exp(-32) < 2^-24), so the
output is bf16(32 * u) = 32 * u exactly.  Scales outside the dequant's
precondition (non-finite, or |s| >= 2^128 / 1032, where -1032 * s overflows)
are replaced by 0.  Both weight layouts must give the same bits.
"""
import numpy as np
import pytest
import torch

from oracle import formats as F
from tests.gpu_helpers import bf16_out

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ops(hip):
    from ferret_amd import ops as O
    return O


def test_int4_dequant_every_bf16_scale_and_nibble(ops):
    print("[case] int4 dequant, all bf16 scales x all nibbles", flush=True)
    N, K = 2048, 2048
    half, groups = N // 2, K // 32
    pat = np.arange(65536, dtype=np.uint32).astype(np.uint16).reshape(half, groups)
    s = F.bf16_bits_to_f32(pat)
    with np.errstate(over="ignore", invalid="ignore"):
        ok = np.isfinite(s) & np.isfinite(np.float32(-1032.0) * s)
    up_scales = np.where(ok, pat, 0).astype(np.uint16)
    nib = np.arange(K, dtype=np.int64) % 16
    row_words = (nib.reshape(K // 8, 8) << (4 * np.arange(8, dtype=np.int64))).sum(axis=1)
    up_words = np.broadcast_to(row_words.astype(np.uint32).view(np.int32), (half, K // 8))
    gate_words = np.full((half, K // 8), 0xCCCCCCCC, dtype=np.uint32).view(np.int32)
    gate_scales = np.full((half, groups), 0x4100, dtype=np.uint16)           # 8.0
    wq_np = np.concatenate([gate_words, up_words])[None]                       # [1, N, K/8]
    ws_np = np.concatenate([gate_scales, up_scales])[None]                     # [1, N, K/32]
    assert wq_np.shape == (1, N, K // 8) and ws_np.shape == (1, N, groups)
    wq = torch.from_numpy(np.ascontiguousarray(wq_np)).cuda()
    ws = torch.from_numpy(np.ascontiguousarray(ws_np).view(np.int16)).cuda().view(torch.bfloat16)
    T = K
    x = torch.zeros((T, K), dtype=torch.bfloat16, device="cuda")
    x[torch.arange(T), torch.arange(T)] = 1.0
    ids = torch.zeros((T, 1), dtype=torch.int32, device="cuda")
    rt = ops.moe_permute(ids, 1, 16)
    out = ops.moe_w13_w4a16(x, wq, ws, rt)
    out_t = ops.moe_w13_w4a16(x, ops.int4_tile_weights(wq), ws, rt)
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), out_t.view(torch.int16)), "the two INT4 layouts differ"
    u = F.int4_dequant(np.ascontiguousarray(up_words), up_scales)              # [half, K] bf16-exact
    want = (np.float32(32.0) * u).T                                             # [T, half], exact
    got = bf16_out(out)
    same = got == want                                                          # +0 == -0
    bad = np.argwhere(~same)
    assert same.all(), (f"{len(bad)} weights differ, e.g. (t, n) = {bad[:4].tolist()}: "
                        f"got {got[tuple(bad[0])] if len(bad) else None}, want {want[tuple(bad[0])] if len(bad) else None}")
