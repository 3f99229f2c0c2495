"""Every OCP e4m3 code through every FP8 GEMM kernel, exactly.

With unit block scales, one operand one-hot (the code of 1.0 at one K index
per row) and the other carrying every non-NaN e4m3 code, each output is a
single e4m3 value, which bf16 holds exactly: c[m, n] = b[n, m % K] (codes on
the weight side) or a[m, n % K] (codes on the token side).  The shapes pick
the square kernel (M = N = 4096), the 256 x 128 tiled kernel (M = 300), its
split-K form (M = 128) and the decode stream kernel (M = 16, M = 1), so the
widening of both operands in each kernel is checked code by code against the
oracle's decoding of the code.  The grouped down projection (routed rows, one
expert empty) gets the same check on both tile tables.
"""
import numpy as np
import pytest
import torch

from oracle import formats as F
from tests.gpu_helpers import bf16_out

pytestmark = pytest.mark.gpu

ONE = 0x38  # e4m3 1.0


@pytest.fixture(scope="module")
def ops(hip):
    from ferret_amd import ops as O
    return O


def _codes(rows, K):
    """Every code in turn (NaN codes 0x7F / 0xFF replaced by 0)."""
    c = (np.arange(rows * K, dtype=np.int64) * 7 + np.arange(rows * K, dtype=np.int64) // 256) % 256
    c = c.astype(np.uint8).reshape(rows, K)
    c[(c & 0x7F) == 0x7F] = 0
    return c


def _one_hot(rows, K):
    c = np.zeros((rows, K), dtype=np.uint8)
    c[np.arange(rows), np.arange(rows) % K] = ONE
    return c


@pytest.mark.parametrize("M,N,K", [(4096, 4096, 256), (300, 512, 384), (128, 512, 512), (16, 1024, 512),
                                   (1, 512, 256)])
@pytest.mark.parametrize("side", ["weights", "tokens"])
def test_every_e4m3_code_exactly(ops, M, N, K, side):
    print(f"[case] e4m3 codes M={M} N={N} K={K} codes on {side}", flush=True)
    if side == "weights":
        a_np, b_np = _one_hot(M, K), _codes(N, K)
        want = F.e4m3_to_f32(b_np)[:, np.arange(M) % K].T                     # [M, N]
    else:
        a_np, b_np = _codes(M, K), _one_hot(N, K)
        want = F.e4m3_to_f32(a_np)[:, np.arange(N) % K]                       # [M, N]
    codes = np.unique(b_np if side == "weights" else a_np)
    assert len(codes) == 254                                                   # all but the two NaNs
    a = torch.from_numpy(a_np).cuda().view(torch.float8_e4m3fn)
    b = torch.from_numpy(b_np).cuda().view(torch.float8_e4m3fn)
    sa = torch.ones((M, K // 128), dtype=torch.float32, device="cuda")
    sb = torch.ones((N // 128, K // 128), dtype=torch.float32, device="cuda")
    out = ops.fp8_gemm_blockscale(a, sa, b, sb)
    torch.cuda.synchronize()
    got = bf16_out(out)
    same = got == want                                                         # +0 == -0
    bad = np.argwhere(~same)
    assert same.all(), f"{len(bad)} outputs differ, first (m, n) = {bad[:3].tolist()}"


@pytest.mark.parametrize("tile_m,rows", [(16, [20, 0, 37, 3]), (128, [140, 0, 300, 17])])
@pytest.mark.parametrize("side", ["weights", "tokens"])
def test_every_e4m3_code_through_the_grouped_down_projection(ops, tile_m, rows, side):
    """The same through moe_w2_fp8 (routed rows, pair order), on the decode
    (16-row) and prefill (128-row) tile tables: out[p, n] = w[e_p, n, p % K]
    or h[p, n % K]."""
    N, K = 512, 384
    print(f"[case] e4m3 codes w2 tile_m={tile_m} codes on {side}", flush=True)
    E = len(rows)
    ids_np = np.concatenate([np.full(n, e, dtype=np.int32) for e, n in enumerate(rows)])
    np.random.default_rng(tile_m).shuffle(ids_np)
    P = len(ids_np)
    if side == "weights":
        h_np = _one_hot(P, K)
        w_np = np.stack([_codes(N, K) for _ in range(E)])
        want = F.e4m3_to_f32(w_np)[ids_np[:, None], np.arange(N)[None, :], (np.arange(P) % K)[:, None]]
        codes = np.unique(w_np)
    else:
        h_np = _codes(P, K)
        w_np = np.stack([_one_hot(N, K) for _ in range(E)])
        want = F.e4m3_to_f32(h_np)[:, np.arange(N) % K]
        codes = np.unique(h_np)
    assert len(codes) == 254
    h = torch.from_numpy(h_np).cuda().view(torch.float8_e4m3fn)
    w = torch.from_numpy(np.ascontiguousarray(w_np)).cuda().view(torch.float8_e4m3fn)
    sh = torch.ones((P, K // 128), dtype=torch.float32, device="cuda")
    sw = torch.ones((E, N // 128, K // 128), dtype=torch.float32, device="cuda")
    ids = torch.from_numpy(ids_np.reshape(-1, 1)).cuda()
    rt = ops.moe_permute(ids, E, tile_m)
    out = torch.full((P, N), float("nan"), dtype=torch.bfloat16, device="cuda")
    ops.moe_w2_fp8(h, sh, w, sw, rt, out=out)
    torch.cuda.synchronize()
    got = bf16_out(out)
    same = got == want
    bad = np.argwhere(~same)
    assert same.all(), f"{len(bad)} outputs differ, first (p, n) = {bad[:3].tolist()}"


@pytest.mark.parametrize("tile_m,rows", [(16, [20, 0, 37, 3]), (128, [140, 0, 300, 17])])
def test_every_e4m3_code_through_the_grouped_gate_up_projection(ops, tile_m, rows):
    """moe_w13_fp8 with every gate weight 32.0 and one-hot activations: gate =
    32 and silu(32) = 32 in fp32 (exp(-32) < 2^-24), so out[p, n] = 32 *
    up[e_p, n, t % K] exactly, with every code on the up rows."""
    N, K = 512, 384
    print(f"[case] e4m3 codes w13 tile_m={tile_m}", flush=True)
    E = len(rows)
    ids_np = np.concatenate([np.full(n, e, dtype=np.int32) for e, n in enumerate(rows)])
    np.random.default_rng(tile_m + 1).shuffle(ids_np)
    T = len(ids_np)
    x_np = _one_hot(T, K)
    up = np.stack([_codes(N // 2, K) for _ in range(E)])
    w_np = np.concatenate([np.full((E, N // 2, K), 0x60, dtype=np.uint8), up], axis=1)  # 0x60 = 32.0
    assert F.e4m3_to_f32(np.array([0x60], dtype=np.uint8))[0] == 32.0 and len(np.unique(up)) == 254
    want = 32.0 * F.e4m3_to_f32(up)[ids_np[:, None], np.arange(N // 2)[None, :], (np.arange(T) % K)[:, None]]
    x = torch.from_numpy(x_np).cuda().view(torch.float8_e4m3fn)
    w = torch.from_numpy(np.ascontiguousarray(w_np)).cuda().view(torch.float8_e4m3fn)
    sx = torch.ones((T, K // 128), dtype=torch.float32, device="cuda")
    sw = torch.ones((E, N // 128, K // 128), dtype=torch.float32, device="cuda")
    ids = torch.from_numpy(ids_np.reshape(-1, 1)).cuda()
    rt = ops.moe_permute(ids, E, tile_m)
    out = torch.full((T, N // 2), float("nan"), dtype=torch.bfloat16, device="cuda")
    ops.moe_w13_fp8(x, sx, w, sw, rt, out=out)
    torch.cuda.synchronize()
    got = bf16_out(out)
    same = got == want
    bad = np.argwhere(~same)
    assert same.all(), f"{len(bad)} outputs differ, first (t, n) = {bad[:3].tolist()}"


@pytest.mark.parametrize("M,N,K", [(4096, 4096, 2048), (300, 2048, 2048)])
@pytest.mark.parametrize("side", ["weights", "tokens"])
def test_every_ue8m0_scale_byte_exactly(ops, M, N, K, side):
    """UE8M0 mode: unit e4m3 values, one side one-hot, and every scale byte
    1..254 on the other side's blocks (byte 127 on this side), so c[m, n] =
    2^(e - 127) exactly for the byte e of its block.  M = N = 4096 runs the
    square kernel with the bytes folded into the widening; M = 300 the decoded
    fp32 scales through the tiled kernel."""
    print(f"[case] ue8m0 bytes M={M} N={N} K={K} bytes on {side}", flush=True)
    nk = K // 128
    if side == "weights":
        a_np = _one_hot(M, K)
        b_np = np.full((N, K), ONE, dtype=np.uint8)
        blk = (np.arange(N // 128)[:, None] * nk + np.arange(nk)[None, :])
        eb = (1 + blk % 254).astype(np.uint8)                                   # [N/128, nk]
        ue_a = np.full((M, nk), 127, dtype=np.uint8)
        ue_b = np.repeat(eb, 128, axis=0)                                       # one row per weight row
        want = np.ldexp(1.0, eb[(np.arange(N) // 128)[None, :], ((np.arange(M) % K) // 128)[:, None]].astype(np.int64)
                        - 127).astype(np.float32)
        used = np.unique(eb)
    else:
        a_np = np.full((M, K), ONE, dtype=np.uint8)
        b_np = _one_hot(N, K)
        ea = (1 + (np.arange(M)[:, None] * nk + np.arange(nk)[None, :]) % 254).astype(np.uint8)   # [M, nk]
        ue_a = ea
        ue_b = np.full((N, nk), 127, dtype=np.uint8)
        want = np.ldexp(1.0, ea[:, ((np.arange(N) % K) // 128)].astype(np.int64) - 127).astype(np.float32)
        used = np.unique(ea)
    assert len(used) == 254 and used.min() == 1 and used.max() == 254
    a = torch.from_numpy(a_np).cuda().view(torch.float8_e4m3fn)
    b = torch.from_numpy(b_np).cuda().view(torch.float8_e4m3fn)
    sfa = ops.pack_ue8m0(torch.from_numpy(ue_a).cuda())
    sfb = ops.pack_ue8m0(torch.from_numpy(np.ascontiguousarray(ue_b)).cuda())
    out = ops.fp8_gemm_ue8m0(a, sfa, b, sfb)
    torch.cuda.synchronize()
    got = bf16_out(out)
    same = got == want
    bad = np.argwhere(~same)
    assert same.all(), f"{len(bad)} outputs differ, first (m, n) = {bad[:3].tolist()}"
