"""GPU parity of ferret_fp8_gemm_ue8m0 (UE8M0 power-of-two block scales in the
packed layout of examples/fp8-gemm/v009_large_m_block_scale_mma_080.cu) against
the oracle ref_bs (oracle.ue8m0), on the reference's own input draw (random e4m3
codes without NaN, scales 0.5 + (rand() % 100) / 200, v009:549-552) and on wider
scale ranges with zero scales; full-size v009 configs on sampled rows."""
import sys

import numpy as np
import pytest
import torch

from oracle import ue8m0 as U
from tests.gpu_helpers import assert_gemm_close, bf16_out

pytestmark = pytest.mark.gpu


def _say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def ops(hip):
    from ferret_amd import ops as _ops
    return _ops


def _inputs(M, N, K, seed, wide=False):
    rng = np.random.default_rng(seed)
    a = rng.integers(0, 254, (M, K)).astype(np.uint8)
    a = np.where(a >= 0x7F, a + 1, a).astype(np.uint8)
    b = rng.integers(0, 254, (N, K)).astype(np.uint8)
    b = np.where(b >= 0x7F, b + 1, b).astype(np.uint8)
    nk, nbk = K // 128, (N + 127) // 128
    if wide:
        sa = np.exp(rng.uniform(-6, 6, (M, nk))).astype(np.float32)
        sb = np.exp(rng.uniform(-6, 6, (nbk, nk))).astype(np.float32)
        sa[rng.random(sa.shape) < 0.05] = 0.0     # zero scales drop their blocks
        sb[rng.random(sb.shape) < 0.05] = 0.0
    else:
        sa = (0.5 + rng.integers(0, 100, (M, nk)) / 200.0).astype(np.float32)
        sb = (0.5 + rng.integers(0, 100, (nbk, nk)) / 200.0).astype(np.float32)
    return a, sa, b, sb


def _run(ops, a, sa, b, sb, rows=None):
    M, K = a.shape
    N = b.shape[0]
    sfa_np, sfb_np = U.packed_inputs(sa, sb, N)
    ad = torch.from_numpy(a).cuda()
    bd = torch.from_numpy(b).cuda()
    # the torch host helpers give the same words on the GPU
    sfa = ops.pack_ue8m0(ops.ue8m0_from_float(torch.from_numpy(sa).cuda()))
    sfb = ops.pack_ue8m0(ops.ue8m0_from_float(ops.expand_block_scales(torch.from_numpy(sb).cuda(), N)))
    assert np.array_equal(sfa.cpu().numpy().view(np.uint32), sfa_np)
    assert np.array_equal(sfb.cpu().numpy().view(np.uint32), sfb_np)
    c = ops.fp8_gemm_ue8m0(ad, sfa, bd, sfb)
    torch.cuda.synchronize()
    got = bf16_out(c)
    if rows is None:
        rows = np.arange(M)
    ref = U.ref_bs(a[rows], sa[rows], b, sb)
    return got[rows], ref


@pytest.mark.parametrize("M,N,K,wide", [(1, 128, 128, False), (16, 256, 640, True), (5, 400, 384, True),
                                        (77, 1024, 512, False), (128, 256, 1024, True), (300, 512, 640, False),
                                        (256, 4096, 7168, False), (512, 1024, 2048, True)])
def test_ue8m0_gemm_small(ops, M, N, K, wide):
    _say(f"fp8_gemm_ue8m0 M={M} N={N} K={K} wide={wide}")
    a, sa, b, sb = _inputs(M, N, K, seed=M * 7 + N + K, wide=wide)
    got, ref = _run(ops, a, sa, b, sb)
    assert_gemm_close(got, ref, f"ue8m0 M={M} N={N} K={K}")


# examples/fp8-gemm/v009_large_m_block_scale_mma_080.cu:526-532
@pytest.mark.parametrize("name,M,K,N", [("o_proj_M2048", 2048, 2048, 7168), ("q_b_proj_M8192", 8192, 1536, 3072),
                                        ("kv_b_proj_M8192", 8192, 512, 4096)])
def test_ue8m0_gemm_reference_configs(ops, name, M, K, N):
    _say(f"fp8_gemm_ue8m0 {name}")
    a, sa, b, sb = _inputs(M, N, K, seed=len(name) + M)
    rows = np.sort(np.random.default_rng(0).choice(M, 48, replace=False))
    got, ref = _run(ops, a, sa, b, sb, rows)
    assert_gemm_close(got, ref, f"ue8m0 {name}")


@pytest.mark.parametrize("M,N,K", [(3072, 4096, 640), (2048, 7168, 384), (3000, 4096, 640)])
def test_ue8m0_square_kernel_wide_scales(ops, M, N, K):
    """Shapes of the 256 x 256 kernel, which applies the packed scale bytes
    while widening each operand: scales over e^-6 .. e^6 with 5 % zero bytes
    (zeroed blocks, never 2^-127), on sampled rows plus the last rows.  At
    M = 3000 the last token tile is partial: its rows past M load scale words
    of the next K-block row or, in the last one, past the array (read as 0 by
    the buffer range check), and are never stored."""
    _say(f"fp8_gemm_ue8m0 square M={M} N={N} K={K} wide")
    a, sa, b, sb = _inputs(M, N, K, seed=M + N + K, wide=True)
    rows = np.unique(np.concatenate([np.random.default_rng(1).choice(M, 40, replace=False), [M - 2, M - 1]]))
    got, ref = _run(ops, a, sa, b, sb, rows)
    assert_gemm_close(got, ref, f"ue8m0 square M={M} N={N} K={K}")


def test_ue8m0_matches_fp32_scale_path_on_powers_of_two(ops):
    """With power-of-two fp32 scales both entry points compute the same product."""
    M, N, K = 200, 512, 1024
    a, _, b, _ = _inputs(M, N, K, seed=5)
    rng = np.random.default_rng(6)
    sa = np.ldexp(np.float32(1), rng.integers(-8, 8, (M, K // 128))).astype(np.float32)
    sb = np.ldexp(np.float32(1), rng.integers(-8, 8, (N // 128, K // 128))).astype(np.float32)
    got, ref = _run(ops, a, sa, b, sb)
    c2 = ops.fp8_gemm_blockscale(torch.from_numpy(a).cuda(), torch.from_numpy(sa).cuda(),
                                 torch.from_numpy(b).cuda(), torch.from_numpy(sb).cuda())
    torch.cuda.synchronize()
    assert np.array_equal(got, bf16_out(c2))
    assert_gemm_close(got, ref, "ue8m0 powers of two")
