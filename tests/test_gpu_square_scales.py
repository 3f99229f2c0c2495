"""The large-M square kernel (fp8_square.hip, 256 x 256 tiles) keeps its fp32
accumulator in units of the running block scale s = sa * sb and rescales it by
s_prev / s at every 128-K block.  These parity tests drive that rescale across
a wide range against the fp32 oracle (oracle.gemm.fp8_blockscale_gemm, the
reference's ref at examples/fp8-gemm/v002_dense_tp8_validated_065.cu:277-288):
activation scales log-uniform over 40 octaves within each token row around a
per-row offset, weight-block scales over another 40, so the products of one
output span up to 80 octaves and reach the fp32 subnormal range (below 2^-126,
where the kernel divides instead of taking a reciprocal) and underflow to 0;
5 % zero scales.  Each check runs on sampled rows plus the last rows of the
last (partial) token tile, both with the reference's metric over the sample
and per row (floor 1e-3 of that row's own max), so rows whose scales are tiny
are held to the same relative accuracy as the rest."""
import sys

import numpy as np
import pytest
import torch

from oracle import gemm as G
from tests.gpu_helpers import GEMM_TOL, assert_gemm_close, bf16_out

pytestmark = pytest.mark.gpu


def _codes(rng, shape):
    c = rng.integers(0, 254, shape).astype(np.uint8)
    return np.where(c >= 0x7F, c + 1, c).astype(np.uint8)     # no NaN codes


def _wide_scales(rng, M, N, K):
    nk, nbk = K // 128, N // 128
    row_off = rng.uniform(-95.0, -35.0, (M, 1))
    sa = np.exp2(row_off + rng.uniform(-20.0, 20.0, (M, nk))) * rng.uniform(1.0, 2.0, (M, nk))
    sb = np.exp2(rng.uniform(-40.0, 0.0, (nbk, nk))) * rng.uniform(1.0, 2.0, (nbk, nk))
    sa, sb = sa.astype(np.float32), sb.astype(np.float32)
    sa[rng.random(sa.shape) < 0.05] = 0.0
    sb[rng.random(sb.shape) < 0.05] = 0.0
    return sa, sb


# (3072, 4096) and (3000, 4096): 192 square-kernel tiles (the second with a
# partial last token tile).  Below the square kernel's threshold the tiled
# kernel (per-block folds) runs the same check: (1100, 4096) on 144 tiles of
# 256 x 128, and (1000, 4096), whose 128 such tiles would fill half the CUs,
# on 256 tiles of 128 x 128 (both with a partial last token tile).
@pytest.mark.parametrize("M,N,K", [(3072, 4096, 1024), (3000, 4096, 1024), (1100, 4096, 1024), (1000, 4096, 1024)])
def test_square_kernel_scales_over_80_octaves(hip, M, N, K):
    from ferret_amd import ops
    L = hip
    print(f"square kernel wide scales M={M} N={N} K={K}", flush=True)
    sys.stdout.flush()
    rng = np.random.default_rng(M + K)
    a, b = _codes(rng, (M, K)), _codes(rng, (N, K))
    sa, sb = _wide_scales(rng, M, N, K)
    prod = sa[:, :, None] * sb.T[None, :, :]                     # [M, nk, nbk] products as the kernel forms them
    nz = prod[prod != 0]
    assert (nz < 2.0 ** -126).any() and (nz > 2.0 ** -60).any()  # subnormal and ordinary products both occur
    c = ops.fp8_gemm_blockscale(torch.from_numpy(a).cuda(), torch.from_numpy(sa).cuda(),
                                torch.from_numpy(b).cuda(), torch.from_numpy(sb).cuda())
    torch.cuda.synchronize()
    rows = np.unique(np.concatenate([rng.choice(M, 40, replace=False), np.arange(M - 3, M)]))
    got = bf16_out(c)[rows]
    ref = G.fp8_blockscale_gemm(a[rows], sa[rows], b, sb)
    assert_gemm_close(got, ref, f"square wide scales M={M}")
    worst = 0.0
    for i, r in enumerate(rows):
        if np.abs(ref[i]).max() == 0:
            assert not got[i].any(), f"row {r}: all scale products are 0 but the output is not"
            continue
        worst = max(worst, assert_gemm_close(got[i], ref[i], f"square wide scales M={M} row {r}"))
    assert worst < GEMM_TOL
