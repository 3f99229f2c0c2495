"""UE8M0 block scales: the oracle (oracle.ue8m0) pinned by facts independent of
its formulas, and the torch host helpers (ops.ue8m0_from_float / pack_ue8m0 /
expand_block_scales, CPU tensors) against it."""
import math

import numpy as np
import pytest
import torch

from oracle import formats as F
from oracle import gemm as G
from oracle import ue8m0 as U


def test_powers_of_two_map_to_their_own_byte():
    k = np.arange(-126, 128)
    v = np.ldexp(np.float32(1.0), k).astype(np.float32)
    assert np.array_equal(U.float_to_ue8m0(v), (k + 127).astype(np.uint8))
    assert np.array_equal(U.ue8m0_to_float((k + 127).astype(np.uint8)), v)


def _brute_nearest(v: float) -> int:
    """Exponent byte e in 1..254 minimising |log2(2^(e-127)) - log2(v)|, by search."""
    lv = math.log2(v)
    return min(range(1, 255), key=lambda e: abs((e - 127) - lv))


def test_log2_nearest_by_brute_force():
    rng = np.random.default_rng(0)
    v = np.exp(rng.uniform(-80, 80, 4000)).astype(np.float32)
    # values just either side of the midpoints 2^(k+1/2)
    mids = np.ldexp(np.sqrt(2.0), np.arange(-60, 60))
    v = np.concatenate([v, np.nextafter(mids.astype(np.float32), np.float32(0)),
                        np.nextafter(mids.astype(np.float32), np.float32(np.inf))])
    got = U.float_to_ue8m0(v)
    want = np.array([_brute_nearest(float(x)) for x in v], dtype=np.uint8)
    assert np.array_equal(got, want)


def test_reference_scale_range_splits_at_root_half():
    # v009 draws scales as 0.5 + (rand() % 100) / 200 -> [0.5, 0.995]
    v = (0.5 + np.arange(100) / 200.0).astype(np.float32)
    got = U.float_to_ue8m0(v)
    assert set(np.unique(got)) == {126, 127}
    assert np.array_equal(got == 127, v >= np.float32(0.7075))   # first grid value above 2^-0.5 = 0.70711


def test_special_values():
    v = np.array([0.0, -0.0, -3.0, np.inf, np.nan, -np.inf, 1e-45, 3.0e38], dtype=np.float32)
    assert U.float_to_ue8m0(v).tolist() == [0, 0, 0, 255, 255, 0, 0, 255]
    assert U.ue8m0_to_float(np.array([0], dtype=np.uint8))[0] == 0.0
    assert np.isinf(U.ue8m0_to_float(np.array([255], dtype=np.uint8))[0])


def test_packing_hand_example_and_round_trip():
    ue = np.array([[1, 2, 3, 4, 5], [6, 7, 8, 9, 10]], dtype=np.uint8)   # dim 2, nk 5
    words = U.prepare_sf(ue)
    assert words.shape == (2, 2)
    assert words.tolist() == [[0x04030201, 0x09080706], [0x00000005, 0x0000000A]]
    rng = np.random.default_rng(1)
    for dim, nk in [(1, 1), (3, 4), (7, 9), (128, 56), (5, 16)]:
        x = rng.integers(0, 256, (dim, nk), dtype=np.uint8)
        assert np.array_equal(U.unpack_sf(U.prepare_sf(x), nk), x)


def test_expand_sb_definition():
    sb = np.arange(3 * 4, dtype=np.float32).reshape(3, 4)
    e = U.expand_sb(sb, 300)
    assert e.shape == (300, 4)
    for n in (0, 127, 128, 255, 256, 299):
        assert np.array_equal(e[n], sb[n // 128])


def _brute_ref_bs(a, sa, b, sb):
    af, bf = F.e4m3_to_f32(a).astype(np.float64), F.e4m3_to_f32(b).astype(np.float64)
    M, K = a.shape
    N = b.shape[0]
    out = np.zeros((M, N))
    for m in range(M):
        for n in range(N):
            for kb in range(K // 128):
                s = 2.0 ** (np.round(np.log2(sa[m, kb]))) * 2.0 ** (np.round(np.log2(sb[n // 128, kb])))
                out[m, n] += float(np.dot(af[m, kb * 128:(kb + 1) * 128], bf[n, kb * 128:(kb + 1) * 128])) * s
    return out


def _codes(rng, shape):
    c = rng.integers(0, 254, shape).astype(np.uint8)
    return np.where(c >= 0x7F, c + 1, c).astype(np.uint8)   # v009's draw: skips the NaN codes


def test_ref_bs_against_float64_loops_and_a_mutant():
    rng = np.random.default_rng(2)
    M, N, K = 3, 130, 256
    a, b = _codes(rng, (M, K)), _codes(rng, (N, K))
    sa = rng.uniform(0.3, 3.0, (M, 2)).astype(np.float32)
    sb = rng.uniform(0.3, 3.0, (2, 2)).astype(np.float32)
    got = U.ref_bs(a, sa, b, sb).astype(np.float64)
    want = _brute_ref_bs(a, sa, b, sb)
    assert np.abs(got - want).max() <= 1e-5 * np.abs(want).max()
    # a wrong exponent on one block is visible
    bad_sb = sb.copy()
    bad_sb[1, 0] *= 2.0
    assert np.abs(U.ref_bs(a, sa, b, bad_sb) - want).max() > 1e-3 * np.abs(want).max()
    # with power-of-two scales ref_bs is the plain block-scaled oracle
    sa2 = np.ldexp(np.float32(1), rng.integers(-3, 4, sa.shape)).astype(np.float32)
    sb2 = np.ldexp(np.float32(1), rng.integers(-3, 4, sb.shape)).astype(np.float32)
    assert np.array_equal(U.ref_bs(a, sa2, b, sb2), G.fp8_blockscale_gemm(a, sa2, b, sb2))


def test_torch_helpers_match_the_oracle():
    from ferret_amd import ops
    rng = np.random.default_rng(3)
    v = np.concatenate([np.exp(rng.uniform(-60, 60, 2000)).astype(np.float32),
                        np.array([0, -1, np.inf, np.nan, 1e-45, 3e38], dtype=np.float32),
                        np.nextafter(np.ldexp(np.float32(np.sqrt(0.5)), np.arange(-5, 5)).astype(np.float32),
                                     np.float32(0))])
    assert np.array_equal(ops.ue8m0_from_float(torch.from_numpy(v)).numpy(), U.float_to_ue8m0(v))
    ue = rng.integers(0, 256, (37, 9), dtype=np.uint8)
    words = ops.pack_ue8m0(torch.from_numpy(ue)).numpy().view(np.uint32)
    assert np.array_equal(words, U.prepare_sf(ue))
    sb = rng.standard_normal((3, 5)).astype(np.float32)
    assert np.array_equal(ops.expand_block_scales(torch.from_numpy(sb), 300).numpy(), U.expand_sb(sb, 300))
    with pytest.raises(ValueError):
        ops.expand_block_scales(torch.from_numpy(sb), 500)
