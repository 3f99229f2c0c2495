"""Pin the oracle's GEMM restatements: brute force, closed forms, special cases, mutants."""
import numpy as np
import pytest

from oracle import formats as F
from oracle import gemm as G
from oracle import quant as Q

RNG = np.random.default_rng(1234)


def _rand_fp8(shape, rng=RNG):
    codes = rng.integers(0, 254, size=shape).astype(np.uint8)
    codes[codes >= 0x7F] += 1          # skip the 0x7F NaN code, as v002:325-328
    return codes


def _brute_fp8(a, sa, b, sb):
    """Triple loop straight from the block-scaled definition (float64 accumulate)."""
    av = F.e4m3_to_f32(a).astype(np.float64)
    bv = F.e4m3_to_f32(b).astype(np.float64)
    m, k = a.shape
    n = b.shape[0]
    c = np.zeros((m, n))
    for i in range(m):
        for j in range(n):
            s = 0.0
            for kk in range(k):
                s += av[i, kk] * bv[j, kk] * sa[i, kk // 128] * sb[j // 128, kk // 128]
            c[i, j] = s
    return c


def test_fp8_gemm_brute_force_tiny():
    m, n, k = 3, 130, 256
    a = _rand_fp8((m, k)); b = _rand_fp8((n, k))
    sa = RNG.uniform(0.5, 1.0, size=(m, 2)).astype(np.float32)
    sb = RNG.uniform(0.5, 1.0, size=(2, 2)).astype(np.float32)
    ours = G.fp8_blockscale_gemm(a, sa, b, sb)
    ref = _brute_fp8(a, sa, b, sb)
    assert np.allclose(ours, ref, rtol=1e-5, atol=1e-3 * np.abs(ref).max())


def test_fp8_gemm_unit_scales_is_plain_matmul():
    m, n, k = 5, 128, 384
    a = _rand_fp8((m, k)); b = _rand_fp8((n, k))
    ours = G.fp8_blockscale_gemm(a, np.ones((m, 3), np.float32), b, np.ones((1, 3), np.float32))
    ref = F.e4m3_to_f32(a).astype(np.float64) @ F.e4m3_to_f32(b).astype(np.float64).T
    assert np.allclose(ours, ref, rtol=1e-5, atol=1e-3 * np.abs(ref).max())


def test_fp8_gemm_power_of_two_scales_small_ints_exact():
    # Codes for small integers: 1.0=0x38, 2.0=0x40, -1.0=0xB8, 0.5=0x30
    vals = np.array([0x38, 0x40, 0xB8, 0x30], dtype=np.uint8)
    m, n, k = 4, 128, 256
    a = RNG.choice(vals, size=(m, k)); b = RNG.choice(vals, size=(n, k))
    sa = np.float32(2.0) ** RNG.integers(-3, 3, size=(m, 2)).astype(np.float32)
    sb = np.float32(2.0) ** RNG.integers(-3, 3, size=(1, 2)).astype(np.float32)
    ours = G.fp8_blockscale_gemm(a, sa, b, sb)
    ref = _brute_fp8(a, sa, b, sb)
    assert np.array_equal(ours.astype(np.float64), ref)


def test_fp8_gemm_single_block_closed_form():
    m, n, k = 2, 128, 128
    a = _rand_fp8((m, k)); b = _rand_fp8((n, k))
    sa = np.array([[0.75], [1.5]], np.float32); sb = np.array([[0.25]], np.float32)
    ours = G.fp8_blockscale_gemm(a, sa, b, sb)
    dot = F.e4m3_to_f32(a).astype(np.float64) @ F.e4m3_to_f32(b).astype(np.float64).T
    ref = dot * sa.astype(np.float64) * 0.25
    assert np.allclose(ours, ref, rtol=1e-5, atol=1e-5 * np.abs(ref).max())


def test_fp8_gemm_rejects_planted_mutants():
    """A dropped K block, a transposed operand or a wrong scale index must fail the gate."""
    from oracle.metrics import gate_fp8
    m, n, k = 8, 256, 512
    x = RNG.standard_normal((m, k)).astype(np.float32)
    w = RNG.standard_normal((n, k)).astype(np.float32)
    a, sa = Q.quant_act_1x128(x); b, sb = Q.quant_weight_128x128(w)
    good = G.fp8_blockscale_gemm(a, sa, b, sb)
    # dropped last block
    bad1 = G.fp8_blockscale_gemm(a[:, :384], sa[:, :3], b[:, :384], sb[:, :3])
    # scale blocks of the weight swapped along N
    bad2 = G.fp8_blockscale_gemm(a, sa, b, sb[::-1].copy())
    # activation scale transposed in K-block order
    bad3 = G.fp8_blockscale_gemm(a, sa[:, ::-1].copy(), b, sb)
    assert gate_fp8(good, good)
    for bad in (bad1, bad2, bad3):
        assert not gate_fp8(bad, good)


def test_quantized_gemm_tracks_fp32_product():
    m, n, k = 4, 256, 512
    x = RNG.standard_normal((m, k)).astype(np.float32)
    w = RNG.standard_normal((n, k)).astype(np.float32)
    a, sa = Q.quant_act_1x128(x); b, sb = Q.quant_weight_128x128(w)
    c = G.fp8_blockscale_gemm(a, sa, b, sb)
    exact = x.astype(np.float64) @ w.astype(np.float64).T
    # e4m3 has 3 mantissa bits: relative rounding <= 1/16 per operand, errors average out.
    assert np.abs(c - exact).max() < 0.1 * np.abs(exact).max()


def test_linear_bf16_brute_force_and_residual():
    m, n, k = 3, 5, 40
    x = F.f32_to_bf16_bits(RNG.standard_normal((m, k)).astype(np.float32))
    w = F.f32_to_bf16_bits(RNG.standard_normal((n, k)).astype(np.float32))
    r = F.f32_to_bf16_bits(RNG.standard_normal((m, n)).astype(np.float32))
    xs = F.bf16_bits_to_f32(x).astype(np.float64); ws = F.bf16_bits_to_f32(w).astype(np.float64)
    brute = np.array([[sum(xs[i, kk] * ws[j, kk] for kk in range(k)) for j in range(n)] for i in range(m)])
    assert np.allclose(G.linear_bf16(x, w), brute, rtol=1e-5, atol=1e-5)
    assert np.allclose(G.linear_bf16(x, w, r), brute + F.bf16_bits_to_f32(r), rtol=1e-5, atol=1e-5)


def test_linear_bf16_small_integers_exact():
    m, n, k = 4, 6, 64
    x = F.f32_to_bf16_bits(RNG.integers(-4, 5, size=(m, k)).astype(np.float32))
    w = F.f32_to_bf16_bits(RNG.integers(-4, 5, size=(n, k)).astype(np.float32))
    exact = F.bf16_bits_to_f32(x).astype(np.int64) @ F.bf16_bits_to_f32(w).astype(np.int64).T
    assert np.array_equal(G.linear_bf16(x, w), exact.astype(np.float32))


def test_silu_mul_closed_form():
    g = np.array([0.0, 1.0, -1.0, 20.0, -100.0], np.float32)
    u = np.array([3.0, 2.0, 2.0, 1.0, 5.0], np.float32)
    out = G.silu_mul(g, u)
    expect = g.astype(np.float64) / (1 + np.exp(-g.astype(np.float64))) * u
    assert out[0] == 0.0
    assert np.allclose(out, expect, rtol=1e-6, atol=1e-30)
    assert abs(out[4]) < 1e-30          # large negative gate -> 0 (no NaN)


def _moe_inputs_fp8(T, E, N, K, topk, rng):
    x = rng.standard_normal((T, K)).astype(np.float32)
    xq, sx = Q.quant_act_1x128(x)
    wq = np.empty((E, N, K), np.uint8); sw = np.empty((E, N // 128, K // 128), np.float32)
    for e in range(E):
        wq[e], sw[e] = Q.quant_weight_128x128(rng.standard_normal((N, K)).astype(np.float32))
    ids = np.stack([rng.choice(E, size=topk, replace=False) for _ in range(T)]).astype(np.int32)
    return xq, sx, wq, sw, ids


def test_moe_fp8_per_row_expert_matches_dense_per_pair():
    rng = np.random.default_rng(7)
    T, E, N, K, topk = 5, 6, 256, 256, 3
    xq, sx, wq, sw, ids = _moe_inputs_fp8(T, E, N, K, topk, rng)
    out = G.moe_w13_fp8(xq, sx, wq, sw, ids)
    assert out.shape == (T * topk, N // 2)
    for t in range(T):
        for j in range(topk):
            e = ids[t, j]
            gu = G.fp8_blockscale_gemm(xq[t:t + 1], sx[t:t + 1], wq[e], sw[e])[0]
            ref = G.silu_mul(gu[:N // 2], gu[N // 2:])
            assert np.allclose(out[t * topk + j], ref, rtol=1e-5, atol=1e-5 * np.abs(ref).max())
    # A wrong-expert mutant (tile-uniform expert, the reference's F2 behaviour) differs.
    wrong = ids.copy(); wrong[:, 1] = wrong[:, 0]
    assert not np.allclose(G.moe_w13_fp8(xq, sx, wq, sw, wrong), out)


def test_moe_fp8_pair_subset():
    rng = np.random.default_rng(8)
    T, E, N, K, topk = 4, 5, 256, 128, 2
    xq, sx, wq, sw, ids = _moe_inputs_fp8(T, E, N, K, topk, rng)
    full = G.moe_w13_fp8(xq, sx, wq, sw, ids)
    sub = G.moe_w13_fp8(xq, sx, wq, sw, ids, pairs=np.array([7, 0, 3]))
    assert np.array_equal(sub, full[[7, 0, 3]])


def test_moe_w4a16_matches_explicit_dequant_matmul():
    rng = np.random.default_rng(9)
    T, E, N, K, topk = 3, 4, 64, 128, 2
    x = F.f32_to_bf16_bits(rng.standard_normal((T, K)).astype(np.float32))
    wq = rng.integers(-2 ** 31, 2 ** 31, size=(E, N, K // 8), dtype=np.int64).astype(np.int32)
    ws = F.f32_to_bf16_bits((rng.standard_normal((E, N, K // 32)) * 0.01).astype(np.float32))
    ids = np.array([[0, 3], [3, 1], [2, 0]], np.int32)
    out = G.moe_w13_w4a16(x, wq, ws, ids)
    xf = F.bf16_bits_to_f32(x).astype(np.float64)
    for t in range(T):
        for j in range(topk):
            e = ids[t, j]
            q = F.int4_unpack(wq[e]).astype(np.float64)                 # [N, K]
            s = np.repeat(F.bf16_bits_to_f32(ws[e]).astype(np.float64), 32, axis=1)
            w = F.bf16_round((q * s).astype(np.float32)).astype(np.float64)
            gu = xf[t] @ w.T
            g, u = gu[:N // 2], gu[N // 2:]
            ref = g / (1 + np.exp(-g)) * u
            assert np.allclose(out[t * topk + j], ref, rtol=1e-4, atol=1e-6)


def test_moe_w2_brute_force_per_pair():
    """Each output row is the block-scaled product of the pair's own h row with
    its expert's W, checked by the float64 triple loop; a wrong-expert and a
    token-indexed (p // topk) mutant are both rejected."""
    rng = np.random.default_rng(21)
    T, E, N, K, topk = 3, 4, 130, 256, 2
    P = T * topk
    h = _rand_fp8((P, K), rng)
    sh = rng.uniform(0.5, 1.0, size=(P, K // 128)).astype(np.float32)
    w = _rand_fp8((E, N, K), rng)
    sw = rng.uniform(0.5, 1.0, size=(E, 2, K // 128)).astype(np.float32)
    ids = np.stack([rng.permutation(E)[:topk] for _ in range(T)]).astype(np.int32)
    out = G.moe_w2_fp8(h, sh, w, sw, ids)
    assert out.shape == (P, N)
    for p in range(P):
        e = ids.reshape(-1)[p]
        ref = _brute_fp8(h[p:p + 1], sh[p:p + 1], w[e], sw[e])[0]
        assert np.allclose(out[p], ref, rtol=1e-5, atol=1e-4 * np.abs(ref).max())
    wrong = ids[:, ::-1].copy()
    assert not np.allclose(G.moe_w2_fp8(h, sh, w, sw, wrong), out)
    tok_rows = np.repeat(np.arange(T), topk)                      # mutant: h indexed by token
    mut = G.moe_w2_fp8(h[tok_rows * topk], sh[tok_rows * topk], w, sw, ids)
    assert not np.allclose(mut, out)


def test_moe_w2_matches_dense_gemm_per_expert_and_subset():
    rng = np.random.default_rng(22)
    T, E, N, K, topk = 6, 3, 256, 384, 2
    P = T * topk
    h = _rand_fp8((P, K), rng)
    sh = rng.uniform(0.1, 2.0, size=(P, K // 128)).astype(np.float32)
    w = _rand_fp8((E, N, K), rng)
    sw = rng.uniform(0.1, 2.0, size=(E, N // 128, K // 128)).astype(np.float32)
    ids = rng.integers(0, E, size=(T, topk)).astype(np.int32)
    out = G.moe_w2_fp8(h, sh, w, sw, ids)
    flat = ids.reshape(-1)
    for e in range(E):
        rows = np.nonzero(flat == e)[0]
        if rows.size:
            ref = G.fp8_blockscale_gemm(h[rows], sh[rows], w[e], sw[e])
            assert np.allclose(out[rows], ref, rtol=1e-6, atol=1e-6 * np.abs(ref).max())
    sub = G.moe_w2_fp8(h, sh, w, sw, ids, pairs=np.array([5, 0, 11]))
    # BLAS may sum a different row count in another order: equal to fp32 rounding
    assert np.allclose(sub, out[[5, 0, 11]], rtol=1e-6, atol=1e-6 * np.abs(out).max())


def test_moe_combine_one_hot_selects_rows_exactly():
    rng = np.random.default_rng(23)
    T, topk, N = 5, 4, 64
    o = F.f32_to_bf16_bits(rng.standard_normal((T * topk, N)).astype(np.float32))
    sel = rng.integers(0, topk, size=T)
    wts = np.zeros((T, topk), np.float32)
    wts[np.arange(T), sel] = 1.0
    y = G.moe_combine(o, wts)
    assert np.array_equal(y, F.bf16_bits_to_f32(o)[np.arange(T) * topk + sel])


def test_moe_combine_power_of_two_mean_exact_and_order_mutant():
    """Values in [1, 2) with 8-bit significands and weights 1/8: every partial
    sum is exact in fp32, so y is the exact mean; summing a shifted row (a
    wrong pair index) is rejected."""
    rng = np.random.default_rng(24)
    T, topk, N = 4, 8, 32
    vals = (1.0 + rng.integers(0, 128, size=(T * topk, N)) / 128.0).astype(np.float32)
    o = F.f32_to_bf16_bits(vals)
    assert np.array_equal(F.bf16_bits_to_f32(o), vals)
    wts = np.full((T, topk), 0.125, np.float32)
    y = G.moe_combine(o, wts)
    exact = vals.astype(np.float64).reshape(T, topk, N).mean(axis=1)
    assert np.array_equal(y.astype(np.float64), exact)
    shifted = np.roll(o, 1, axis=0)
    assert not np.array_equal(G.moe_combine(shifted, wts), y)
