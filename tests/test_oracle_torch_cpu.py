"""The PyTorch-CPU fp32 path (oracle.torch_cpu, the timed CPU baseline) agrees
with the pinned numpy oracle (oracle.gemm) on small shapes, to fp32 summation
tolerance; a dropped scale block is caught."""
import numpy as np
import pytest
import torch

from oracle import formats as F
from oracle import gemm as G
from oracle import quant as Q
from oracle import torch_cpu as TC


def _close(t, ref, tol=2e-5):
    got = t.numpy().astype(np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    scale = max(np.abs(ref).max(), 1e-30)
    return np.abs(got - ref).max() / scale < tol


def _fp8(rng, m, k):
    return Q.quant_act_1x128(rng.standard_normal((m, k)).astype(np.float32))


def _fp8w(rng, n, k):
    return Q.quant_weight_128x128(rng.standard_normal((n, k)).astype(np.float32))


def test_dense_fp8_and_linear():
    rng = np.random.default_rng(0)
    a, sa = _fp8(rng, 9, 384)
    b, sb = _fp8w(rng, 256, 384)
    ref = G.fp8_blockscale_gemm(a, sa, b, sb)
    assert _close(TC.fp8_blockscale_gemm(a, sa, b, sb), ref)
    sb2 = sb.copy()
    sb2[1, 2] = 0.0
    assert not _close(TC.fp8_blockscale_gemm(a, sa, b, sb2), ref)   # a dropped block is visible
    x = F.f32_to_bf16_bits(rng.standard_normal((5, 256)).astype(np.float32))
    w = F.f32_to_bf16_bits((0.02 * rng.standard_normal((64, 256))).astype(np.float32))
    r = F.f32_to_bf16_bits(rng.standard_normal((5, 64)).astype(np.float32))
    assert _close(TC.linear_bf16(x, w, r), G.linear_bf16(x, w, r))


def test_moe_paths():
    rng = np.random.default_rng(1)
    T, E, N, K, topk = 6, 4, 256, 256, 2
    ids = np.stack([rng.permutation(E)[:topk] for _ in range(T)]).astype(np.int32)
    pairs = np.array([0, 3, 4, 7, 11, 2], dtype=np.int64)
    x, sx = _fp8(rng, T, K)
    w = np.empty((E, N, K), dtype=np.uint8)
    sw = np.empty((E, N // 128, K // 128), dtype=np.float32)
    for e in range(E):
        w[e], sw[e] = _fp8w(rng, N, K)
    assert _close(TC.moe_w13_fp8(x, sx, w, sw, ids, pairs), G.moe_w13_fp8(x, sx, w, sw, ids, pairs=pairs))
    h, sh = _fp8(rng, T * topk, K)
    assert _close(TC.moe_w2_fp8(h, sh, w, sw, ids, pairs), G.moe_w2_fp8(h, sh, w, sw, ids, pairs=pairs))
    xb = F.f32_to_bf16_bits(rng.standard_normal((T, K)).astype(np.float32))
    wq = rng.integers(-2 ** 31, 2 ** 31, size=(E, N, K // 8), dtype=np.int64).astype(np.int32)
    ws = F.f32_to_bf16_bits((0.01 * rng.standard_normal((E, N, K // 32))).astype(np.float32))
    assert _close(TC.moe_w13_w4a16(xb, wq, ws, ids, pairs), G.moe_w13_w4a16(xb, wq, ws, ids, pairs=pairs))
    o = F.f32_to_bf16_bits(rng.standard_normal((T * topk, 64)).astype(np.float32))
    wts = rng.random((T, topk)).astype(np.float32)
    assert _close(TC.moe_combine(o, wts), G.moe_combine(o, wts))


def test_int4_dequant_matches_format_oracle():
    rng = np.random.default_rng(2)
    wq = rng.integers(-2 ** 31, 2 ** 31, size=(32, 16), dtype=np.int64).astype(np.int32)
    ws = F.f32_to_bf16_bits((0.01 * rng.standard_normal((32, 4))).astype(np.float32))
    assert np.array_equal(TC.int4_dequant(wq, ws).numpy(), F.int4_dequant(wq, ws))


@pytest.mark.parametrize("m", [1, 7])
def test_quant_matches_oracle_quantizer(m):
    rng = np.random.default_rng(3)
    x = (rng.standard_normal((m, 256)) * 3).astype(np.float32)
    q, s = TC.quant_act_1x128(x)
    qo, so = Q.quant_act_1x128(x)
    assert np.array_equal(q.view(torch.uint8).numpy(), qo) and np.array_equal(s.numpy(), so)
