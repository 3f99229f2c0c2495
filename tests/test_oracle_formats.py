"""Pin the oracle's number formats against library routines and the format definitions."""
import numpy as np
import pytest
import torch

from oracle import formats as F


def test_e4m3_table_matches_torch_all_codes():
    codes = torch.arange(256, dtype=torch.uint8)
    ref = codes.view(torch.float8_e4m3fn).float().numpy()
    ours = F.e4m3_to_f32(np.arange(256, dtype=np.uint8))
    nan_ref = np.isnan(ref)
    assert np.array_equal(nan_ref, np.isnan(ours))
    assert np.array_equal(ref[~nan_ref], ours[~nan_ref])


def test_e4m3_definition_known_codes():
    # Hand-picked codes from the OCP definition (bias 7, subnormal at e=0).
    t = F.E4M3_TABLE
    assert t[0x7E] == 448.0                  # max finite
    assert t[0x38] == 1.0                    # e=7, m=0
    assert t[0x01] == 2.0 ** -9              # smallest subnormal
    assert t[0x08] == 2.0 ** -6              # smallest normal
    assert t[0xB8] == -1.0
    assert np.isnan(t[0x7F]) and np.isnan(t[0xFF])
    assert t[0x80] == 0.0 and np.signbit(t[0x80])


def test_e4m3_encode_matches_torch_on_midpoints_and_random():
    finite = np.array([v for v in F.E4M3_TABLE if np.isfinite(v)], dtype=np.float32)
    pos = np.unique(np.abs(finite))
    mids = ((pos[1:] + pos[:-1]) / 2).astype(np.float32)
    probes = np.concatenate([
        pos, -pos, mids, -mids,
        np.nextafter(mids, np.float32(np.inf)), np.nextafter(mids, np.float32(-np.inf)),
        np.array([448.0, 449.0, 463.9, 464.0, 464.1, 500.0, 1e9, -1e9, np.nan], dtype=np.float32),
        np.random.default_rng(0).standard_normal(20000).astype(np.float32) * 100,
    ]).astype(np.float32)
    ref = torch.from_numpy(probes).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    ours = F.f32_to_e4m3(probes)
    # NaN codes may differ in sign only if both are NaN.
    ref_nan = np.isnan(F.e4m3_to_f32(ref))
    ours_nan = np.isnan(F.e4m3_to_f32(ours))
    assert np.array_equal(ref_nan, ours_nan)
    assert np.array_equal(ref[~ref_nan], ours[~ours_nan])


def test_bf16_rne_matches_torch():
    rng = np.random.default_rng(1)
    bits = rng.integers(0, 2 ** 32, size=200000, dtype=np.uint64).astype(np.uint32)
    x = bits.view(np.float32)
    x = x[np.isfinite(x)]
    edge = np.array([0.0, -0.0, 1.0, 1.00390625, 1.0039062500001, 3.3895314e38, 1e-40, -2.5], dtype=np.float32)
    x = np.concatenate([x, edge]).astype(np.float32)
    ref = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    ours = F.f32_to_bf16_bits(x)
    assert np.array_equal(ref, ours)
    assert np.array_equal(F.bf16_bits_to_f32(ours), torch.from_numpy(x).to(torch.bfloat16).float().numpy())


def test_bf16_ties_to_even():
    # 1 + 2^-8 is exactly half-way between 1 and 1 + 2^-7: rounds to even (1.0).
    assert F.bf16_round(np.array([1.0 + 2 ** -8], dtype=np.float32))[0] == 1.0
    # 1 + 3*2^-8 is half-way between 1+2^-7 and 1+2^-6: rounds to 1+2^-6.
    assert F.bf16_round(np.array([1.0 + 3 * 2 ** -8], dtype=np.float32))[0] == 1.0 + 2 ** -6


def test_int4_known_answers():
    w = np.array([[0x76543210, np.int64(0xFEDCBA98) - 2 ** 32]], dtype=np.int64).astype(np.int32)
    nib = F.int4_unpack(w)
    assert nib.tolist() == [[-8, -7, -6, -5, -4, -3, -2, -1, 0, 1, 2, 3, 4, 5, 6, 7]]


def test_int4_exhaustive_value_position():
    for v in range(16):
        for s in range(8):
            word = np.array([[(v << (4 * s))]], dtype=np.int64)
            word = np.where(word >= 2 ** 31, word - 2 ** 32, word).astype(np.int32)
            nib = F.int4_unpack(word)[0]
            expect = np.full(8, -8)
            expect[s] = v - 8
            assert nib.tolist() == expect.tolist(), (v, s)


def test_int4_dequant_group_boundary_and_rounding():
    # K = 64: two scale groups; all nibbles = 15 (+7); scales chosen so the
    # product needs bf16 rounding: 7 * bf16(1.0078125) = 7.0546875 -> bf16 7.0625? check via torch
    k = 64
    words = np.full((1, k // 8), np.int64(0xFFFFFFFF) - 2 ** 32, dtype=np.int64).astype(np.int32)
    sc = np.array([[1.0078125, 3.0]], dtype=np.float32)
    sc_bits = F.f32_to_bf16_bits(sc)
    deq = F.int4_dequant(words, sc_bits)
    ref_first = torch.tensor(7.0 * 1.0078125, dtype=torch.float32).to(torch.bfloat16).float().item()
    assert np.all(deq[0, :32] == ref_first)
    assert np.all(deq[0, 32:] == 21.0)
    assert ref_first != 7.0 * 1.0078125      # rounding really happened


def test_int4_layouts_agree():
    rng = np.random.default_rng(3)
    n, k = 8, 64
    wq = rng.integers(-2 ** 31, 2 ** 31, size=(n, k // 8), dtype=np.int64).astype(np.int32)
    sc = F.f32_to_bf16_bits(rng.standard_normal((n, k // 32)).astype(np.float32) * 0.01)
    a = F.int4_dequant(wq, sc)
    b = F.int4_dequant_kmajor(np.ascontiguousarray(wq.T), np.ascontiguousarray(sc.T))
    assert np.array_equal(a, b)


def test_int4_dequant_matches_reference_torch_formula():
    """Re-evaluate the reference oracle's torch steps (compare_marlin_vs_ref.py:68-84)
    on a [K/8, N] layout and compare with the numpy restatement."""
    rng = np.random.default_rng(4)
    H, N = 64, 16
    raw = torch.from_numpy(rng.integers(-2 ** 31, 2 ** 31, size=(H // 8, N), dtype=np.int64).astype(np.int32))
    scales = (torch.from_numpy(rng.standard_normal((H // 32, N)).astype(np.float32)) * 0.01).to(torch.bfloat16)
    u = raw.unsqueeze(0).expand(8, -1, -1)
    shifts = torch.arange(8, dtype=torch.int32) * 4
    nibbles = (u >> shifts.view(8, 1, 1)) & 0xF
    nibbles = nibbles.permute(1, 0, 2).contiguous().view(H, N)
    signed = nibbles.to(torch.float32) - 8.0
    sc = scales.to(torch.float32).repeat_interleave(32, dim=0)
    ref = (signed * sc).to(torch.bfloat16).to(torch.float32).t().contiguous().numpy()
    ours = F.int4_dequant_kmajor(raw.numpy(), scales.view(torch.int16).numpy().view(np.uint16))
    assert np.array_equal(ref, ours)


def test_int4_tile_weights_against_loops_and_inverse():
    """Tile (e, b, k), row r, word j is word 16k + j of weight row 16b + r of
    expert e -- checked word by word on a small tensor of distinct values, and
    the inverse restores the checkpoint words."""
    E, N, K = 2, 48, 384
    wq = np.arange(E * N * K // 8, dtype=np.int64).astype(np.int32).reshape(E, N, K // 8)
    t = F.int4_tile_weights(wq)
    assert t.shape == (E, N // 16, K // 128, 16, 16)
    for e in range(E):
        for b in range(N // 16):
            for k in range(K // 128):
                for r in range(16):
                    for j in range(16):
                        assert t[e, b, k, r, j] == wq[e, 16 * b + r, 16 * k + j]
    # the 1-KB tile of (e, b, k) is contiguous in memory
    flat = t.reshape(-1)
    off = ((1 * (N // 16) + 2) * (K // 128) + 1) * 256
    assert np.array_equal(flat[off:off + 256].reshape(16, 16), wq[1, 32:48, 16:32])
    assert np.array_equal(F.int4_untile_weights(t), wq)
    rnd = np.random.default_rng(3).integers(-2 ** 31, 2 ** 31, (3, 32, 256 // 8)).astype(np.int32)
    assert np.array_equal(F.int4_untile_weights(F.int4_tile_weights(rnd)), rnd)
