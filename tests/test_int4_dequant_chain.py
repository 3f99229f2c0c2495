"""The INT4 dequant chain of the GPU kernels (dequant_int4x8, skinny_kernel.hpp),
emulated exactly on the CPU over every finite bf16 group scale and every
nibble, against the oracle's bf16_RNE(float(q - 8) * s).

The kernel places nibble q in an fp16 mantissa under the exponent of 1024 and
forms the weight with one mixed fma:
  nibbles 0, 2, 4, 6:  fma(1024 + q,      s,      c1),  c1 = fp32(-1032 * s)
  nibbles 1, 3, 5, 7:  fma(1024 + 16 q,   s / 16, c2),  c2 = fp32(-72 * s)
then packs the fp32 result to bf16 with round-to-nearest-even.  A fused
multiply-add rounds its exact result once, so it is emulated by the exact sum
in float64 (the product has at most 19 significant bits, c1 / c2 at most 16)
rounded once to float32.  The weights agree with the oracle's for every scale
|s| < 2^128 / 1032, where -1032 * s is a finite float; above it c1 overflows to
-inf and the chain breaks down, so that bound is the dequant's stated
precondition (include/ferret_hip.h).  The one other difference is the sign of
a zero weight (q = 8 with s < 0: the chain gives +0, the oracle -0), which adds
nothing to a dot product.
"""
import numpy as np

from oracle import formats as F


def _chain(q: np.ndarray, s: np.ndarray, odd: bool) -> np.ndarray:
    """The kernel's weight for nibble value q under scale s (float32 arrays)."""
    with np.errstate(over="ignore", invalid="ignore"):
        if odd:
            a = (1024.0 + 16.0 * q.astype(np.float64))
            b = (s * np.float32(0.0625)).astype(np.float32)
            c = (np.float32(-72.0) * s).astype(np.float32)
        else:
            a = (1024.0 + q.astype(np.float64))
            b = s
            c = (np.float32(-1032.0) * s).astype(np.float32)
        exact = a * b.astype(np.float64) + c.astype(np.float64)
        return F.bf16_round(exact.astype(np.float32))


def _all_finite_scales():
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    s = F.bf16_bits_to_f32(bits)
    keep = np.isfinite(s)
    return bits[keep], s[keep]


def test_chain_equals_the_oracle_for_every_scale_below_the_bound():
    bits, s = _all_finite_scales()
    q = np.arange(16, dtype=np.int64)
    # the oracle itself: one word holding nibble q in all 8 positions, one 8-wide group
    words = (q * 0x11111111).astype(np.uint32).view(np.int32)              # [16]
    with np.errstate(over="ignore"):  # the largest scales overflow the oracle's fp32 product too
        ref = F.int4_dequant(np.broadcast_to(words[None, :, None], (len(s), 16, 1)),
                             np.broadcast_to(bits[:, None, None], (len(s), 16, 1)), group=8)  # [S, 16, 8]
    with np.errstate(over="ignore"):
        ok = np.isfinite(np.float32(-1032.0) * s)                          # the precondition
    assert ok.sum() > 60000 and (~ok).sum() > 0
    for pos in range(8):
        got = _chain(np.broadcast_to(q[None, :], (len(s), 16)), np.broadcast_to(s[:, None], (len(s), 16)),
                     odd=bool(pos & 1))
        r = ref[:, :, pos]
        same = (got == r) | (np.isnan(got) & np.isnan(r))                  # value equality: +0 == -0
        assert same[ok].all(), f"nibble position {pos}: {np.argwhere(~same & ok[:, None])[:5]}"
        # above the bound the chain is wrong for some nibble: the bound is needed
        assert not same[~ok].all()


def test_chain_bound_is_the_overflow_of_1032_s():
    bits, s = _all_finite_scales()
    with np.errstate(over="ignore"):
        ok = np.isfinite(np.float32(-1032.0) * s)
    a = np.abs(s)
    # every scale below 2^128 / 1032 passes, every one at or above fails
    assert a[ok].max() < 2.0 ** 128 / 1032 <= a[~ok].min()
    assert 2.0 ** 117 < a[~ok].min() < 2.0 ** 118
    # the oracle's own fp32 product (q - 8) * s stays finite over the whole allowed range
    assert np.isfinite(np.float32(7.0) * a[ok].max())


def test_chain_spot_values():
    # s = 0.0078125 (bf16 0x3C00), q = 15: 7 * 2^-7 exactly; q = 3: -5 * 2^-7
    s = np.float32(0.0078125)
    for odd in (False, True):
        assert _chain(np.array([15]), np.array([s]), odd)[0] == np.float32(7 * 0.0078125)
        assert _chain(np.array([3]), np.array([s]), odd)[0] == np.float32(-5 * 0.0078125)
    # a rounding case: s with all 8 mantissa bits, q - 8 = 7 -> 11 significant bits -> RNE to 8
    s = F.bf16_bits_to_f32(np.array([0x3FFF], dtype=np.uint16))[0]            # 1.9921875
    want = F.bf16_round(np.array([np.float32(7.0) * s], dtype=np.float32))[0]
    assert want != np.float32(7.0) * s                                      # the product is rounded
    for odd in (False, True):
        assert _chain(np.array([15]), np.array([s]), odd)[0] == want
