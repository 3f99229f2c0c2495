"""Number formats on the path: OCP e4m3fn, bf16, packed INT4 (test infrastructure).

Reference usage this restates:

* e4m3 decode: ``examples/fp8-gemm/v002_dense_tp8_validated_065.cu:283-284``
  (``__nv_cvt_fp8_to_halfraw(..., __NV_E4M3)``), the NaN-code avoidance at
  ``v002...cu:325-328``.
* bf16 RNE: ``examples/qwen3-8b-decode-linear-bs16/v019_swapab_cg2_l2hints.cu:361``
  and ``correctness/compare_marlin_vs_ref.py:84,100`` (``.to(torch.bfloat16)``).
* INT4 unpack: ``correctness/compare_marlin_vs_ref.py:63-86`` and the layout
  contract ``tasks/kimi-moe-w13-int4-grouped-gemm.yaml:68-83,158``.

Pinned by (tests/test_oracle_formats.py): the 256-code e4m3 table against
``torch.float8_e4m3fn`` and against the format definition at hand-picked codes;
encode against torch's cast on every code midpoint; bf16 against
``torch.Tensor.to(torch.bfloat16)`` on random and edge bit patterns; INT4 on the
known-answer words 0x76543210 / 0xFEDCBA98 and exhaustively over 16 values x 8
nibble positions; the INT4 tile regrouping against an element-by-element loop
over the contract's description and by its inverse.
"""
from __future__ import annotations

import numpy as np

E4M3_MAX = 448.0


def _build_e4m3_table() -> np.ndarray:
    """Value of every e4m3fn code, from the OCP FP8 definition.

    1 sign bit, 4 exponent bits (bias 7), 3 mantissa bits; exponent 0 is
    subnormal (m/8 * 2^-6); codes 0x7F and 0xFF are NaN; no infinities.
    """
    t = np.empty(256, dtype=np.float32)
    for code in range(256):
        s = -1.0 if code & 0x80 else 1.0
        e = (code >> 3) & 0xF
        m = code & 0x7
        if e == 0xF and m == 0x7:
            t[code] = np.nan
        elif e == 0:
            t[code] = s * (m / 8.0) * 2.0 ** -6
        else:
            t[code] = s * (1.0 + m / 8.0) * 2.0 ** (e - 7)
    return t


E4M3_TABLE = _build_e4m3_table()


def e4m3_to_f32(codes: np.ndarray) -> np.ndarray:
    """Decode e4m3fn bytes to float32 (exact)."""
    return E4M3_TABLE[np.asarray(codes, dtype=np.uint8)]


# Finite non-negative e4m3 values in increasing order, with their codes.
_POS_CODES = np.arange(0, 0x7F, dtype=np.uint8)          # 0x00..0x7E
_POS_VALS = E4M3_TABLE[_POS_CODES].astype(np.float64)


def f32_to_e4m3(x: np.ndarray) -> np.ndarray:
    """Encode float32 -> e4m3fn with round-to-nearest-even.

    Magnitudes above 464 (half-way between 448 and the first unrepresentable
    step; 464 itself ties to even, i.e. 448) and NaN become the NaN code,
    matching ``Tensor.to(torch.float8_e4m3fn)`` (non-saturating).
    """
    x = np.asarray(x, dtype=np.float32)
    a = np.abs(x).astype(np.float64)
    idx = np.searchsorted(_POS_VALS, a, side="left")      # first value >= a
    idx = np.clip(idx, 0, len(_POS_VALS) - 1)
    hi = idx
    lo = np.maximum(idx - 1, 0)
    vhi = _POS_VALS[hi]
    vlo = _POS_VALS[lo]
    dlo = a - vlo
    dhi = vhi - a
    pick_hi = (dhi < dlo) | ((dhi == dlo) & ((_POS_CODES[hi] & 1) == 0))
    pick_hi |= a <= vlo                                    # exact hit / below 0
    code = np.where(pick_hi, _POS_CODES[hi], _POS_CODES[lo]).astype(np.uint8)
    code = np.where(a == vhi, _POS_CODES[hi], code).astype(np.uint8)
    code = code | np.where(np.signbit(x), np.uint8(0x80), np.uint8(0))
    nan_mask = np.isnan(x) | (a > 464.0)
    code = np.where(nan_mask, np.uint8(0x7F) | (code & 0x80), code)
    return code.astype(np.uint8)


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """float32 -> bf16 bit pattern (uint16), round-to-nearest-even; NaN stays NaN."""
    x = np.ascontiguousarray(np.asarray(x, dtype=np.float32))
    b = x.view(np.uint32).astype(np.uint64)
    rounded = (b + 0x7FFF + ((b >> 16) & 1)) >> 16
    out = rounded.astype(np.uint16)
    nan = np.isnan(x)
    if nan.any():
        out = np.where(nan, ((b >> 16).astype(np.uint16) | np.uint16(0x0040)), out)
    return out.astype(np.uint16)


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    """bf16 bit pattern (uint16) -> float32 (exact)."""
    b = np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16
    return b.view(np.float32)


def bf16_round(x: np.ndarray) -> np.ndarray:
    """Round float32 values to the nearest bf16 value (RNE), returned as float32."""
    return bf16_bits_to_f32(f32_to_bf16_bits(x))


def int4_unpack(words: np.ndarray) -> np.ndarray:
    """Unpack int32 words along the last axis into signed nibbles.

    Nibble s (bits 4s..4s+3, low nibble first) of word k holds K index 8k+s;
    the stored value is offset-8 unsigned, so the signed value is ``nib - 8``
    (``correctness/compare_marlin_vs_ref.py:68-79``,
    ``tasks/kimi-moe-w13-int4-grouped-gemm.yaml:72-77``).
    Returns int8 with the last axis 8x longer.
    """
    w = np.asarray(words).astype(np.int64) & 0xFFFFFFFF
    shifts = np.arange(8, dtype=np.int64) * 4
    nib = (w[..., None] >> shifts) & 0xF                      # [..., K/8, 8]
    signed = (nib - 8).astype(np.int8)
    return signed.reshape(*w.shape[:-1], w.shape[-1] * 8)


def int4_dequant(words: np.ndarray, scales_bf16_bits: np.ndarray, group: int = 32) -> np.ndarray:
    """Dequantize packed INT4 rows to bf16-exact float32 values.

    ``words``: int32 [..., K/8] (K contiguous, N-major rows, the per-expert
    layout of ``kimi-moe-w13-int4-grouped-gemm.yaml:78-82``);
    ``scales_bf16_bits``: uint16 [..., K/group].
    Value = bf16_RNE(float(nib - 8) * float(scale[k // group])) as in
    ``compare_marlin_vs_ref.py:80-84``: the fp32 product is exact, then one
    rounding to bf16.
    """
    q = int4_unpack(words).astype(np.float32)                 # [..., K]
    s = bf16_bits_to_f32(scales_bf16_bits)                    # [..., K/group]
    s_full = np.repeat(s, group, axis=-1)
    return bf16_round(q * s_full)


def int4_dequant_kmajor(raw_q: np.ndarray, scales_bf16_bits: np.ndarray, group: int = 32) -> np.ndarray:
    """Same dequant for the reference oracle's ``[K/8, N]`` layout.

    ``correctness/compare_marlin_vs_ref.py:50-51``: ``raw_q`` int32 [K/8, N] and
    scales [K/group, N]; returns [N, K] float32 (so it is comparable with
    :func:`int4_dequant` on the transposed packing).
    """
    return int4_dequant(np.ascontiguousarray(raw_q.T), np.ascontiguousarray(scales_bf16_bits.T), group)


def int4_tile_weights(wq: np.ndarray) -> np.ndarray:
    """INT4 w13 words ``[E, N, K/8]`` regrouped into 16-row x 128-K tiles
    ``[E, N/16, K/128, 16, 16]`` (int32): tile ``(e, b, k)`` row ``r`` holds the
    16 words (64 bytes, K = 128k .. 128k+127) of weight row ``16b + r``.

    A pure permutation of the checkpoint words, the kind of one-time load-time
    pre-permutation ``tasks/kimi-moe-w13-int4-grouped-gemm.yaml:68-71`` allows
    (the reference runs ``gptq_marlin_moe_repack`` there,
    ``baselines/kimi-moe-w13-int4/baseline_marlin.py:62-89``).
    """
    E, N, K8 = wq.shape
    assert N % 16 == 0 and K8 % 16 == 0
    return np.ascontiguousarray(wq.reshape(E, N // 16, 16, K8 // 16, 16).transpose(0, 1, 3, 2, 4))


def int4_untile_weights(t: np.ndarray) -> np.ndarray:
    """Inverse of :func:`int4_tile_weights`."""
    E, NB, KB, R, C = t.shape
    return np.ascontiguousarray(t.transpose(0, 1, 3, 2, 4).reshape(E, NB * R, KB * C))
