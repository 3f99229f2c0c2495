"""UE8M0 (power-of-two) block scales for the dense FP8 GEMM (test infrastructure).

Restates the scale handling of the reference's block-scale FP8 GEMM,
``examples/fp8-gemm/v009_large_m_block_scale_mma_080.cu``:

* ``float_to_ue8m0`` (:375-384): a positive fp32 scale becomes the exponent
  byte of the power of two nearest to it in log2 (``exp2f(roundf(log2f(v)))``);
  ``v <= 0`` gives byte 0.  Restated here exactly, without a logarithm: with
  ``v = m * 2^e`` (``m`` in [0.5, 1)), the nearest power is ``2^(e-1)`` when
  ``m < 2^-0.5`` and ``2^e`` otherwise (no float equals ``2^(k+1/2)``, so there
  is no tie); the byte is that exponent + 127, clamped to [0, 255] (the
  reference's ``bits >> 23`` gives 0 for subnormal powers and 255 for inf).
  Parity unpinned in one band: ``log2f`` may round a value within ~1 ulp of
  ``2^(k+1/2)`` to the other side, so the reference's host helper can disagree
  with this exact rule there (never on the scales its own tests draw).
* ``ue8m0_to_float`` (:477-484): byte e -> 2^(e-127), byte 0 -> 0.0.
* ``prepare_sf`` (:386-403): scales [dim, nk] -> uint32 words [ceil(nk/4), dim]
  column-major, byte j of word [sk, d] = scale of (d, K-block 4 sk + j),
  missing K-blocks 0.
* ``expand_sb`` (:405-412): weight scales [ceil(N/128), nk] -> one row per
  weight row, row n taking block n // 128.
* ``ref_bs`` (:486-505): the block-scaled product with both scales rounded
  through UE8M0, ``C = sum_kb (sum_k a*b) * (sa_ue * sb_ue)`` — here
  ``oracle.gemm.fp8_blockscale_gemm`` on the decoded scales (the product of two
  powers of two is exact, so the rounding commutes with the scale product).

Pinned by tests/test_oracle_ue8m0.py: every power of two maps to its own byte,
a brute-force search over all 255 exponents for the log2-nearest one on random
and boundary values, the reference's own scale range ([0.5, 0.995] -> 126/127
split at 2^-0.5), packing round trips with ragged nk and a hand-written word
example, the block expansion by its definition, and ref_bs against a float64
triple loop with a planted wrong-exponent mutant rejected.
"""
from __future__ import annotations

import numpy as np

from .gemm import fp8_blockscale_gemm

_SQRT_HALF = 2.0 ** -0.5


def float_to_ue8m0(v: np.ndarray) -> np.ndarray:
    """fp32 scales -> UE8M0 bytes (uint8), log2-nearest power of two."""
    x = np.asarray(v, dtype=np.float32).astype(np.float64)
    pos = x > 0
    nan_or_inf = ~np.isfinite(x)
    m, e = np.frexp(np.where(pos & ~nan_or_inf, x, 1.0))
    k = e - 1 + (m >= _SQRT_HALF)
    out = np.where(pos, np.clip(k + 127, 0, 255), 0)
    out = np.where(nan_or_inf & ~(x < 0), 255, out)      # +inf and NaN: the exponent field of inf / NaN
    return out.astype(np.uint8)


def ue8m0_to_float(e: np.ndarray) -> np.ndarray:
    """UE8M0 bytes -> fp32 (2^(e-127); 0 for byte 0)."""
    b = np.atleast_1d(np.asarray(e, dtype=np.uint32))
    v = (b << np.uint32(23)).view(np.float32)
    out = np.where(b == 0, np.float32(0.0), v).astype(np.float32)
    return out.reshape(np.shape(e))


def prepare_sf(ue: np.ndarray) -> np.ndarray:
    """UE8M0 bytes [dim, nk] -> uint32 words [ceil(nk/4), dim] (column-major packing)."""
    ue = np.asarray(ue, dtype=np.uint8)
    dim, nk = ue.shape
    nsk = (nk + 3) // 4
    padded = np.zeros((dim, nsk * 4), dtype=np.uint32)
    padded[:, :nk] = ue
    p = padded.reshape(dim, nsk, 4)
    words = p[..., 0] | (p[..., 1] << 8) | (p[..., 2] << 16) | (p[..., 3] << 24)
    return np.ascontiguousarray(words.T.astype(np.uint32))


def unpack_sf(words: np.ndarray, nk: int) -> np.ndarray:
    """uint32 words [ceil(nk/4), dim] -> UE8M0 bytes [dim, nk]."""
    w = np.asarray(words, dtype=np.uint32)
    nsk, dim = w.shape
    out = np.zeros((dim, nsk * 4), dtype=np.uint8)
    for j in range(4):
        out[:, j::4] = ((w.T >> (8 * j)) & 0xFF).astype(np.uint8)
    return out[:, :nk]


def expand_sb(sb: np.ndarray, N: int) -> np.ndarray:
    """Weight block scales [ceil(N/128), nk] -> per-row [N, nk] (row n <- block n // 128)."""
    sb = np.asarray(sb)
    return sb[np.arange(N) // 128]


def ref_bs(a_codes, sa, b_codes, sb) -> np.ndarray:
    """fp32 C[M, N] with both fp32 scale sets rounded through UE8M0 (sb per 128-row block)."""
    sa_ue = ue8m0_to_float(float_to_ue8m0(sa))
    sb_ue = ue8m0_to_float(float_to_ue8m0(sb))
    return fp8_blockscale_gemm(a_codes, sa_ue, b_codes, sb_ue)


def packed_inputs(sa: np.ndarray, sb: np.ndarray, N: int):
    """The reference's host preparation: (sfa words [ceil(nk/4), M], sfb words [ceil(nk/4), N])."""
    return prepare_sf(float_to_ue8m0(sa)), prepare_sf(expand_sb(float_to_ue8m0(sb), N))
