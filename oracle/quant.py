"""absmax/448 FP8 quantizers (test infrastructure).

The reference calls DeepGEMM's ``per_token_cast_to_fp8`` (1x128 activation
blocks) and ``per_block_cast_to_fp8`` (128x128 weight blocks) with fp32 scales
(``baselines/fp8-gemm/baseline_prefill.py:41-42``,
``baselines/fp8-group-gemm/baseline_dsv3_decode.py:45-53``).  DeepGEMM is not
vendored (empty submodule), so its exact epsilon clamp cannot be imported; this
module defines the library's own quantizer, stated once here and mirrored by the
torch input generator:

    amax = max(|x| over the block, 1e-4);  q = e4m3_RNE(x * (448 / amax));
    scale = amax / 448                       (all in float32)

Parity with DeepGEMM's helper itself is UNPINNED (no import possible).
Pinned by: the invariants ``max|q| == 448`` on every block with amax > 1e-4,
``|q*scale - x| <= half an e4m3 ulp * scale``, ``scale > 0``; and bit-exact
agreement with the torch generator (tests/test_oracle_quant.py).
"""
from __future__ import annotations

import numpy as np

from .formats import f32_to_e4m3

AMAX_FLOOR = np.float32(1e-4)
FP8_MAX = np.float32(448.0)


def quant_act_1x128(x: np.ndarray):
    """x float32 [M, K] -> (q uint8 [M, K], scale float32 [M, K/128])."""
    x = np.asarray(x, dtype=np.float32)
    m, k = x.shape
    assert k % 128 == 0, "K must be a multiple of 128"
    xv = x.reshape(m, k // 128, 128)
    amax = np.maximum(np.abs(xv).max(axis=2), AMAX_FLOOR).astype(np.float32)
    mult = (FP8_MAX / amax).astype(np.float32)
    q = f32_to_e4m3((xv * mult[:, :, None]).astype(np.float32)).reshape(m, k)
    return q, (amax / FP8_MAX).astype(np.float32)


def quant_weight_128x128(w: np.ndarray):
    """w float32 [N, K] -> (q uint8 [N, K], scale float32 [N/128, K/128])."""
    w = np.asarray(w, dtype=np.float32)
    n, k = w.shape
    assert n % 128 == 0 and k % 128 == 0, "N and K must be multiples of 128"
    wv = w.reshape(n // 128, 128, k // 128, 128)
    amax = np.maximum(np.abs(wv).max(axis=(1, 3)), AMAX_FLOOR).astype(np.float32)
    mult = (FP8_MAX / amax).astype(np.float32)
    q = f32_to_e4m3((wv * mult[:, None, :, None]).astype(np.float32)).reshape(n, k)
    return q, (amax / FP8_MAX).astype(np.float32)
