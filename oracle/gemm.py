"""fp32 restatements of the four GEMM cases (test infrastructure).

All products are formed from exactly decoded operands and accumulated in
float32, in the reference's summation form:

* bf16 decode linear: ``tests/compare_decode_linear.py:263-274``
  (``torch.matmul(x.float(), w.float().t()) (+ r)``) and the harness check at
  ``examples/qwen3-8b-decode-linear-bs16/v019_swapab_cg2_l2hints.cu:641-668``.
* FP8 block-scaled GEMM: host ``ref`` at
  ``examples/fp8-gemm/v002_dense_tp8_validated_065.cu:277-288`` — per 128-K
  block, ``p = sum a*b`` then ``s += p * (sa[m,kb] * sb[n/128,kb])``.
* FP8 MoE w13: ``cpu_ref_bs`` at
  ``examples/fp8-group-gemm/v007_dsv3_decode_verified_105.cu:442-467`` with the
  expert taken per ROW (the reference takes it per 128-row tile, line 449-450,
  which is only right for 128-padded segments) and the SiLU(gate)*up epilogue of
  ``correctness/compare_marlin_vs_ref.py:93-97``.
* INT4 W4A16 MoE w13: ``fp32_oracle_w13_silu`` at
  ``correctness/compare_marlin_vs_ref.py:44-100``.
* FP8 MoE w2 (down, K = 2048 -> N = 7168 at
  ``tasks/fp8-group-gemm-dsv3-decode.yaml:11-13``): the block-scaled product of
  ``cpu_ref_bs`` per routed pair, the pair's own activation row.
* Top-k combine: sum_j w[t,j] * o[t*topk+j] in float32 (the library's own
  contract; the reference's routing weights are left unused by w13,
  ``baselines/kimi-moe-w13-int4/baseline_marlin.py:158``).

Pinned by (tests/test_oracle_gemm.py): brute-force triple loops on tiny shapes,
the all-scales-one reduction to a plain fp8 matmul, power-of-two scales (exact),
single-K-block closed form, small-integer operands with exact sums, a planted
transposition / dropped-block / wrong-expert mutant that each check rejects, and
the SiLU closed form at known points; w2 against a per-pair brute-force loop
and against fp8_blockscale_gemm on each expert's rows; the combine by one-hot
weights (exact row selection) and power-of-two uniform weights (exact mean).
"""
from __future__ import annotations

import numpy as np

from .formats import bf16_bits_to_f32, e4m3_to_f32, int4_dequant


def _f32(a):
    return np.asarray(a, dtype=np.float32)


def linear_bf16(x_bits: np.ndarray, w_bits: np.ndarray, residual_bits: np.ndarray | None = None) -> np.ndarray:
    """Y = X . W^T (+ residual) in float32.

    x_bits uint16 [M, K], w_bits uint16 [N, K], residual uint16 [M, N] or None
    (all bf16 bit patterns). Returns float32 [M, N] (not rounded).
    """
    x = bf16_bits_to_f32(x_bits)
    w = bf16_bits_to_f32(w_bits)
    y = (x @ w.T).astype(np.float32)
    if residual_bits is not None:
        y = (y + bf16_bits_to_f32(residual_bits)).astype(np.float32)
    return y


def fp8_blockscale_gemm(a_codes, sa, b_codes, sb, block: int = 128) -> np.ndarray:
    """C[m,n] = sum_kb (sum_{k in kb} A[m,k] B[n,k]) * sa[m,kb] * sb[n//128,kb].

    a_codes uint8 [M,K], sa float32 [M,K/128], b_codes uint8 [N,K],
    sb float32 [ceil(N/128), K/128]. Returns float32 [M, N].
    Follows ``v002_dense_tp8_validated_065.cu:277-288`` block by block.
    """
    a = e4m3_to_f32(a_codes)
    b = e4m3_to_f32(b_codes)
    sa = _f32(sa)
    sb = _f32(sb)
    m, k = a.shape
    n = b.shape[0]
    nk = (k + block - 1) // block
    sb_rows = sb[np.arange(n) // block]                       # [N, nk]
    c = np.zeros((m, n), dtype=np.float32)
    for kb in range(nk):
        ks = slice(kb * block, min((kb + 1) * block, k))
        p = (a[:, ks] @ b[:, ks].T).astype(np.float32)
        sc = (sa[:, kb][:, None] * sb_rows[:, kb][None, :]).astype(np.float32)
        c = (c + p * sc).astype(np.float32)
    return c


def silu_mul(gate: np.ndarray, up: np.ndarray) -> np.ndarray:
    """silu(g) * u = g / (1 + exp(-g)) * u in float32 (``compare_marlin_vs_ref.py:93-97``)."""
    g = _f32(gate)
    with np.errstate(over="ignore"):
        s = (g / (np.float32(1.0) + np.exp(-g))).astype(np.float32)
    return (s * _f32(up)).astype(np.float32)


def _pairs_by_expert(topk_ids: np.ndarray, pairs: np.ndarray | None):
    ids = np.asarray(topk_ids).reshape(-1)
    if pairs is None:
        pairs = np.arange(ids.size)
    pairs = np.asarray(pairs, dtype=np.int64)
    groups: dict[int, list[int]] = {}
    for p in pairs:
        groups.setdefault(int(ids[p]), []).append(int(p))
    return pairs, groups


def moe_w13_fp8(x_codes, sx, w_codes, sw, topk_ids, pairs=None) -> np.ndarray:
    """FP8 block-scaled MoE gate-up projection with SiLU(gate)*up.

    x_codes uint8 [T,K], sx float32 [T,K/128]; w_codes uint8 [E,N,K] (gate rows
    [0,N/2), up rows [N/2,N)); sw float32 [E,N/128,K/128]; topk_ids int [T,topk].
    Pair p = t*topk + j routes token t to expert topk_ids[t,j] (row order of
    ``compare_marlin_vs_ref.py:97``).  Returns float32 [len(pairs), N/2] for the
    requested pairs (all pairs by default), in the order given.
    """
    topk = np.asarray(topk_ids).shape[1]
    n = w_codes.shape[1]
    half = n // 2
    pairs, groups = _pairs_by_expert(topk_ids, pairs)
    out = np.zeros((pairs.size, half), dtype=np.float32)
    pos = {int(p): i for i, p in enumerate(pairs)}
    for e, plist in groups.items():
        toks = np.array(plist) // topk
        gu = fp8_blockscale_gemm(x_codes[toks], sx[toks], w_codes[e], sw[e])
        res = silu_mul(gu[:, :half], gu[:, half:])
        for r, p in enumerate(plist):
            out[pos[p]] = res[r]
    return out


def moe_w13_w4a16(x_bits, wq, ws_bits, topk_ids, pairs=None, group: int = 32) -> np.ndarray:
    """INT4 W4A16 MoE gate-up projection with SiLU(gate)*up.

    x_bits uint16 [T,K] (bf16); wq int32 [E,N,K/8] (8 nibbles per word along K,
    low nibble first, offset-8); ws_bits uint16 [E,N,K/32] (bf16 scales);
    topk_ids int [T,topk].  Per ``compare_marlin_vs_ref.py:63-100``: dequant to
    bf16, fp32 accumulate, silu(gate)*up in fp32.  Returns float32
    [len(pairs), N/2].
    """
    topk = np.asarray(topk_ids).shape[1]
    n = wq.shape[1]
    half = n // 2
    x = bf16_bits_to_f32(x_bits)
    pairs, groups = _pairs_by_expert(topk_ids, pairs)
    out = np.zeros((pairs.size, half), dtype=np.float32)
    pos = {int(p): i for i, p in enumerate(pairs)}
    for e, plist in groups.items():
        w = int4_dequant(wq[e], ws_bits[e], group)            # [N, K] bf16-exact
        toks = np.array(plist) // topk
        gu = (x[toks] @ w.T).astype(np.float32)
        res = silu_mul(gu[:, :half], gu[:, half:])
        for r, p in enumerate(plist):
            out[pos[p]] = res[r]
    return out


def moe_w2_fp8(h_codes, sh, w_codes, sw, topk_ids, pairs=None) -> np.ndarray:
    """FP8 block-scaled MoE down projection.

    h_codes uint8 [P,K], sh float32 [P,K/128] (pair order: row p is pair p);
    w_codes uint8 [E,N,K]; sw float32 [E,N/128,K/128]; topk_ids int [T,topk]
    with T*topk = P.  out[p] = fp8_blockscale_gemm(h[p], W[expert(p)]).
    Returns float32 [len(pairs), N] for the requested pairs, in the order given.
    """
    n = w_codes.shape[1]
    pairs, groups = _pairs_by_expert(topk_ids, pairs)
    out = np.zeros((pairs.size, n), dtype=np.float32)
    pos = {int(p): i for i, p in enumerate(pairs)}
    for e, plist in groups.items():
        rows = np.array(plist)
        res = fp8_blockscale_gemm(h_codes[rows], sh[rows], w_codes[e], sw[e])
        for r, p in enumerate(plist):
            out[pos[p]] = res[r]
    return out


def moe_combine(o_bits: np.ndarray, weights: np.ndarray) -> np.ndarray:
    """y[t] = sum_j weights[t,j] * o[t*topk + j] in float32, j in order.

    o_bits uint16 [T*topk, N] (bf16, pair order); weights float32 [T, topk].
    Returns float32 [T, N] (not rounded).
    """
    w = _f32(weights)
    t, topk = w.shape
    o = bf16_bits_to_f32(o_bits).reshape(t, topk, -1)
    y = np.zeros((t, o.shape[2]), dtype=np.float32)
    for j in range(topk):
        y = (y + w[:, j][:, None] * o[:, j, :]).astype(np.float32)
    return y
