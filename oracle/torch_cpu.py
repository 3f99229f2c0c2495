"""PyTorch-CPU fp32 dequantize-then-matmul path (test infrastructure).

The CPU baseline that bench.py times beside the GPU kernels: the same math as
``oracle.gemm``, written the way the reference's own torch baselines and
oracle are (dequantize every operand to fp32, one ``torch.matmul`` per GEMM or
per expert, SiLU(gate)*up in fp32), so it runs on torch's multi-threaded CPU
GEMM.  Only ``bench.py``'s ``cpu_baseline`` leg and ``tests/`` use it; the
correctness verdict of a bench run comes from ``oracle.gemm``.

Follows:
* dense FP8: dequantize A by its 1x128 scales and B by its 128x128 scales,
  then fp32 matmul (the reference's baselines feed DeepGEMM the same scaled
  operands, ``baselines/fp8-gemm/baseline_prefill.py:41-54``; the block-order
  fp32 oracle is ``examples/fp8-gemm/v002_dense_tp8_validated_065.cu:277-288``);
* bf16 linear: ``tests/compare_decode_linear.py:263-274``;
* INT4 W4A16 w13: ``correctness/compare_marlin_vs_ref.py:44-100``
  (dequantize to bf16, fp32 matmul per expert, silu(gate)*up);
* FP8 MoE w13 / w2: the dense FP8 product per expert over its routed rows.

Pinned by ``tests/test_oracle_torch_cpu.py`` against ``oracle.gemm`` (itself
pinned by brute force and closed forms) on small shapes, to fp32 summation
tolerance (the two sum in different orders).
"""
from __future__ import annotations

import numpy as np
import torch


def _e4m3(codes: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(codes)).view(torch.float8_e4m3fn).to(torch.float32)


def _bf16(bits: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(torch.bfloat16).to(torch.float32)


def dequant_act(codes: np.ndarray, scales: np.ndarray) -> torch.Tensor:
    """e4m3 [M, K] x fp32 [M, K/128] -> fp32 [M, K]."""
    a = _e4m3(codes)
    m, k = a.shape
    s = torch.from_numpy(np.ascontiguousarray(scales, dtype=np.float32))
    return (a.view(m, k // 128, 128) * s[:, :, None]).view(m, k)


def dequant_weight(codes: np.ndarray, scales: np.ndarray) -> torch.Tensor:
    """e4m3 [N, K] x fp32 [ceil(N/128), K/128] -> fp32 [N, K]."""
    b = _e4m3(codes)
    n, k = b.shape
    s = torch.from_numpy(np.ascontiguousarray(scales, dtype=np.float32))
    s_rows = s.repeat_interleave(128, dim=0)[:n]                     # [N, K/128]
    return (b.view(n, k // 128, 128) * s_rows[:, :, None]).view(n, k)


def fp8_blockscale_gemm(a_codes, sa, b_codes, sb) -> torch.Tensor:
    return dequant_act(a_codes, sa) @ dequant_weight(b_codes, sb).T


def linear_bf16(x_bits, w_bits, residual_bits=None) -> torch.Tensor:
    y = _bf16(x_bits) @ _bf16(w_bits).T
    return y + _bf16(residual_bits) if residual_bits is not None else y


def silu_mul(g: torch.Tensor, u: torch.Tensor) -> torch.Tensor:
    return g / (1.0 + torch.exp(-g)) * u


def int4_dequant(wq: np.ndarray, ws_bits: np.ndarray, group: int = 32) -> torch.Tensor:
    """int32 [N, K/8] (low nibble first, value = nibble - 8) x bf16 [N, K/group]
    -> fp32 [N, K] of bf16-rounded values (compare_marlin_vs_ref.py:63-86)."""
    w = torch.from_numpy(np.ascontiguousarray(wq))
    shifts = torch.arange(0, 32, 4, dtype=torch.int32)
    q = ((w[:, :, None] >> shifts) & 0xF).reshape(w.shape[0], -1).to(torch.float32) - 8.0
    s = _bf16(ws_bits).repeat_interleave(group, dim=1)
    return (q * s).to(torch.bfloat16).to(torch.float32)


def _by_expert(topk_ids: np.ndarray, pairs: np.ndarray):
    ids = np.asarray(topk_ids).reshape(-1)[pairs]
    order = np.argsort(ids, kind="stable")
    for e in np.unique(ids):
        sel = order[ids[order] == e]
        yield int(e), sel


def moe_w13_fp8(x_codes, sx, w_codes, sw, topk_ids, pairs) -> torch.Tensor:
    topk = np.asarray(topk_ids).shape[1]
    half = w_codes.shape[1] // 2
    pairs = np.asarray(pairs, dtype=np.int64)
    out = torch.empty((pairs.size, half), dtype=torch.float32)
    for e, sel in _by_expert(topk_ids, pairs):
        toks = pairs[sel] // topk
        gu = dequant_act(x_codes[toks], sx[toks]) @ dequant_weight(w_codes[e], sw[e]).T
        out[torch.from_numpy(sel)] = silu_mul(gu[:, :half], gu[:, half:])
    return out


def moe_w13_w4a16(x_bits, wq, ws_bits, topk_ids, pairs) -> torch.Tensor:
    topk = np.asarray(topk_ids).shape[1]
    half = wq.shape[1] // 2
    pairs = np.asarray(pairs, dtype=np.int64)
    x = _bf16(x_bits)
    out = torch.empty((pairs.size, half), dtype=torch.float32)
    for e, sel in _by_expert(topk_ids, pairs):
        toks = torch.from_numpy(pairs[sel] // topk)
        gu = x[toks] @ int4_dequant(wq[e], ws_bits[e]).T
        out[torch.from_numpy(sel)] = silu_mul(gu[:, :half], gu[:, half:])
    return out


def moe_w2_fp8(h_codes, sh, w_codes, sw, topk_ids, pairs) -> torch.Tensor:
    pairs = np.asarray(pairs, dtype=np.int64)
    out = torch.empty((pairs.size, w_codes.shape[1]), dtype=torch.float32)
    for e, sel in _by_expert(topk_ids, pairs):
        rows = pairs[sel]
        out[torch.from_numpy(sel)] = dequant_act(h_codes[rows], sh[rows]) @ dequant_weight(w_codes[e], sw[e]).T
    return out


def moe_combine(o_bits, weights) -> torch.Tensor:
    w = torch.from_numpy(np.ascontiguousarray(weights, dtype=np.float32))
    t, topk = w.shape
    o = _bf16(o_bits).view(t, topk, -1)
    return (w[:, :, None] * o).sum(dim=1)


def quant_act_1x128(x: np.ndarray):
    """absmax/448 1x128 quantizer in torch (fp32 in, e4m3 codes + fp32 scales out)."""
    xt = torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32))
    m, k = xt.shape
    xv = xt.view(m, k // 128, 128)
    amax = xv.abs().amax(dim=2).clamp_min(1e-4)
    q = (xv * (448.0 / amax)[:, :, None]).to(torch.float8_e4m3fn).view(m, k)
    return q, amax / 448.0
