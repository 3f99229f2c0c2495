"""Shared helpers for the GPU parity tests (host-side conversions, oracle calls)."""
from __future__ import annotations

import numpy as np
import torch

from oracle import formats as F
from oracle import gemm as G
from oracle import metrics as MT
from oracle import routing as R

# Max relative error |g - r| / max(|r|, 1e-3 max|r|) allowed for every GEMM
# output against the fp32 dequantize-then-matmul oracle.
GEMM_TOL = 1e-2


def bits16(t: torch.Tensor) -> np.ndarray:
    """bf16 tensor -> uint16 bit patterns on the host."""
    return t.detach().contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def codes8(t: torch.Tensor) -> np.ndarray:
    return t.detach().contiguous().view(torch.uint8).cpu().numpy()


def f32(t: torch.Tensor) -> np.ndarray:
    return t.detach().float().cpu().numpy()


def bf16_out(t: torch.Tensor) -> np.ndarray:
    return F.bf16_bits_to_f32(bits16(t))


def assert_gemm_close(got: np.ndarray, ref: np.ndarray, what: str, tol: float = GEMM_TOL):
    err, nbad = MT.fp8_rel_err(got, ref)
    assert nbad == 0, f"{what}: {nbad} non-finite values"
    assert err < tol, f"{what}: max rel err {err:.4g} >= {tol}"
    return err


def oracle_routing(ids: np.ndarray, E: int, tile_m: int):
    counts, offsets, sp = R.permute(ids, E)
    tiles = R.tile_table(counts, offsets, tile_m)
    return counts, offsets, sp, tiles


def moe_sample_pairs(ids: np.ndarray, E: int, max_experts: int = 6, max_rows: int = 96, seed: int = 0):
    """Pairs of a few experts: the most and least loaded hit experts plus random ones."""
    counts, offsets, sp = R.permute(ids, E)
    hit = np.nonzero(counts)[0]
    order = hit[np.argsort(counts[hit], kind="stable")]
    rng = np.random.default_rng(seed)
    chosen = {int(order[0]), int(order[-1])}
    extra = rng.permutation(hit)
    for e in extra:
        if len(chosen) >= max_experts:
            break
        chosen.add(int(e))
    pairs = []
    for e in sorted(chosen):
        seg = sp[offsets[e]:offsets[e + 1]]
        if len(seg) > max_rows:
            seg = np.concatenate([seg[: max_rows // 2], seg[-max_rows // 2:]])
        pairs.extend(int(p) for p in seg)
    return np.array(pairs, dtype=np.int64), sorted(chosen)
