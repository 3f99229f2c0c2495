"""MoE routing, histogram, permutation and tile table (test infrastructure).

The reference has no routing kernel: DSv3 tasks use synthetic uniform segments
``m_indices = arange(M_total) // M_per_e``
(``baselines/fp8-group-gemm/baseline_dsv3_decode.py:50``,
``baseline_dsv3_prefill.py:53``), and Kimi uses randperm routing plus vLLM's
``moe_align_block_size`` (``baselines/kimi-moe-w13-int4/baseline_marlin.py:92-104,123-126``).
The contract restated here is therefore the library's own, fixed as follows:

* top-k is taken on fp32 LOGITS (softmax is monotonic), ordered by
  (value descending, expert index ascending); NaN logits rank as -inf;
* pair p = t*topk + j (``correctness/compare_marlin_vs_ref.py:97``);
* pairs are grouped by expert with a STABLE order (ascending pair index inside
  each expert), never arrival order;
* expert ids outside [0, E) are not routed (they get no row);
* the tile table lists, expert by expert in ascending order, tiles of at most
  ``tile_m`` consecutive sorted rows: (expert, first sorted row, row count).

vLLM's ``moe_align_block_size`` output format (padding sentinels) is only
pinnable by import, which is unavailable: parity with it is UNPINNED; the
build's tile table replaces it.  Pinned by (tests/test_oracle_routing.py):
brute force with ``np.argsort(kind="stable")`` on random and crafted-tie
inputs, bijection / histogram / cumsum invariants, and hand-written fixtures.
"""
from __future__ import annotations

import numpy as np


def route_topk(logits: np.ndarray, topk: int):
    """Top-k experts per token. Returns (ids int32 [T,topk], weights float32 [T,topk]).

    weights are the full softmax over E evaluated at the chosen experts (not
    renormalised); they are not used by the w13 projection.
    """
    lg = np.asarray(logits, dtype=np.float32)
    key = np.where(np.isnan(lg), -np.inf, lg)
    # np.argsort on -key is stable: equal values keep ascending index order.
    order = np.argsort(-key, axis=1, kind="stable")[:, :topk].astype(np.int32)
    mx = key.max(axis=1, keepdims=True)
    ex = np.exp((key - mx).astype(np.float32)).astype(np.float32)
    sm = (ex / ex.sum(axis=1, keepdims=True)).astype(np.float32)
    w = np.take_along_axis(sm, order.astype(np.int64), axis=1).astype(np.float32)
    return order, w


def expert_histogram(topk_ids: np.ndarray, num_experts: int) -> np.ndarray:
    ids = np.asarray(topk_ids).reshape(-1).astype(np.int64)
    valid = (ids >= 0) & (ids < num_experts)
    return np.bincount(ids[valid], minlength=num_experts).astype(np.int32)


def permute(topk_ids: np.ndarray, num_experts: int):
    """Stable expert-major order of the routed pairs.

    Returns (counts int32 [E], offsets int32 [E+1], sorted_pair int32 [P_valid])
    with sorted_pair[offsets[e] + r] = the r-th pair (ascending) routed to e.
    """
    ids = np.asarray(topk_ids).reshape(-1).astype(np.int64)
    valid = (ids >= 0) & (ids < num_experts)
    counts = np.bincount(ids[valid], minlength=num_experts).astype(np.int32)
    offsets = np.zeros(num_experts + 1, dtype=np.int32)
    offsets[1:] = np.cumsum(counts)
    key = np.where(valid, ids, num_experts)                     # invalid last
    order = np.argsort(key, kind="stable")
    sorted_pair = order[: int(valid.sum())].astype(np.int32)
    return counts, offsets, sorted_pair


def tile_table(counts: np.ndarray, offsets: np.ndarray, tile_m: int) -> np.ndarray:
    """int32 [ntiles, 3] rows (expert, first sorted row, row count)."""
    rows = []
    for e, c in enumerate(np.asarray(counts)):
        c = int(c)
        for j in range(0, c, tile_m):
            rows.append((e, int(offsets[e]) + j, min(tile_m, c - j)))
    if not rows:
        return np.zeros((0, 3), dtype=np.int32)
    return np.asarray(rows, dtype=np.int32)


def max_tiles(num_pairs: int, num_experts: int, tile_m: int) -> int:
    """Upper bound on the tile count for any routing of ``num_pairs`` pairs."""
    return min(num_pairs, (num_pairs + tile_m - 1) // tile_m + num_experts)


def m_indices(counts: np.ndarray) -> np.ndarray:
    """Expert id of every sorted row (DeepGEMM 'contiguous' layout), int32 [P]."""
    return np.repeat(np.arange(len(counts), dtype=np.int32), np.asarray(counts))
