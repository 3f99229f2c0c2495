"""Pin the oracle's routing / histogram / permutation / tile table."""
import numpy as np
import pytest
from hypothesis import given, settings, strategies as st

from oracle import routing as R


def test_topk_crafted_ties_and_nan():
    logits = np.array([
        [1.0, 3.0, 3.0, 2.0, np.nan, 3.0],
        [0.0, -0.0, 0.0, -1.0, -1.0, 5.0],
    ], dtype=np.float32)
    ids, w = R.route_topk(logits, 4)
    assert ids.tolist() == [[1, 2, 5, 3], [5, 0, 1, 2]]
    assert np.all(np.isfinite(w[0])) and np.all(w > 0)


def test_topk_brute_force_random():
    rng = np.random.default_rng(0)
    for _ in range(20):
        T, E, k = int(rng.integers(1, 9)), int(rng.integers(8, 70)), int(rng.integers(1, 8))
        lg = rng.integers(-3, 4, size=(T, E)).astype(np.float32)   # many ties
        ids, _ = R.route_topk(lg, k)
        for t in range(T):
            order = sorted(range(E), key=lambda e: (-lg[t, e], e))[:k]
            assert ids[t].tolist() == order


def test_topk_weights_are_softmax():
    rng = np.random.default_rng(1)
    lg = rng.standard_normal((4, 16)).astype(np.float32)
    ids, w = R.route_topk(lg, 3)
    sm = np.exp(lg.astype(np.float64)); sm /= sm.sum(1, keepdims=True)
    assert np.allclose(w, np.take_along_axis(sm, ids.astype(np.int64), 1), rtol=1e-5)


def test_permute_fixture():
    ids = np.array([[2, 0], [0, 2], [1, 2]], np.int32)      # pairs 0..5
    counts, offsets, sp = R.permute(ids, 4)
    assert counts.tolist() == [2, 1, 3, 0]
    assert offsets.tolist() == [0, 2, 3, 6, 6]
    assert sp.tolist() == [1, 2, 4, 0, 3, 5]
    tiles = R.tile_table(counts, offsets, 2)
    assert tiles.tolist() == [[0, 0, 2], [1, 2, 1], [2, 3, 2], [2, 5, 1]]
    assert R.m_indices(counts).tolist() == [0, 0, 1, 2, 2, 2]


def test_permute_skips_invalid_ids():
    ids = np.array([[0, 7], [-1, 1]], np.int32)
    counts, offsets, sp = R.permute(ids, 2)
    assert counts.tolist() == [1, 1] and offsets.tolist() == [0, 1, 2]
    assert sp.tolist() == [0, 3]


@settings(max_examples=60, deadline=None)
@given(st.integers(1, 40), st.integers(1, 20), st.integers(1, 6), st.integers(1, 9), st.integers(0, 2 ** 31 - 1))
def test_permute_invariants(T, E, k, tile_m, seed):
    rng = np.random.default_rng(seed)
    ids = rng.integers(0, E, size=(T, k)).astype(np.int32)
    counts, offsets, sp = R.permute(ids, E)
    flat = ids.reshape(-1)
    assert sorted(sp.tolist()) == list(range(T * k))                         # bijection
    assert counts.tolist() == np.bincount(flat, minlength=E).tolist()
    assert offsets[0] == 0 and np.array_equal(np.diff(offsets), counts)
    for e in range(E):
        seg = sp[offsets[e]:offsets[e + 1]]
        assert np.all(flat[seg] == e) and np.all(np.diff(seg) > 0)          # stable
    tiles = R.tile_table(counts, offsets, tile_m)
    assert tiles.shape[0] <= R.max_tiles(T * k, E, tile_m)
    assert int(tiles[:, 2].sum()) == T * k
    assert np.all(tiles[:, 2] >= 1) and np.all(tiles[:, 2] <= tile_m)
    covered = np.concatenate([np.arange(r0, r0 + n) for _, r0, n in tiles]) if len(tiles) else np.array([])
    assert covered.tolist() == list(range(T * k))
