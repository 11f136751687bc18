"""Pin the oracle's restatement of the reference MoE block
(reference python/ccut/blocks/moe.py)."""

from __future__ import annotations

import numpy as np
import pytest

from oracle import moe


def _topk_argsort(x: np.ndarray, k: int):
    """Brute force: stable descending sort keeps the lowest index first among
    equal values."""
    idx = np.argsort(-x.astype(np.float64), axis=1, kind="stable")[:, :k]
    return np.take_along_axis(x, idx, axis=1), idx


def test_topk_matches_stable_argsort_with_ties():
    rng = np.random.default_rng(0)
    x = rng.integers(-3, 4, size=(50, 20)).astype(np.float32)  # many ties
    v, i = moe.topk(x, 6)
    v2, i2 = _topk_argsort(x, 6)
    assert np.array_equal(i, i2) and np.array_equal(v, v2)


def test_topk_nan_and_sentinel_quirk():
    x = np.array([[np.nan, 1.0, np.nan, 0.5],
                  [np.nan, np.nan, np.nan, np.nan]], dtype=np.float32)
    v, i = moe.topk(x, 3)
    assert i[0].tolist() == [1, 3, -1]          # NaN never selected
    # row of NaN: nothing > -1e30 -> (-1e30, -1); used[-1] marks the last column
    assert i[1].tolist() == [-1, -1, -1]
    assert np.all(v[1] == np.float32(-1.0e30))


def test_reference_topk_softmax_invariants_rehosted():
    """reference python/tests/test_blocks.py:127-134."""
    np.random.seed(5)
    gl = np.random.randn(6, 32).astype(np.float32)
    w, idx = moe.topk_softmax(gl, 4)
    assert np.allclose(w.sum(axis=1), 1.0, atol=1e-5)
    assert all(len(set(idx[i].tolist())) == 4 for i in range(6))
    for i in range(6):
        assert bool((np.diff(w[i]) <= 1e-6).all())


def test_topk_softmax_closed_forms():
    rng = np.random.default_rng(1)
    lg = rng.standard_normal((40, 64)).astype(np.float32)
    w, idx = moe.topk_softmax(lg, 6, True)
    _, idx2 = _topk_argsort(lg, 6)
    assert np.array_equal(idx, idx2)
    sel = np.take_along_axis(lg, idx, 1).astype(np.float64)
    ref = np.exp(sel - sel.max(1, keepdims=True))
    ref /= ref.sum(1, keepdims=True)
    assert np.allclose(w, ref, atol=1e-6)
    w0, idx0 = moe.topk_softmax(lg, 6, False)
    p = np.exp(lg.astype(np.float64) - lg.max(1, keepdims=True))
    p /= p.sum(1, keepdims=True)
    assert np.array_equal(idx0, idx2)  # softmax is monotonic
    assert np.allclose(w0, np.take_along_axis(p, idx0, 1), atol=1e-6)
    assert np.all(w0.sum(1) < 1.0)  # not renormalised


def test_route_experts_modes():
    rng = np.random.default_rng(2)
    lg = rng.standard_normal((10, 16)).astype(np.float32)
    w1, i1 = moe.route_experts(lg, 4, 1)
    wr, ir = moe.topk_softmax(lg, 4, True)
    assert np.array_equal(i1, ir) and np.allclose(w1, wr, atol=1e-6)
    w0, i0 = moe.route_experts(lg, 4, 0)
    sel = np.take_along_axis(lg, i0, 1).astype(np.float64)
    assert np.allclose(w0, np.exp(sel) / np.exp(sel).sum(1, keepdims=True), atol=1e-6)


def test_routing_special_rows_closed_forms():
    """Rows where numpy's float32 softmax and the float64 route_experts loop
    part ways (IEEE arithmetic fixes every value here)."""
    k = 3
    assert float(np.float32(-1e30)) < -1e30  # the slot filler sits below the loop's start
    empty = np.full((1, 5), -1e30, np.float32)  # nothing selectable
    w, i = moe.topk_softmax(empty, k, True)
    assert (i == -1).all() and np.allclose(w, 1.0 / k)  # exp(0) / k
    w, i = moe.route_experts(empty, k, 1)
    assert (w == 0).all()  # exp(-1e30f - (-1e30)) underflows: sum 0 -> weights 0
    w, i = moe.route_experts(empty, k, 0)
    assert (w == 0).all()
    inf_row = np.array([[1.0, np.inf, 0.5, 2.0, -1.0]], np.float32)
    with np.errstate(invalid="ignore"):
        w, i = moe.topk_softmax(inf_row, k, True)
        assert list(i[0]) == [1, 3, 0] and np.isnan(w).all()  # inf - inf in the max shift
        w, i = moe.route_experts(inf_row, k, 1)
        assert (w == 0).all()  # NaN sum is not > 0
        w, i = moe.route_experts(inf_row, k, 0)
        assert np.isnan(w[0, 0]) and (w[0, 1:] == 0).all()  # inf / inf, finite / inf
        nan_row = np.array([[1.0, np.nan, 0.5, 2.0, -1.0]], np.float32)
        w, i = moe.topk_softmax(nan_row, k, False)
        assert (i == -1).all()  # every probability NaN: nothing selectable


def test_expert_order_and_align_contract():
    ids = np.array([[3, 1], [1, 0], [2, 3], [3, 1]])
    order = moe.expert_order(ids)
    assert list(order.keys()) == [3, 1, 0, 2]
    assert order == {3: [0, 2, 3], 1: [0, 1, 3], 0: [1], 2: [2]}
    al = moe.moe_align(ids, num_experts=5, tile_m=2)
    # expert 3: a = 0, 5, 6 ; expert 1: a = 1, 2, 7 ; expert 0: a = 3 ; expert 2: a = 4
    assert al["sorted_ids"].tolist() == [0, 5, 6, -1, 1, 2, 7, -1, 3, -1, 4, -1]
    assert al["tile_expert"].tolist() == [3, 3, 1, 1, 0, 2]
    assert al["counts"].tolist() == [1, 3, 1, 3, 0]
    assert al["expert_rank"].tolist() == [2, 1, 3, 0, -1]


def test_moe_combine_bruteforce():
    rng = np.random.default_rng(3)
    T, H, I, E, k = 7, 8, 6, 5, 2
    x = rng.standard_normal((T, H)).astype(np.float32)
    W = {e: (rng.standard_normal((H, I)).astype(np.float32), rng.standard_normal((H, I)).astype(np.float32),
             rng.standard_normal((I, H)).astype(np.float32)) for e in range(E)}
    lg = rng.standard_normal((T, E)).astype(np.float32)
    w, ids = moe.topk_softmax(lg, k)
    out = moe.moe_combine(x, ids, w, W.__getitem__)
    ref = np.zeros((T, H))
    for t in range(T):
        for s in range(k):
            g, u, d = (a.astype(np.float64) for a in W[int(ids[t, s])])
            xt = x[t].astype(np.float64)
            gg = xt @ g
            h = gg / (1 + np.exp(-gg)) * (xt @ u)
            ref[t] += float(w[t, s]) * (h @ d)
    assert np.allclose(out, ref, rtol=1e-4, atol=1e-4)
    out2 = moe.moe_ffn_dense(x, ids, w, W.__getitem__)
    assert np.allclose(out2, ref, rtol=1e-4, atol=1e-4)
