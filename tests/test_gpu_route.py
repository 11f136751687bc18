"""GPU parity of routing: top-k ids and the expert-sorted permutation are
bit-exact with the oracle; routing weights within 1e-6 (float32 exp)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import moe as omoe

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("E,k", [(64, 6), (256, 8), (128, 8), (32, 4), (1000, 16), (8, 8), (1, 1)])
@pytest.mark.parametrize("norm", [True, False])
def test_topk_softmax_parity(gpu, E, k, norm):
    from ccut.blocks import moe

    rng = np.random.default_rng(E * 10 + k)
    lg = rng.standard_normal((67, E)).astype(np.float32)
    w, ids = moe.topk_softmax(lg, k, norm)
    w0, ids0 = omoe.topk_softmax(lg, k, norm)
    assert ids.dtype == np.int64 and w.dtype == np.float32
    assert np.array_equal(ids, ids0)
    assert np.allclose(w, w0, atol=1e-6, rtol=1e-6)


def test_topk_ties_and_plain_values(gpu):
    from ccut.blocks import moe

    rng = np.random.default_rng(7)
    x = rng.integers(-2, 3, size=(200, 96)).astype(np.float32)  # heavy ties
    v, i = moe.topk(x, 8)
    v0, i0 = omoe.topk(x, 8)
    assert np.array_equal(i, i0) and np.array_equal(v, v0)
    w, ids = moe.topk_softmax(x, 8, True)
    assert np.array_equal(ids, omoe.topk_softmax(x, 8, True)[1])


def test_topk_nan_rows_and_sentinel(gpu):
    from ccut.blocks import moe

    x = np.array([[np.nan, 1.0, np.nan, 0.5, -np.inf],
                  [np.nan] * 5,
                  [-1e31, 2.0, -1e31, -1e31, -1e31]], dtype=np.float32)
    v, i = moe.topk(x, 3)
    v0, i0 = omoe.topk(x, 3)
    assert np.array_equal(i, i0)
    assert np.array_equal(v, v0)


@pytest.mark.parametrize("E,k", [(64, 8), (64, 16), (40, 6), (64, 1), (96, 8)])
def test_topk_edge_cases_all_modes(gpu, E, k):
    """Heavy ties, +0 next to -0, exact -1e30 and NaN (never selected), rows
    with fewer selectable values than k (slots filled with -1e30 / -1), and
    NaN / +inf logits, which numpy's softmax turns into NaN rows and the
    route_experts loop into zero weights.  E <= 64 is the one column per lane
    selection, E = 96 two columns per lane."""
    from ccut.blocks import moe

    rng = np.random.default_rng(E + k)
    x = rng.integers(-2, 3, size=(96, E)).astype(np.float32)
    x[x == 0] = np.where(rng.random(np.count_nonzero(x == 0)) < 0.5, -0.0, 0.0)
    x[rng.random(x.shape) < 0.05] = -1e30
    x[rng.random(x.shape) < 0.05] = np.nan
    x[5, :] = -1e30
    x[6, : E - 3] = np.nan
    x[7, :] = -0.0
    x[7, 9] = 0.0
    x[8:12] = np.where(np.isnan(x[8:12]), 1.0, x[8:12])  # rows 8-11: no NaN
    x[9, 3] = np.inf
    x[10, [2, 30]] = np.inf
    x[11, :] = rng.integers(-2, 3, size=E)
    x[11, 17] = -np.inf
    v, i = moe.topk(x, k)
    v0, i0 = omoe.topk(x, k)
    assert np.array_equal(i, i0)
    assert np.array_equal(v.view(np.uint32), v0.view(np.uint32))  # -0 stays -0
    for norm in (True, False):
        w, ids = moe.topk_softmax(x, k, norm)
        w0, ids0 = omoe.topk_softmax(x, k, norm)
        assert np.array_equal(ids, ids0)
        assert np.allclose(w, w0, atol=1e-6, rtol=1e-6, equal_nan=True)
    assert np.isnan(omoe.topk_softmax(x, k, True)[0][9]).all()  # the +inf row
    assert (omoe.topk_softmax(x, k, False)[1][9] == -1).all()  # NaN probabilities
    for norm in (0, 1):
        w, ids = moe.route_experts(x, k, norm)
        w0, ids0 = omoe.route_experts(x, k, norm)
        assert np.array_equal(ids, ids0)
        assert np.allclose(w, w0, atol=1e-6, rtol=1e-6, equal_nan=True)
    assert (omoe.route_experts(x, k, 1)[0][9] == 0).all()


def test_route_experts_modes(gpu):
    from ccut.blocks import moe

    rng = np.random.default_rng(8)
    lg = rng.standard_normal((33, 64)).astype(np.float32)
    for norm in (0, 1):
        w, i = moe.route_experts(lg, 6, norm)
        w0, i0 = omoe.route_experts(lg, 6, norm)
        assert np.array_equal(i, i0) and np.allclose(w, w0, atol=1e-6)


def test_reference_topk_softmax_invariants_on_gpu(gpu):
    """reference python/tests/test_blocks.py:127-134 against this API."""
    from ccut.blocks import moe

    np.random.seed(5)
    gl = np.random.randn(6, 32).astype(np.float32)
    w, idx = moe.topk_softmax(gl, 4)
    assert np.allclose(w.sum(axis=1), 1.0, atol=1e-5)
    assert all(len(set(idx[i].tolist())) == 4 for i in range(6))
    for i in range(6):
        assert bool((np.diff(w[i]) <= 1e-6).all())


def _align_check(ids: np.ndarray, E: int, tile_m: int):
    from ccut.blocks import moe

    got = moe.moe_align(ids, E, tile_m).host()
    ref = omoe.moe_align(ids, E, tile_m)
    assert got["num_tiles"] == ref["num_tiles"]
    assert np.array_equal(got["sorted_ids"], ref["sorted_ids"])
    assert np.array_equal(got["tile_expert"], ref["tile_expert"])
    assert np.array_equal(got["counts"], ref["counts"])
    assert got["num_experts_active"] == int((ref["counts"] > 0).sum())


@pytest.mark.parametrize("T,E,k,tile_m", [(1, 64, 6, 16), (16, 64, 6, 16), (100, 256, 8, 64),
                                          (2048, 256, 8, 128), (513, 128, 8, 32), (7, 8, 8, 1),
                                          # one-wave schedule of small batches (<= 256 assignments): the
                                          # largest batch, 10 id bits, 128-row tiles, one expert; 257 is
                                          # the first batch of the workgroup kernel
                                          (32, 256, 8, 16), (20, 1000, 8, 16), (16, 8, 8, 128), (10, 1, 1, 16),
                                          (257, 16, 1, 16),
                                          # one-workgroup schedule of mid-size batches (257 .. 8192
                                          # assignments, 1 .. 8 chunks per wave): 1024 experts, 8 experts
                                          # (many repeats per chunk), the largest batch, 7-row tiles
                                          (512, 256, 8, 16), (200, 1024, 10, 128), (1024, 8, 8, 64),
                                          (300, 1000, 3, 7), (129, 64, 8, 128), (1025, 64, 8, 128)])
def test_align_permutation_bitexact(gpu, T, E, k, tile_m):
    rng = np.random.default_rng(T + E)
    lg = rng.standard_normal((T, E)).astype(np.float32)
    _, ids = omoe.topk_softmax(lg, k)
    _align_check(ids, E, tile_m)


@pytest.mark.parametrize("T,E", [(512, 128), (512, 256)])
def test_align_skewed_router_mid(gpu, T, E):
    """The int4 (128 experts) and FP8 per-row (256 experts) prefill
    layers at T=512 top-8: skewed experts with several 128-row tiles."""
    rng = np.random.default_rng(T + E + 1)
    lg = (rng.standard_normal((T, E)) + rng.standard_normal((1, E)) * 2.0).astype(np.float32)
    _, ids = omoe.topk_softmax(lg, 8)
    _align_check(ids, E, 128)


@pytest.mark.parametrize("n,E", [(3000, 37), (8192, 1024), (300, 5)])
def test_align_raw_ids_mid(gpu, n, E):
    """Arbitrary id streams (repeats inside a chunk, ids outside [0, E)
    dropped) on the mid-size schedule."""
    rng = np.random.default_rng(n + E)
    ids = rng.integers(-2, E + 3, size=(n, 1)).astype(np.int64)
    _align_check(ids, E, 16)


def test_align_skewed_router_t4096(gpu):
    rng = np.random.default_rng(42)
    lg = (rng.standard_normal((4096, 128)) + rng.standard_normal((1, 128)) * 2.0).astype(np.float32)
    _, ids = omoe.topk_softmax(lg, 8)
    _align_check(ids, 128, 64)


def test_align_drops_invalid_ids_and_handles_duplicates(gpu):
    ids = np.array([[3, -1], [1, 3], [7, 1], [3, 3]], dtype=np.int64)
    from ccut.blocks import moe

    got = moe.moe_align(ids, 5, 2).host()
    # expert 3: a = 0, 3, 6, 7 ; expert 1: a = 2, 5 ; ids -1 and 7 dropped
    assert got["sorted_ids"].tolist() == [0, 3, 6, 7, 2, 5]
    assert got["tile_expert"].tolist() == [3, 3, 1]
    assert got["counts"].tolist() == [0, 2, 0, 4, 0]


@pytest.mark.parametrize("k,H", [(3, 70), (20, 128), (6, 2048)])
def test_combine_slot_order(gpu, k, H):
    """Slot-order float32 sums; k above 16 runs in chunks of 16 slots, H a
    multiple of 4 on the 16-byte path."""
    from ccut._lib import call
    from ccut import _dev

    rng = np.random.default_rng(9 + k)
    T = 5
    rows = torch.from_numpy(rng.standard_normal((T * k, H)).astype(np.float32)).to(gpu)
    w = torch.from_numpy(rng.random((T, k)).astype(np.float32)).to(gpu)
    y = torch.empty((T, H), dtype=torch.float32, device=gpu)
    call("ccq_moe_combine", rows.data_ptr(), w.data_ptr(), y.data_ptr(), 0, T, k, H, _dev.stream_ptr())
    r = rows.cpu().numpy().reshape(T, k, H)
    ref = np.zeros((T, H), dtype=np.float32)
    for s in range(k):
        ref += w.cpu().numpy()[:, s:s + 1] * r[:, s]
    assert np.allclose(y.cpu().numpy(), ref, atol=1e-6)
