"""Oracle: restatement of the reference's MoE routing, expert FFN and combine.

Test infrastructure only (see ``oracle/__init__.py``).
"""

from __future__ import annotations

import numpy as np

from oracle.ref_quant import silu_mul_fused


def topk(x: np.ndarray, k: int) -> tuple[np.ndarray, np.ndarray]:
    """Per row, k passes of "first strictly greater than the running best".
    Follows ``blocks/moe.py:46-68``.

    The running best starts at -1e30 and ``x > best`` is strict, so ties go to
    the lowest column, NaN and values <= -1e30 are never picked.  When a pass
    finds nothing, the reference stores ``(-1e30, -1)`` and its ``used[-1] = 1``
    marks the LAST column as used; that quirk is kept.
    """
    x = np.asarray(x)
    rows, cols = x.shape
    vals = np.empty((rows, k), dtype=x.dtype)
    idx = np.empty((rows, k), dtype=np.int64)
    xd = x.astype(np.float64)
    for r in range(rows):
        used = np.zeros(cols, dtype=bool)
        row = xd[r]
        for j in range(k):
            cand = np.where(used | ~(row > -1.0e30), -np.inf, row)
            bi = int(np.argmax(cand))  # first maximum = lowest index
            if not (cand[bi] > -1.0e30):
                bi = -1
                best = -1.0e30
            else:
                best = row[bi]
            used[bi] = True
            vals[r, j] = best
            idx[r, j] = bi
    return vals, idx


def topk_softmax(logits: np.ndarray, k: int, norm_topk_prob: bool = True) -> tuple[np.ndarray, np.ndarray]:
    """Routing weights.  Follows ``blocks/moe.py:71-89`` with the same numpy
    float32 operations.

    ``norm_topk_prob=True``: top-k of the logits, then softmax over the k.
    ``False``: float32 softmax over all experts, then top-k of the
    probabilities, no renormalisation.
    """
    logits = np.asarray(logits, dtype=np.float32)
    if not norm_topk_prob:
        e = np.exp(logits - logits.max(axis=1, keepdims=True))
        p = e / np.maximum(e.sum(axis=1, keepdims=True), 1e-30)
        vals, idx = topk(p, k)
        return vals.astype(np.float32), idx
    vals, idx = topk(logits, k)
    v = vals - vals.max(axis=1, keepdims=True)
    ex = np.exp(v)
    w = ex / np.maximum(ex.sum(axis=1, keepdims=True), 1e-30)
    return w.astype(np.float32), idx


def route_experts(gate_logits: np.ndarray, top_k: int, norm_topk: int) -> tuple[np.ndarray, np.ndarray]:
    """Fused top-k + softmax.  Follows ``blocks/moe.py:92-119`` (numba
    semantics: the sum is a float64 scalar).

    ``norm_topk=1``: softmax over the k selected logits with the max
    subtracted.  ``norm_topk=0``: ``exp(v)/sum(exp(v))`` over the k selected
    raw logits (no max subtraction) -- this disagrees with
    ``topk_softmax(norm_topk_prob=False)``, as in the reference.  The running
    maximum is a float64 starting at -1e30, above the float32 slot filler
    -1e30f, so a row with nothing selectable gets weights 0 (``s > 0`` fails),
    where ``topk_softmax`` gives 1/k.
    """
    vals, idx = topk(np.asarray(gate_logits, dtype=np.float32), top_k)
    rows = vals.shape[0]
    w = np.empty((rows, top_k), dtype=np.float32)
    for r in range(rows):
        if norm_topk:
            m = -1.0e30
            for j in range(top_k):
                if vals[r, j] > m:
                    m = vals[r, j]
            e = np.exp((vals[r].astype(np.float64) - m)).astype(np.float32)
        else:
            e = np.exp(vals[r].astype(np.float64)).astype(np.float32)
        s = 0.0
        for j in range(top_k):  # sequential float64 sum, as the numba loop
            s += float(e[j])
        w[r] = (e.astype(np.float64) / s).astype(np.float32) if s > 0 else 0.0
    return w, idx


def expert_ffn(x: np.ndarray, w_gate: np.ndarray, w_up: np.ndarray, w_down: np.ndarray) -> np.ndarray:
    """``down(silu(x @ Wg) * (x @ Wu))`` with ``Wg, Wu [hidden, inter]`` and
    ``Wd [inter, hidden]`` already dequantized.  Follows ``blocks/moe.py:122-141``.
    """
    x = np.asarray(x, dtype=np.float32)
    gate = x @ w_gate
    up = x @ w_up
    inter = silu_mul_fused(gate, up)
    return inter @ w_down


def expert_order(expert_ids: np.ndarray) -> dict[int, list[int]]:
    """The token permutation contract of ``blocks/moe.py:163-167`` (and
    ``models/generic.py:366-370``): experts in first-appearance order scanning
    tokens ascending then slots ascending; each expert's token list ascending.
    """
    ids = np.asarray(expert_ids)
    by_expert: dict[int, list[int]] = {}
    for t in range(ids.shape[0]):
        for e in range(ids.shape[1]):
            by_expert.setdefault(int(ids[t, e]), []).append(t)
    return by_expert


def moe_combine(x, expert_ids, weights, w_lookup, expert_fn=expert_ffn) -> np.ndarray:
    """``y[t] = sum_e w[t,e] * expert_e(x[t])`` grouped by expert.
    Follows ``blocks/moe.py:144-174``: one batch per expert in first-appearance
    order; ``out[t] += w[t, slot] * y[i]`` in float32 with the slot found by
    ``list(ids[t]).index(eid)``."""
    x = np.asarray(x, dtype=np.float32)
    ids = np.asarray(expert_ids)
    weights = np.asarray(weights, dtype=np.float32)
    seq, hidden = x.shape
    out = np.zeros((seq, hidden), dtype=np.float32)
    for eid, toks in expert_order(ids).items():
        wg, wu, wd = w_lookup(eid)
        y = expert_fn(x[np.array(toks, dtype=np.int64)], wg, wu, wd)
        for i, t in enumerate(toks):
            out[t] += weights[t, list(ids[t]).index(eid)] * y[i]
    return out


def moe_align(expert_ids: np.ndarray, num_experts: int, tile_m: int) -> dict:
    """Expert-sorted, tile-padded assignment schedule.

    The permutation itself is the reference's (``expert_order``): experts in
    first-appearance order, within an expert the flat assignments
    ``a = t*k + slot`` ascending.  Each expert's list is padded with -1 to a
    multiple of ``tile_m``.  Returns ``sorted_ids`` (padded), ``tile_expert``
    (expert of each tile), ``expert_rank`` (first-appearance rank per expert,
    -1 when unused) and ``counts`` (assignments per expert).
    """
    ids = np.asarray(expert_ids).astype(np.int64)
    T, k = ids.shape
    flat = ids.reshape(-1)
    order: list[int] = []
    seen = set()
    for e in flat:
        e = int(e)
        if 0 <= e < num_experts and e not in seen:
            seen.add(e)
            order.append(e)
    sorted_ids: list[int] = []
    tile_expert: list[int] = []
    counts = np.zeros(num_experts, dtype=np.int64)
    rank = np.full(num_experts, -1, dtype=np.int64)
    for r, e in enumerate(order):
        rank[e] = r
        a = [int(i) for i in np.nonzero(flat == e)[0]]
        counts[e] = len(a)
        ntile = (len(a) + tile_m - 1) // tile_m
        a = a + [-1] * (ntile * tile_m - len(a))
        sorted_ids.extend(a)
        tile_expert.extend([e] * ntile)
    return {
        "sorted_ids": np.array(sorted_ids, dtype=np.int32),
        "tile_expert": np.array(tile_expert, dtype=np.int32),
        "expert_rank": rank.astype(np.int32),
        "counts": counts.astype(np.int32),
        "num_tiles": len(tile_expert),
    }


def moe_ffn_dense(x, expert_ids, weights, w_lookup) -> np.ndarray:
    """Same result as ``moe_combine`` but accumulating each token's k expert
    outputs in slot order (the order the GPU combine uses).  Used where the
    float32 summation order should not be part of the comparison."""
    x = np.asarray(x, dtype=np.float32)
    ids = np.asarray(expert_ids)
    weights = np.asarray(weights, dtype=np.float32)
    T, k = ids.shape
    per: dict[int, np.ndarray] = {}
    rows: dict[int, list[int]] = {}
    for eid, toks in expert_order(ids).items():
        wg, wu, wd = w_lookup(eid)
        per[eid] = expert_ffn(x[np.array(toks, dtype=np.int64)], wg, wu, wd)
        rows[eid] = toks
    out = np.zeros_like(x)
    pos = {eid: {t: i for i, t in enumerate(toks)} for eid, toks in rows.items()}
    for t in range(T):
        for s in range(k):
            eid = int(ids[t, s])
            out[t] += weights[t, s] * per[eid][pos[eid][t]]
    return out
