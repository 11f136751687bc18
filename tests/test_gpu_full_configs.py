"""GPU parity at the full benchmark workloads of the two prefill layers,
through the same entry points the benchmark times:

* FP8 block MoE prefill: 256 experts, top-8 of N(0,1) router logits,
  T = 2048 tokens, hidden 7168, expert intermediate 2048, e4m3 weights from
  clip(N(0, 0.02), +-448) with float32 128x128 block scales, bf16
  activations quantized per token per 128 channels;
* int4 (AWQ, group 128) MoE prefill: 128 experts, top-8 of a skewed router
  (logits N(0,1) + a per-expert bias N(0,2)), hidden 2048, intermediate 768,
  T = 512 and 4096.

Routing ids and the expert-sorted token permutation the FFN ran on are
checked bit for bit on the whole batch against the oracle; outputs within
max|dy| <= 2e-2 * max|y_ref| of the oracle's restatement of the reference
algorithm (dequantize, then float32 matmuls with a float32 intermediate,
expert_ffn + moe_combine of blocks/moe.py:122-174): every token for the int4
layer, 256 tokens spread over the batch for the FP8 layer (its oracle
dequantizes each routed expert's 44 MB of weights on the host)."""

from __future__ import annotations

import os
from concurrent.futures import ThreadPoolExecutor

import numpy as np
import pytest
import torch

from oracle import awq as oawq
from oracle import fp8_block as ofb
from oracle import moe as omoe

pytestmark = pytest.mark.gpu

TOL = 2e-2
# regression bounds: about 3x the error measured on MI355X, below the
# contract (FP8 layer 2.2e-3 over 256 tokens: the e4m3 activations and the
# two-part e4m3 intermediate; int4 layers 3.8e-3 / 3.4e-3 at T = 512 / 4096:
# the bf16 intermediate and down rows)
REGRESS_C4 = 7e-3
REGRESS_C5 = 1.2e-2


def _ffn_schedule(ws: torch.Tensor, n: int, E: int, tile_m: int):
    """The schedule an FFN call left at the head of its workspace: sorted
    assignment ids (max_tiles * tile_m int32), then the tile -> expert table
    and the meta words, each region rounded to 256 bytes (the workspace
    layout of ccq_moe_w4_ffn / ccq_moe_fp8_ffn)."""
    from ccut._lib import lib

    mt = int(lib().ccq_moe_align_max_tiles(n, E, tile_m))
    a256 = lambda b: (b + 255) & ~255  # noqa: E731
    w = ws.view(torch.int32)
    o_te = a256(mt * tile_m * 4) // 4
    o_meta = o_te + a256(mt * 4) // 4
    ntiles = int(w[o_meta].item())
    return {"num_tiles": ntiles, "sorted_ids": w[: ntiles * tile_m].cpu().numpy(),
            "tile_expert": w[o_te: o_te + ntiles].cpu().numpy()}


def _check_routing(lg: torch.Tensor, w: torch.Tensor, ids: torch.Tensor, k: int):
    w0, ids0 = omoe.topk_softmax(lg.cpu().numpy(), k)
    assert np.array_equal(ids.cpu().numpy(), ids0)
    assert np.abs(w.cpu().numpy() - w0).max() <= 1e-6
    return w0, ids0


def _check_schedule(sch: dict, ids0: np.ndarray, E: int, tile_m: int):
    ref = omoe.moe_align(ids0, E, tile_m)
    assert sch["num_tiles"] == ref["num_tiles"]
    assert np.array_equal(sch["sorted_ids"], ref["sorted_ids"])
    assert np.array_equal(sch["tile_expert"], ref["tile_expert"])


def test_fp8_block_moe_prefill_full_layer(gpu):
    from ccut import _dev
    from ccut import workloads as wl
    from ccut.blocks import moe

    E, H, I, T, k = 256, 7168, 2048, 2048, 8
    print(f"[fp8 full layer] E={E} H={H} I={I} T={T} k={k}", flush=True)
    gate = wl.fp8_block_weights(E, I, H, seed=81, device=gpu)
    up = wl.fp8_block_weights(E, I, H, seed=82, device=gpu)
    down = wl.fp8_block_weights(E, H, I, seed=83, device=gpu)
    ex = moe.Fp8Experts.from_block(gate, up, down)
    x = wl.activations(T, H, seed=84, device=gpu)
    lg = wl.router_logits(T, E, seed=85, device=gpu)
    w, ids = moe.topk_softmax(lg, k, True)
    y = moe.moe_ffn_fp8(x, ids, w, ex, out_dtype=torch.float32)
    torch.cuda.synchronize()
    w0, ids0 = _check_routing(lg, w, ids, k)
    _check_schedule(_ffn_schedule(_dev.workspace("moe_fp8", 0, gpu), T * k, E, 128), ids0, E, 128)
    yh = y.cpu().numpy()
    assert np.isfinite(yh).all()

    toks = np.arange(0, T, T // 256)
    xs = x[torch.from_numpy(toks).to(gpu)].float().cpu().numpy()
    need: dict[int, list[int]] = {}
    for j, t in enumerate(toks):
        for e in ids0[t]:
            need.setdefault(int(e), []).append(j)

    def one(e):
        mats = [(t_[0][e].cpu().numpy(), t_[1][e].cpu().numpy()) for t_ in (gate, up, down)]
        rows = need[e]
        out = ofb.expert_ffn(xs[rows], mats[0][0], mats[0][1], mats[1][0], mats[1][1], mats[2][0], mats[2][1])
        return e, rows, out

    per = {}
    with ThreadPoolExecutor(max_workers=min(8, os.cpu_count() or 1)) as pool:
        for e, rows, out in pool.map(one, sorted(need)):
            for r, o in zip(rows, out):
                per[(r, e)] = o
    ref = np.zeros((len(toks), H), dtype=np.float32)
    for j, t in enumerate(toks):
        for s in range(k):
            ref[j] += w0[t, s] * per[(j, int(ids0[t, s]))]
    err = np.abs(yh[toks] - ref).max() / np.abs(ref).max()
    print(f"[fp8 full layer] {len(need)} experts checked, rel err {err:.3e}", flush=True)
    assert err <= TOL
    assert err <= REGRESS_C4


@pytest.mark.parametrize("T", [512, 4096])
def test_int4_moe_prefill_full_layer(gpu, T):
    from ccut import _dev
    from ccut import workloads as wl
    from ccut.blocks import moe

    E, H, I, G, k = 128, 2048, 768, 128, 8
    print(f"[int4 full layer] E={E} H={H} I={I} T={T} k={k} skewed router", flush=True)
    gate = wl.awq_experts(E, H, I, G, seed=71, device=gpu)
    up = wl.awq_experts(E, H, I, G, seed=72, device=gpu)
    down = wl.awq_experts(E, I, H, G, seed=73, device=gpu)
    ex = moe.W4Experts.from_awq(gate, up, down, G)
    x = wl.activations(T, H, seed=74, device=gpu)
    lg = wl.router_logits(T, E, seed=75, device=gpu, skew_std=2.0)
    w, ids = moe.topk_softmax(lg, k, True)
    y = moe.moe_ffn_w4(x, ids, w, ex, out_dtype=torch.float32)
    torch.cuda.synchronize()
    w0, ids0 = _check_routing(lg, w, ids, k)
    _check_schedule(_ffn_schedule(_dev.workspace("moe_w4", 0, gpu), T * k, E, 128), ids0, E, 128)
    yh = y.cpu().numpy()
    host = [tuple(a.cpu().numpy() for a in t_) for t_ in (gate, up, down)]
    cache = {}

    def lookup(e):
        if e not in cache:
            cache[e] = tuple(oawq.dequant(m[0][e], m[1][e], m[2][e], G) for m in host)
        return cache[e]

    ref = omoe.moe_combine(x.float().cpu().numpy(), ids0, w0, lookup)
    err = np.abs(yh - ref).max() / np.abs(ref).max()
    counts = np.bincount(ids0.reshape(-1), minlength=E)
    print(f"[int4 full layer] T={T}: experts used {int((counts > 0).sum())}, rows per expert "
          f"{int(counts.min())}..{int(counts.max())}, rel err {err:.3e}", flush=True)
    assert err <= TOL
    assert err <= REGRESS_C5
