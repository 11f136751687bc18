"""The shared expert's add (reference python/ccut/blocks/moe.py:177-179,
experts/pipeline.py:181-190) as its own kernel and in the combine's
epilogue: bit-identical to combine-then-add, and to numpy's float32
``y + gate * shared``."""

from __future__ import annotations

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def test_shared_expert_add_matches_numpy(gpu):
    from ccut.blocks import moe

    rng = np.random.default_rng(4)
    y = rng.standard_normal((7, 300)).astype(np.float32)
    s = rng.standard_normal((7, 300)).astype(np.float32)
    g = 0.37
    ref = y + np.float32(g) * s  # numpy: the product in float32, then the add
    yh = y.copy()
    moe.shared_expert_add(yh, s, g)
    assert np.array_equal(yh, ref)
    yd = torch.from_numpy(y).to(gpu)
    moe.shared_expert_add(yd, torch.from_numpy(s).to(gpu), g)
    assert np.array_equal(yd.cpu().numpy(), ref)


@pytest.mark.parametrize("k,H", [(6, 2048), (3, 70), (20, 128)])
def test_combine_shared_epilogue(gpu, k, H):
    from ccut import _dev
    from ccut._lib import call

    rng = np.random.default_rng(k + H)
    T = 5
    rows = torch.from_numpy(rng.standard_normal((T * k, H)).astype(np.float32)).to(gpu)
    w = torch.from_numpy(rng.random((T, k)).astype(np.float32)).to(gpu)
    sh = torch.from_numpy(rng.standard_normal((T, H)).astype(np.float32)).to(gpu)
    g = np.float32(0.61)
    y0 = torch.empty((T, H), device=gpu)
    call("ccq_moe_combine", rows.data_ptr(), w.data_ptr(), y0.data_ptr(), 0, T, k, H, _dev.stream_ptr())
    y1 = torch.empty((T, H), device=gpu)
    call("ccq_moe_combine_shared", rows.data_ptr(), w.data_ptr(), sh.data_ptr(), float(g), y1.data_ptr(), 0, T, k,
         H, _dev.stream_ptr())
    ref = y0.cpu().numpy() + g * sh.cpu().numpy()
    assert np.array_equal(y1.cpu().numpy(), ref)


def test_moe_ffn_w4_shared_epilogue(gpu):
    from ccut.blocks import moe
    from oracle import awq as oawq

    E, H, I, G, T, k = 8, 256, 384, 128, 5, 2
    rng = np.random.default_rng(12)

    def one(K, N):
        q = rng.integers(0, 16, size=(E, K, N), dtype=np.uint8)
        z = rng.integers(0, 16, size=(E, K // G, N), dtype=np.uint8)
        s = (np.abs(rng.standard_normal((E, K // G, N))) * 0.01 + 1e-3).astype(np.float16)
        return (torch.from_numpy(np.stack([oawq.pack(q[e]) for e in range(E)])).to(gpu),
                torch.from_numpy(np.stack([oawq.pack(z[e]) for e in range(E)])).to(gpu), torch.from_numpy(s).to(gpu))

    ex = moe.W4Experts.from_awq(one(H, I), one(H, I), one(I, H), group_size=G)
    x = torch.from_numpy(rng.standard_normal((T, H)).astype(np.float32)).to(gpu).to(torch.bfloat16)
    lg = torch.from_numpy(rng.standard_normal((T, E)).astype(np.float32)).to(gpu)
    w, ids = moe.topk_softmax(lg, k, True)
    sh = torch.from_numpy(rng.standard_normal((T, H)).astype(np.float32)).to(gpu)
    y0 = moe.moe_ffn_w4(x, ids, w, ex, out_dtype=torch.float32)
    moe.shared_expert_add(y0, sh, 1.25)
    y1 = moe.moe_ffn_w4(x, ids, w, ex, out_dtype=torch.float32, shared=sh, shared_gate=1.25)
    assert np.array_equal(y1.cpu().numpy(), y0.cpu().numpy())


def test_moe_ffn_fp8_shared_epilogue(gpu):
    from ccut.blocks import moe

    E, H, I, T, k = 8, 256, 384, 20, 2
    rng = np.random.default_rng(21)

    def fp8w(N, K):
        v = np.clip(rng.standard_normal((E, N, K)) * 0.02, -448, 448).astype(np.float32)
        w = torch.from_numpy(v).to(torch.float8_e4m3fn).view(torch.uint8).to(gpu)
        s = torch.from_numpy((np.abs(rng.standard_normal((E, N // 128, K // 128))) * 0.01 + 1e-3)
                             .astype(np.float32)).to(gpu)
        return w, s

    ex = moe.Fp8Experts.from_block(fp8w(I, H), fp8w(I, H), fp8w(H, I))
    x = torch.from_numpy(rng.standard_normal((T, H)).astype(np.float32)).to(gpu).to(torch.bfloat16)
    lg = torch.from_numpy(rng.standard_normal((T, E)).astype(np.float32)).to(gpu)
    w, ids = moe.topk_softmax(lg, k, True)
    sh = torch.from_numpy(rng.standard_normal((T, H)).astype(np.float32)).to(gpu)
    y0 = moe.moe_ffn_fp8(x, ids, w, ex, out_dtype=torch.float32)
    moe.shared_expert_add(y0, sh, 0.8)
    y1 = moe.moe_ffn_fp8(x, ids, w, ex, out_dtype=torch.float32, shared=sh, shared_gate=0.8)
    assert np.array_equal(y1.cpu().numpy(), y0.cpu().numpy())


def _awq_stack(rng, E, K, N, G):
    from oracle import awq as oawq

    q = rng.integers(0, 16, size=(E, K, N), dtype=np.uint8)
    z = rng.integers(0, 16, size=(E, K // G, N), dtype=np.uint8)
    s = (np.abs(rng.standard_normal((E, K // G, N))) * 0.01 + 1e-3).astype(np.float16)
    return (np.stack([oawq.pack(a) for a in q]), np.stack([oawq.pack(a) for a in z]), s)


@pytest.mark.parametrize("T,k,E", [(1, 2, 8), (5, 3, 8), (16, 6, 64), (40, 2, 8)])
def test_shared_expert_ffn_in_the_layer(gpu, T, k, E):
    """The shared expert's FFN as the stack's last expert (every token's slot
    k, weight shared_gate) through ccq_moe_w4_forward_shared: in-kernel
    routing for decode batches (T <= 16), the routing kernel above; the
    routed sum then shared_gate * shared_ffn(x), against the oracle's
    expert_ffn on dequantized weights (reference pipeline.py:145-190)."""
    from ccut.blocks import moe
    from oracle import awq as oawq
    from oracle import moe as omoe

    H, I, G = 256, 384, 128
    rng = np.random.default_rng(T * 100 + k * 10 + E)
    gate, up, down = _awq_stack(rng, E + 1, H, I, G), _awq_stack(rng, E + 1, H, I, G), _awq_stack(rng, E + 1, I, H, G)
    routed = [tuple(a[:E] for a in t) for t in (gate, up, down)]
    shared = tuple(tuple(a[E] for a in t) for t in (gate, up, down))
    to = lambda t: tuple(torch.from_numpy(np.ascontiguousarray(a)).to(gpu) for a in t)  # noqa: E731
    ex = moe.W4Experts.from_awq(to(routed[0]), to(routed[1]), to(routed[2]), G,
                                shared=tuple(to(s) for s in shared))
    assert ex.shared_expert and ex.num_experts == E + 1 and ex.routed_experts == E
    x = torch.from_numpy(rng.standard_normal((T, H)).astype(np.float32)).to(torch.bfloat16)
    lg = rng.standard_normal((T, E)).astype(np.float32)
    g = 0.625
    y = moe.moe_forward_w4(x.to(gpu), torch.from_numpy(lg).to(gpu), ex, top_k=k, out_dtype=torch.float32,
                           shared_gate=g).cpu().numpy()
    lut = {e: tuple(oawq.dequant(t[0][e], t[1][e], t[2][e], G) for t in (gate, up, down)) for e in range(E + 1)}
    w0, ids0 = omoe.topk_softmax(lg, k)
    xf = x.float().numpy()
    ref = omoe.moe_combine(xf, ids0, w0, lut.__getitem__) + np.float32(g) * omoe.expert_ffn(xf, *lut[E])
    assert np.max(np.abs(y - ref)) <= 2e-2 * np.max(np.abs(ref))
    # the ids-given form appends the same slot: the same kernels, the same result
    yi = moe.moe_ffn_w4(x.to(gpu), torch.from_numpy(ids0.astype(np.int64)).to(gpu), torch.from_numpy(w0).to(gpu), ex,
                        out_dtype=torch.float32, shared_gate=g).cpu().numpy()
    assert np.max(np.abs(yi - ref)) <= 2e-2 * np.max(np.abs(ref))
