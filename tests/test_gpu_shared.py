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
