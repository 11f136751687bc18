"""Pin the oracle's FP8 block-scaled restatement (absent from the reference:
parity unpinned there; pinned here by torch's RNE e4m3fn cast and the
scheme's invariants)."""

from __future__ import annotations

import numpy as np
import torch

from oracle import fp8_block as fb
from oracle.ref_quant import FP8_TABLE


def test_rne_encode_matches_torch_cast():
    rng = np.random.default_rng(0)
    mids = ((FP8_TABLE[0:0x7E].astype(np.float64) + FP8_TABLE[1:0x7F]) / 2).astype(np.float32)
    vals = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * 100,
        rng.standard_normal(5000).astype(np.float32) * 0.005,
        mids, -mids,                      # ties: to even
        np.array([0.0, -0.0, 448.0, -448.0, 2.0 ** -10, 3 * 2.0 ** -11], dtype=np.float32),
    ])
    vals = np.clip(vals, -448, 448)
    got = fb.float32_to_fp8_rne(vals)
    ref = torch.from_numpy(vals).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(got, ref)


def test_act_quant_invariants():
    rng = np.random.default_rng(1)
    x = (rng.standard_normal((9, 384)) * rng.random((9, 1)) * 10).astype(np.float32)
    x[3, 128:256] = 0.0  # an all-zero block
    q, s = fb.act_quant(x)
    assert q.shape == x.shape and s.shape == (9, 3)
    dec = FP8_TABLE[q].astype(np.float64)
    assert np.all(np.abs(dec) <= 448)
    # the block maximum maps to +-448 exactly
    xb = np.abs(x.reshape(9, 3, 128))
    am = xb.argmax(2)
    for t in range(9):
        for b in range(3):
            if xb[t, b].max() > 0:
                assert abs(dec[t, b * 128 + am[t, b]]) == 448.0
    assert np.all(q[3, 128:256] == 0)
    # round trip within half an e4m3 ulp of the scaled value (relative 2^-4)
    back = fb.act_dequant(q, s)
    err = np.abs(back - x)
    tol = np.maximum(np.abs(x) * 2.0 ** -4, np.repeat(s, 128, axis=1) * 2.0 ** -10)
    assert np.all(err <= tol + 1e-30)


def test_block_dequant_loop():
    rng = np.random.default_rng(2)
    w = rng.integers(0, 0x7E, size=(256, 384), dtype=np.uint8)
    s = rng.random((2, 3)).astype(np.float32)
    W = fb.block_dequant(w, s)
    for n in (0, 127, 128, 255):
        for k in (0, 127, 128, 383):
            assert W[n, k] == np.float32(float(FP8_TABLE[w[n, k]]) * float(s[n // 128, k // 128]))


def test_to_bf16_rne():
    x = np.array([1.0, 1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, -3.0], dtype=np.float32)
    got = fb.to_bf16(x)
    ref = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    assert np.array_equal(got, ref)


def _f64_linear_loop(x, w, s_w):
    """y[t, n] = sum_k deq(q[t,k]) s_a[t, k//128] * fp8(w[n,k]) s_w[n//128, k//128]
    element by element in float64 (q, s_a from the oracle's act_quant, which
    the tests above pin)."""
    q, sa = fb.act_quant(x)
    T, K = x.shape
    N = w.shape[0]
    y = np.zeros((T, N), dtype=np.float64)
    for t in range(T):
        for n in range(N):
            acc = 0.0
            for k in range(K):
                acc += (float(FP8_TABLE[q[t, k]]) * float(sa[t, k // 128])) * \
                       (float(FP8_TABLE[w[n, k]]) * float(s_w[n // 128, k // 128]))
            y[t, n] = acc
    return y


def _tiny_block_weights(rng, N, K):
    w = rng.integers(0, 0x7E, size=(N, K), dtype=np.uint8) | (rng.integers(0, 2, size=(N, K)) * 0x80).astype(np.uint8)
    s = (rng.random((-(-N // 128), K // 128)) + 0.5).astype(np.float32)
    return w, s


def test_linear_against_float64_loop():
    """Non-square N != K, distinct block scales: a transposed operand, a
    swapped scale index or a dropped activation scale all fail."""
    rng = np.random.default_rng(5)
    x = (rng.standard_normal((3, 256)) * np.array([[1.0], [7.0], [0.01]])).astype(np.float32)
    w, s = _tiny_block_weights(rng, 130, 256)  # N = 130: a partial last row block
    got = fb.linear(x, w, s)
    ref = _f64_linear_loop(x, w, s)
    assert got.shape == (3, 130)
    assert np.allclose(got, ref, rtol=1e-5, atol=1e-5 * np.abs(ref).max())


def test_expert_ffn_against_float64_loop():
    """down(silu(gate) * up) with gate/up [I, H] and down [H, I] (row = output
    channel), the intermediate in full precision: float64 loops."""
    rng = np.random.default_rng(6)
    H, I, T = 256, 384, 2
    x = rng.standard_normal((T, H)).astype(np.float32)
    wg, sg = _tiny_block_weights(rng, I, H)
    wu, su = _tiny_block_weights(rng, I, H)
    wd, sd = _tiny_block_weights(rng, H, I)
    # keep the products moderate: scale the weight scales down
    sg, su, sd = sg * 1e-3, su * 1e-3, sd * 1e-3
    got = fb.expert_ffn(x, wg, sg, wu, su, wd, sd)
    g = _f64_linear_loop(x, wg, sg)
    u = _f64_linear_loop(x, wu, su)
    h = g / (1.0 + np.exp(-g)) * u
    ref = np.zeros((T, H))
    for t in range(T):
        for n in range(H):
            ref[t, n] = sum(h[t, i] * float(FP8_TABLE[wd[n, i]]) * float(sd[n // 128, i // 128]) for i in range(I))
    assert got.shape == (T, H)
    assert np.abs(got - ref).max() <= 1e-4 * np.abs(ref).max()
    # the intermediate is not re-quantized: a re-quantized one is visibly off
    hq = fb.act_dequant(*fb.act_quant(h.astype(np.float32)))
    requant = hq @ fb.block_dequant(wd, sd).T
    assert np.abs(requant - ref).max() > 10 * np.abs(got - ref).max()
