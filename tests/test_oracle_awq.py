"""Pin the oracle's AWQ restatement by the format's own definition
(AutoAWQ GEMM packing; absent from the reference, so parity against the
reference is unpinned and these invariants are the pin)."""

from __future__ import annotations

import numpy as np

from oracle import awq


def test_known_answer_word():
    # columns 0..7 hold 1..8; nibble i holds column AWQ_ORDER[i] = 0,2,4,6,1,3,5,7
    q = np.arange(1, 9, dtype=np.uint8)[None, :]
    word = awq.pack(q).view(np.uint32)[0, 0]
    assert word == 0x86427531
    assert awq.unpack(np.array([[0x86427531]], dtype=np.uint32).view(np.int32)).tolist() == [list(range(1, 9))]


def test_single_column_bit_positions():
    for j in range(8):
        q = np.zeros((1, 8), dtype=np.uint8)
        q[0, j] = 0xF
        w = int(awq.pack(q).view(np.uint32)[0, 0])
        assert w == 0xF << (4 * awq.AWQ_REVERSE_ORDER[j])


def test_pack_unpack_round_trip_random_words():
    rng = np.random.default_rng(0)
    words = rng.integers(0, 2 ** 32, size=(64, 32), dtype=np.uint64).astype(np.uint32).view(np.int32)
    assert np.array_equal(awq.pack(awq.unpack(words)), words)
    q = rng.integers(0, 16, size=(33, 48), dtype=np.uint8)
    assert np.array_equal(awq.unpack(awq.pack(q)), q)


def test_dequant_exact_and_grouped():
    rng = np.random.default_rng(1)
    K, N, G = 256, 40, 64
    q = rng.integers(0, 16, size=(K, N), dtype=np.uint8)
    z = rng.integers(0, 16, size=(K // G, N), dtype=np.uint8)
    s = (np.abs(rng.standard_normal((K // G, N))) * 0.01 + 1e-3).astype(np.float16)
    W = awq.dequant(awq.pack(q), awq.pack(z), s, G)
    g = np.arange(K) // G
    exact = (q.astype(np.float64) - z[g].astype(np.float64)) * s[g].astype(np.float64)
    assert np.array_equal(W.astype(np.float64), exact)  # exact in float32
    # a zero-point equal to q gives exactly zero
    W2 = awq.dequant(awq.pack(q), awq.pack(np.repeat(q[::G], 1, axis=0)), s, G)
    assert np.all(W2[::G] == 0)


def test_linear_matches_float64():
    rng = np.random.default_rng(2)
    K, N, G = 256, 64, 128
    q = rng.integers(0, 16, size=(K, N), dtype=np.uint8)
    z = rng.integers(0, 16, size=(K // G, N), dtype=np.uint8)
    s = (np.abs(rng.standard_normal((K // G, N))) * 0.01 + 1e-3).astype(np.float16)
    x = rng.standard_normal((3, K)).astype(np.float32)
    y = awq.linear(x, awq.pack(q), awq.pack(z), s, G)
    g = np.arange(K) // G
    W = (q - z[g].astype(np.float64)) * s[g].astype(np.float64)
    assert np.allclose(y, x.astype(np.float64) @ W, rtol=1e-5, atol=1e-5)
