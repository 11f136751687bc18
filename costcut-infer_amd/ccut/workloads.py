"""Seeded synthetic inputs of the benchmark workloads (no checkpoints exist
offline).  Distributions:

* AWQ linear: ``q``, ``z`` uniform in 0..15, scales ``|N(0,1)| * 0.01 + 1e-3``
  (fp16), activations ``N(0,1)``;
* MoE routing: logits ``N(0,1)`` (plus a per-expert bias ``N(0, 2)`` for the
  skewed router), softmax, top-k;
* FP8 block weights: ``clip(N(0, 0.02), +-448)`` cast to e4m3fn, float32
  ``128x128`` block scales ``|N(0,1)| * 0.01 + 1e-3``;
* FP8 per-row weights (the reference checkpoint's expert format):
  ``clip(N(0, 0.02), +-448)`` cast to e4m3fn, one scale per output row
  ``|N(0,1)| * 0.01 + 1e-3`` rounded to BF16 as the checkpoint stores it.

Everything is drawn from a ``torch.Generator`` on the target device so the
large expert sets are generated in HBM.
"""

from __future__ import annotations

import torch

from ccut.quant.awq import pack_awq


def gen(seed: int, device) -> torch.Generator:
    return torch.Generator(device=device).manual_seed(int(seed))


def awq_linear(K: int, N: int, group: int = 128, seed: int = 0, device="cuda",
               scale_dtype: torch.dtype = torch.float16):
    """``(qweight [K, N/8] i32, qzeros [K/G, N/8] i32, scales [K/G, N])``."""
    g = gen(seed, device)
    q = torch.randint(0, 16, (K, N), generator=g, device=device, dtype=torch.int32)
    z = torch.randint(0, 16, (K // group, N), generator=g, device=device, dtype=torch.int32)
    s = (torch.randn((K // group, N), generator=g, device=device).abs() * 0.01 + 1e-3).to(scale_dtype)
    return pack_awq(q), pack_awq(z), s


def awq_experts(E: int, K: int, N: int, group: int = 128, seed: int = 0, device="cuda",
                scale_dtype: torch.dtype = torch.float16):
    """Stacked ``(qweight [E, K, N/8], qzeros [E, K/G, N/8], scales [E, K/G, N])``."""
    qw = torch.empty((E, K, N // 8), dtype=torch.int32, device=device)
    qz = torch.empty((E, K // group, N // 8), dtype=torch.int32, device=device)
    sc = torch.empty((E, K // group, N), dtype=scale_dtype, device=device)
    for e in range(E):
        a, b, c = awq_linear(K, N, group, seed * 100003 + e, device, scale_dtype)
        qw[e], qz[e], sc[e] = a, b, c
    return qw, qz, sc


def activations(T: int, H: int, seed: int = 0, device="cuda", dtype: torch.dtype = torch.bfloat16):
    return torch.randn((T, H), generator=gen(seed, device), device=device).to(dtype)


def router_logits(T: int, E: int, seed: int = 0, device="cuda", skew_std: float = 0.0):
    g = gen(seed, device)
    lg = torch.randn((T, E), generator=g, device=device)
    if skew_std > 0:
        lg = lg + torch.randn((1, E), generator=g, device=device) * skew_std
    return lg.float().contiguous()


def fp8_block_weights(E: int, N: int, K: int, seed: int = 0, device="cuda", block: int = 128):
    """``(w [E, N, K] e4m3fn bytes as uint8, s_w [E, N/128, K/128] f32)``."""
    g = gen(seed, device)
    w = torch.empty((E, N, K), dtype=torch.uint8, device=device)
    for e in range(E):
        v = (torch.randn((N, K), generator=g, device=device) * 0.02).clamp_(-448, 448)
        w[e] = v.to(torch.float8_e4m3fn).view(torch.uint8)
    s = torch.randn((E, N // block, K // block), generator=g, device=device).abs() * 0.01 + 1e-3
    return w, s.float().contiguous()


def fp8_row_weights(E: int, N: int, K: int, seed: int = 0, device="cuda"):
    """``(w [E, N, K] e4m3fn bytes as uint8, s [E, N] f32 holding BF16 values)``."""
    g = gen(seed, device)
    w = torch.empty((E, N, K), dtype=torch.uint8, device=device)
    for e in range(E):
        v = (torch.randn((N, K), generator=g, device=device) * 0.02).clamp_(-448, 448)
        w[e] = v.to(torch.float8_e4m3fn).view(torch.uint8)
    s = torch.randn((E, N), generator=g, device=device).abs() * 0.01 + 1e-3
    return w, s.to(torch.bfloat16).float().contiguous()
