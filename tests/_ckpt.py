"""Small synthetic MoE checkpoints in safetensors (two shards and a
model.safetensors.index.json) for the expert index / reader tests."""

from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import torch
from safetensors.torch import save_file

PATTERN = "model.layers.{layer}.mlp.experts.{expert}.{proj}_proj"


def write_fp8(d: Path, L=2, E=3, H=64, I=32, seed=0) -> dict:
    """FP8 e4m3 experts [out, in] with per-row BF16 scales [out, 1] (the
    Ornith layout); layer l in shard l+1, plus a non-expert tensor.  Returns
    {(l, e, proj): (codes u8 [out, in], scale f32 [out])}."""
    rng = np.random.default_rng(seed)
    shards, wm, ref = [{}, {}], {}, {}
    for l in range(L):
        for e in range(E):
            for proj, (o, i) in (("gate", (I, H)), ("up", (I, H)), ("down", (H, I))):
                w = torch.from_numpy((rng.standard_normal((o, i)) * 40).astype(np.float32)).to(torch.float8_e4m3fn)
                s = torch.from_numpy((np.abs(rng.standard_normal((o, 1))) * 0.01 + 1e-3).astype(np.float32))
                s = s.to(torch.bfloat16)
                name = f"model.layers.{l}.mlp.experts.{e}.{proj}_proj"
                shards[l % 2][name + ".weight"] = w
                shards[l % 2][name + ".weight_scale"] = s
                ref[(l, e, proj)] = (w.view(torch.uint8).numpy().copy(), s.float().numpy().reshape(-1))
        shards[l % 2][f"model.layers.{l}.mlp.gate.weight"] = torch.zeros((E, H), dtype=torch.bfloat16)
    return _save(d, shards, ref)


def write_awq(d: Path, L=1, E=4, H=256, I=128, G=128, seed=0) -> dict:
    """AWQ experts: qweight int32 [K, N/8], qzeros int32 [K/G, N/8], scales
    F16 [K/G, N] per projection (K = in, N = out).  Returns
    {(l, e, proj): (qweight, qzeros, scales) numpy}."""
    from oracle import awq as oawq

    rng = np.random.default_rng(seed)
    shards, ref = [{}, {}], {}
    for l in range(L):
        for e in range(E):
            for proj, (K, N) in (("gate", (H, I)), ("up", (H, I)), ("down", (I, H))):
                q = rng.integers(0, 16, size=(K, N), dtype=np.uint8)
                z = rng.integers(0, 16, size=(K // G, N), dtype=np.uint8)
                s = (np.abs(rng.standard_normal((K // G, N))) * 0.01 + 1e-3).astype(np.float16)
                qw, qz = oawq.pack(q), oawq.pack(z)
                name = f"model.layers.{l}.mlp.experts.{e}.{proj}_proj"
                sh = shards[e % 2]
                sh[name + ".qweight"] = torch.from_numpy(qw.view(np.int32).copy())
                sh[name + ".qzeros"] = torch.from_numpy(qz.view(np.int32).copy())
                sh[name + ".scales"] = torch.from_numpy(s.copy())
                ref[(l, e, proj)] = (qw, qz, s)
    return _save(d, shards, ref)


def _save(d: Path, shards, ref) -> dict:
    d.mkdir(parents=True, exist_ok=True)
    wm = {}
    for i, sh in enumerate(shards):
        fn = f"model-{i + 1:05d}-of-{len(shards):05d}.safetensors"
        save_file(sh, str(d / fn))
        wm.update({k: fn for k in sh})
    (d / "model.safetensors.index.json").write_text(json.dumps({"metadata": {}, "weight_map": wm}))
    return ref


def write_fp8_block(d: Path, L=1, E=4, H=256, I=256, seed=0, scale_name="weight_scale_inv") -> dict:
    """Block-FP8 experts: e4m3 [out, in] from clip(N(0, 0.02), +-448) and
    float32 128x128 block scales [ceil(out/128), ceil(in/128)] named
    ``scale_name``.  Returns {(l, e, proj): (codes u8 [out, in], scales f32)}."""
    rng = np.random.default_rng(seed)
    shards, ref = [{}, {}], {}
    for l in range(L):
        for e in range(E):
            for proj, (o, i) in (("gate", (I, H)), ("up", (I, H)), ("down", (H, I))):
                v = np.clip(rng.standard_normal((o, i)) * 0.02, -448, 448).astype(np.float32)
                w = torch.from_numpy(v).to(torch.float8_e4m3fn)
                s = (np.abs(rng.standard_normal((-(-o // 128), -(-i // 128)))) * 0.5 + 0.25).astype(np.float32)
                name = f"model.layers.{l}.mlp.experts.{e}.{proj}_proj"
                shards[e % 2][name + ".weight"] = w
                shards[e % 2][name + "." + scale_name] = torch.from_numpy(s)
                ref[(l, e, proj)] = (w.view(torch.uint8).numpy().copy(), s)
    return _save(d, shards, ref)


def write_ct_int4(d: Path, L=1, E=4, H=256, I=128, G=128, seed=0) -> dict:
    """int4 group experts in the AWQ GEMM packing under compressed-tensors'
    group tensor names: ``.weight`` int32 [K, N/8], ``.zero_points`` int32
    [K/G, N/8], ``.scales`` F16 [K/G, N].  Returns {(l, e, proj): (qweight,
    qzeros, scales)}."""
    from oracle import awq as oawq

    rng = np.random.default_rng(seed)
    shards, ref = [{}, {}], {}
    for l in range(L):
        for e in range(E):
            for proj, (K, N) in (("gate", (H, I)), ("up", (H, I)), ("down", (I, H))):
                q = rng.integers(0, 16, size=(K, N), dtype=np.uint8)
                z = rng.integers(0, 16, size=(K // G, N), dtype=np.uint8)
                s = (np.abs(rng.standard_normal((K // G, N))) * 0.01 + 1e-3).astype(np.float16)
                qw, qz = oawq.pack(q), oawq.pack(z)
                name = f"model.layers.{l}.mlp.experts.{e}.{proj}_proj"
                sh = shards[e % 2]
                sh[name + ".weight"] = torch.from_numpy(qw.view(np.int32).copy())
                sh[name + ".zero_points"] = torch.from_numpy(qz.view(np.int32).copy())
                sh[name + ".scales"] = torch.from_numpy(s.copy())
                ref[(l, e, proj)] = (qw, qz, s)
    return _save(d, shards, ref)
