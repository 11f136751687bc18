"""Expert index over safetensors shard headers (reference python/ccut/
experts/index.py:40-276): pattern parsing, segment offsets and shapes,
coverage check, cache.  Host only."""

from __future__ import annotations

import os

import numpy as np
import pytest

from _ckpt import PATTERN, write_fp8
from ccut.experts.index import ExpertIndex, build_expert_index, parse_expert_pattern, read_header


def test_pattern_plain_and_regex():
    rx = parse_expert_pattern(PATTERN)
    m = rx.match("model.layers.12.mlp.experts.255.down_proj.weight_scale")
    assert (m.group("layer"), m.group("expert"), m.group("proj")) == ("12", "255", "down")
    assert rx.match("xmodel.layers.1.mlp.experts.2.up_proj.weight") is None  # anchored at the start
    assert rx.match("model.layers.1.mlp.experts.x.up_proj.weight") is None
    rx2 = parse_expert_pattern(r"model\.layers\.{layer}\.mlp\.experts\.{expert}\.{proj}_proj")
    assert rx2.match("model.layers.3.mlp.experts.7.gate_proj.weight").group("proj") == "gate"


def test_index_segments_match_tensor_bytes(tmp_path):
    ref = write_fp8(tmp_path, L=2, E=3)
    idx = build_expert_index(tmp_path, PATTERN, num_layers=2, num_experts=3, top_k=2)
    assert idx.coverage() == (6, 6)
    assert idx.tensors_total == 2 * 3 * 6 + 2
    e = idx.get(1, 2)
    assert set(e.segments) == {f"{p}.{s}" for p in ("gate", "up", "down") for s in ("weight", "weight_scale")}
    assert e.shapes["gate.weight"] == (32, 64) and e.shapes["down.weight_scale"] == (64, 1)
    off, length, numel, dtype = e.segments["up.weight"]
    assert (length, numel, dtype) == (32 * 64, 32 * 64, "F8_E4M3")
    start, _ = read_header(tmp_path / e.shard)
    fd = os.open(tmp_path / e.shard, os.O_RDONLY)
    try:
        raw = np.frombuffer(os.pread(fd, length, start + off), dtype=np.uint8)
    finally:
        os.close(fd)
    assert np.array_equal(raw.reshape(32, 64), ref[(1, 2, "up")][0])
    assert e.bytes_total() == 3 * 32 * 64 + 2 * 32 * 2 + 64 * 2


def test_index_coverage_error_and_cache(tmp_path):
    write_fp8(tmp_path / "m", L=2, E=3)
    with pytest.raises(ValueError, match="covers 6 of 8"):
        build_expert_index(tmp_path / "m", PATTERN, num_layers=2, num_experts=4)
    cache = tmp_path / "cache" / "expert_index.json"
    a = build_expert_index(tmp_path / "m", PATTERN, 2, 3, cache_path=cache)
    assert cache.exists()
    b = build_expert_index(tmp_path / "m", PATTERN, 2, 3, cache_path=cache)
    assert b.build_ms == 0.0 and b.entries == a.entries  # served from the cache
    c = ExpertIndex.from_dict(a.to_dict())
    assert c.entries == a.entries and c.manifest_hash == a.manifest_hash
    # a changed checkpoint invalidates the cache
    write_fp8(tmp_path / "m", L=2, E=3, seed=5, H=128)
    d = build_expert_index(tmp_path / "m", PATTERN, 2, 3, cache_path=cache)
    assert d.get(0, 0).shapes["gate.weight"] == (32, 128)
