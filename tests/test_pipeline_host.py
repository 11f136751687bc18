"""Host logic of the expert pipeline (reference python/ccut/experts/
pipeline.py:34-84): route history and metrics, no GPU."""

from __future__ import annotations

from ccut.experts.pipeline import PipelineMetrics, RouteHistory


def test_route_history_predicts_most_frequent_in_window():
    h = RouteHistory(window=3)
    assert h.predict(4) == []
    h.record([5, 1, 2])
    h.record([1, 2])
    h.record([2, 7])
    assert h.predict(2) == [2, 1]  # 2 seen 3 times, 1 twice
    assert h.predict(10)[:2] == [2, 1] and set(h.predict(10)) == {1, 2, 5, 7}
    h.record([9])  # the window drops [5, 1, 2]
    assert h.predict(1) == [2] and 5 not in h.predict(10)


def test_metrics_ratios_and_dict():
    m = PipelineMetrics()
    assert m.overlap_ratio() == 0.0 and m.speculative_accept_rate() == 0.0
    m.compute_ns, m.overlap_ns, m.speculative_total, m.speculative_correct = 200, 50, 4, 3
    d = m.to_dict()
    assert d["overlap_ratio"] == 0.25 and d["spec_accept_rate"] == 0.75
    assert set(d) == {"compute_ns", "prefetch_ns", "overlap_ns", "overlap_ratio", "steps", "spec_accept_rate",
                      "ring_hits", "ring_misses", "expert_timeouts", "dropped_assignments"}


def test_kv_mode_and_bytes(tmp_path):
    """reference python/ccut/quant/kv.py:37-67 (host logic)."""
    import json

    import pytest

    from ccut.quant.kv import KVQuantMode, kv_bytes_per_token, resolve_kv_dtype

    assert resolve_kv_dtype(None) == "bf16" and resolve_kv_dtype(None, "FP8") == "fp8"
    (tmp_path / "config.json").write_text(json.dumps({"text_config": {"kv_cache_scheme": {"type": "fp8_e4m3"}}}))
    assert resolve_kv_dtype(tmp_path) == KVQuantMode.FP8
    (tmp_path / "config.json").write_text(json.dumps({"kv_cache_scheme": None}))
    assert resolve_kv_dtype(tmp_path, "auto") == KVQuantMode.BF16
    with pytest.raises(ValueError):
        resolve_kv_dtype(tmp_path, "int8")
    assert kv_bytes_per_token(4, 128, "bf16") == 2048 and kv_bytes_per_token(4, 128, "fp8") == 1032
    with pytest.raises(ValueError):
        kv_bytes_per_token(4, 128, "int4")
