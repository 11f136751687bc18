"""Expert pipeline, index and reader on the GPU operators (reference
``python/ccut/experts/``)."""

from ccut.experts.index import ExpertEntry, ExpertIndex, build_expert_index, load_expert_index, parse_expert_pattern
from ccut.experts.pipeline import ExpertPipeline, PipelineMetrics, RouteHistory
from ccut.experts.reader import ExpertReader, ExpertRing, RingFullError

__all__ = ["ExpertEntry", "ExpertIndex", "ExpertPipeline", "ExpertReader", "ExpertRing", "PipelineMetrics",
           "RingFullError", "RouteHistory", "build_expert_index", "load_expert_index", "parse_expert_pattern"]
