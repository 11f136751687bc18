"""Expert pipeline step on the GPU operators (reference ``python/ccut/experts/``)."""

from ccut.experts.pipeline import ExpertPipeline, PipelineMetrics, RouteHistory

__all__ = ["ExpertPipeline", "PipelineMetrics", "RouteHistory"]
