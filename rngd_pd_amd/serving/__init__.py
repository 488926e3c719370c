"""Serving-side pieces of the decode worker: continuous scheduling onto the
paged cache and request prefetch (serving/cluster.py:350-467,832-1134)."""
from .scheduler import ContinuousScheduler, Prefetcher

__all__ = ["ContinuousScheduler", "Prefetcher"]
