"""Timing helpers."""
from .benchmarking import benchmark_repeat, time_ms

__all__ = ["benchmark_repeat", "time_ms"]
