"""Continuous-batching scheduler for graph decode."""
from .scheduler import ContinuousBatchScheduler, greedy_next_tokens
