"""Compact token-selection contract."""
from .selector import TokenSelection, canonical_selection

__all__ = ['TokenSelection', 'canonical_selection']
