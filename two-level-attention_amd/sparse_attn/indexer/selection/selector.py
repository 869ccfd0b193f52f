"""Compact decode selection: sorted unique token ids + per-head counts.

Reference: sparse_attn/indexer/selection/selector.py:6-66.
"""
from typing import NamedTuple

import torch


class TokenSelection(NamedTuple):
    """``indices`` [B, Hkv, K] int32, the first ``counts[b, h]`` entries are
    sorted, unique and valid (the rest are 0); ``counts`` [B, Hkv] int32."""
    indices: torch.Tensor
    counts: torch.Tensor

    def valid(self):
        width = self.indices.shape[-1]
        return torch.arange(width, device=self.indices.device) < self.counts[..., None]

    def to_mask(self, capacity):
        """Dense [B, Hkv, capacity] bool mask of the selected ids."""
        mask = torch.zeros((*self.indices.shape[:-1], capacity + 1),
                           dtype=torch.bool, device=self.indices.device)
        ids = torch.where(self.valid(), self.indices.long(), capacity)
        mask.scatter_(-1, ids, True)
        return mask[..., :capacity]


def canonical_selection(ids, valid, capacity, width=None):
    """Sort, de-duplicate and compact ``ids[valid & 0 <= ids < capacity]``."""
    if ids.ndim != 3 or valid.shape != ids.shape or capacity < 1:
        raise ValueError(
            'selection requires [B,Hkv,K] ids/valid and positive capacity, got '
            f'ids.shape={tuple(ids.shape)} valid.shape={tuple(valid.shape)} '
            f'capacity={capacity}')
    width = ids.shape[-1] if width is None else min(width, ids.shape[-1])
    keep = valid & (ids >= 0) & (ids < capacity)
    ordered = torch.where(keep, ids, capacity).sort(-1).values
    prev = torch.cat((torch.full_like(ordered[..., :1], -1), ordered[..., :-1]), -1)
    first = (ordered < capacity) & (ordered != prev)
    packed = torch.where(first, ordered, capacity).sort(-1).values[..., :width]
    count = (packed < capacity).sum(-1, dtype=torch.int32)
    return TokenSelection(
        torch.where(packed < capacity, packed, 0).to(torch.int32).contiguous(),
        count.contiguous())
