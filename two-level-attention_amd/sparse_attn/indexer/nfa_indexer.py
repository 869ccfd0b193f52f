"""NFA indexer: validated configuration and subspace dimension tables.

Reference: sparse_attn/indexer/nfa_indexer.py:22-154.  Validation covers the
same conditions and raises ``ValueError`` like the reference; the production
selection itself is ``nfa_layer_batch_selector.select_topk_for_layer_batched``.
"""
import operator

import torch

from .tia_indexer import TIAIndexer

SUBSPACES = ('full', 'rope', 'nope', 'tail', 'random', 'highfreq', 'mla_rope')


def _count(name, value, *, allow_off=False):
    if allow_off and isinstance(value, str) and value.strip().lower() == 'off':
        return None
    if value is None:
        return None
    if isinstance(value, bool):
        raise ValueError(f'{name} must be an integer count, got {value!r}')
    try:
        return int(value) if isinstance(value, str) else operator.index(value)
    except (TypeError, ValueError, OverflowError) as exc:
        raise ValueError(f'{name} must be an integer count, got {value!r}') from exc


class NFAIndexer(TIAIndexer):
    """Immutable selector configuration and dimension maps."""

    def __init__(self, args, snapshot=None) -> None:
        super().__init__(args)
        self.layer_idx = None
        self.subspace = getattr(args, 'nfa_subspace', 'full')
        if self.subspace not in SUBSPACES:
            raise ValueError(f'invalid nfa_subspace: {self.subspace}')
        self.enable_subspace = (bool(getattr(args, 'nfa_enable_subspace', True))
                                and self.subspace != 'full')
        if self.subspace in ('rope', 'nope', 'mla_rope'):
            self.enable_subspace = True
        self.l2_subspace = getattr(args, 'nfa_l2_subspace', 'same')
        if self.l2_subspace not in ('same', 'full'):
            raise ValueError(f'invalid nfa_l2_subspace: {self.l2_subspace}')
        self.head_dim = 192 if self.subspace == 'mla_rope' else 128
        self.far_method = getattr(args, 'nfa_far_method', 'minmax')
        self.near_method = getattr(args, 'nfa_near_method', 'avg')
        self.l2_quant = bool(getattr(args, 'nfa_l2_quant', False))
        self.sink_tokens = int(getattr(args, 'nfa_sink_tokens', 128))
        if self.sink_tokens < 0:
            raise ValueError('nfa_sink_tokens must be >= 0')
        if self.sliding_window_size < 1:
            raise ValueError('nfa_swa_size must be >= 1')
        block_size = int(args.tia_block_size)
        if self.sliding_window_size % block_size:
            raise ValueError('nfa_swa_size must be a multiple of tia_block_size')

        near_tokens_raw = getattr(args, 'nfa_near_tokens', None)
        self.nt_near_pages = _count('nfa_near_pages',
                                    getattr(args, 'nfa_near_pages', None))
        self.nt_near_tokens = _count('nfa_near_tokens', near_tokens_raw,
                                     allow_off=True)
        self.nt_near_len = _count('nfa_near_len',
                                  getattr(args, 'nfa_near_len', None))
        near_tokens_off = (isinstance(near_tokens_raw, str)
                           and near_tokens_raw.strip().lower() == 'off')
        if self.nt_near_pages is None or self.nt_near_len is None:
            raise ValueError('NFA needs explicit nfa_near_pages and nfa_near_len')
        if self.nt_near_tokens is None and not near_tokens_off:
            raise ValueError("nfa_near_tokens must be a non-negative integer or 'off'")
        if self.nt_near_pages < 0 or self.nt_near_len < 0:
            raise ValueError('nfa_near_pages / nfa_near_len must be >= 0')
        if self.nt_near_pages > args.tia_level1_topk:
            raise ValueError('nfa_near_pages cannot exceed tia_level1_topk')
        if self.nt_near_pages * block_size > self.nt_near_len:
            raise ValueError('geometry: nfa_near_pages * block_size must be <= nfa_near_len')
        k2 = int(args.tia_level2_topk)
        if k2 < self.sink_tokens + self.sliding_window_size:
            raise ValueError('tia_level2_topk cannot be smaller than sink + swa')
        if not near_tokens_off:
            if self.nt_near_tokens < 0:
                raise ValueError('nfa_near_tokens must be >= 0')
            if self.nt_near_tokens > self.nt_near_pages * block_size:
                raise ValueError('geometry: nfa_near_tokens must be <= near_pages * block_size')
            if k2 - self.sink_tokens - self.sliding_window_size - self.nt_near_tokens < 0:
                raise ValueError('geometry: K2 - sink - swa - nfa_near_tokens must be >= 0')
        if getattr(args, 'nfa_proj_basis', None):
            raise ValueError('nfa_proj_basis (projection basis) is not supported')
        if getattr(args, 'nfa_static_pair', False):
            raise ValueError('nfa_static_pair (prefill pair calibration) is not supported')
        if getattr(args, 'nfa_far_skip_backend', 'legacy') != 'legacy':
            raise ValueError('only the graph-ready paged cache is supported')
        if getattr(args, 'nfa_far_skip_cache', 'retain') != 'retain':
            raise ValueError('only the graph-ready paged cache is supported')

    @property
    def _sink_pool_lo_blk(self):
        return max(0, self.sink_tokens // self.args.tia_block_size)

    def _tail_indices(self, device):
        """Low-frequency RoPE dims: the top ``half/cmp_ratio`` of each half."""
        if self.head_dim == 256:
            return torch.cat((torch.arange(208, 224, device=device),
                              torch.arange(240, 256, device=device)))
        half = self.head_dim // 2
        delta = half // self.cmp_ratio
        return torch.cat((torch.arange(half - delta, half, device=device),
                          torch.arange(self.head_dim - delta, self.head_dim,
                                       device=device)))

    def _subspace_indices(self, device):
        key = (self.head_dim, self.subspace, self.cmp_ratio, str(device))
        cached = getattr(self, '_dims_cache', None)
        if cached is not None and cached[0] == key:
            return cached[1]
        if self.subspace == 'rope':
            out = torch.arange(0, 64, device=device)
        elif self.subspace == 'nope':
            out = (torch.arange(0, 64, device=device) if self.head_dim == 256
                   else torch.arange(64, 128, device=device))
        elif self.subspace == 'mla_rope':
            out = torch.arange(128, 192, device=device)
        elif self.subspace == 'random':
            gen = torch.Generator().manual_seed(20261002)
            out = torch.randperm(128, generator=gen)[:32].sort().values.to(device)
        elif self.subspace == 'highfreq':
            delta = 64 // self.cmp_ratio
            out = torch.tensor(list(range(delta)) + list(range(64, 64 + delta)),
                               device=device)
        else:
            out = self._tail_indices(device)
        self._dims_cache = (key, out)
        return out

    def _qat_indices(self, device):
        return self._tail_indices(device)
