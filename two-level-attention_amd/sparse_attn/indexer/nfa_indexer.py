"""NFA indexer: the selector's validated configuration and dimension tables.

Reference interface: sparse_attn/indexer/nfa_indexer.py:22-154 (``NFAIndexer``).
The configuration checks are the reference's conditions with its own
``ValueError`` messages (:32-106), which are part of the error contract of
a drop-in; on top of them, a flag value whose selection semantics this path
does not implement (``arguments.UNIMPLEMENTED``) is rejected here, before any
launch, instead of being silently ignored.  The production selection itself
is ``nfa_layer_batch_selector.select_topk_for_layer_batched``.
"""
import operator

import torch

from ..arguments import UNIMPLEMENTED
from .tia_indexer import TIAIndexer

SUBSPACES = ('full', 'rope', 'nope', 'tail', 'random', 'highfreq', 'mla_rope')


def _count(name, value, *, allow_off=False):
    """An explicit integer count (``None`` when absent or ``off``)."""
    if value is None or (allow_off and isinstance(value, str)
                         and value.strip().lower() == 'off'):
        return None
    bad = ValueError(f'{name} 须为整数计数，收到 {value!r}')
    if isinstance(value, bool):
        raise bad
    try:
        return int(value) if isinstance(value, str) else operator.index(value)
    except (TypeError, ValueError, OverflowError) as exc:
        raise bad from exc


def _reject_unimplemented(args):
    for flag, (default, what) in UNIMPLEMENTED.items():
        value = getattr(args, flag, default)
        if value != default:
            raise ValueError(f'--{flag}={value!r} asks for {what}, which the HIP '
                             f'NFA selector does not implement (default {default!r})')


class NFAIndexer(TIAIndexer):
    """Immutable selector configuration and dimension maps."""

    def __init__(self, args, snapshot=None) -> None:
        super().__init__(args)
        self.layer_idx = None
        self.subspace = getattr(args, 'nfa_subspace', 'full')
        if self.subspace not in SUBSPACES:
            raise ValueError(f'nfa_subspace 非法取值: {self.subspace}')
        self.enable_subspace = (self.subspace in ('rope', 'nope', 'mla_rope')
                                or (bool(getattr(args, 'nfa_enable_subspace', True))
                                    and self.subspace != 'full'))
        self.l2_subspace = getattr(args, 'nfa_l2_subspace', 'same')
        if self.l2_subspace not in ('same', 'full'):
            raise ValueError(f'nfa_l2_subspace 非法取值: {self.l2_subspace}')
        self.head_dim = 192 if self.subspace == 'mla_rope' else 128
        self.far_method = getattr(args, 'nfa_far_method', 'minmax')
        self.near_method = getattr(args, 'nfa_near_method', 'avg')
        self.l2_quant = bool(getattr(args, 'nfa_l2_quant', False))
        self.sink_tokens = int(getattr(args, 'nfa_sink_tokens', 128))
        self._check_geometry(args)
        self._check_removed_paths(args)
        _reject_unimplemented(args)

    def _check_geometry(self, args):
        """Window, sink and the near-quota geometry (reference :39-95)."""
        if self.sink_tokens < 0:
            raise ValueError('nfa_sink_tokens 必须 >= 0')
        if self.sliding_window_size < 1:
            raise ValueError('nfa_swa_size 必须 >= 1')
        bs = int(args.tia_block_size)
        if self.sliding_window_size % bs:
            raise ValueError('nfa_swa_size 必须是 tia_block_size 的整数倍')
        raw_nt = getattr(args, 'nfa_near_tokens', None)
        nt_off = isinstance(raw_nt, str) and raw_nt.strip().lower() == 'off'
        self.nt_near_pages = _count('nfa_near_pages', getattr(args, 'nfa_near_pages', None))
        self.nt_near_tokens = _count('nfa_near_tokens', raw_nt, allow_off=True)
        self.nt_near_len = _count('nfa_near_len', getattr(args, 'nfa_near_len', None))
        nb, nt, nl = self.nt_near_pages, self.nt_near_tokens, self.nt_near_len
        if nb is None or nl is None:
            raise ValueError('生产 NFA 必须显式传 nfa_near_pages 与 nfa_near_len')
        if nt is None and not nt_off:
            raise ValueError("nfa_near_tokens 须传非负整数或 'off'")
        if nb < 0 or nl < 0:
            raise ValueError('nfa_near_pages/nfa_near_len 必须非负')
        if nb > args.tia_level1_topk:
            raise ValueError('nfa_near_pages 不可超过 tia_level1_topk')
        if nb * bs > nl:
            raise ValueError('网格约束破坏：nfa_near_pages * block_size <= nfa_near_len')
        protected = self.sink_tokens + self.sliding_window_size
        k2 = int(args.tia_level2_topk)
        if k2 < protected:
            raise ValueError('tia_level2_topk 不可小于 sink+swa')
        if nt_off:
            return
        if nt < 0:
            raise ValueError('nfa_near_tokens 必须非负')
        if nt > nb * bs:
            raise ValueError('网格约束破坏：nt <= nb * bs')
        if k2 - protected - nt < 0:
            raise ValueError('网格约束破坏：far = K2-sink-swa-nt >= 0')

    @staticmethod
    def _check_removed_paths(args):
        """Experiment paths the reference removed (reference :97-106)."""
        if getattr(args, 'nfa_proj_basis', None):
            raise ValueError('nfa_proj_basis 旧 HF Cache 路径已删除')
        if getattr(args, 'nfa_static_pair', False):
            raise ValueError('nfa_static_pair 旧 prefill 标定路径已删除')
        if (getattr(args, 'nfa_far_skip_backend', 'legacy') != 'legacy'
                or getattr(args, 'nfa_far_skip_cache', 'retain') != 'retain'):
            raise ValueError('仅支持 GraphReadyPagedRegionCache')

    @property
    def _sink_pool_lo_blk(self):
        return max(0, self.sink_tokens // self.args.tia_block_size)

    def _tail_indices(self, device):
        """Low-frequency RoPE dims: the top ``half/cmp_ratio`` of each half
        (for head_dim 256, the layout [NoPE 192 | RoPE 64]: 16 of each RoPE
        half)."""
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
