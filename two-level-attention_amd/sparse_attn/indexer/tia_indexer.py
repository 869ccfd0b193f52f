"""TIA indexer base: window size, L2 compression ratio and 4-bit key quant.

Reference: sparse_attn/indexer/tia_indexer.py:10-31.
"""
import torch

from .base import Indexer


class TIAIndexer(Indexer):

    def __init__(self, args) -> None:
        super().__init__(args)
        self.group_size = None
        self.sliding_window_size = getattr(args, 'nfa_swa_size', 128)
        self.cmp_ratio = args.tia_level2_cmp_ratio
        self.enable_async = getattr(args, 'tia_enable_async_topk', False)
        self.prev_mask = None

    @staticmethod
    def min_max_per_token_quant(x: torch.Tensor, num_bits: int = 4) -> torch.Tensor:
        """Quantise-dequantise each row of ``x`` to ``num_bits`` with its own
        min/max, computed op by op in the dtype of ``x``."""
        hi = x.amax(dim=-1, keepdim=True)
        lo = x.amin(dim=-1, keepdim=True)
        levels = 2 ** num_bits - 1
        step = (hi - lo).clamp(min=1e-9) / levels
        shift = -lo
        code = torch.clamp(torch.round((x + shift) / step), 0, levels)
        return code * step - shift

    def clear(self):
        self.prev_mask = None
