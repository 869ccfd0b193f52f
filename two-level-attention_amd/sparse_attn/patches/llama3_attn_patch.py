"""Llama-3.1 attention forward on the graph-ready paged cache.

Reference: the v1 ``sparse_attn/patches/llama3_attn_patch.py:30-261`` (kept in the
reference's archived v1 source tree) patches ``LlamaAttention`` for the same
two-level decode.  This forward shares the Qwen3 one's prefill and decode
steps; Llama has no per-head q/k RMSNorm.
"""
from typing import Optional

import torch

from .qwen3_attn_patch import (_check_cache, _decode_fusable, _rope, decode_qkv,
                               nfa_decode_attention, paged_prefill_attention)


def llama3_attn_forward(
    self,
    hidden_states: torch.Tensor,
    position_embeddings,
    attention_mask: Optional[torch.Tensor],
    past_key_values=None,
    cache_position=None,
    **kwargs,
):
    """Llama attention with the single GraphReadyPagedRegionCache path."""
    _check_cache(self, past_key_values)
    input_shape = hidden_states.shape[:-1]
    if _decode_fusable(hidden_states):
        q, k, v = decode_qkv(self, hidden_states, position_embeddings)
        return nfa_decode_attention(self, q, k, v, past_key_values, input_shape), None
    hidden_shape = (*input_shape, -1, self.head_dim)
    query_states = self.q_proj(hidden_states).view(hidden_shape).transpose(1, 2)
    key_states = self.k_proj(hidden_states).view(hidden_shape).transpose(1, 2)
    value_states = self.v_proj(hidden_states).view(hidden_shape).transpose(1, 2)
    cos, sin = position_embeddings
    query_states, key_states = _rope(self, query_states, key_states, cos, sin)

    if input_shape[1] != 1:
        return paged_prefill_attention(
            self, query_states, key_states, value_states, attention_mask,
            past_key_values, input_shape, **kwargs)
    return nfa_decode_attention(
        self, query_states, key_states, value_states, past_key_values,
        input_shape), None
