"""DeepSeek-V2 attention forward on the graph-ready paged cache.

Reference: the archived v1 tree's ``sparse_attn/patches/deepseek_v2_attn_patch.py``
(agent_doc/results/frozen_near_far_v1_16_independent005_20261030/
ai_supervision/independent_final_20261030T0715/source/v1/) and the
``mla_rope`` dims of ``indexer/nfa_indexer.py:133-134``.  Same contract: the
latent attention is expanded per head -- K = [k_nope (128) | k_pe (64)] = 192
dims, V = 128 dims, H = HKV (a GQA group of one) -- and the two-level
selection scores the RoPE part of the key, dims 128..191 (``--nfa_subspace
mla_rope``); attention consumes q.k over all 192 dims and p.v over the 128
value dims.  Here the expanded K/V of every token live in the paged arena
(KV heads = query heads, head_dim_k 192, head_dim_v 128): a prompt is written
with ``write_prefill`` and attended densely by the model's own attention; a
decode step selects from its current query and attends to the selection with
the sparse gather attention, both through the HIP kernels and capturable into
a hipGraph.  The absorbed form (selection and attention in the 512 + 64
latent space) has no reference semantics and is not built.

The projections follow transformers' ``DeepseekV2Attention`` (q_proj or the
q LoRA pair, kv_a_proj_with_mqa, kv_a_layernorm, the module's own
``expand_kv`` and the module-level ``apply_rotary_emb``), so the arena holds
exactly the keys and values the unpatched module attends to.
"""
import sys

import torch

from .qwen3_attn_patch import _check_cache, nfa_decode_attention


def _expanded_qkv(module, hidden_states, position_embeddings):
    """Per-head query [B, H, S, 192], key [B, H, S, 192] and value
    [B, H, S, 128] of the module's latent attention, post-RoPE."""
    rope = getattr(sys.modules[type(module).__module__], 'apply_rotary_emb', None)
    if rope is None:
        raise RuntimeError(f'{type(module).__module__} has no apply_rotary_emb')
    b, s = hidden_states.shape[:2]
    if module.q_lora_rank is None:
        q = module.q_proj(hidden_states)
    else:
        q = module.q_b_proj(module.q_a_layernorm(module.q_a_proj(hidden_states)))
    q = q.view(b, s, -1, module.qk_head_dim).transpose(1, 2)
    q_nope, q_pe = torch.split(q, [module.qk_nope_head_dim, module.qk_rope_head_dim],
                               dim=-1)
    latent = module.kv_a_proj_with_mqa(hidden_states)
    kv_nope, k_pe = torch.split(latent, [module.kv_lora_rank, module.qk_rope_head_dim],
                                dim=-1)
    k_nope = module.kv_a_layernorm(kv_nope).view(b, 1, s, module.kv_lora_rank)
    k_pe = k_pe.view(b, 1, s, module.qk_rope_head_dim)
    q_pe, k_pe = rope(q_pe, k_pe, position_embeddings.to(q_pe.device))
    query = torch.cat((q_nope, q_pe), dim=-1)
    key, value = module.expand_kv(k_nope, k_pe)
    return query, key, value


def deepseek_v2_attn_forward(
    self,
    hidden_states: torch.Tensor,
    attention_mask=None,
    past_key_values=None,
    position_embeddings=None,
    **kwargs,
):
    """DeepSeek-V2 attention with the single GraphReadyPagedRegionCache path."""
    from .qwen3_attn_patch import _attention_interface
    _check_cache(self, past_key_values)
    input_shape = hidden_states.shape[:-1]
    query, key, value = _expanded_qkv(self, hidden_states, position_embeddings)
    cache = past_key_values
    if input_shape[1] == 1:
        return nfa_decode_attention(self, query, key.contiguous(), value.contiguous(),
                                    cache, input_shape), None
    request_id = cache.active_request_id
    if request_id is None:
        raise ValueError('GraphReady prefill requires an active request id')
    cache.write_prefill(self.layer_idx, request_id, key.contiguous(), value.contiguous())
    attention = _attention_interface(self)
    out, weights = attention(self, query, key, value, attention_mask, dropout=0.0,
                             scaling=self.scaling, **kwargs)
    return self.o_proj(out.reshape(*input_shape, -1).contiguous()), weights
