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
a hipGraph.

Absorbed form (``register_patch(..., mla='absorbed')``, a latent cache): the
arena holds one row per token, ``[kv_a_layernorm(c) | k_pe]`` (kv_lora_rank +
64 dims, 1.15 KB at DeepSeek-V2-Lite's 512 + 64 instead of 16 x (192 + 128)
x 2 B = 10 KB expanded).  Every expanded head holds the same k_pe, so the
selection -- per query head, on the RoPE dims -- is the expanded path's bit
for bit when each head selects from the shared rows; attention runs in the
latent space, q_h = [W_uk,h^T q_nope,h | q_pe,h] against the rows and
out_h = W_uv,h (sum_i p_i c_i), which equals the expanded attention up to
rounding.  The reference builds no absorbed decode; this is its algebraic
equivalent over the same selections.

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


def _latent_parts(module, hidden_states, position_embeddings):
    """Per-head q_nope [B, H, S, nope] and post-RoPE q_pe [B, H, S, rope],
    c [B, 1, S, rank] and k_pe [B, 1, S, rope], and the latent rows
    [B, S, rank + rope] = [kv_a_layernorm(c) | k_pe]."""
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
    c = module.kv_a_layernorm(kv_nope).view(b, 1, s, module.kv_lora_rank)
    k_pe = k_pe.view(b, 1, s, module.qk_rope_head_dim)
    q_pe, k_pe = rope(q_pe, k_pe, position_embeddings.to(q_pe.device))
    rows = torch.cat((c[:, 0], k_pe[:, 0]), dim=-1)
    return q_nope, q_pe, c, k_pe, rows


def absorbed_weights(module):
    """The head-wise halves of kv_b_proj: W_uk [H, nope, rank] and W_uv
    [H, v, rank], contiguous (cached until the weight changes)."""
    w = module.kv_b_proj.weight
    held = module.__dict__.get('_nfa_absorbed')
    if held is not None and held[0] is w and held[1] == w._version:
        return held[2], held[3]
    heads = module.num_heads
    wv = w.detach().view(heads, module.qk_nope_head_dim + module.v_head_dim,
                         module.kv_lora_rank)
    w_uk = wv[:, :module.qk_nope_head_dim, :].contiguous()
    w_uv = wv[:, module.qk_nope_head_dim:, :].contiguous()
    module._nfa_absorbed = (w, w._version, w_uk, w_uv)
    return w_uk, w_uv


def absorbed_decode_attention(module, q_nope, q_pe, rows, cache, batch):
    """One decode token per row on a latent arena: write the latent row,
    select per query head on the RoPE dims, attend in the latent space and
    up-project each head's result.  Returns the o_proj output [B, 1, hidden]."""
    from ..indexer.nfa_layer_batch_selector import select_topk_for_layer_batched
    from ..ops.paged_region_kernels import sparse_mla_attention_gather

    layer_idx = module.layer_idx
    w_uk, w_uv = absorbed_weights(module)
    heads = module.num_heads
    # q_abs = W_uk^T q_nope per head: [H, B, nope] x [H, nope, rank] (both
    # operands contiguous)
    q_abs = torch.bmm(q_nope[:, :, 0].transpose(0, 1).contiguous(), w_uk)
    q_lat = torch.cat((q_abs.transpose(0, 1), q_pe[:, :, 0]), dim=-1).contiguous()
    keys = rows.view(batch, 1, 1, -1).contiguous()
    slot_mapping = cache.slot_mapping_for_layer(layer_idx)[:batch]
    select_topk_for_layer_batched(
        cache, layer_idx, cache.active_req_ids, q_lat, attention=module,
        decode_write=(keys, None, slot_mapping))
    # out_h = W_uv,h (sum_i p_i c_i), the up-projection fused into the kernel
    out = sparse_mla_attention_gather(
        cache.layers[layer_idx], q_lat, cache.gather_indices_for_layer(layer_idx),
        cache.visible_lens_for_layer(layer_idx), cache.query_to_req_buf,
        scale=module.scaling, w_uv=w_uv,
        workspace=cache.__dict__.setdefault('_nfa_selector_workspace', {}))
    return module.o_proj(out.reshape(batch, 1, heads * module.v_head_dim))


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
    cache = past_key_values
    if getattr(cache, 'latent', False):
        return _absorbed_forward(self, hidden_states, attention_mask, cache,
                                 position_embeddings, input_shape, **kwargs)
    query, key, value = _expanded_qkv(self, hidden_states, position_embeddings)
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


def _absorbed_forward(module, hidden_states, attention_mask, cache,
                      position_embeddings, input_shape, **kwargs):
    """A latent arena: decode through the absorbed path; a prompt writes its
    latent rows and is attended densely by the module's own attention over
    the expanded heads (as the unpatched module does)."""
    from .qwen3_attn_patch import _attention_interface
    q_nope, q_pe, c, k_pe, rows = _latent_parts(module, hidden_states,
                                                position_embeddings)
    if input_shape[1] == 1:
        return absorbed_decode_attention(module, q_nope, q_pe, rows[:, 0], cache,
                                         input_shape[0]), None
    request_id = cache.active_request_id
    if request_id is None:
        raise ValueError('GraphReady prefill requires an active request id')
    cache.write_prefill(module.layer_idx, request_id, rows.unsqueeze(1).contiguous(), None)
    query = torch.cat((q_nope, q_pe), dim=-1)
    key, value = module.expand_kv(c, k_pe)
    attention = _attention_interface(module)
    out, weights = attention(module, query, key, value, attention_mask, dropout=0.0,
                             scaling=module.scaling, **kwargs)
    return module.o_proj(out.reshape(*input_shape, -1).contiguous()), weights
