"""Qwen3 attention forward on the graph-ready paged cache.

Reference: sparse_attn/patches/qwen3_attn_patch.py:22-196 (``qwen3_attn_forward``).
Same contract: a prompt (more than one token per row) is written into the
paged arena with ``write_prefill`` and attended densely by the model's own
attention implementation; a decode step (one token per row) selects this
layer's tokens from the current post-RoPE query with
``select_topk_for_layer_batched`` — which also writes the current K/V — and
attends to them with the sparse gather attention.  For bf16 decode the q/k
RMSNorm and RoPE run as one launch (the reference's qwen3_decode_rope,
ops/qwen3_rope_triton.py:118, plus the two norms).  Every device step is a
HIP kernel with fixed buffers, so the decode forward can be captured into a
hipGraph.  ``--nfa_operator_mode serial|overlap`` attends the protected
sink/SWA set and the selected middle apart and merges the two softmax
states (reference :123-195); an unknown mode raises ``ValueError``.
"""
from typing import Optional

import torch


def _attention_interface(module):
    from transformers.modeling_utils import ALL_ATTENTION_FUNCTIONS
    from transformers.models.qwen3.modeling_qwen3 import eager_attention_forward
    impl = module.config._attn_implementation
    getter = getattr(ALL_ATTENTION_FUNCTIONS, 'get_interface', None)
    if getter is not None:
        return getter(impl, eager_attention_forward)
    return ALL_ATTENTION_FUNCTIONS.get(impl, eager_attention_forward)


def _check_cache(module, cache):
    from ..cache import GraphReadyPagedRegionCache
    from ..ops.selector_options import validate_selector_options
    if getattr(module, 'layer_idx', 0) == 0:
        capacity = cache.get_max_cache_shape() if cache is not None else None
        validate_selector_options(
            capacity if isinstance(capacity, int) and capacity > 0 else None)
    if not isinstance(cache, GraphReadyPagedRegionCache):
        raise ValueError(
            'NFA requires GraphReadyPagedRegionCache; use prefill_frozen_request')


def paged_prefill_attention(module, query_states, key_states, value_states,
                            attention_mask, cache, input_shape, **kwargs):
    """Write the prompt K/V into the arena, then dense causal attention."""
    request_id = cache.active_request_id
    if request_id is None:
        raise ValueError('GraphReady prefill requires an active request id')
    cache.write_prefill(module.layer_idx, request_id, key_states, value_states)
    attention = _attention_interface(module)
    attn_output, attn_weights = attention(
        module, query_states, key_states, value_states, attention_mask,
        dropout=0.0 if not module.training else module.attention_dropout,
        scaling=module.scaling,
        sliding_window=getattr(module, 'sliding_window', None),
        **kwargs)
    return module.o_proj(attn_output.reshape(*input_shape, -1).contiguous()), attn_weights


def nfa_decode_attention(module, query_states, key_states, value_states, cache,
                         input_shape):
    """One decode token per row: select, write the current K/V, attend.

    ``query_states`` ``[B, HQ, 1, D]`` and ``key_states`` / ``value_states``
    ``[B, HKV, 1, D]`` are post-RoPE.  Returns the o_proj output
    ``[B, 1, hidden]``.  ``--nfa_operator_mode`` (reference
    qwen3_attn_patch.py:103-195): ``off`` selects the union and attends it
    in one pass; ``serial`` and ``overlap`` attend the protected sink/SWA set
    and the selected middle apart and merge the two softmax states
    (protected first), ``overlap`` running the protected part on a side
    stream while the selection runs.
    """
    from ..indexer.nfa_layer_batch_selector import select_topk_for_layer_batched
    from ..ops.paged_region_kernels_nfa import decode_graph_ready

    operator_mode = getattr(module.indexer.args, 'nfa_operator_mode', 'off')
    batch = input_shape[0]
    layer_idx = module.layer_idx
    slot_mapping = cache.slot_mapping_for_layer(layer_idx)[:batch]
    q_flat = query_states[:, :, 0]
    if operator_mode == 'off':
        select_topk_for_layer_batched(
            cache, layer_idx, cache.active_req_ids, q_flat, attention=module,
            decode_write=(key_states, value_states, slot_mapping))
        result = decode_graph_ready(
            module, q_flat, cache,
            gather_indices=cache.gather_indices_for_layer(layer_idx),
            visible_lens=cache.visible_lens_for_layer(layer_idx),
            query_to_req=cache.query_to_req_buf)
    elif operator_mode in ('serial', 'overlap'):
        result = disjoint_regions_attention(
            module, q_flat, key_states, value_states, cache, slot_mapping,
            operator_mode == 'overlap')
    else:
        raise ValueError(f'unknown NFA operator mode: {operator_mode}')
    return module.o_proj(result.reshape(*input_shape, -1).contiguous())


def disjoint_regions_attention(module, q_flat, key_states, value_states, cache,
                                slot_mapping, overlap):
    """Protected ∥ middle attention of one layer (reference
    qwen3_attn_patch.py:123-195): the current K/V is written first, so both
    arms read the same committed arena; serial and overlap differ only in
    the stream of the protected arm, the merge order is the same."""
    from ..indexer.nfa_layer_batch_selector import select_topk_for_layer_batched
    from ..ops.paged_region_kernels import (sparse_paged_attention_gather_partial,
                                            sparse_paged_attention_regions_combine)
    from ..ops.paged_region_kernels_nfa import build_protected_gather, split_gather_buffers

    layer_idx = module.layer_idx
    batch = q_flat.shape[0]
    cache.write_decode(layer_idx, key_states, value_states, slot_mapping)
    prot_gather, prot_lens, mid_gather, mid_lens = split_gather_buffers(
        cache, layer_idx, batch)
    workspace = cache.__dict__.setdefault('_nfa_selector_workspace', {})
    q_flat = q_flat if q_flat.is_contiguous() else q_flat.contiguous()
    layer = cache.layers[layer_idx]

    def protected_partial():
        build_protected_gather(cache, layer_idx, module.indexer, prot_gather, prot_lens)
        return sparse_paged_attention_gather_partial(
            layer, q_flat, prot_gather, prot_lens, cache.query_to_req_buf,
            scale=module.scaling, workspace=workspace, name='protected', nsplit=1)

    def middle_partial():
        select_topk_for_layer_batched(
            cache, layer_idx, cache.active_req_ids, q_flat, attention=module,
            middle_only=True, selection_output=(mid_gather, mid_lens))
        return sparse_paged_attention_gather_partial(
            layer, q_flat, mid_gather, mid_lens, cache.query_to_req_buf,
            scale=module.scaling, workspace=workspace, name='middle', nsplit=4)

    if overlap:
        primitives = workspace.get('nfa_overlap_primitives')
        if primitives is None:
            if torch.cuda.is_current_stream_capturing():
                raise RuntimeError('overlap streams must be warmed before capture')
            # default priority, like every stream of this package
            primitives = (torch.cuda.Stream(device=q_flat.device), torch.cuda.Event(),
                          torch.cuda.Event())
            workspace['nfa_overlap_primitives'] = primitives
        side, fork, join = primitives
        main = torch.cuda.current_stream()
        fork.record(main)
        side.wait_event(fork)
        with torch.cuda.stream(side):
            prot_parts = protected_partial()
            join.record(side)
        mid_parts = middle_partial()
        main.wait_event(join)
        # the protected arm's buffers are reused by the next layer's side
        # launches only after this join
    else:
        prot_parts = protected_partial()
        mid_parts = middle_partial()
    return sparse_paged_attention_regions_combine(
        q_flat, prot_parts, mid_parts, workspace=workspace)


def _rope(module, query_states, key_states, cos, sin):
    from transformers.models.qwen3.modeling_qwen3 import apply_rotary_pos_emb
    return apply_rotary_pos_emb(query_states, key_states, cos, sin)


def decode_qkv(module, hidden_states, position_embeddings):
    """q/k/v of one decode token per row: projections, then per-head q/k
    RMSNorm (when the module has q_norm/k_norm) and RoPE in one launch.
    Returns ``q`` [B, HQ, 1, D], ``k``/``v`` [B, HKV, 1, D], post-RoPE."""
    from ..ops.decode_fused import qk_norm_rope_decode
    b = hidden_states.shape[0]
    d = module.head_dim
    q = module.q_proj(hidden_states).view(b, -1)
    k = module.k_proj(hidden_states).view(b, -1)
    v = module.v_proj(hidden_states).view(b, -1, 1, d)
    hq, hkv = q.shape[1] // d, k.shape[1] // d
    q_norm = getattr(module, 'q_norm', None)
    k_norm = getattr(module, 'k_norm', None)
    cos, sin = position_embeddings
    q, k = qk_norm_rope_decode(
        q, k, None if q_norm is None else q_norm.weight,
        None if k_norm is None else k_norm.weight, cos, sin,
        0.0 if q_norm is None else q_norm.variance_epsilon,
        hq=hq, hkv=hkv, head_dim=d)
    return q.view(b, hq, 1, d), k.view(b, hkv, 1, d), v


def _decode_fusable(hidden_states):
    return (hidden_states.dim() == 3 and hidden_states.shape[1] == 1
            and hidden_states.dtype == torch.bfloat16 and hidden_states.is_cuda)


def qwen3_attn_forward(
    self,
    hidden_states: torch.Tensor,
    position_embeddings,
    attention_mask: Optional[torch.Tensor],
    past_key_values=None,
    cache_position=None,
    **kwargs,
):
    """Qwen3 attention with the single GraphReadyPagedRegionCache path."""
    _check_cache(self, past_key_values)
    input_shape = hidden_states.shape[:-1]
    if _decode_fusable(hidden_states):
        q, k, v = decode_qkv(self, hidden_states, position_embeddings)
        return nfa_decode_attention(self, q, k, v, past_key_values, input_shape), None
    hidden_shape = (*input_shape, -1, self.head_dim)
    query_states = self.q_norm(
        self.q_proj(hidden_states).view(hidden_shape)).transpose(1, 2)
    key_states = self.k_norm(
        self.k_proj(hidden_states).view(hidden_shape)).transpose(1, 2)
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
