"""Fused decode step of a whole Qwen3 / Llama decoder layer.

The reference speeds up the decode step of HF's Qwen3 decoder layer with
instance-level patches of its pieces: RMSNorm (patches/qwen3_rmsnorm_patch.py:
48-75), SiLU*up (patches/qwen3_mlp_silu_patch.py:42-75) and q/k RoPE
(ops/qwen3_rope_triton.py:118, called from patches/qwen3_attn_patch.py:53-57),
leaving about 20 separate launches per layer.  This patch replaces the
layer's decode forward with seven launches over the same HF parameters:

    [input norm + q/k/v projections]  nfa_decode_linear (3 segments)
    [q/k norm + RoPE]                 nfa_qk_norm_rope_decode
    [selection + K/V write]           nfa_select_layer
    [sparse attention]                nfa_sparse_attn_decode
    [o_proj + residual]               nfa_decode_linear (residual epilogue)
    [post norm + gate/up + SiLU*up]   nfa_decode_linear (SiLU-gate epilogue)
    [down_proj + residual]            nfa_decode_linear (residual epilogue)

Prefill, batches above the kernels' limits and other dtypes run the layer's
original forward (whose attention is the patched paged-cache forward).
"""
from types import MethodType

import torch

_ORIG = '_nfa_decode_layer_original_forward'


def _decoder_layer_classes():
    from transformers.models.llama.modeling_llama import LlamaDecoderLayer
    from transformers.models.qwen3.modeling_qwen3 import Qwen3DecoderLayer
    return (Qwen3DecoderLayer, LlamaDecoderLayer)


def is_silu(act):
    """HF's SiLU activation module (``SiLUActivation``) or torch's."""
    return (isinstance(act, torch.nn.SiLU) or type(act).__name__ == 'SiLUActivation') \
        and not getattr(act, 'inplace', False)


def _fusable(layer, hidden_states, cache):
    from ..cache import GraphReadyPagedRegionCache
    from ..ops.decode_fused import LINEAR_MAX_ROWS
    attn = layer.self_attn
    return (isinstance(cache, GraphReadyPagedRegionCache)
            and hasattr(attn, 'indexer')
            and hidden_states.dim() == 3 and hidden_states.shape[1] == 1
            and hidden_states.shape[0] <= LINEAR_MAX_ROWS
            and hidden_states.dtype == torch.bfloat16 and hidden_states.is_cuda
            and hidden_states.is_contiguous()
            and attn.q_proj.bias is None and attn.k_proj.bias is None
            and attn.v_proj.bias is None and attn.o_proj.bias is None
            and is_silu(layer.mlp.act_fn)
            and layer.mlp.gate_proj.bias is None and layer.mlp.down_proj.bias is None)


def nfa_decode_layer_forward(self, hidden_states, attention_mask=None,
                             position_ids=None, past_key_values=None,
                             use_cache=False, position_embeddings=None, **kwargs):
    """Decoder-layer forward: seven fused launches for one decode token per
    row, the original forward otherwise."""
    if not _fusable(self, hidden_states, past_key_values):
        return getattr(self, _ORIG)(
            hidden_states, attention_mask=attention_mask, position_ids=position_ids,
            past_key_values=past_key_values, use_cache=use_cache,
            position_embeddings=position_embeddings, **kwargs)
    from ..indexer.nfa_layer_batch_selector import select_topk_for_layer_batched
    from ..ops.decode_fused import decode_linear, qk_norm_rope_decode
    from ..ops.paged_region_kernels_nfa import decode_graph_ready

    self._nfa_fused_calls = getattr(self, '_nfa_fused_calls', 0) + 1
    attn, mlp, cache = self.self_attn, self.mlp, past_key_values
    b, _, hidden = hidden_states.shape
    d = attn.head_dim
    hq = attn.q_proj.weight.shape[0] // d
    hkv = attn.k_proj.weight.shape[0] // d
    x = hidden_states.view(b, hidden)
    q, k, v = decode_linear(
        x, (attn.q_proj.weight, attn.k_proj.weight, attn.v_proj.weight),
        norm_weight=self.input_layernorm.weight,
        eps=self.input_layernorm.variance_epsilon)
    cos, sin = position_embeddings
    q_norm = getattr(attn, 'q_norm', None)
    k_norm = getattr(attn, 'k_norm', None)
    q, k = qk_norm_rope_decode(
        q, k, None if q_norm is None else q_norm.weight,
        None if k_norm is None else k_norm.weight, cos, sin,
        q_norm.variance_epsilon if q_norm is not None else 0.0,
        hq=hq, hkv=hkv, head_dim=d)
    layer_idx = attn.layer_idx
    slots = cache.slot_mapping_for_layer(layer_idx)[:b]
    mode = getattr(attn.indexer.args, 'nfa_operator_mode', 'off')
    if mode == 'off':
        select_topk_for_layer_batched(
            cache, layer_idx, cache.active_req_ids, q, attention=attn,
            decode_write=(k.view(b, hkv, 1, d), v.view(b, hkv, 1, d), slots))
        o = decode_graph_ready(
            attn, q, cache, gather_indices=cache.gather_indices_for_layer(layer_idx),
            visible_lens=cache.visible_lens_for_layer(layer_idx),
            query_to_req=cache.query_to_req_buf)
    elif mode in ('serial', 'overlap'):
        from .qwen3_attn_patch import disjoint_regions_attention
        o = disjoint_regions_attention(attn, q, k.view(b, hkv, 1, d),
                                        v.view(b, hkv, 1, d), cache, slots,
                                        mode == 'overlap')
    else:
        raise ValueError(f'unknown NFA operator mode: {mode}')
    h1, = decode_linear(o.view(b, hq * d), (attn.o_proj.weight,), residual=x)
    a, = decode_linear(h1, (mlp.gate_proj.weight, mlp.up_proj.weight),
                       norm_weight=self.post_attention_layernorm.weight,
                       eps=self.post_attention_layernorm.variance_epsilon,
                       silu_gate=True)
    h2, = decode_linear(a, (mlp.down_proj.weight,), residual=h1)
    return h2.view(b, 1, hidden)


def register_decode_layer_patch(model, expected=None):
    """Patch every Qwen3 / Llama decoder layer; returns the count.  With
    ``expected`` a different count raises instead of half-patching."""
    classes = _decoder_layer_classes()
    n = 0
    for module in model.modules():
        if isinstance(module, classes):
            if not hasattr(module, _ORIG):
                setattr(module, _ORIG, module.forward)
            module.forward = MethodType(nfa_decode_layer_forward, module)
            n += 1
    if expected is not None and n != expected:
        raise RuntimeError(f'decode layer patch count {n} != expected {expected}')
    return n


def unregister_decode_layer_patch(model):
    n = 0
    for module in model.modules():
        original = getattr(module, _ORIG, None)
        if original is not None:
            module.forward = original
            delattr(module, _ORIG)
            n += 1
    return n
