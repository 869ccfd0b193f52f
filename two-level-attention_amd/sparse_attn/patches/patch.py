"""Attach the NFA indexer and the paged-cache attention forward to a model.

Reference: sparse_attn/patches/patch.py:28-132 (``register_patch``).  Same
contract: every Qwen3 attention module (and, as in the reference's v1 tree,
every Llama and DeepSeek-V2 attention module) gets ``module.indexer`` built
from ``args`` and
its ``forward`` replaced on the instance (the original is kept in
``_nfa_original_forward``); the number of patched modules is returned, and a
sparse method that matches no module raises instead of silently running dense
attention.  GLM-4.7 (absorbed latent attention) is not built here.
"""
from types import MethodType

import torch.nn as nn

from ..indexer import indexer_type_dict
from ..indexer.nfa_indexer import NFAIndexer


def _reject_removed_cache_args(args):
    backend = getattr(args, 'nfa_far_skip_backend', 'legacy')
    cache = getattr(args, 'nfa_far_skip_cache', 'retain')
    if backend != 'legacy' or cache != 'retain':
        raise ValueError(
            'far-skip/static/batch cache paths have been removed; '
            'only GraphReadyPagedRegionCache is supported '
            '(nfa_far_skip_backend=legacy, nfa_far_skip_cache=retain)')


def _attention_classes():
    """(class, forward) pairs of the attention modules this build patches."""
    from transformers.models.deepseek_v2.modeling_deepseek_v2 import DeepseekV2Attention
    from transformers.models.llama.modeling_llama import LlamaAttention
    from transformers.models.qwen3.modeling_qwen3 import Qwen3Attention
    from .deepseek_v2_attn_patch import deepseek_v2_attn_forward
    from .llama3_attn_patch import llama3_attn_forward
    from .qwen3_attn_patch import qwen3_attn_forward
    return ((Qwen3Attention, qwen3_attn_forward),
            (LlamaAttention, llama3_attn_forward),
            (DeepseekV2Attention, deepseek_v2_attn_forward))


def _key_dim(module):
    """Per-head key width the selector sees (DeepSeek-V2: the expanded
    nope + rope key)."""
    if hasattr(module, 'qk_head_dim'):
        return module.qk_head_dim
    return module.head_dim


def register_patch(model: nn.Module, args, snapshot=None,
                   rmsnorm_decode: bool = False,
                   mlp_silu_decode: bool = False,
                   decode_layers: bool = False,
                   mla: str = 'expanded') -> int:
    """Patch the model's attention modules; returns how many were patched.

    ``rmsnorm_decode`` / ``mlp_silu_decode`` also move the decode-step
    RMSNorm and MLP onto fused HIP kernels; ``decode_layers`` runs the whole
    decoder layer's decode step as seven fused launches.  ``mla`` chooses how
    a DeepSeek-V2 model's caches hold its latent attention: ``expanded``
    (per-head keys and values, as the reference's patch) or ``absorbed``
    (one latent row per token, selection and attention in the latent space;
    no reference counterpart).
    """
    _reject_removed_cache_args(args)
    if mla not in ('expanded', 'absorbed'):
        raise ValueError(f'unknown MLA layout {mla!r} (expanded or absorbed)')
    indexer_type = indexer_type_dict.get(args.method, None)
    if args.method != 'none' and indexer_type is None:
        raise ValueError(f'not support {args.method}')
    if args.method != 'none' and any(
            type(m).__name__ == 'Glm4MoeLiteAttention' for m in model.modules()):
        raise ValueError('GLM-4.7 latent attention is not built in this package')

    n_patched = 0
    if indexer_type is not None:
        classes = _attention_classes()
        for name, module in model.named_modules():
            forward = next((f for c, f in classes if isinstance(module, c)), None)
            if forward is None:
                continue
            if snapshot is not None and indexer_type is NFAIndexer:
                module.indexer = indexer_type(args, snapshot=snapshot)
            else:
                module.indexer = indexer_type(args)
            module.indexer.head_dim = _key_dim(module)
            if hasattr(module, 'layer_idx'):
                module.indexer.layer_idx = module.layer_idx
            if not hasattr(module, '_nfa_original_forward'):
                module._nfa_original_forward = module.forward
            module.forward = MethodType(forward, module)
            n_patched += 1
    model_type = getattr(getattr(model, 'config', None), 'model_type', None)
    if mla == 'absorbed':
        if model_type != 'deepseek_v2':
            raise ValueError('the absorbed MLA layout needs a DeepSeek-V2 model')
        if getattr(args, 'nfa_subspace', None) != 'mla_rope':
            raise ValueError('the absorbed MLA layout selects on --nfa_subspace mla_rope')
    if model_type == 'deepseek_v2':
        # read by build_frozen_cache: the arena layout of the model's caches
        model._nfa_mla = mla
    if (rmsnorm_decode or mlp_silu_decode or decode_layers) and n_patched:
        if model_type not in ('qwen3', 'llama'):
            raise ValueError('fused decode patches cover Qwen3 and Llama models')
        layers = model.config.num_hidden_layers
        norms_per_layer = 4 if model_type == 'qwen3' else 2
        if rmsnorm_decode:
            from .qwen3_rmsnorm_patch import register_rmsnorm_patch
            register_rmsnorm_patch(model, expected=layers * norms_per_layer + 1)
        if mlp_silu_decode:
            from .qwen3_mlp_silu_patch import register_mlp_silu_patch
            register_mlp_silu_patch(model, expected=layers)
        if decode_layers:
            from .decode_layer_patch import register_decode_layer_patch
            register_decode_layer_patch(model, expected=layers)
    if args.method != 'none' and n_patched == 0:
        kinds = sorted({type(m).__name__ for _, m in model.named_modules()})
        raise RuntimeError(
            f'method={args.method!r} but the model has no Qwen3Attention, '
            f'LlamaAttention or DeepseekV2Attention module to patch (patched=0); '
            f'running on would label dense output as sparse. Module types: '
            f'{kinds[:8]}')
    return n_patched


def unregister_patch(model: nn.Module) -> int:
    """Restore the original attention forwards (and undo the fused decode
    patches); returns how many attention modules were restored."""
    from .decode_layer_patch import unregister_decode_layer_patch
    from .qwen3_mlp_silu_patch import unregister_mlp_silu_patch
    from .qwen3_rmsnorm_patch import unregister_rmsnorm_patch
    unregister_decode_layer_patch(model)
    unregister_mlp_silu_patch(model)
    unregister_rmsnorm_patch(model)
    n = 0
    for module in model.modules():
        original = getattr(module, '_nfa_original_forward', None)
        if original is None:
            continue
        module.forward = original
        del module._nfa_original_forward
        n += 1
    return n
