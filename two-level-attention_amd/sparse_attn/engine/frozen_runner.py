"""Prefill, freeze and graph decode of one request on the paged cache.

Reference: sparse_attn/engine/frozen_runner.py:62-90 (``build_frozen_cache``),
:93-155 (``prefill_frozen_request``) and :158-300 (``decode_frozen_request``).
Same lifecycle: dense prefill straight into the arena, per-layer far/near
skip decisions frozen into the cache, then greedy decode steps through the
graph runner with asynchronous token receipts.

Skip decisions come from a static gate decision (``static_gate``), from the
request-time gate (``config``, a ``GateConfig``: the near/far attention mass
of the last prompt rows, profiled in every layer during the prefill by one
HIP kernel), or, with neither, are all False (every region kept).
"""
from contextlib import contextmanager
from dataclasses import replace

import torch

from ..cache.paged_region_cache import GraphReadyPagedRegionCache, RequestPhase
from ..policies.frozen_gate import decide_regions, profile_regions, region_present
from ..scheduler.scheduler import greedy_next_tokens


@contextmanager
def capture_profiles(model, geometry, config):
    """Profile each layer's prefill attention once (reference
    engine/frozen_runner.py:15-35): the model's attention function is wrapped
    for the duration; the wrapped call still computes the attention."""
    from transformers.modeling_utils import ALL_ATTENTION_FUNCTIONS
    impl = model.config._attn_implementation
    original = ALL_ATTENTION_FUNCTIONS[impl]
    profiles = {}

    def profiled(module, query, key, value, *args, **kwargs):
        layer_idx = module.layer_idx
        if layer_idx in profiles:
            raise ValueError('multiple prefill chunks unsupported')
        profiles[layer_idx] = profile_regions(
            query, key, geometry, rows=config.rows,
            scale=kwargs.get('scaling', module.scaling))
        return original(module, query, key, value, *args, **kwargs)

    ALL_ATTENTION_FUNCTIONS[impl] = profiled
    try:
        yield profiles
    finally:
        ALL_ATTENTION_FUNCTIONS[impl] = original


@contextmanager
def _request_failure_guard(cache, request_id):
    try:
        yield
    except Exception:
        if cache.request_phases.get(request_id) != RequestPhase.FAILED:
            cache.transition_request(request_id, RequestPhase.FAILED)
        raise


def _model_dims(model):
    """(config, kv heads, key dim, value dim, latent) of the paged arena: a
    DeepSeek-V2 model stores its latent attention expanded per head (key =
    nope + rope dims, one kv head per query head), or -- patched with
    ``mla='absorbed'`` -- as latent rows (one kv head of kv_lora_rank + rope
    dims, the values their first kv_lora_rank dims)."""
    cfg = model.config
    if getattr(cfg, 'model_type', None) == 'deepseek_v2':
        if getattr(model, '_nfa_mla', 'expanded') == 'absorbed':
            return (cfg, 1, cfg.kv_lora_rank + cfg.qk_rope_head_dim, cfg.kv_lora_rank,
                    True)
        return (cfg, cfg.num_attention_heads, cfg.qk_nope_head_dim + cfg.qk_rope_head_dim,
                cfg.v_head_dim, False)
    head_dim = getattr(cfg, 'head_dim', None) or cfg.hidden_size // cfg.num_attention_heads
    return (cfg, cfg.num_key_value_heads, head_dim,
            int(getattr(cfg, 'v_head_dim', None) or head_dim), False)


def build_frozen_cache(model, geometry, sequence_capacity, *, max_requests=1,
                       max_visible_len=None, physical_pages=None):
    """Fixed-address cache for ``max_requests`` requests of up to
    ``sequence_capacity`` prompt tokens plus ``geometry.max_new_tokens``.
    ``physical_pages`` sizes the K/V arena when the requests together need
    fewer pages than ``max_requests`` full-length ones (ragged batches)."""
    page = geometry.page
    max_blocks = (sequence_capacity + geometry.max_new_tokens + page - 1) // page + 8
    if max_visible_len is None:
        max_visible_len = sequence_capacity + geometry.max_new_tokens + 16
    if physical_pages is None:
        physical_pages = max_requests * max_blocks + 8
    cfg, hkv, head_dim, head_dim_v, latent = _model_dims(model)
    return GraphReadyPagedRegionCache(
        cfg.num_hidden_layers, geometry, max_requests=max_requests,
        max_physical_pages=physical_pages, max_blocks=max_blocks,
        max_visible_len=max_visible_len, max_query_tokens=max_requests,
        num_kv_heads=hkv, num_query_heads=cfg.num_attention_heads,
        head_dim_k=head_dim, head_dim_v=head_dim_v, dtype=model.dtype,
        device=next(model.parameters()).device, latent=latent)


def _prefill_mask_arg(model):
    if getattr(model.config, 'model_type', None) == 'qwen3':
        return {'full_attention': None}
    return None


def prefill_frozen_request(model, input_ids, config=None, geometry=None,
                           static_gate=None, suffix_length=0, *, cache=None,
                           request_id=None):
    """Dense one-shot prefill of ``input_ids`` [1, L] into the cache, then
    freeze the request's per-layer skip decisions.  Returns ``(output,
    audit)`` like the reference; ``output.past_key_values`` is the cache."""
    if geometry is None:
        raise ValueError('prefill_frozen_request needs a RegionGeometry')
    n_layers = model.config.num_hidden_layers
    prompt_length = int(input_ids.shape[-1])
    if not isinstance(suffix_length, int) or suffix_length < 0:
        raise ValueError('suffix_length must be a non-negative integer')
    capacity = prompt_length + suffix_length
    geo = (replace(geometry, max_new_tokens=geometry.max_new_tokens + suffix_length)
           if suffix_length else geometry)
    if cache is None:
        cache = build_frozen_cache(model, geo, capacity)
    if cache.n_layers != n_layers or cache.geometry != geo:
        raise ValueError('shared cache does not match model layers or geometry')
    if capacity + geometry.max_new_tokens > cache.max_blocks * geometry.page:
        raise ValueError('request exceeds shared cache sequence capacity')
    if static_gate is not None and static_gate.num_layers != n_layers:
        raise ValueError(f'static gate num_layers={static_gate.num_layers} does '
                         f'not match the model ({n_layers})')
    request_id = cache.add_request(request_id)
    cache.set_active_request(request_id)
    profiles = None
    with _request_failure_guard(cache, request_id):
        positions = torch.arange(prompt_length, device=input_ids.device)[None]

        def prefill():
            return model(input_ids=input_ids, position_ids=positions,
                         past_key_values=cache, use_cache=True, logits_to_keep=1,
                         attention_mask=_prefill_mask_arg(model))

        if static_gate is None and config is not None:
            with capture_profiles(model, geometry, config) as profiles:
                output = prefill()
            if len(profiles) != n_layers:
                raise ValueError('incomplete native layer profiling')
            present_near, present_far = region_present(prompt_length, geometry)
            decisions = {l: decide_regions(profiles[l], config, present_near,
                                           present_far) for l in range(n_layers)}
            skip_far = [decisions[l]['skip_far'] for l in range(n_layers)]
            skip_near = [decisions[l]['skip_near'] for l in range(n_layers)]
        else:
            output = prefill()
            if static_gate is not None:
                skip_far = list(static_gate.skip_far)
                skip_near = list(static_gate.skip_near)
            else:
                skip_far, skip_near = [False] * n_layers, [False] * n_layers
            decisions = {l: {'skip_near': skip_near[l], 'skip_far': skip_far[l]}
                         for l in range(n_layers)}
        cache.freeze(request_id, skip_far, skip_near)
    return output, dict(profiles=profiles, decisions=decisions, request_id=request_id,
                        material_length=prompt_length, suffix_length=suffix_length)


def decode_frozen_request(model, output, *, max_new_tokens, eos_ids, pad_token_id=0,
                          capture_graph=True, min_new_tokens=0, receipt=None):
    """Greedy decode of the active request after ``prefill_frozen_request``.
    Returns ``(generated_tokens, cache)``."""
    from .graph_runner import session_graph_runner
    from ..scheduler.scheduler import ContinuousBatchScheduler

    if max_new_tokens < 0:
        raise ValueError('max_new_tokens must be non-negative')
    if not 0 <= min_new_tokens <= max_new_tokens:
        raise ValueError('min_new_tokens must be in [0, max_new_tokens]')
    cache = output.past_key_values
    request_id = cache.active_request_id
    if request_id is None:
        raise ValueError('frozen decode requires an active request')
    eos_ids = frozenset(int(t) for t in eos_ids)
    generated = []
    with _request_failure_guard(cache, request_id):
        if max_new_tokens == 0:
            cache.transition_request(request_id, RequestPhase.FINISHED)
            return generated, cache
        cache.transition_request(request_id, RequestPhase.GENERATE)
        first = greedy_next_tokens(output.logits, eos_ids, generated_counts=0,
                                   min_new_tokens=min_new_tokens)
        generated.append(int(first[0]))  # the one synchronisation per request

        def stop(tokens):
            return (len(tokens) >= min_new_tokens and tokens[-1] in eos_ids) \
                or len(tokens) >= max_new_tokens

        runner = None
        if not stop(generated):
            scheduler = ContinuousBatchScheduler(
                cache=cache, max_batch=1, eos_ids=eos_ids, pad_token_id=pad_token_id,
                track_receipts=True, auto_finish_requests=False)
            scheduler.add_request(request_id)
            scheduler.next_tokens[request_id] = generated[0]
            runner = session_graph_runner(
                model, cache, scheduler, buckets=(1,),
                device=next(model.parameters()).device, capture=capture_graph)
            submitted = 1
            done = False

            def consume(receipts):
                nonlocal done
                for rid, tok in receipts:
                    if rid == request_id and not done:
                        generated.append(int(tok))
                        done = stop(generated)

            while submitted < max_new_tokens and not done:
                runner.step(model, cache, generated_counts=submitted,
                            min_new_tokens=min_new_tokens)
                submitted += 1
                consume(scheduler.pop_ready_receipts())
            consume(scheduler.flush_ready_receipts())
            # steps submitted after the stop token are rolled back
            extra = max(0, submitted - len(generated))
            if extra:
                cache.states[request_id].logical_length -= extra
                cache.nfa_decode_steps = max(0, cache.nfa_decode_steps - extra)
            model._nfa_graph_session_pool.release(runner)
        cache.transition_request(request_id, RequestPhase.FINISHED)
        if receipt is not None:
            receipt.update(
                generated_tokens=len(generated),
                nfa_decode_steps=cache.nfa_decode_steps,
                graph_capture_count=runner.capture_count if runner else 0,
                graph_replays=runner.replay_count if runner else 0,
                graph_eager_fallbacks=runner.eager_fallback_count if runner else 0)
    return generated, cache
