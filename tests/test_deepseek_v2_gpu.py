"""Patched DeepSeek-V2 on the paged cache, on the GPU.

A tiny random-init bf16 DeepSeek-V2 (2 layers, 16 heads, kv LoRA rank 64,
nope 128 + rope 64 key dims, 128 value dims, dense MLPs) with a 9000-token
prompt, run through the expanded-head path: the arena holds per-head keys of
192 dims and values of 128, one kv head per query head, and the selector
scores the rope dims 128..191 (``--nfa_subspace mla_rope``).

* prefill: the arena holds exactly the keys and values the unpatched module
  expands from its latent cache, and the prefill logits agree (atol 1e-5);
* one eager decode step: each layer's selection equals the oracle's on a
  snapshot of that layer (bit-exact gather rows and visible lengths), the
  attention output matches a float64 attention over the selected rows
  (rtol 2e-2, atol 2e-3), and the logits match the unpatched model with its
  attention restricted to the same token sets;
* graph decode: replayed steps give bit-identical logits and the same tokens
  as eager steps.
"""
import copy

import numpy as np
import pytest
import torch

from nfa_case import cfg_from, run_oracle
from sparse_attn.engine.frozen_runner import prefill_frozen_request
from sparse_attn.engine.graph_runner import GraphRunner
from sparse_attn.ops.paged_region_kernels_nfa import nfa_args
from sparse_attn.patches.patch import register_patch
from sparse_attn.policies.region_geometry import RegionGeometry
from sparse_attn.scheduler.scheduler import ContinuousBatchScheduler
from test_model_patch_gpu import _arena_rows, _masked_sdpa, _recording

pytestmark = pytest.mark.gpu

DEV = 'cuda'
PROMPT = 9000
GEO = RegionGeometry(sink=4, near=4096, window=128, page=16, max_new_tokens=16)


def _tiny_dsv2(seed=20261201):
    from transformers import DeepseekV2Config, DeepseekV2ForCausalLM
    torch.manual_seed(seed)
    cfg = DeepseekV2Config(
        vocab_size=1024, hidden_size=512, intermediate_size=1024,
        num_hidden_layers=2, num_attention_heads=16, num_key_value_heads=16,
        q_lora_rank=None, kv_lora_rank=64, qk_nope_head_dim=128,
        qk_rope_head_dim=64, v_head_dim=128, first_k_dense_replace=2,
        max_position_embeddings=16384)
    cfg._attn_implementation = 'sdpa'
    return DeepseekV2ForCausalLM(cfg).to(device=DEV, dtype=torch.bfloat16).eval()


def _args():
    args = nfa_args('mla_rope')
    args.tia_block_size = 16
    return args


def _prefill(model, ids):
    assert register_patch(model, _args()) == model.config.num_hidden_layers
    with torch.no_grad():
        out, audit = prefill_frozen_request(model, ids, None, GEO)
    return out, out.past_key_values, audit['request_id']


def _expanded_reference(ref_model, ref_cache, layer_idx):
    """The keys and values the unpatched module expands from its latent cache."""
    layer = ref_cache.layers[layer_idx]
    attn = ref_model.model.layers[layer_idx].self_attn
    key, value = attn.expand_kv(layer.keys, layer.values)
    return key[0], value[0]


def test_prefill_writes_expanded_heads_and_logits():
    model = _tiny_dsv2()
    ref_model = copy.deepcopy(model)
    ids = torch.randint(0, 1024, (1, PROMPT),
                        generator=torch.Generator().manual_seed(7)).to(DEV)
    print(f'# deepseek_v2 prefill {PROMPT}', flush=True)
    with torch.no_grad():
        ref = ref_model(ids, use_cache=True)
    out, cache, rid = _prefill(model, ids)
    assert cache.num_kv_heads == 16
    assert cache.layers[0].head_dim_k == 192 and cache.layers[0].head_dim_v == 128
    # the same attention on the same K/V; the unpatched model's attention
    # runs with an implicit causal mask, the patched one with the mask built
    # from the paged cache, which may pick another kernel for the same sum
    torch.testing.assert_close(out.logits[:, -1], ref.logits[:, -1], rtol=1e-2,
                               atol=1e-5)
    for layer_idx in range(model.config.num_hidden_layers):
        k, v = _arena_rows(cache, layer_idx, rid, PROMPT)
        want_k, want_v = _expanded_reference(ref_model, ref.past_key_values, layer_idx)
        assert torch.equal(k, want_k)
        assert torch.equal(v, want_v)


def test_decode_step_selection_attention_and_logits():
    model = _tiny_dsv2()
    ref_model = copy.deepcopy(model)
    ids = torch.randint(0, 1024, (1, PROMPT),
                        generator=torch.Generator().manual_seed(11)).to(DEV)
    with torch.no_grad():
        ref = ref_model(ids, use_cache=True)
    out, cache, rid = _prefill(model, ids)
    token = out.logits[:, -1].argmax(-1, keepdim=True)
    pos = torch.full((1, 1), PROMPT, dtype=torch.long, device=DEV)
    cache.new_step([rid])
    cache.plan_common([rid])
    print(f'# deepseek_v2 decode step at {PROMPT}', flush=True)
    with torch.no_grad(), _recording() as calls:
        logits = model(input_ids=token, position_ids=pos, past_key_values=cache,
                       use_cache=True).logits
    torch.cuda.synchronize()
    cache.commit_step()

    page = GEO.page
    allowed = {}
    for layer_idx in range(model.config.num_hidden_layers):
        rec = calls[layer_idx]
        assert rec['indexer'].subspace == 'mla_rope' and rec['indexer'].head_dim == 192
        cfg = cfg_from(cache, rec['indexer'], rec['scaling'])
        assert list(cfg.dims) == list(range(128, 192))
        width = cache.gather_indices_for_layer(layer_idx).shape[-1]
        res, k_pool, v_pool = run_oracle(cfg, rec['snap'], rec['q'], rec['decode'],
                                         max_vis=width)
        gather = cache.gather_indices_for_layer(layer_idx).cpu().numpy()
        vis = cache.visible_lens_for_layer(layer_idx).cpu().numpy()
        inverse = {p: lp for lp, p in cache.states[rid].block_tables[layer_idx].items()}
        masks = []
        want = np.zeros_like(rec['out'].numpy())
        for kv in range(cache.num_kv_heads):
            r = res[0][kv]
            tag = f'layer={layer_idx} kv={kv}'
            assert vis[0, kv] == r.vis_len, tag
            np.testing.assert_array_equal(gather[0, kv, :r.vis_len],
                                          r.gather[:r.vis_len], err_msg=tag)
            assert 0 < r.vis_len <= 1024 < PROMPT, tag
            slots = r.gather[:r.vis_len]
            keys = k_pool[slots // page, 0, kv, slots % page].astype(np.float64)
            vals = v_pool[slots // page, 0, kv, slots % page].astype(np.float64)
            s = rec['q'][0, kv].astype(np.float64) @ keys.T * rec['scaling']
            p = np.exp(s - s.max())
            want[0, kv] = (p / p.sum()) @ vals
            mask = torch.zeros(PROMPT + 1, dtype=torch.bool, device=DEV)
            logical = [inverse[x // page] * page + x % page for x in slots.tolist()]
            mask[torch.tensor(logical, device=DEV)] = True
            masks.append(mask)
        allowed[layer_idx] = masks
        assert rec['out'].shape[-1] == 128
        np.testing.assert_allclose(rec['out'].numpy(), want, rtol=2e-2, atol=2e-3,
                                   err_msg=f'layer={layer_idx} attention')

    with torch.no_grad(), _masked_sdpa(allowed):
        ref_logits = ref_model(input_ids=token, position_ids=pos,
                               past_key_values=ref.past_key_values,
                               use_cache=True).logits
    diff = (logits.float() - ref_logits.float()).abs().max().item()
    scale = ref_logits.float().abs().max().item()
    assert diff <= 2e-2 * scale, (diff, scale)


def test_graph_replay_matches_eager_steps():
    steps = 5
    model = _tiny_dsv2()
    ids = torch.randint(0, 1024, (1, PROMPT),
                        generator=torch.Generator().manual_seed(13)).to(DEV)
    runs = {}
    for mode in ('eager', 'graph'):
        print(f'# deepseek_v2 {mode} decode {steps} steps', flush=True)
        out, cache, rid = _prefill(model, ids)
        sched = ContinuousBatchScheduler(cache=cache, max_batch=1, eos_ids=(),
                                         pad_token_id=0, track_receipts=True)
        sched.add_request(rid)
        sched.next_tokens[rid] = int(out.logits[0, -1].argmax())
        runner = GraphRunner(scheduler=sched, buckets=(1,), device=DEV)
        if mode == 'graph':
            runner.capture_all(model, cache)
        logits = []
        with torch.no_grad():
            for i in range(steps):
                logits.append(runner.step(model, cache, generated_counts=i + 1)
                              .logits.float().clone())
        tokens = [t for _, t in sched.flush_ready_receipts()]
        if mode == 'graph':
            assert runner.replay_count == steps and runner.eager_fallback_count == 0
        runs[mode] = (tokens, torch.stack(logits))
        del runner, sched, cache, out
    assert runs['graph'][0] == runs['eager'][0]
    assert torch.equal(runs['graph'][1], runs['eager'][1])
