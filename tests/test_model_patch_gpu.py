"""Patched Qwen3 / Llama models on the paged cache, on the GPU.

Tiny random-init bf16 models (2 layers, 8 query / 2 kv heads, head_dim 128)
with a 9000-token prompt, so that the decode selection is sparse (far, near,
sink and window regions all present):

* prefill: the arena holds exactly the K/V that the unpatched model's own
  cache holds, and the prefill logits are identical;
* one eager decode step: every layer's selection (gather rows and visible
  lengths) equals the oracle's on a snapshot of that layer, the attention
  output matches an fp32 attention over the selected rows (rtol 2e-2,
  atol 2e-3), and the logits match the unpatched model restricted to the
  same token sets;
* graph decode: replayed steps give bit-identical logits and the same tokens
  as eager steps through the same runner.
"""
import copy
from contextlib import contextmanager

import numpy as np
import pytest
import torch

from nfa_case import cfg_from, run_oracle, snapshot
from sparse_attn.engine.frozen_runner import prefill_frozen_request
from sparse_attn.engine.graph_runner import GraphRunner
from sparse_attn.indexer import nfa_layer_batch_selector as selmod
from sparse_attn.ops import paged_region_kernels_nfa as opsmod
from sparse_attn.ops.paged_region_kernels_nfa import nfa_args
from sparse_attn.patches.patch import register_patch
from sparse_attn.policies.region_geometry import RegionGeometry
from sparse_attn.scheduler.scheduler import ContinuousBatchScheduler

pytestmark = pytest.mark.gpu

DEV = 'cuda'
PROMPT = 9000
GEO = RegionGeometry(sink=4, near=4096, window=128, page=16, max_new_tokens=16)


def _tiny_model(kind, seed=20261201):
    torch.manual_seed(seed)
    common = dict(vocab_size=1024, hidden_size=512, intermediate_size=1024,
                  num_hidden_layers=2, num_attention_heads=8,
                  num_key_value_heads=2, head_dim=128,
                  max_position_embeddings=16384, rope_theta=1e6)
    if kind == 'qwen3':
        from transformers import Qwen3Config, Qwen3ForCausalLM
        cfg = Qwen3Config(**common)
        cls = Qwen3ForCausalLM
    else:
        from transformers import LlamaConfig, LlamaForCausalLM
        cfg = LlamaConfig(**common)
        cls = LlamaForCausalLM
    cfg._attn_implementation = 'sdpa'
    model = cls(cfg).to(device=DEV, dtype=torch.bfloat16).eval()
    return model


def _args():
    args = nfa_args('tail')
    args.tia_block_size = 16
    return args


def _mask_arg(model):
    return {'full_attention': None} if model.config.model_type == 'qwen3' else None


@contextmanager
def _recording():
    """Record, per layer, the selector's inputs (snapshot, q, decode K/V) and
    the gather attention's output of the decode step."""
    calls = {}
    real_select = selmod.select_topk_for_layer_batched
    real_attn = opsmod.decode_graph_ready

    def select(cache, layer_idx, req_ids, q, attention=None, decode_write=None, **kw):
        calls[layer_idx] = dict(
            snap=snapshot(cache, layer_idx, len(req_ids)),
            q=q.float().cpu().numpy(),
            decode=tuple(t.float().cpu().numpy() if t.is_floating_point()
                         else t.cpu().numpy() for t in decode_write),
            scaling=attention.scaling, indexer=attention.indexer)
        return real_select(cache, layer_idx, req_ids, q, attention=attention,
                           decode_write=decode_write, **kw)

    def attn(module, q, cache, **kw):
        out = real_attn(module, q, cache, **kw)
        calls[module.layer_idx]['out'] = out.float().cpu()
        return out

    selmod.select_topk_for_layer_batched = select
    opsmod.decode_graph_ready = attn
    try:
        yield calls
    finally:
        selmod.select_topk_for_layer_batched = real_select
        opsmod.decode_graph_ready = real_attn


@contextmanager
def _masked_sdpa(allowed):
    """Replace the models' sdpa attention by fp32 attention restricted, per
    layer and kv head, to ``allowed[layer][kv]`` (bool over key positions)."""
    from transformers.modeling_utils import ALL_ATTENTION_FUNCTIONS
    original = ALL_ATTENTION_FUNCTIONS['sdpa']

    def masked(module, query, key, value, attention_mask, scaling=None, **kw):
        b, hq, t, d = query.shape
        hkv = key.shape[1]
        g = hq // hkv
        q = query.float()
        k = key.float().repeat_interleave(g, dim=1)
        v = value.float().repeat_interleave(g, dim=1)
        s = torch.matmul(q, k.transpose(-1, -2).contiguous()) * scaling
        keep = torch.stack([allowed[module.layer_idx][h // g] for h in range(hq)])
        s = s.masked_fill(~keep[None, :, None, :], float('-inf'))
        out = torch.matmul(torch.softmax(s, dim=-1), v).to(query.dtype)
        return out.transpose(1, 2).contiguous(), None

    ALL_ATTENTION_FUNCTIONS['sdpa'] = masked
    try:
        yield
    finally:
        ALL_ATTENTION_FUNCTIONS['sdpa'] = original


def _arena_rows(cache, layer_idx, rid, n):
    layer = cache.layers[layer_idx]
    page = cache.geometry.page
    table = cache.states[rid].block_tables[layer_idx]
    pids = torch.tensor([table[lp] for lp in range((n + page - 1) // page)],
                        device=DEV)
    k = layer.kv_pool_k[pids, 0].permute(1, 0, 2, 3).reshape(
        layer.num_kv_heads, -1, layer.head_dim_k)[:, :n]
    v = layer.kv_pool_v[pids, 0].permute(1, 0, 2, 3).reshape(
        layer.num_kv_heads, -1, layer.head_dim_v)[:, :n]
    return k, v


def _prefill(model, ids, fused=False):
    register_patch(model, _args(), rmsnorm_decode=fused, mlp_silu_decode=fused,
                   decode_layers=fused)
    with torch.no_grad():
        out, audit = prefill_frozen_request(model, ids, None, GEO)
    return out, out.past_key_values, audit['request_id']


@pytest.mark.parametrize('kind', ['qwen3', 'llama'])
def test_prefill_writes_model_kv_and_logits(kind):
    model = _tiny_model(kind)
    ref_model = copy.deepcopy(model)
    gen = torch.Generator(device='cpu').manual_seed(7)
    ids = torch.randint(0, 1024, (1, PROMPT), generator=gen).to(DEV)
    print(f'# {kind} prefill {PROMPT}', flush=True)
    with torch.no_grad():
        ref = ref_model(ids, use_cache=True)
    out, cache, rid = _prefill(model, ids)
    torch.testing.assert_close(out.logits[:, -1], ref.logits[:, -1], rtol=0, atol=0)
    for layer_idx in range(model.config.num_hidden_layers):
        k, v = _arena_rows(cache, layer_idx, rid, PROMPT)
        assert torch.equal(k, ref.past_key_values.layers[layer_idx].keys[0])
        assert torch.equal(v, ref.past_key_values.layers[layer_idx].values[0])


@pytest.mark.parametrize('kind', ['qwen3', 'llama'])
def test_decode_step_selection_attention_and_logits(kind):
    model = _tiny_model(kind)
    ref_model = copy.deepcopy(model)
    gen = torch.Generator(device='cpu').manual_seed(11)
    ids = torch.randint(0, 1024, (1, PROMPT), generator=gen).to(DEV)
    with torch.no_grad():
        ref = ref_model(ids, use_cache=True)
    out, cache, rid = _prefill(model, ids)
    token = out.logits[:, -1].argmax(-1, keepdim=True)
    pos = torch.full((1, 1), PROMPT, dtype=torch.long, device=DEV)
    cache.new_step([rid])
    cache.plan_common([rid])
    print(f'# {kind} decode step at {PROMPT}', flush=True)
    with torch.no_grad(), _recording() as calls:
        logits = model(input_ids=token, position_ids=pos, past_key_values=cache,
                       use_cache=True, attention_mask=_mask_arg(model)).logits
    torch.cuda.synchronize()
    cache.commit_step()

    n_layers = model.config.num_hidden_layers
    hkv = cache.num_kv_heads
    page = GEO.page
    allowed = {}
    for layer_idx in range(n_layers):
        rec = calls[layer_idx]
        cfg = cfg_from(cache, rec['indexer'], rec['scaling'])
        width = cache.gather_indices_for_layer(layer_idx).shape[-1]
        res, k_pool, v_pool = run_oracle(cfg, rec['snap'], rec['q'], rec['decode'],
                                         max_vis=width)
        gather = cache.gather_indices_for_layer(layer_idx).cpu().numpy()
        vis = cache.visible_lens_for_layer(layer_idx).cpu().numpy()
        inverse = {p: lp for lp, p in
                   cache.states[rid].block_tables[layer_idx].items()}
        masks = []
        want = np.zeros_like(rec['out'].numpy())
        for kv in range(hkv):
            r = res[0][kv]
            tag = f'{kind} layer={layer_idx} kv={kv}'
            assert vis[0, kv] == r.vis_len, tag
            np.testing.assert_array_equal(gather[0, kv, :r.vis_len],
                                          r.gather[:r.vis_len], err_msg=tag)
            assert 0 < r.vis_len <= 1024 < PROMPT, tag
            slots = r.gather[:r.vis_len]
            keys = k_pool[slots // page, 0, kv, slots % page]
            vals = v_pool[slots // page, 0, kv, slots % page]
            g = cfg.hq // hkv
            q = rec['q'][0, kv * g:(kv + 1) * g]
            s = q @ keys.T * rec['scaling']
            p = np.exp(s - s.max(-1, keepdims=True))
            want[0, kv * g:(kv + 1) * g] = (p / p.sum(-1, keepdims=True)) @ vals
            mask = torch.zeros(PROMPT + 1, dtype=torch.bool, device=DEV)
            logical = [inverse[s // page] * page + s % page for s in slots.tolist()]
            mask[torch.tensor(logical, device=DEV)] = True
            masks.append(mask)
        allowed[layer_idx] = masks
        np.testing.assert_allclose(rec['out'].numpy(), want, rtol=2e-2, atol=2e-3,
                                   err_msg=f'{kind} layer={layer_idx} attention')

    with torch.no_grad(), _masked_sdpa(allowed):
        ref_logits = ref_model(input_ids=token, position_ids=pos,
                               past_key_values=ref.past_key_values,
                               use_cache=True).logits
    diff = (logits.float() - ref_logits.float()).abs().max().item()
    scale = ref_logits.float().abs().max().item()
    assert diff <= 2e-2 * scale, (diff, scale)


@pytest.mark.parametrize('kind', ['qwen3', 'llama'])
def test_fused_decode_layers_match_unfused(kind):
    """Seven-launch decoder layers against the layer-by-layer HF modules
    (with the patched attention), fed the same tokens for three steps."""
    fused = _tiny_model(kind)
    plain = copy.deepcopy(fused)
    gen = torch.Generator(device='cpu').manual_seed(17)
    ids = torch.randint(0, 1024, (1, PROMPT), generator=gen).to(DEV)
    out_f, cache_f, rid_f = _prefill(fused, ids, fused=True)
    out_p, cache_p, rid_p = _prefill(plain, ids)
    assert torch.equal(out_f.logits, out_p.logits)  # prefill is not fused
    token = out_p.logits[:, -1].argmax(-1, keepdim=True)
    for step in range(3):
        print(f'# {kind} fused vs plain decode step {step}', flush=True)
        pos = torch.full((1, 1), PROMPT + step, dtype=torch.long, device=DEV)
        logits = []
        for model, cache, rid in ((fused, cache_f, rid_f), (plain, cache_p, rid_p)):
            cache.new_step([rid])
            cache.plan_common([rid])
            with torch.no_grad():
                logits.append(model(input_ids=token, position_ids=pos,
                                    past_key_values=cache, use_cache=True,
                                    attention_mask=_mask_arg(model)).logits.float())
            cache.commit_step()
        diff = (logits[0] - logits[1]).abs().max().item()
        scale = logits[1].abs().max().item()
        assert diff <= 3e-2 * scale, (step, diff, scale)
        token = logits[1][:, -1].argmax(-1, keepdim=True)
    layers = fused.model.layers
    assert all(getattr(l, '_nfa_fused_calls', 0) == 3 for l in layers)
    assert not any(hasattr(l, '_nfa_fused_calls') for l in plain.model.layers)


@pytest.mark.parametrize('fused', [False, True])
@pytest.mark.parametrize('kind', ['qwen3', 'llama'])
def test_graph_replay_matches_eager_steps(kind, fused):
    steps = 6
    model = _tiny_model(kind)
    gen = torch.Generator(device='cpu').manual_seed(13)
    ids = torch.randint(0, 1024, (1, PROMPT), generator=gen).to(DEV)
    runs = {}
    for mode in ('eager', 'graph'):
        print(f'# {kind} fused={fused} {mode} decode {steps} steps', flush=True)
        out, cache, rid = _prefill(model, ids, fused=fused)
        sched = ContinuousBatchScheduler(cache=cache, max_batch=1, eos_ids=(),
                                         pad_token_id=0, track_receipts=True)
        sched.add_request(rid)
        sched.next_tokens[rid] = int(out.logits[0, -1].argmax())
        runner = GraphRunner(scheduler=sched, buckets=(1,), device=DEV)
        if mode == 'graph':
            runner.capture_all(model, cache)
            assert runner.capture_count >= 1
        logits = []
        with torch.no_grad():
            for i in range(steps):
                lg = runner.step(model, cache, generated_counts=i + 1)
                logits.append(lg.logits.float().clone())
        tokens = [t for _, t in sched.flush_ready_receipts()]
        if mode == 'graph':
            assert runner.replay_count == steps and runner.eager_fallback_count == 0
        else:
            assert runner.eager_fallback_count == steps
        calls = [getattr(l, '_nfa_fused_calls', 0) for l in model.model.layers]
        assert all(c > 0 for c in calls) == fused, calls
        assert cache.states[rid].logical_length == PROMPT + steps
        runs[mode] = (tokens, torch.stack(logits))
    assert runs['graph'][0] == runs['eager'][0]
    assert len(runs['graph'][0]) == steps
    assert torch.equal(runs['graph'][1], runs['eager'][1])
