"""Several ragged requests decoded together through one paged cache (GPU).

A tiny random-init bf16 Llama (2 layers, 8 query / 2 kv heads, head_dim 128),
three prompts of 5000, 9000 and 6500 tokens prefilled into one cache, then
decoded as one batch (the reference's continuous-batching decode,
``scheduler/scheduler.py:38-328`` and ``engine/graph_runner.py:7-302``):

* one eager batched step: every layer's selection for every request (gather
  rows and visible lengths) equals the oracle's on a snapshot of that layer,
  and each request's row of the logits equals the same step decoded alone
  from an identical cache (tolerance: the dense layers see batch 3 vs 1);
* graph decode with a padded bucket of 4: replayed steps give bit-identical
  logits and the same tokens as eager steps through the same runner, and
  every request advances by one token per step.
"""
import numpy as np
import pytest
import torch

from nfa_case import cfg_from, run_oracle
from sparse_attn.engine.frozen_runner import build_frozen_cache, prefill_frozen_request
from sparse_attn.engine.graph_runner import GraphRunner
from sparse_attn.scheduler.scheduler import ContinuousBatchScheduler
from test_model_patch_gpu import GEO, _args, _mask_arg, _recording, _tiny_model

pytestmark = pytest.mark.gpu

DEV = 'cuda'
PROMPTS = (5000, 9000, 6500)


def _prefilled(seed=17):
    """A patched tiny Llama and one cache holding the three prompts."""
    from sparse_attn.patches.patch import register_patch
    model = _tiny_model('llama')
    register_patch(model, _args())
    cache = build_frozen_cache(model, GEO, max(PROMPTS), max_requests=4,
                               max_visible_len=1024)
    gen = torch.Generator(device='cpu').manual_seed(seed)
    rids, firsts = [], []
    with torch.no_grad():
        for n in PROMPTS:
            ids = torch.randint(0, 1024, (1, n), generator=gen).to(DEV)
            out, audit = prefill_frozen_request(model, ids, None, GEO, cache=cache)
            rids.append(audit['request_id'])
            firsts.append(int(out.logits[0, -1].argmax()))
    return model, cache, rids, firsts


def _step(model, cache, rids, tokens):
    """One eager decode step of `rids` (one token each) straight through the
    model; returns the logits [B, V]."""
    tok = torch.tensor(tokens, dtype=torch.long, device=DEV)[:, None]
    pos = torch.tensor([[cache.states[r].logical_length] for r in rids],
                       dtype=torch.long, device=DEV)
    cache.new_step(rids)
    cache.plan_common(rids)
    with torch.no_grad():
        logits = model(input_ids=tok, position_ids=pos, past_key_values=cache,
                       use_cache=True, attention_mask=_mask_arg(model)).logits
    torch.cuda.synchronize()
    cache.commit_step()
    return logits[:, -1].float()


def test_batched_step_selections_and_logits():
    model, cache, rids, firsts = _prefilled()
    print(f'# batched llama decode step, prompts {PROMPTS}', flush=True)
    with _recording() as calls:
        logits = _step(model, cache, rids, firsts)
    page = GEO.page
    for layer_idx in range(model.config.num_hidden_layers):
        rec = calls[layer_idx]
        cfg = cfg_from(cache, rec['indexer'], rec['scaling'])
        width = cache.gather_indices_for_layer(layer_idx).shape[-1]
        res, _, _ = run_oracle(cfg, rec['snap'], rec['q'], rec['decode'], max_vis=width)
        gather = cache.gather_indices_for_layer(layer_idx).cpu().numpy()
        vis = cache.visible_lens_for_layer(layer_idx).cpu().numpy()
        for b, n in enumerate(PROMPTS):
            for kv in range(cache.num_kv_heads):
                r = res[b][kv]
                tag = f'layer={layer_idx} request={b} kv={kv}'
                assert vis[b, kv] == r.vis_len, tag
                np.testing.assert_array_equal(gather[b, kv, :r.vis_len],
                                              r.gather[:r.vis_len], err_msg=tag)
                assert 0 < r.vis_len <= 1024 < n, tag
    # each request's row against the same step decoded alone
    for b in range(len(PROMPTS)):
        model1, cache1, rids1, firsts1 = _prefilled()
        assert firsts1 == firsts
        alone = _step(model1, cache1, [rids1[b]], [firsts1[b]])[0]
        diff = (logits[b] - alone).abs().max().item()
        scale = alone.abs().max().item()
        assert diff <= 2e-2 * scale, (b, diff, scale)
        del model1, cache1


def test_batched_graph_replay_matches_eager():
    steps = 5
    runs = {}
    for mode in ('eager', 'graph'):
        print(f'# batched llama {mode} decode {steps} steps', flush=True)
        model, cache, rids, firsts = _prefilled()
        sched = ContinuousBatchScheduler(cache=cache, max_batch=4, eos_ids=(),
                                         pad_token_id=0, track_receipts=True)
        for rid, tok in zip(rids, firsts):
            sched.add_request(rid)
            sched.next_tokens[rid] = tok
        runner = GraphRunner(scheduler=sched, buckets=(4,), device=DEV)
        if mode == 'graph':
            runner.capture_all(model, cache)
        logits = []
        with torch.no_grad():
            for i in range(steps):
                out = runner.step(model, cache, generated_counts=i + 1)
                logits.append(out.logits[:len(rids)].float().clone())
        receipts = sched.flush_ready_receipts()
        if mode == 'graph':
            assert runner.replay_count == steps and runner.eager_fallback_count == 0
        for rid, n in zip(rids, PROMPTS):
            assert cache.states[rid].logical_length == n + steps
        runs[mode] = (sorted(receipts), torch.stack(logits))
        del runner, sched, cache, model
    assert runs['graph'][0] == runs['eager'][0]
    assert len(runs['graph'][0]) == steps * len(PROMPTS)
    assert torch.equal(runs['graph'][1], runs['eager'][1])
