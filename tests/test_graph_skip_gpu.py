"""hipGraph capture and replay under frozen skip signatures (GPU).

Mirrors the reference's capture tests
(tests/test_nfa_current_query_selector.py:826-993): a captured selector step
reads the live current query and decode K/V, a both-skip replay still writes
the decode K/V, and a capture on padding rows does not specialise the replay
to the padding rows' skip state.

* selector + attention captured in region modes 1 (far skipped), 2 (near
  skipped) and 3 (both skipped: the protected-only union) and replayed over
  four decode steps with fresh inputs in the captured buffers: gather rows,
  visible lengths and the decode-written K/V rows bit-exact against the
  oracle at every replay, attention against the float64 oracle (rtol 2e-2 /
  atol 2e-3);
* a capture on padding rows only (region mode 0), replayed with live rows of
  all four skip states plus a padding row: every row as the oracle's and as
  the same launch run eagerly;
* the graph runner over a tiny Llama with three requests in a padded bucket
  of 4, their skip states mixed (region mode 0) or uniform (modes 2 and 3):
  replayed steps give bit-identical logits, tokens and KV arenas to eager
  steps through the same runner.
"""
from types import SimpleNamespace

import numpy as np
import pytest
import torch

from nfa_case import (GPU, attention_ns, bf16_randn, cfg_from, make_indexer,
                      prod_cache, run_oracle, snapshot)
from oracle import nfa_oracle as orc
from sparse_attn.indexer.nfa_layer_batch_selector import \
    select_topk_for_layer_batched
from sparse_attn.ops.paged_region_kernels_nfa import decode_graph_ready

pytestmark = pytest.mark.gpu

SCALE = 128 ** -0.5


def _compare_rows(cache, res, rows, tag):
    gather = cache.gather_indices_for_layer(0)[:rows].cpu().numpy()
    vis = cache.visible_lens_for_layer(0)[:rows].cpu().numpy()
    for b in range(rows):
        for kv in range(cache.num_kv_heads):
            r = res[b][kv]
            assert vis[b, kv] == r.vis_len, (tag, b, kv)
            np.testing.assert_array_equal(gather[b, kv, :r.vis_len], r.gather,
                                          err_msg=f'{tag} row={b} kv={kv}')


@pytest.mark.parametrize('skip,mode', [((True, False), 1), ((False, True), 2),
                                       ((True, True), 3)],
                         ids=['far_skipped', 'near_skipped', 'both_skipped'])
def test_selector_capture_replay_in_region_mode(skip, mode):
    lengths = [9000, 12345]
    cache, gen, req_ids = prod_cache(lengths, skips=[skip] * 2)
    indexer = make_indexer()
    attn = attention_ns(indexer, SCALE)
    b, hq, hkv = 2, cache.num_query_heads, cache.num_kv_heads
    # the captured inputs: the step's query, decode K/V and slots
    q = bf16_randn((b, hq, 128), gen, GPU)
    keys = bf16_randn((b, hkv, 1, 128), gen, GPU)
    values = bf16_randn((b, hkv, 1, 128), gen, GPU)
    slots = torch.zeros(b, dtype=torch.int32, device=GPU)
    module = SimpleNamespace(layer_idx=0, scaling=SCALE)
    assert cache.nfa_region_mode(cache.nfa_skip_signature(req_ids), 0) == mode

    def run():
        select_topk_for_layer_batched(cache, 0, req_ids, q, attention=attn,
                                      decode_write=(keys, values, slots))
        return decode_graph_ready(module, q, cache)

    cache.new_step(req_ids)
    cache.plan_common(req_ids)
    slots.copy_(cache.slot_mapping_for_layer(0)[:b])
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            run()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = run()
    torch.cuda.synchronize()
    cache.commit_step()
    print(f'# region mode {mode}: captured', flush=True)
    for step in range(4):
        cache.new_step(req_ids)
        cache.plan_common(req_ids)
        q.copy_(bf16_randn((b, hq, 128), gen, GPU))
        keys.copy_(bf16_randn((b, hkv, 1, 128), gen, GPU))
        values.copy_(bf16_randn((b, hkv, 1, 128), gen, GPU))
        slots.copy_(cache.slot_mapping_for_layer(0)[:b])
        torch.cuda.synchronize()
        snap = snapshot(cache, 0, b)
        graph.replay()
        torch.cuda.synchronize()
        cfg = cfg_from(cache, indexer, SCALE)
        dec = (keys.float().cpu().numpy(), values.float().cpu().numpy(),
               slots.cpu().numpy())
        res, k_pool, v_pool = run_oracle(cfg, snap, q.float().cpu().numpy(), dec,
                                         max_vis=1024, copy=False)
        _compare_rows(cache, res, b, f'mode {mode} replay {step}')
        layer = cache.layers[0]
        for row, slot in enumerate(dec[2].tolist()):
            phys, off = divmod(slot, cache.geometry.page)
            # the replay wrote this step's K/V (also with both regions skipped)
            np.testing.assert_array_equal(
                layer.kv_pool_k[phys, 0, :, off].float().cpu().numpy(), dec[0][row, :, 0])
            np.testing.assert_array_equal(
                layer.kv_pool_v[phys, 0, :, off].float().cpu().numpy(), dec[1][row, :, 0])
        gather = cache.gather_indices_for_layer(0)[:b].cpu().numpy()
        vis = cache.visible_lens_for_layer(0)[:b].cpu().numpy()
        ref = orc.sparse_attention(k_pool, v_pool, q.float().cpu().numpy(), gather,
                                   vis, np.arange(b), SCALE, cache.geometry.page)
        np.testing.assert_allclose(out.float().cpu().numpy(), ref, rtol=2e-2, atol=2e-3)
        print(f'# region mode {mode}: replay {step + 1} as the oracle', flush=True)
        del snap, k_pool, v_pool
        cache.commit_step()


def test_padded_capture_replays_live_rows_of_every_skip_state():
    lengths = [9000, 9100, 12000, 8000]
    skips = [(False, False), (True, False), (False, True), (True, True)]
    cache, gen, live = prod_cache(lengths, skips=skips, max_req=5)
    indexer = make_indexer()
    attn = attention_ns(indexer, SCALE)
    b = 5
    q = bf16_randn((b, cache.num_query_heads, 128), gen, GPU)
    padding = [-1] * b

    def run(rows):
        select_topk_for_layer_batched(cache, 0, rows, q, attention=attn)

    # capture on padding rows only: no live signature, region mode 0
    cache.new_step(padding)
    cache.plan_common(padding)
    assert cache.nfa_region_mode(cache.nfa_skip_signature(padding), 0) == 0
    run(padding)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        run(padding)
    rows = live + [-1]
    cache.new_step(rows)
    cache.plan_common(rows)
    torch.cuda.synchronize()
    snap = snapshot(cache, 0, b)
    graph.replay()
    torch.cuda.synchronize()
    replay = (cache.gather_indices_for_layer(0)[:b].clone(),
              cache.visible_lens_for_layer(0)[:b].clone())
    res, _, _ = run_oracle(cfg_from(cache, indexer, SCALE), snap,
                           q.float().cpu().numpy(), None, max_vis=1024, copy=False)
    _compare_rows(cache, res, len(live), 'padded capture replay')
    assert int(replay[1][len(live)].max()) == 0  # the padding row selects nothing
    run(rows)  # the same launch, eager
    torch.cuda.synchronize()
    w = cache.gather_indices_for_layer(0).shape[-1]
    for r in range(len(live)):
        for kv in range(cache.num_kv_heads):
            n = min(int(replay[1][r, kv]), w)
            assert int(cache.visible_lens_for_layer(0)[r, kv]) == int(replay[1][r, kv])
            assert torch.equal(cache.gather_indices_for_layer(0)[r, kv, :n],
                               replay[0][r, kv, :n])


@pytest.mark.parametrize('assign', ['mixed', 'near_skipped', 'both_skipped'])
def test_graph_runner_skip_signatures_match_eager(assign):
    from sparse_attn.engine.graph_runner import GraphRunner
    from sparse_attn.scheduler.scheduler import ContinuousBatchScheduler
    from test_batched_decode_gpu import PROMPTS, _prefilled

    skips = {'mixed': [(False, False), (True, False), (True, True)],
             'near_skipped': [(False, True)] * 3,
             'both_skipped': [(True, True)] * 3}[assign]
    want_mode = {'mixed': 0, 'near_skipped': 2, 'both_skipped': 3}[assign]
    steps = 4
    runs = {}
    for how in ('eager', 'graph'):
        print(f'# skip signature {assign}: {how} decode {steps} steps', flush=True)
        model, cache, rids, firsts = _prefilled()
        layers = model.config.num_hidden_layers
        for rid, (sf, sn) in zip(rids, skips):
            cache.freeze(rid, [sf] * layers, [sn] * layers)
        sig = cache.nfa_skip_signature(rids + [-1])
        assert cache.nfa_region_mode(sig, 0) == want_mode
        sched = ContinuousBatchScheduler(cache=cache, max_batch=4, eos_ids=(),
                                         pad_token_id=0, track_receipts=True)
        for rid, tok in zip(rids, firsts):
            sched.add_request(rid)
            sched.next_tokens[rid] = tok
        runner = GraphRunner(scheduler=sched, buckets=(4,), device=GPU)
        if how == 'graph':
            runner.capture_all(model, cache)
            assert all(key[2] == sig for key in runner.graphs)
        logits = []
        with torch.no_grad():
            for i in range(steps):
                out = runner.step(model, cache, generated_counts=i + 1)
                logits.append(out.logits[:len(rids)].float().clone())
        receipts = sched.flush_ready_receipts()
        if how == 'graph':
            assert runner.replay_count == steps and runner.eager_fallback_count == 0
        for rid, n in zip(rids, PROMPTS):
            assert cache.states[rid].logical_length == n + steps
        arena = [_token_rows(cache, li, rids) for li in range(layers)]
        runs[how] = (sorted(receipts), torch.stack(logits), arena)
        del runner, sched, cache, model
    assert runs['graph'][0] == runs['eager'][0]
    assert torch.equal(runs['graph'][1], runs['eager'][1])
    for (kg, vg), (ke, ve) in zip(runs['graph'][2], runs['eager'][2]):
        # every request's K/V rows, the decode tokens' included, are identical
        # (both regions skipped too)
        assert torch.equal(kg, ke) and torch.equal(vg, ve)


def _token_rows(cache, layer_idx, rids):
    """K and V rows of every logical token of the requests, in order, read
    through their block tables (slots never written hold no data)."""
    page = cache.geometry.page
    layer = cache.layers[layer_idx]
    ks, vs = [], []
    for rid in rids:
        n = cache.states[rid].logical_length
        table = cache.states[rid].block_tables[layer_idx]
        tok = torch.arange(n)
        phys = torch.tensor([table[int(t)] for t in tok // page], device=GPU)
        off = (tok % page).to(GPU)
        ks.append(layer.kv_pool_k[phys, 0, :, off].clone())
        vs.append(layer.kv_pool_v[phys, 0, :, off].clone())
    return torch.cat(ks), torch.cat(vs)
