"""Selector and attention parity at the benchmarked workload shapes.

Each case builds the layer a benchmark configuration runs -- Qwen3-8B /
Llama-3.1-8B attention geometry (32 query / 8 KV heads, head_dim 128),
page = block = 16, the production NFA flags -- with the outlier-channel keys
of the benchmark (N(0,1) x a per-channel LogNormal(0,1) scale, RoPE theta 1e6
at the token positions), and compares the HIP path with the oracle:

* selector: far/near score bits, I_F / I_N, L2 bounds, every scored
  candidate and its logit bits, the middle selection, gather rows and
  visible lengths (all bit-exact), and the decode-written K/V rows;
* attention over the selected rows: rtol 2e-2 / atol 2e-3 (bf16 KV) or
  rtol 1e-4 / atol 1e-5 (fp32 KV) against the float64 oracle.

Workloads: 131072-token context at batch 1 with 20 incremental decode steps
(compared at the rebuild step and three incremental steps), a 32768-token
context with fp32 KV and fp32 queries, 16 requests of lengths drawn
uniformly from [32768, 131072] in one shared cache, and a 1M-token context
with the 32/8 heads (the multi-pass selector instance whose tiles list their
own top-K pages for the tail).

Every workload also runs the production launch -- no debug buffers, the
launch the benchmarks and the model patches time -- for at least one step,
whose gather rows, visible lengths and decode-written rows are compared with
the oracle.
"""
from types import SimpleNamespace

import numpy as np
import pytest
import torch

from bench import synthetic_keys
from nfa_case import (GPU, attention_ns, bf16_randn, make_indexer, prod_cache,
                      run_and_compare)
from oracle import nfa_oracle as orc
from sparse_attn.indexer.nfa_layer_batch_selector import \
    select_topk_for_layer_batched
from sparse_attn.ops.paged_region_kernels_nfa import decode_graph_ready
from sparse_attn.policies.region_geometry import RegionGeometry

pytestmark = pytest.mark.gpu

HQ, HKV, D = 32, 8, 128
SCALE = D ** -0.5


def _outlier_keys(n, hkv, d, gen):
    return synthetic_keys(torch, n, hkv, d, gen, GPU, dtype=torch.float32)


def _decode_token(cache, b, gen, dtype, positions):
    """Current-token K (outlier recipe at the row's position) and V."""
    keys = torch.cat([synthetic_keys(torch, 1, HKV, D, gen, GPU, start=p,
                                     dtype=dtype)[0].transpose(0, 1)
                      for p in positions])           # [b, hkv, d]
    keys = keys.unsqueeze(2).contiguous()            # [b, hkv, 1, d]
    values = torch.randn(b, HKV, 1, D, generator=gen, device=GPU).to(dtype)
    slots = cache.slot_mapping_for_layer(0)[:b].clone()
    return keys, values, slots


def _check_attention(cache, q, k_pool, v_pool, rows, dtype):
    """Attention over the selected rows vs the float64 oracle on the
    oracle's post-write pools."""
    out = decode_graph_ready(SimpleNamespace(layer_idx=0, scaling=SCALE), q, cache)
    torch.cuda.synchronize()
    gather = cache.gather_indices_for_layer(0)[:rows].cpu().numpy()
    vis = cache.visible_lens_for_layer(0)[:rows].cpu().numpy()
    ref = orc.sparse_attention(k_pool, v_pool, q.float().cpu().numpy(), gather,
                               vis, np.arange(rows), SCALE, cache.geometry.page)
    got = out.float().cpu().numpy()
    if dtype == torch.bfloat16:
        np.testing.assert_allclose(got, ref, rtol=2e-2, atol=2e-3)
    else:
        np.testing.assert_allclose(got, ref, rtol=1e-4, atol=1e-5)


def test_128k_context_batch1_incremental_steps():
    """131072-token context, 32/8 heads, bf16: 20 decode steps, the first
    one rebuilding the page statistics and the rest incremental; the full
    comparison at steps 1, 10 and 20, attention at step 20."""
    length = 131072
    geo = RegionGeometry(sink=4, near=4096, window=128, page=16, max_new_tokens=32)
    cache, gen, req_ids = prod_cache([length], hkv=HKV, hq=HQ, max_req=1,
                                     geometry=geo, key_fn=_outlier_keys)
    indexer = make_indexer()
    print('# 128K workload ready', flush=True)
    for step in range(20):
        cache.new_step(req_ids)
        cache.plan_common(req_ids)
        q = bf16_randn((1, HQ, D), gen, GPU)
        decode = _decode_token(cache, 1, gen, torch.bfloat16, [length + step])
        if step == 14:
            # the production launch (no debug buffers), incremental statistics
            plan = {}
            res = run_and_compare(cache, indexer, req_ids, q, decode,
                                  scaling=SCALE, check_debug=False, plan=plan)
            assert plan['instance'] == 0 and plan['passes'] == 1, plan
            assert all(res[0][kv].vis_len == 1024 for kv in range(HKV))
            print('# 128K step 15 (production launch): selections bit-exact',
                  flush=True)
        elif step in (0, 9, 19):
            res, k_pool, v_pool = run_and_compare(
                cache, indexer, req_ids, q, decode, scaling=SCALE,
                return_pools=True)
            assert all(res[0][kv].vis_len == 1024 for kv in range(HKV))
            assert all(res[0][kv].quota == 892 for kv in range(HKV))
            print(f'# 128K step {step + 1}: selections bit-exact', flush=True)
            if step == 19:
                _check_attention(cache, q, k_pool, v_pool, 1, torch.bfloat16)
            del k_pool, v_pool
        else:
            select_topk_for_layer_batched(cache, 0, req_ids, q,
                                          attention=attention_ns(indexer, SCALE),
                                          decode_write=decode)
        cache.commit_step()


def test_32k_context_fp32_kv():
    """32768-token context with fp32 KV and fp32 queries, 32/8 heads."""
    length = 32768
    cache, gen, req_ids = prod_cache([length], hkv=HKV, hq=HQ, max_req=1,
                                     dtype=torch.float32, key_fn=_outlier_keys)
    indexer = make_indexer()
    cache.new_step(req_ids)
    cache.plan_common(req_ids)
    q = torch.randn(1, HQ, D, generator=gen, device=GPU)
    decode = _decode_token(cache, 1, gen, torch.float32, [length])
    res, k_pool, v_pool = run_and_compare(cache, indexer, req_ids, q, decode,
                                          scaling=SCALE, return_pools=True)
    assert all(res[0][kv].vis_len == 1024 for kv in range(HKV))
    _check_attention(cache, q, k_pool, v_pool, 1, torch.float32)


def test_16_ragged_requests_32k_to_128k():
    """16 requests with lengths U(32768, 131072) in one shared cache: the
    rebuild step through the production launch, the next (incremental) step
    with every debug output and attention."""
    lengths = torch.randint(32768, 131073, (16,),
                            generator=torch.Generator().manual_seed(20261201)).tolist()
    cache, gen, req_ids = prod_cache(lengths, hkv=HKV, hq=HQ, max_req=16,
                                     key_fn=_outlier_keys)
    indexer = make_indexer()
    print(f'# 16 ragged requests, {sum(lengths)} tokens', flush=True)
    for step in range(2):
        cache.new_step(req_ids)
        cache.plan_common(req_ids)
        q = bf16_randn((16, HQ, D), gen, GPU)
        decode = _decode_token(cache, 16, gen, torch.bfloat16,
                               [n + step for n in lengths])
        plan = {}
        res, k_pool, v_pool = run_and_compare(cache, indexer, req_ids, q, decode,
                                              scaling=SCALE, return_pools=True,
                                              check_debug=step == 1, plan=plan)
        assert plan['instance'] == 1, plan  # multi-pass tiles, no page lists
        assert all(res[r][kv].vis_len == 1024 for r in range(16) for kv in range(HKV))
        print(f'# 16 ragged step {step + 1} (debug {step == 1}): selections '
              'bit-exact', flush=True)
        if step == 1:
            _check_attention(cache, q, k_pool, v_pool, 16, torch.bfloat16)
        del k_pool, v_pool
        cache.commit_step()


def test_1m_context_8_kv_heads_page_lists():
    """1M-token context (plus 8192 tokens, so that every near-pool page id
    passes 16 bits) with the benchmark's 32/8 heads: 32 tiles per row of 5
    passes each, whose tiles list their own top-K pages for the tail (the
    instance the 1M benchmark times).  The rebuild step is compared with
    every debug output, the next (incremental) step through the production
    launch."""
    length = (1 << 20) + 8192
    geo = RegionGeometry(sink=4, near=4096, window=128, page=16, max_new_tokens=32)
    cache, gen, req_ids = prod_cache([length], hkv=HKV, hq=HQ, max_req=1,
                                     geometry=geo, key_fn=_outlier_keys)
    indexer = make_indexer()
    print('# 1M workload (8 kv heads) ready', flush=True)
    for step in range(2):
        cache.new_step(req_ids)
        cache.plan_common(req_ids)
        q = bf16_randn((1, HQ, D), gen, GPU)
        decode = _decode_token(cache, 1, gen, torch.bfloat16, [length + step])
        plan = {}
        res = run_and_compare(cache, indexer, req_ids, q, decode, scaling=SCALE,
                              check_debug=step == 0, with_v=False, plan=plan)
        assert plan['instance'] == 2 and plan['round_tiles'] == 32, plan
        assert plan['passes'] == 5, plan
        for kv in range(HKV):
            r = res[0][kv]
            assert r.vis_len == 1024
            # the near pool's pages (and its page-list entries) lie past
            # 16-bit ids; far pages reach 65783 at this length
            assert int(r.i_n.min()) > 65535
        print(f'# 1M step {step + 1} (debug {step == 0}): selections bit-exact',
              flush=True)
        del res
        cache.commit_step()
