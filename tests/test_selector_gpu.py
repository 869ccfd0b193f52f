"""Bit-exact parity of the HIP selector with the CPU oracle.

Every case runs ``select_topk_for_layer_batched`` through libnfa_hip.so on
the GPU and the oracle on a snapshot of the same cache, then compares: L1
far/near score bits, I_F / I_N, L2 bounds, the scored candidates and their
logit bits, the middle selection, the final physical gather rows and
visible lengths (all exact), plus the decode-written K/V rows.
"""
import numpy as np
import pytest
import torch

from nfa_case import (GEO16, attention_ns, bf16_randn, cfg_from,
                      decode_inputs, make_indexer, prefill_request, prod_cache,
                      run_and_compare, run_oracle, snapshot, u16)
from sparse_attn.indexer.nfa_layer_batch_selector import \
    select_topk_for_layer_batched
from sparse_attn.policies.region_geometry import RegionGeometry

pytestmark = pytest.mark.gpu

DEV = 'cuda'


_prefill = prefill_request
_decode_inputs = decode_inputs
_u16 = u16
_prod_cache = prod_cache


@pytest.mark.parametrize('lengths', [[20000], [9000, 20500], [5000, 700, 12345]])
def test_production_flags_bit_exact(lengths):
    cache, gen, req_ids = _prod_cache(lengths)
    indexer = make_indexer()
    b = len(req_ids)
    cache.new_step(req_ids)
    cache.plan_common(req_ids)
    q = bf16_randn((b, cache.num_query_heads, 128), gen, DEV)
    decode = _decode_inputs(cache, b, gen, torch.bfloat16)
    run_and_compare(cache, indexer, req_ids, q, decode, scaling=0.08838834764831845)


def test_sixteen_ragged_requests():
    """The batched decode shape: 16 requests of ragged lengths in one cache."""
    lengths = torch.randint(3000, 24001, (16,),
                            generator=torch.Generator().manual_seed(16)).tolist()
    cache, gen, req_ids = _prod_cache(lengths, max_req=16)
    indexer = make_indexer()
    cache.new_step(req_ids)
    cache.plan_common(req_ids)
    q = bf16_randn((16, cache.num_query_heads, 128), gen, DEV)
    decode = _decode_inputs(cache, 16, gen, torch.bfloat16)
    run_and_compare(cache, indexer, req_ids, q, decode, scaling=0.08838834764831845)


def test_one_million_token_context():
    """1M-token row (plus 8192, so that the near pool's pages have ids past
    16 bits): 66048 pages over several dispatch rounds of tiles, the L1
    top-k over every page."""
    cache, gen, req_ids = _prod_cache([(1 << 20) + 8192], hkv=1, hq=4, max_req=1)
    indexer = make_indexer()
    cache.new_step(req_ids)
    cache.plan_common(req_ids)
    q = bf16_randn((1, 4, 128), gen, DEV)
    decode = _decode_inputs(cache, 1, gen, torch.bfloat16)
    print('# 1M context: selector + oracle', flush=True)
    res = run_and_compare(cache, indexer, req_ids, q, decode,
                          scaling=0.08838834764831845)
    assert res[0][0].vis_len == 1024
    assert int(res[0][0].i_n.min()) > 65535  # near pages past 16-bit ids


@pytest.mark.parametrize('zero_keys', [False, True])
def test_long_and_short_rows_in_one_launch(zero_keys):
    """A row of 19375 pages (past 16384: its tiles list their own top-K
    pages for the tail) beside a short row that leaves the tail every key,
    in the multi-pass instance; with all-zero keys (ties everywhere) every
    page of the long row survives its tile and the tail reads every key."""
    cache, gen, req_ids = _prod_cache([310000, 20000], hkv=2, hq=8, max_req=2,
                                      zero_keys=zero_keys)
    indexer = make_indexer()
    cache.new_step(req_ids)
    cache.plan_common(req_ids)
    q = bf16_randn((2, 8, 128), gen, DEV)
    decode = _decode_inputs(cache, 2, gen, torch.bfloat16)
    print(f'# long and short rows (zero keys {zero_keys}): selector + oracle', flush=True)
    res = run_and_compare(cache, indexer, req_ids, q, decode,
                          scaling=0.08838834764831845)
    assert res[0][0].vis_len == 1024 and res[1][0].vis_len == 1024


@pytest.mark.parametrize('side_copy', [True, False])
def test_l2_from_side_copy_or_k_pool(side_copy):
    # the L2 logits read the L2 side copy, or the K pool when it is off
    cache, gen, req_ids = _prod_cache([9000, 20500])
    cache.nfa_l2_side_copy = side_copy
    indexer = make_indexer()
    cache.new_step(req_ids)
    cache.plan_common(req_ids)
    q = bf16_randn((2, cache.num_query_heads, 128), gen, DEV)
    decode = _decode_inputs(cache, 2, gen, torch.bfloat16)
    run_and_compare(cache, indexer, req_ids, q, decode, scaling=0.08838834764831845)


def test_incremental_side_rows_become_candidates():
    # tokens appended by incremental steps leave the 128-token window and
    # are scored from the side rows those steps wrote
    geo = RegionGeometry(sink=4, near=4096, window=128, page=16,
                         max_new_tokens=256)
    cache, gen, req_ids = _prod_cache([3000], geometry=geo)
    indexer = make_indexer()
    for step in range(150):
        cache.new_step(req_ids)
        cache.plan_common(req_ids)
        q = bf16_randn((1, cache.num_query_heads, 128), gen, DEV)
        decode = _decode_inputs(cache, 1, gen, torch.bfloat16)
        if step < 149:
            select_topk_for_layer_batched(cache, 0, req_ids, q,
                                          attention=attention_ns(indexer, 1.0),
                                          decode_write=decode)
        else:
            run_and_compare(cache, indexer, req_ids, q, decode)
        cache.commit_step()


@pytest.mark.parametrize('lengths,subspace', [([20000], 'tail'), ([5000, 700, 12345], 'tail'),
                                              ([20000], 'rope'), ([5000, 700, 12345], 'rope')])
def test_l2_quant_4bit_keys_bit_exact(lengths, subspace):
    """--nfa_l2_quant: L2 logits over the packed 4-bit side cache (written by
    the statistics rebuild) against the oracle's min_max_per_token_quant
    semantics: every candidate's logit bits, the middle and the gather; 32
    L2 dims (tail subspace) and 64 (rope subspace)."""
    cache, gen, req_ids = _prod_cache(lengths)
    indexer = make_indexer(l2_quant=True, subspace=subspace)
    b = len(req_ids)
    cache.new_step(req_ids)
    cache.plan_common(req_ids)
    q = bf16_randn((b, cache.num_query_heads, 128), gen, DEV)
    decode = _decode_inputs(cache, b, gen, torch.bfloat16)
    run_and_compare(cache, indexer, req_ids, q, decode, scaling=0.08838834764831845)


@pytest.mark.parametrize('subspace', ['tail', 'rope'])
def test_l2_quant_incremental_rows_and_raw_differ(subspace):
    """4-bit rows written by decode steps (32 or 64 lanes quantising the new
    token) become candidates and score as the oracle's quantised keys; the
    4-bit and raw modes pick different tokens (so the flag is live)."""
    geo = RegionGeometry(sink=4, near=4096, window=128, page=16,
                         max_new_tokens=256)
    # long enough that the L2 quota (892) is below the candidate count, so
    # the logits decide
    cache, gen, req_ids = _prod_cache([12000], geometry=geo)
    indexer = make_indexer(l2_quant=True, subspace=subspace)
    for step in range(150):
        cache.new_step(req_ids)
        cache.plan_common(req_ids)
        q = bf16_randn((1, cache.num_query_heads, 128), gen, DEV)
        decode = _decode_inputs(cache, 1, gen, torch.bfloat16)
        if step < 149:
            select_topk_for_layer_batched(cache, 0, req_ids, q,
                                          attention=attention_ns(indexer, 1.0),
                                          decode_write=decode)
            cache.commit_step()
        else:
            res = run_and_compare(cache, indexer, req_ids, q, decode)
    raw, _, _ = run_oracle(cfg_from(cache, make_indexer(subspace=subspace), 1.0),
                           snapshot(cache, 0, 1),
                           q.float().cpu().numpy(), None, max_vis=1024)
    assert any(not np.array_equal(res[0][kv].middle, raw[0][kv].middle)
               for kv in range(cache.num_kv_heads))


def test_l2_quant_rejects_unsupported_geometry():
    cache, gen, req_ids = _prod_cache([3000])
    cache.new_step(req_ids)
    cache.plan_common(req_ids)
    q = bf16_randn((1, cache.num_query_heads, 128), gen, DEV)
    wide = make_indexer(l2_quant=True, l2_subspace='full')  # 128 L2 dims
    with pytest.raises(ValueError, match='l2_quant'):
        select_topk_for_layer_batched(cache, 0, req_ids, q,
                                      attention=attention_ns(wide, 1.0))
    cache.nfa_l2_side_copy = False
    with pytest.raises(ValueError, match='side cache'):
        select_topk_for_layer_batched(cache, 0, req_ids, q,
                                      attention=attention_ns(make_indexer(l2_quant=True),
                                                             1.0))


def test_incremental_stats_over_decode_steps():
    cache, gen, req_ids = _prod_cache([6000, 6015])
    indexer = make_indexer()
    for step in range(20):
        cache.new_step(req_ids)
        cache.plan_common(req_ids)
        q = bf16_randn((2, cache.num_query_heads, 128), gen, DEV)
        decode = _decode_inputs(cache, 2, gen, torch.bfloat16)
        run_and_compare(cache, indexer, req_ids, q, decode,
                        check_debug=step % 5 == 0)
        cache.commit_step()


def test_mixed_skip_states_padding_rows_and_noncontiguous_slots():
    lengths = [4500, 4501, 5100, 5133]
    skips = [(False, False), (True, False), (False, True), (True, True)]
    cache, gen, _ = _prod_cache(lengths, skips=skips, req_ids=[1, 3, 6, 7],
                                max_req=8)
    indexer = make_indexer()
    req_ids = [1, -1, 3, 6, 7]
    cache.new_step(req_ids)
    cache.plan_common(req_ids)
    q = bf16_randn((5, cache.num_query_heads, 128), gen, DEV)
    decode = _decode_inputs(cache, 5, gen, torch.bfloat16)
    run_and_compare(cache, indexer, req_ids, q, decode)


@pytest.mark.parametrize('skip', [(False, True), (True, False)])
def test_uniform_skip_state_long_rows(skip):
    """Every row skips the same region (region modes 1 and 2), with far and
    near pools both long enough to matter."""
    cache, gen, req_ids = _prod_cache([9001, 20000], skips=[skip] * 2)
    indexer = make_indexer()
    cache.new_step(req_ids)
    cache.plan_common(req_ids)
    q = bf16_randn((2, cache.num_query_heads, 128), gen, DEV)
    decode = _decode_inputs(cache, 2, gen, torch.bfloat16)
    run_and_compare(cache, indexer, req_ids, q, decode, scaling=0.08838834764831845)


def _hot_cache(length, hot):
    """One request whose keys are zero except 1.0 in every L1/L2 dim for the
    tokens of `hot` (a range); queries of ones then score those tokens (and
    their pages) above all others, and every other score ties."""
    from nfa_case import indexer_dims
    cache, gen, req_ids = _prod_cache([length], zero_keys=True)
    dims, _ = indexer_dims(make_indexer())
    layer = cache.layers[0]
    page = cache.geometry.page
    table = cache.states[0].block_tables[0]
    for t in hot:
        layer.kv_pool_k[table[t // page], 0, :, t % page, torch.as_tensor(dims)] = 1.0
    return cache, gen, req_ids


@pytest.mark.parametrize('case', ['l2_quota_fills_a_bin', 'l1_budget_fills_a_bin'])
def test_threshold_bin_taken_whole(case):
    """The K-th largest key closes its high-byte bin exactly: exactly 892
    tokens (the L2 quota) or exactly 96 far pages (K_F) score above all the
    rest, all tied.  The second-level threshold pass must then take the whole
    bin."""
    hot = range(16, 16 + 892) if case == 'l2_quota_fills_a_bin' else range(16, 16 + 96 * 16)
    cache, gen, req_ids = _hot_cache(9000, hot)
    indexer = make_indexer()
    cache.new_step(req_ids)
    cache.plan_common(req_ids)
    q = torch.ones((1, cache.num_query_heads, 128), dtype=torch.bfloat16, device=DEV)
    keys, values, slots = _decode_inputs(cache, 1, gen, torch.bfloat16)
    res = run_and_compare(cache, indexer, req_ids, q, (keys * 0, values, slots))
    r = res[0][0]
    if case == 'l2_quota_fills_a_bin':
        assert r.count == 892 and set(r.middle[:892]) == set(hot)
    else:
        assert sorted(r.i_f) == list(range(1, 97))


def test_all_both_skip_uses_protected_path():
    cache, gen, req_ids = _prod_cache([3000, 4100], skips=[(True, True)] * 2)
    indexer = make_indexer()
    cache.new_step(req_ids)
    cache.plan_common(req_ids)
    q = bf16_randn((2, cache.num_query_heads, 128), gen, DEV)
    decode = _decode_inputs(cache, 2, gen, torch.bfloat16)
    run_and_compare(cache, indexer, req_ids, q, decode)


def test_ties_everywhere_lowest_index_wins():
    cache, gen, req_ids = _prod_cache([7000], zero_keys=True)
    indexer = make_indexer()
    cache.new_step(req_ids)
    cache.plan_common(req_ids)
    q = bf16_randn((1, cache.num_query_heads, 128), gen, DEV)
    run_and_compare(cache, indexer, req_ids, q, None)


def test_fixed_near_token_quota():
    cache, gen, req_ids = _prod_cache([9000, 6000])
    indexer = make_indexer(near_tokens=256)
    cache.new_step(req_ids)
    cache.plan_common(req_ids)
    q = bf16_randn((2, cache.num_query_heads, 128), gen, DEV)
    decode = _decode_inputs(cache, 2, gen, torch.bfloat16)
    run_and_compare(cache, indexer, req_ids, q, decode)


def test_middle_only_output():
    cache, gen, req_ids = _prod_cache([8000])
    indexer = make_indexer()
    cache.new_step(req_ids)
    cache.plan_common(req_ids)
    q = bf16_randn((1, cache.num_query_heads, 128), gen, DEV)
    run_and_compare(cache, indexer, req_ids, q, None, middle_only=True)


@pytest.mark.parametrize('subspace,l2', [('full', 'same'), ('rope', 'same'),
                                         ('tail', 'full'), ('nope', 'full')])
def test_subspace_variants(subspace, l2):
    cache, gen, req_ids = _prod_cache([7000])
    indexer = make_indexer(subspace=subspace, l2_subspace=l2)
    cache.new_step(req_ids)
    cache.plan_common(req_ids)
    q = bf16_randn((1, cache.num_query_heads, 128), gen, DEV)
    decode = _decode_inputs(cache, 1, gen, torch.bfloat16)
    run_and_compare(cache, indexer, req_ids, q, decode)


def test_fp32_kv_and_query():
    cache, gen, req_ids = _prod_cache([6000], dtype=torch.float32)
    indexer = make_indexer(far_method='avg', near_method='minmax')
    cache.new_step(req_ids)
    cache.plan_common(req_ids)
    q = bf16_randn((1, cache.num_query_heads, 128), gen, DEV).float()
    decode = _decode_inputs(cache, 1, gen, torch.float32)
    run_and_compare(cache, indexer, req_ids, q, decode, scaling=0.0883883)


@pytest.mark.parametrize('far,near', [('avg', 'minmax'), ('minmax', 'minmax'),
                                      ('avg', 'avg')])
def test_pool_methods_with_staged_bf16_statistics(far, near):
    """Each pool's method swapped on bf16 statistics, which are staged in LDS
    and scored one lane per page in 64-page groups that never hold pages of
    both pools (at these lengths the near pool's first page lies inside a
    64-page stretch of its tile), and the 60000-token row's tiles take two
    passes (32 rows share the launch: 8 tiles per row, at most 448 pages a
    pass)."""
    lengths = [60000, 9000, 33000, 700]
    cache, gen, req_ids = _prod_cache(lengths, hkv=8, hq=32, max_req=4)
    indexer = make_indexer(far_method=far, near_method=near)
    cache.new_step(req_ids)
    cache.plan_common(req_ids)
    q = bf16_randn((4, 32, 128), gen, DEV)
    decode = _decode_inputs(cache, 4, gen, torch.bfloat16)
    plan = {}
    print(f'# pool methods far {far} / near {near}: selector + oracle', flush=True)
    run_and_compare(cache, indexer, req_ids, q, decode,
                    scaling=0.08838834764831845, plan=plan)
    assert plan['instance'] == 1 and plan['passes'] > 1, plan


def test_short_contexts_below_window():
    cache, gen, req_ids = _prod_cache([40, 100, 140, 300])
    indexer = make_indexer()
    cache.new_step(req_ids)
    cache.plan_common(req_ids)
    q = bf16_randn((4, cache.num_query_heads, 128), gen, DEV)
    decode = _decode_inputs(cache, 4, gen, torch.bfloat16)
    run_and_compare(cache, indexer, req_ids, q, decode)


@pytest.mark.parametrize('dtype', [torch.bfloat16, torch.float32])
def test_avg_top2_far_scores(dtype):
    """--nfa_far_method avg_top2 (selector:2412-2427): far scores from the two
    largest per-head page means against the unrounded query, bit-exact with
    the oracle in the staged bf16 path and the fp32 statistics path."""
    cache, gen, req_ids = _prod_cache([20000, 9001], dtype=dtype)
    indexer = make_indexer(far_method='avg_top2')
    cache.new_step(req_ids)
    cache.plan_common(req_ids)
    q = bf16_randn((2, cache.num_query_heads, 128), gen, DEV).to(dtype)
    decode = _decode_inputs(cache, 2, gen, dtype)
    run_and_compare(cache, indexer, req_ids, q, decode, scaling=0.08838834764831845)


def test_avg_top2_needs_two_heads_per_group():
    cache, gen, req_ids = _prod_cache([3000], hkv=2, hq=2)
    cache.new_step(req_ids)
    cache.plan_common(req_ids)
    q = bf16_randn((1, 2, 128), gen, DEV)
    with pytest.raises(ValueError, match='avg_top2'):
        select_topk_for_layer_batched(
            cache, 0, req_ids, q,
            attention=attention_ns(make_indexer(far_method='avg_top2'), 1.0))


@pytest.mark.parametrize('lengths,hkv,hq,instance', [
    ([20000], 2, 8, 0),         # single-pass tiles
    ([540000], 8, 32, 2),       # multi-pass tiles listing their top-K pages
])
def test_block_smaller_than_page_scores_block_table_width(lengths, hkv, hq, instance):
    """--tia_block_size 16 over 32-token pages: ceil(L / 16) exceeds the
    block-table width, and only its first max_blocks L1 blocks are scored
    (selector:205-206).  The tiles split those pages; the tail's key scans
    and the page lists of long rows (second case, 16886 pages per row) must
    cover exactly them."""
    geo = RegionGeometry(sink=4, near=4096, window=128, page=32, max_new_tokens=64)
    cache, gen, req_ids = _prod_cache(lengths, hkv=hkv, hq=hq, max_req=1,
                                      geometry=geo)
    assert -(-lengths[0] // 16) > cache.max_blocks
    indexer = make_indexer()
    cache.new_step(req_ids)
    cache.plan_common(req_ids)
    q = bf16_randn((1, hq, 128), gen, DEV)
    decode = _decode_inputs(cache, 1, gen, torch.bfloat16)
    plan = {}
    print(f'# block 16 / page 32, {lengths[0]} tokens: selector + oracle', flush=True)
    run_and_compare(cache, indexer, req_ids, q, decode,
                    scaling=0.08838834764831845, plan=plan, with_v=False)
    assert plan['instance'] == instance, plan


def test_handover_over_incremental_production_steps():
    """Regression test of the cross-workgroup hand-over without the L2
    writeback: 30 incremental decode steps through the production launch
    (the tiles hand keys, page lists and histograms to the tail through
    device-scope stores and atomics), on 6 rows whose tiles spread over
    several XCDs (workgroup row + 6 * tile), every step compared with the
    oracle."""
    cache, gen, req_ids = _prod_cache([9000, 20500, 14000], max_req=3)
    indexer = make_indexer()
    for step in range(30):
        cache.new_step(req_ids)
        cache.plan_common(req_ids)
        q = bf16_randn((3, cache.num_query_heads, 128), gen, DEV)
        decode = _decode_inputs(cache, 3, gen, torch.bfloat16)
        run_and_compare(cache, indexer, req_ids, q, decode,
                        scaling=0.08838834764831845, check_debug=False)
        cache.commit_step()


def test_batch_wider_than_the_output_rows_is_rejected():
    """A batch of more rows than the cache's gather rows (request slots) is
    rejected before any launch instead of writing past them."""
    cache, gen, req_ids = _prod_cache([3000, 3100], max_req=2)
    rows = req_ids + [-1]   # within max_query_tokens, beyond max_requests
    cache.new_step(rows)
    cache.plan_common(rows)
    q = bf16_randn((3, cache.num_query_heads, 128), gen, DEV)
    before = cache.gather_indices_buf.clone()
    with pytest.raises(ValueError, match='selection outputs hold 2 rows'):
        select_topk_for_layer_batched(cache, 0, rows, q,
                                      attention=attention_ns(make_indexer(), 1.0))
    torch.cuda.synchronize()
    assert torch.equal(cache.gather_indices_buf, before)
