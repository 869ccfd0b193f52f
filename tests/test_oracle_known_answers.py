"""The reference test-suite's known answers, checked on the CPU oracle.

The scenarios restate tests/test_nfa_current_query_selector.py of the
reference (counterfactual current-query block choice :150-184, numeric near
quota counts :226-275, L1/L2 dimension choice :340-396 and the strict region
oracle :434-497) and assert the same counts on the oracle.
"""
import numpy as np
import pytest
import torch

from nfa_case import (attention_ns, cfg_from, make_cache, make_indexer,
                      run_oracle, snapshot)
from sparse_attn.policies.region_geometry import RegionGeometry

PAGE = 64
GEOMETRY = RegionGeometry(sink=4, near=128, window=64, page=PAGE, max_new_tokens=8)


def _indexer(k1=4, near_pages=2, subspace='tail', l2_subspace='same',
             near_tokens='off'):
    return make_indexer(bs=64, k1=k1, near_pages=near_pages, k2=128, sink=4,
                        swa=GEOMETRY.window, near_len=GEOMETRY.near,
                        subspace=subspace, l2_subspace=l2_subspace,
                        near_tokens=near_tokens)


def _cache(keys, skip=(False, False), n=448):
    cache = make_cache('cpu', geometry=GEOMETRY, max_blocks=16,
                       max_physical_pages=64, max_visible_len=640, hkv=1, hq=2,
                       max_requests=8)
    cache.add_request(2)
    cache.write_prefill(0, 2, keys, torch.zeros_like(keys))
    cache.freeze(2, [skip[0]], [skip[1]])
    cache.new_step([2])
    cache.plan_common([2])
    return cache


def _select(cache, indexer, query, decode_key=None):
    cfg = cfg_from(cache, indexer, 1.0)
    snap = snapshot(cache, 0, 1)
    decode = None
    if decode_key is not None:
        slots = cache.slot_mapping_for_layer(0)[:1].numpy()
        decode = (decode_key.float().numpy(), np.zeros_like(decode_key.float().numpy()),
                  slots)
    res, _, _ = run_oracle(cfg, snap, query.float().numpy(), decode, max_vis=640)
    row = res[0][0]
    page = cache.geometry.page
    inverse = {phys: lp for lp, phys in cache.states[2].block_tables[0].items()}
    ids = sorted(inverse[int(s) // page] * page + int(s) % page
                 for s in row.gather[:row.vis_len])
    return ids, row


def _counterfactual_keys():
    keys = torch.zeros(1, 1, 448, 128, dtype=torch.bfloat16)
    keys[:, :, 64:128, 48] = 8
    keys[:, :, 192:256, 49] = 8
    return keys


def test_current_query_selects_its_own_block():
    cache = _cache(_counterfactual_keys())
    indexer = _indexer(k1=1, near_pages=0)
    gen = torch.Generator().manual_seed(20261102)
    dk = torch.randn(1, 1, 1, 128, generator=gen).to(torch.bfloat16)
    current = torch.zeros(1, 2, 128, dtype=torch.bfloat16)
    current[..., 48] = 1
    previous = torch.zeros_like(current)
    previous[..., 49] = 1
    cur_ids, _ = _select(cache, indexer, current, dk)
    assert sum(64 <= t < 128 for t in cur_ids) == 60
    assert not any(192 <= t < 256 for t in cur_ids)
    prev_ids, _ = _select(cache, indexer, previous, dk)
    assert sum(192 <= t < 256 for t in prev_ids) == 60
    assert not any(64 <= t < 128 for t in prev_ids)


def _fixed_quota(near_tokens, skip):
    keys = torch.zeros(1, 1, 448, 128, dtype=torch.bfloat16)
    keys[:, :, 4:256, 48] = 8
    keys[:, :, 256:384, 48] = 1
    cache = _cache(keys, skip)
    query = torch.zeros(1, 2, 128, dtype=torch.bfloat16)
    query[..., 48] = 1
    ids, _ = _select(cache, _indexer(k1=4, near_pages=2, near_tokens=near_tokens),
                     query)
    return (sum(4 <= t < 256 for t in ids), sum(256 <= t < 384 for t in ids),
            len(ids)), ids


def test_near_tokens_off_free_competition():
    counts, ids = _fixed_quota('off', (False, False))
    assert counts == (60, 0, 128)


@pytest.mark.parametrize('skip,expected', [
    ((False, False), (44, 16, 128)),
    ((True, False), (0, 60, 128)),
    ((False, True), (44, 0, 112)),
    ((True, True), (0, 0, 68)),
])
def test_numeric_near_quota_counts(skip, expected):
    counts, ids = _fixed_quota(16, skip)
    assert counts == expected
    assert ids == sorted(set(ids))


@pytest.mark.parametrize('subspace,l2_subspace,block', [
    ('full', 'same', 1), ('full', 'full', 1), ('tail', 'same', 3),
    ('tail', 'full', 3)])
def test_l1_l2_dimension_choice(subspace, l2_subspace, block):
    keys = torch.zeros(1, 1, 448, 128, dtype=torch.bfloat16)
    keys[:, :, 64:128, 0] = 16
    keys[:, :, 64:128, 48] = 1
    keys[:, :, 192:256, 48] = 8
    cache = _cache(keys)
    query = torch.zeros(1, 2, 128, dtype=torch.bfloat16)
    query[..., 0] = 1
    query[..., 48] = 1
    ids, _ = _select(cache, _indexer(k1=1, near_pages=0, subspace=subspace,
                                     l2_subspace=l2_subspace), query)
    lo = block * PAGE
    other = 192 if block == 1 else 64
    assert sum(lo <= t < lo + PAGE for t in ids) == 60
    assert not any(other <= t < other + PAGE for t in ids)


def _strict_region_oracle(length, skip_far, skip_near):
    sink_hi = min(GEOMETRY.sink, length)
    near_hi = max(sink_hi, length - GEOMETRY.window)
    far_hi = min(near_hi, max(sink_hi, ((length - GEOMETRY.window - GEOMETRY.near)
                                        // PAGE) * PAGE))
    protected = set(range(sink_hi)) | set(range(near_hi, length))
    selectable = set(range(sink_hi, far_hi)) | set(range(far_hi, near_hi))
    excluded = set()
    if skip_far:
        excluded |= set(range(sink_hi, far_hi))
    if skip_near:
        excluded |= set(range(far_hi, near_hi))
    return protected, selectable, excluded


@pytest.mark.parametrize('length', [448, 449, 510, 513])
@pytest.mark.parametrize('skip', [(False, False), (True, False), (False, True),
                                  (True, True)])
def test_strict_region_properties(length, skip):
    gen = torch.Generator().manual_seed(20261107 + length)
    keys = torch.randn(1, 1, length, 128, generator=gen).to(torch.bfloat16)
    cache = _cache(keys, skip, n=length)
    query = torch.randn(1, 2, 128, generator=gen).to(torch.bfloat16)
    ids, row = _select(cache, _indexer(), query)
    protected, selectable, excluded = _strict_region_oracle(length + 1, *skip)
    got = set(ids)
    assert len(ids) == len(got)
    assert protected <= got
    assert got <= protected | selectable
    assert not got & excluded
    if skip == (True, True):
        assert got == protected
