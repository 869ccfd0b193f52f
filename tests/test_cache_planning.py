"""Host-side step planning of the paged cache (CPU).

Every decode step, each live row's slot (per layer) must be the physical
slot of its new token through the block table: page ``len // page`` of the
row's request at offset ``len % page``.  Steady steps move slots by one on
the device and append a page for rows whose token opens one; the check runs
over many steps with ragged lengths (rows crossing pages on different steps),
a padding row, and a layout change half way.
"""
import pytest
import torch

from nfa_case import make_cache
from sparse_attn.cache import RequestPhase
from sparse_attn.policies.region_geometry import RegionGeometry

GEO = RegionGeometry(sink=4, near=64, window=16, page=16, max_new_tokens=80)


def _expect_slots(cache, req_ids):
    # slots are indexed by query token: live rows in batch order
    page = cache.geometry.page
    tok = 0
    for b, rid in enumerate(req_ids):
        if rid < 0:
            assert int(cache.planned_lengths_buf[b]) == 0
            continue
        state = cache.states[rid]
        pos = cache.pending_lengths[rid] - 1
        assert pos == state.logical_length
        for layer in range(cache.n_layers):
            pid = state.block_tables[layer][pos // page]
            assert int(cache.block_table_buf[layer, rid, pos // page]) == pid
            assert int(cache.slot_mapping_buf[layer, tok]) == pid * page + pos % page, \
                (layer, b, rid, pos)
        assert int(cache.planned_lengths_buf[b]) == pos + 1
        assert int(cache.query_to_req_buf[tok]) == b
        tok += 1
    for layer in range(cache.n_layers):
        assert (cache.slot_mapping_buf[layer, tok:len(req_ids)] == -1).all()


def test_steady_steps_append_pages_and_move_slots():
    lengths = {0: 100, 1: 111, 3: 96, 5: 47}
    cache = make_cache('cpu', geometry=GEO, n_layers=3, max_requests=6,
                       max_blocks=16, max_physical_pages=80, hkv=1, hq=2,
                       head_dim=16, dtype=torch.float32, max_query_tokens=8)
    for rid, n in lengths.items():
        cache.add_request(rid)
        for layer in range(3):
            k = torch.randn(1, 1, n, 16)
            cache.write_prefill(layer, rid, k, k)
        cache.freeze(rid, [False] * 3, [False] * 3)
    layouts = [[0, 1, -1, 3], [5, 0, 1, 3]]
    crossings = 0
    for step in range(60):
        req_ids = layouts[0] if step < 30 else layouts[1]
        cache.new_step(req_ids)
        crossings += cache.step_opens_page
        cache.plan_common(req_ids)
        _expect_slots(cache, req_ids)
        cache.commit_step()
    assert crossings >= 8
    # every request's pages: distinct per layer, and never shared by requests
    for layer in range(3):
        seen = set()
        for rid in lengths:
            pids = list(cache.states[rid].block_tables[layer].values())
            assert len(set(pids)) == len(pids)
            assert not seen & set(pids)
            seen |= set(pids)


def _small_cache(n_layers=2, max_requests=3, max_visible_len=64):
    return make_cache('cpu', geometry=GEO, n_layers=n_layers,
                      max_requests=max_requests, max_blocks=16,
                      max_physical_pages=40, hkv=2, hq=4, head_dim=16,
                      dtype=torch.float32, max_query_tokens=4,
                      max_visible_len=max_visible_len)


def _prefill_cpu(cache, rid, n, skips=None):
    cache.add_request(rid)
    for layer in range(cache.n_layers):
        k = torch.randn(1, cache.num_kv_heads, n, 16)
        cache.write_prefill(layer, rid, k, k)
    far, near = skips or ([False] * cache.n_layers, [False] * cache.n_layers)
    cache.freeze(rid, far, near)


def _logical(cache, layer, b, rid, width):
    page = cache.geometry.page
    inverse = {pid: lp for lp, pid in cache.states[rid].block_tables[layer].items()}
    slots = cache.gather_indices_buf[layer, b, 0, :width].tolist()
    assert cache.gather_indices_buf[layer, b, 1, :width].tolist() == slots
    return [inverse[s // page] * page + s % page for s in slots]


def test_dense_and_given_gather_rows():
    """Dense rows are the kept region intervals (RegionGeometry.bounds) at
    the planned length; given ids map through the block table; a padding
    row gets length 0."""
    cache = _small_cache(max_visible_len=200)
    # layer 0 keeps everything, layer 1 skips the far region
    _prefill_cpu(cache, 0, 150, ([False, True], [False, False]))
    rows = [0, -1]
    cache.new_step(rows)
    cache.plan_common(rows)
    gather, lens = cache.prepare_metadata(rows, 0)
    length = 151
    assert lens[0].tolist() == [length, length] and lens[1].tolist() == [0, 0]
    assert _logical(cache, 0, 0, 0, length) == list(range(length))
    cache.prepare_metadata(rows, 1)
    sink_hi, far_hi, near_hi = GEO.bounds(length)
    want = list(range(sink_hi)) + list(range(far_hi, length))
    assert far_hi > sink_hi  # the far region is non-empty, so skipping it matters
    assert int(cache.visible_lens_buf[1, 0, 0]) == len(want)
    assert _logical(cache, 1, 0, 0, len(want)) == want
    # given ids, and (ids, count) with the count as the visible length
    cache.prepare_metadata(rows, 0, selected_ids_by_req={0: [3, 40, 149]})
    assert _logical(cache, 0, 0, 0, 3) == [3, 40, 149]
    ids = torch.tensor([7, 9, 100, 0])
    cache.prepare_metadata(rows, 0, selected_ids_by_req={0: (ids, torch.tensor(3))})
    assert int(cache.visible_lens_buf[0, 0, 0]) == 3
    assert _logical(cache, 0, 0, 0, 4) == [7, 9, 100, 0]


def test_prepare_all_layers_fills_the_visible_bucket():
    cache = _small_cache(max_visible_len=200)
    _prefill_cpu(cache, 1, 60)
    rows = [1]
    cache.new_step(rows)
    cache.prepare_all_layers(rows, visible_bucket=64)
    assert cache.active_visible_bucket == 64
    for layer in range(2):
        assert cache.visible_lens_for_layer(layer)[0].tolist() == [61, 61]
        assert torch.equal(cache.gather_indices_for_layer(layer)[0],
                           cache.gather_indices_buf[layer, 0, :, :64])
    with pytest.raises(RuntimeError, match='exceeds fixed capacity'):
        small = _small_cache(max_visible_len=32)
        _prefill_cpu(small, 0, 60)
        small.prepare_metadata([0], 0)


def test_visible_bucket_covers_the_planned_length():
    cache = _small_cache(max_visible_len=200)
    _prefill_cpu(cache, 0, 63)
    _prefill_cpu(cache, 2, 40)
    # the next step plans 64 tokens for request 0: the 64 bucket holds it
    assert cache.choose_visible_bucket([0, 2], (32, 64, 128)) == 64
    cache.states[0].logical_length = 64
    assert cache.choose_visible_bucket([0, 2], (32, 64, 128)) == 128
    assert cache.choose_visible_bucket([2, -1], (32, 64, 128)) == 64
    assert cache.choose_visible_bucket([0], ()) == 200


def test_pages_are_reused_lowest_first_and_pad_is_never_handed_out():
    cache = _small_cache()
    _prefill_cpu(cache, 0, 50)     # 4 pages per layer
    _prefill_cpu(cache, 1, 20)     # 2 pages per layer
    first = cache.states[0].block_tables[0].values()
    assert first == [0, 1, 2, 3]
    cache.remove_request(0)
    _prefill_cpu(cache, 0, 30)     # 2 pages: the lowest returned ids
    assert cache.states[0].block_tables[0].values() == [0, 1]
    layer = cache.layers[0]
    assert layer.PAD_PAGE_ID not in layer.free_ids
    assert len(layer.free_ids) == layer.max_physical_pages - 4
    with pytest.raises(RuntimeError, match='exhausted'):
        layer.alloc_pages(layer.max_physical_pages)


def test_request_phase_transitions():
    cache = _small_cache()
    rid = cache.add_request()
    assert rid == 0 and cache.request_phases[rid] == RequestPhase.PREFILL
    with pytest.raises(ValueError, match='invalid request phase transition'):
        cache.transition_request(rid, 'GENERATE')
    cache.transition_request(rid, 'FREEZE')
    cache.transition_request(rid, 'GENERATE')
    cache.transition_request(rid, 'FINISHED')
    with pytest.raises(ValueError, match='FINISHED -> FAILED'):
        cache.transition_request(rid, 'FAILED')
    with pytest.raises(ValueError, match='unknown request phase slot'):
        cache.transition_request(2, 'FREEZE')
    with pytest.raises(ValueError, match='already active'):
        cache.add_request(rid)
