"""Host-side step planning of the paged cache (CPU).

Every decode step, each live row's slot (per layer) must be the physical
slot of its new token through the block table: page ``len // page`` of the
row's request at offset ``len % page``.  Steady steps move slots by one on
the device and append a page for rows whose token opens one; the check runs
over many steps with ragged lengths (rows crossing pages on different steps),
a padding row, and a layout change half way.
"""
import torch

from nfa_case import make_cache
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
        crossings += cache._page_cross
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
