"""The allocation-free selector entry point against the workspace entry.

``nfa_select_layer_noalloc`` runs the selector with a static device scratch
array instead of a caller workspace.  Two calls in a row -- the second with
a smaller input (fewer rows, shorter contexts, fewer kv heads) and then a
third as large as the first -- must each give exactly what
``nfa_select_layer`` gives on the same cache: gather rows, visible lengths
and every intermediate the debug outputs expose.
"""
import ctypes

import numpy as np
import pytest
import torch

from nfa_case import (attention_ns, bf16_randn, make_indexer, prod_cache)
from sparse_attn import _native as nat
from sparse_attn.indexer.nfa_layer_batch_selector import (_alloc_debug,
                                                          select_layer_params)

pytestmark = pytest.mark.gpu
DEV = 'cuda'


def _launch(lib, cache, req_ids, q, indexer, *, noalloc):
    p, keep = select_layer_params(cache, 0, req_ids, q,
                                  attention_ns(indexer, 0.08838834764831845))
    dbg = {}
    cand_cap = (p.k_f + p.k_n + 2) * p.bs
    _alloc_debug(dbg, p.batch, p.hkv, p.max_blocks, p.k_f, p.k_n, p.k2,
                 cand_cap, torch.device(DEV))
    p.dbg_far, p.dbg_near = dbg['far'].data_ptr(), dbg['near'].data_ptr()
    p.dbg_i_f, p.dbg_i_n = dbg['i_f'].data_ptr(), dbg['i_n'].data_ptr()
    p.dbg_middle, p.dbg_counts = dbg['middle'].data_ptr(), dbg['counts'].data_ptr()
    p.dbg_bounds = dbg['bounds'].data_ptr()
    p.dbg_cand_tok = dbg['cand_tok'].data_ptr()
    p.dbg_cand_logit = dbg['cand_logit'].data_ptr()
    p.dbg_cand_count = dbg['cand_count'].data_ptr()
    p.dbg_cand_cap = cand_cap
    ws = None
    if noalloc:
        rc = lib.nfa_select_layer_noalloc(ctypes.byref(p), nat.stream_handle())
    else:
        need = lib.nfa_select_workspace_bytes(ctypes.byref(p))
        ws = torch.zeros(need, dtype=torch.uint8, device=DEV)
        p.workspace, p.workspace_bytes = ws.data_ptr(), need
        rc = lib.nfa_select_layer(ctypes.byref(p), nat.stream_handle())
    assert rc == 0, lib.nfa_last_error()
    torch.cuda.synchronize()
    b = len(req_ids)
    out = {k: v.cpu().numpy() for k, v in dbg.items()}
    out['gather'] = cache.gather_indices_for_layer(0)[:b].cpu().numpy()
    out['vis'] = cache.visible_lens_for_layer(0)[:b].cpu().numpy()
    del keep, ws
    return out


def _compare(lib, lengths, hkv, hq, seed):
    cache, gen, req_ids = prod_cache(lengths, hkv=hkv, hq=hq,
                                     max_req=len(lengths), seed=seed)
    indexer = make_indexer()
    cache.new_step(req_ids)
    cache.plan_common(req_ids)
    q = bf16_randn((len(req_ids), hq, 128), gen, DEV)
    # each entry rebuilds the page statistics from scratch
    cache._nfa_page_stats_lengths = None
    got = _launch(lib, cache, req_ids, q, indexer, noalloc=True)
    cache._nfa_page_stats_lengths.zero_()
    want = _launch(lib, cache, req_ids, q, indexer, noalloc=False)
    for key in want:
        np.testing.assert_array_equal(got[key], want[key], err_msg=key)
    assert (got['vis'] > 0).all()


def test_noalloc_matches_workspace_entry_on_consecutive_calls():
    lib = nat.load_library()
    # first call: 3 rows x 8 kv heads, the largest input
    _compare(lib, [20000, 9000, 12345], hkv=8, hq=32, seed=1)
    # second call: smaller (one row, 2 kv heads, shorter context); the
    # scratch still holds the first call's keys
    _compare(lib, [5000], hkv=2, hq=8, seed=2)
    # and large again, after the small one
    _compare(lib, [15000, 21000], hkv=8, hq=32, seed=3)


def test_noalloc_rejects_inputs_beyond_the_scratch_array():
    lib = nat.load_library()
    cache, gen, req_ids = prod_cache([3000], hkv=2, hq=8, max_req=1)
    cache.new_step(req_ids)
    cache.plan_common(req_ids)
    q = bf16_randn((1, 8, 128), gen, DEV)
    p, keep = select_layer_params(cache, 0, req_ids, q,
                                  attention_ns(make_indexer(), 1.0))
    p.batch = 200   # 200 x 2 = 400 rows > NFA_SELECT_SCRATCH_ROWS
    rc = lib.nfa_select_layer_noalloc(ctypes.byref(p), nat.stream_handle())
    assert rc == -3
    assert b'static array' in lib.nfa_last_error()
