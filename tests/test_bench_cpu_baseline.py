"""The CPU baseline leg of bench.py computes what it claims (no GPU).

* its L1/L2 dims are the production indexer's (tail subspace at cmp_ratio 4);
* the page-range split of the L1 phase reassembles the oracle's whole-row
  far / near scores bit for bit.
"""
import numpy as np
import torch

import bench
from nfa_case import make_indexer
from oracle import nfa_oracle as orc


def test_baseline_dims_are_the_indexers():
    want = make_indexer().\
        _subspace_indices(torch.device('cpu')).numpy()
    np.testing.assert_array_equal(bench.cpu_tail_dims(128, 4), want)
    np.testing.assert_array_equal(bench.cpu_tail_dims(128, 4),
                                  np.r_[48:64, 112:128])


def test_l1_page_ranges_reassemble_the_row():
    c = bench._cpu_config0(7, 2)
    cfg = c['cfg']
    # a shorter row than the baseline's, same geometry
    length = 6000
    q_full = orc.prepare_q(cfg, c['q'][0, 0], cfg.dims)
    for kv in (0, 5):
        far, near, _ = orc.l1_scores(cfg, c['k_pool'], c['bt'], length, kv, q_full,
                                     False, False)
        kt = -(-length // cfg.bs)
        cuts = [0, 97, kt // 2, kt]
        parts = [bench.cpu_l1_part(cfg, c['k_pool'], c['bt'], length, kv, q_full,
                                   a, b) for a, b in zip(cuts, cuts[1:])]
        np.testing.assert_array_equal(np.concatenate([f for f, _ in parts]), far)
        np.testing.assert_array_equal(np.concatenate([n for _, n in parts]), near)
