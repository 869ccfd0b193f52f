"""Region invariants that pin the oracle's L1 pools and bypass pages.

With unlimited L1 budgets (every pool page selected), the far pool, the near
pool and the two bypass pages (the sink page past the sink tokens, the
SWA-boundary page before the window) must tile the middle interval exactly:
the owned candidate tokens are [max(SINK, lower), min(L - W, upper)) with no
token offered by two active slots.  A page in neither pool that holds middle
tokens must therefore be a bypass page, and no other page may contribute.
This holds whenever the physical page equals the L1 block (page 16 / block 16
as every benchmarked configuration runs, and 64 / 64 as the reference's
tests run); with a 64-token page over 16-token blocks the page-granular far
boundary leaves gaps that the L2 hole fill covers instead, so that geometry
is not asserted here.

The check uses only the oracle's outputs and the interval arithmetic of the
region definition, so a slip in a pool bound or a bypass condition
(``selector:209-262, 1195-1251``) shows up as a missing or doubled token;
two planted mistakes below confirm it does.
"""
import numpy as np
import pytest

from oracle import nfa_oracle as orc

SINK, WINDOW, NEAR = 4, 128, 4096
LENGTHS = (list(range(1, 400)) + list(range(4090, 4500, 7))
           + [8191, 8192, 8193, 20000, 20001, 131072, 131073])


def _cfg(page, length):
    max_blocks = (length + page - 1) // page + 2
    dims = np.arange(96, 128)
    return orc.NfaConfig(
        hq=4, hkv=1, head_dim=128, head_dim_v=128, bs=page, page=page,
        max_blocks=max_blocks, geo_sink=SINK, geo_near=NEAR, geo_window=WINDOW,
        sink_tokens=SINK, swa=WINDOW, near_len=NEAR, k1=2 * max_blocks,
        near_pages=max_blocks, k2=1024, dims=dims, fine_dims=dims, scale=1.0)


def _tiling(page, length, skip_far, skip_near):
    """(owned candidate tokens, expected interval, any token doubled)."""
    cfg = _cfg(page, length)
    far_pool, near_pool, geo = orc.l1_pools(cfg, length, skip_far, skip_near)
    one = 0x3F80  # every pool page scores 1.0
    far = np.where(far_pool, one, orc.NEG_INF_BITS).astype(np.uint16)
    near = np.where(near_pool, one, orc.NEG_INF_BITS).astype(np.uint16)
    i_f = orc.l1_topk(far, 0, geo.far_end, cfg.k_f, cfg.kt_cap)
    i_n = orc.l1_topk(near, geo.near_start, geo.near_end, cfg.k_n, cfg.kt_cap)
    token, active, pack_r = orc.candidate_slots(cfg, i_f, i_n, far, near, length)
    lower, upper, _ = orc.l2_bounds(cfg, length, skip_far, skip_near)
    owned = orc.owned_slots(cfg, token, active, pack_r, lower, upper)
    lo = max(0, length - WINDOW)
    want = np.arange(max(SINK, lower), min(lo, upper))
    offered = token[:pack_r][active[:pack_r]]
    offered = offered[(offered >= lower) & (offered < upper)]
    doubled = len(offered) != len(np.unique(offered))
    return np.sort(token[owned]), want, doubled


@pytest.mark.parametrize('page', [16, 64])
@pytest.mark.parametrize('skip', [(False, False), (True, False), (False, True)])
def test_pools_and_bypass_pages_tile_the_middle(page, skip):
    for length in LENGTHS:
        got, want, doubled = _tiling(page, length, *skip)
        assert not doubled, (page, length, skip)
        np.testing.assert_array_equal(got, want, err_msg=f'{page} {length} {skip}')


def test_planted_bypass_slip_is_caught(monkeypatch):
    """The near pool keeping the SWA-boundary page (a dropped bypass
    exclusion) offers its tokens twice."""
    original = orc.l1_pools

    def leaky(cfg, length, skip_far, skip_near):
        far_pool, near_pool, geo = original(cfg, length, skip_far, skip_near)
        t = np.arange(len(near_pool))
        byp = max(length - cfg.geo_window, 0) // cfg.bs
        near_pool = near_pool | ((t == byp) & (t >= geo.near_start)
                                 & (t < geo.swa_lo_blk))
        return far_pool, near_pool, geo

    monkeypatch.setattr(orc, 'l1_pools', leaky)
    caught = [length for length in LENGTHS
              if _tiling(16, length, False, False)[2]]
    assert caught, 'a doubled boundary page went unnoticed'


def test_planted_pool_bound_slip_is_caught(monkeypatch):
    """A far pool that stops one page short leaves a hole in the tiling."""
    original = orc.l1_pools

    def short(cfg, length, skip_far, skip_near):
        far_pool, near_pool, geo = original(cfg, length, skip_far, skip_near)
        far_pool = far_pool.copy()
        hits = np.nonzero(far_pool)[0]
        if len(hits):
            far_pool[hits[-1]] = False
        return far_pool, near_pool, geo

    monkeypatch.setattr(orc, 'l1_pools', short)
    missing = 0
    for length in (8192, 20001, 131073):
        got, want, _ = _tiling(16, length, False, False)
        missing += len(np.setdiff1d(want, got))
    assert missing > 0
