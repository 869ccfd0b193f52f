"""Pins every function of the CPU oracle against something independent of it.

Each check is chosen so that a plausible slip in the oracle (a dropped term,
a wrong sign or index, a transposed operand, a reordered sum) fails it:
torch's own bf16 conversion and softmax, exact integer arithmetic where the
inputs make every fp32 step exact, order-sensitive fp32 sums whose result
is known in closed form, and brute force over small inputs (full sorts and
set unions instead of the oracle's packed keys, owner tags and binary
searches).  The reference holds no golden vectors for this path; its own
tests' known answers are checked in test_oracle_known_answers.py.
"""
import numpy as np
import pytest
import torch

from oracle import nfa_oracle as orc

F32 = np.float32


def _cfg(**kw):
    base = dict(hq=8, hkv=2, head_dim=16, head_dim_v=16, bs=4, page=4,
                max_blocks=64, geo_sink=4, geo_near=32, geo_window=16,
                sink_tokens=4, swa=16, near_len=32, k1=6, near_pages=2, k2=64,
                dims=np.arange(8), fine_dims=np.arange(8), scale=1.0)
    base.update(kw)
    return orc.NfaConfig(**base)


def _torch_bf16_bits(x):
    t = torch.from_numpy(np.asarray(x, dtype=np.float32)).to(torch.bfloat16)
    return t.view(torch.int16).numpy().astype(np.int64) & 0xFFFF


# ---------------------------------------------------------------------------
# bf16 rounding and the order key
# ---------------------------------------------------------------------------

def test_bf16_rounding_matches_torch():
    rng = np.random.default_rng(1)
    x = rng.standard_normal(20000).astype(F32) * F32(1e3)
    # exact halfway cases (ties to even) and their neighbours
    hi = rng.integers(0, 1 << 15, 4000, dtype=np.uint32) << 16
    half = np.concatenate([hi | 0x8000, hi | 0x7FFF, hi | 0x8001]).view(F32)
    special = np.array([0.0, -0.0, np.inf, -np.inf, 1e-45, -1e-45, 3.4e38,
                        -3.4e38, 1.0, -1.0], dtype=F32)
    vals = np.concatenate([x, half[np.isfinite(half)], special])
    np.testing.assert_array_equal(orc.bf16_bits(vals).astype(np.int64),
                                  _torch_bf16_bits(vals))
    nans = np.array([0x7FC00000, 0xFFC00000, 0x7F800001, 0xFF812345],
                    dtype=np.uint32).view(F32)
    assert (orc.bf16_bits(nans) == orc.NAN_BITS).all()


def test_ord16u_orders_like_the_values():
    bits = np.arange(1 << 16, dtype=np.int64)
    vals = orc.bits_to_f32(bits.astype(np.uint16))
    finite_or_inf = ~np.isnan(vals)
    b = bits[finite_or_inf]
    order = b[np.argsort(orc.ord16u(b), kind='stable')]
    v = orc.bits_to_f32(order.astype(np.uint16))
    assert (np.diff(v.astype(np.float64)) >= 0).all()
    # -0 ranks just below +0, NaN (canonical) above +inf
    assert orc.ord16u(0x8000) + 1 == orc.ord16u(0x0000)
    assert orc.ord16u(orc.NAN_BITS) > orc.ord16u(0x7F80)
    assert len(set(orc.ord16u(b).tolist())) == len(b)


# ---------------------------------------------------------------------------
# declared fp32 reduction order
# ---------------------------------------------------------------------------

def test_seq_dot_is_ascending_fp32_without_fma():
    one = np.ones(3, dtype=F32)
    # the 1 survives only if it is added after the large terms cancel
    assert orc.seq_dot(np.array([1e8, -1e8, 1], dtype=F32), one) == F32(1)
    assert orc.seq_dot(np.array([1e8, 1, -1e8], dtype=F32), one) == F32(0)
    # product rounded before the add: (1 + 2^-12)^2 = 1 + 2^-11 + 2^-24
    a = F32(1 + 2.0 ** -12)
    got = orc.seq_dot(np.array([-1, a], dtype=F32), np.array([1, a], dtype=F32))
    assert got == F32(2.0 ** -11)   # a fused multiply-add would keep 2^-24
    ints = np.random.default_rng(2).integers(-50, 50, (7, 33)).astype(F32)
    w = np.random.default_rng(3).integers(-5, 5, (33,)).astype(F32)
    np.testing.assert_array_equal(orc.seq_dot(ints, w),
                                  (ints.astype(np.int64) @ w.astype(np.int64)).astype(F32))
    np.testing.assert_array_equal(orc.seq_sum(ints), ints.astype(np.int64).sum(0).astype(F32))


def _round_f32_exact(x):
    """Round a Fraction to fp32, round-to-nearest-even, with denormals and
    overflow to inf, by integer arithmetic alone (no float rounding)."""
    from fractions import Fraction
    if x == 0:
        return F32(0.0)
    sign = -1 if x < 0 else 1
    a = abs(x)
    # exponent E with 2^E <= a < 2^(E+1)
    e = a.numerator.bit_length() - a.denominator.bit_length()
    if Fraction(2) ** e > a:
        e -= 1
    q = max(e, -126) - 23                 # the fp32 grid spacing at a
    m = a / Fraction(2) ** q              # a in units of the spacing
    n, r = divmod(m.numerator, m.denominator)
    twice = 2 * r
    if twice > m.denominator or (twice == m.denominator and n % 2 == 1):
        n += 1
    val = Fraction(n) * Fraction(2) ** q
    if val >= Fraction(2) ** 128:
        return F32(sign * np.inf)
    return F32(sign * float(val))


def test_exact_dot_is_the_fused_multiply_add_chain():
    """exact_dot equals the sequential chain acc = round(acc + a*b) computed
    in exact rational arithmetic, on random fp32 vectors with exponents
    spread over the whole range (products that fp32 cannot hold, denormals,
    cancellations), against rounding done by integers alone."""
    from fractions import Fraction
    rng = np.random.default_rng(41)
    n, d = 300, 12
    mant = rng.uniform(1.0, 2.0, (2, n, d))
    ex = rng.integers(-75, 60, (2, n, d))
    sgn = rng.choice([-1.0, 1.0], (2, n, d))
    vals = (sgn * mant * np.exp2(ex)).astype(F32)
    vals[0, :40] = orc.bf16r(vals[0, :40])          # bf16 operands too
    vals[1, :40] = orc.bf16r(vals[1, :40])
    vals[0, 40:60, 3] = -vals[0, 40:60, 2]          # cancellations
    vals[1, 40:60, 3] = vals[1, 40:60, 2]
    a, b = vals
    got = orc.exact_dot(a, b)
    for i in range(n):
        acc = F32(0.0)
        for k in range(d):
            exact = Fraction(float(acc)) + Fraction(float(a[i, k])) * Fraction(float(b[i, k]))
            acc = _round_f32_exact(exact)
        assert got[i].tobytes() == acc.tobytes(), (i, got[i], acc)


def test_exact_dot_ties_overflow_and_specials():
    """The single rounding where a float64 sum would round twice: acc + p on
    an fp32 midpoint in float64 but off it exactly (both directions), the
    overflow threshold, the fused closed form, and inf / NaN / zero terms."""
    one = F32(1.0)
    # true value just above the midpoint 1 + 2^-24: rounds up (ties-to-even
    # of the float64 sum would give 1)
    assert orc.add_exact_f32(one, 2.0 ** -24 + 2.0 ** -70) == F32(1 + 2.0 ** -23)
    assert F32(1.0 + (2.0 ** -24 + 2.0 ** -70)) == one
    # just below the midpoint between 1 + 2^-23 and 1 + 2^-22: rounds down
    lo = F32(1 + 2.0 ** -23)
    assert orc.add_exact_f32(lo, 2.0 ** -24 - 2.0 ** -70) == lo
    assert F32(np.float64(lo) + (2.0 ** -24 - 2.0 ** -70)) == F32(1 + 2.0 ** -22)
    # exactly on the overflow threshold in float64, below it exactly
    fmax = F32(np.finfo(F32).max)
    assert orc.add_exact_f32(fmax, 2.0 ** 103 - 2.0 ** 50) == fmax
    with np.errstate(over='ignore'):
        assert np.isinf(F32(np.float64(fmax) + (2.0 ** 103 - 2.0 ** 50)))
    assert np.isinf(orc.add_exact_f32(fmax, 2.0 ** 103))
    # fused: (1 + 2^-12)^2 - (1 + 2^-11) keeps the 2^-24 a rounded product loses
    a = F32(1 + 2.0 ** -12)
    got = orc.exact_dot(np.array([-(1 + 2.0 ** -11), a], dtype=F32),
                        np.array([1, a], dtype=F32))
    assert got == F32(2.0 ** -24)
    assert orc.seq_dot(np.array([-(1 + 2.0 ** -11), a], dtype=F32),
                       np.array([1, a], dtype=F32)) == F32(0)
    # inf * 0 is NaN, inf survives, zeros keep +0
    assert np.isnan(orc.exact_dot(np.array([np.inf, 1], dtype=F32), np.array([0, 1], dtype=F32)))
    assert orc.exact_dot(np.array([np.inf, 1], dtype=F32), np.array([2, 1], dtype=F32)) == np.inf
    z = orc.exact_dot(np.array([-1, 0], dtype=F32), np.array([0, 5], dtype=F32))
    assert z == 0 and not np.signbit(z)
    # integers: exact whatever the order of rounding
    ints = np.random.default_rng(4).integers(-50, 50, (7, 33)).astype(F32)
    w = np.random.default_rng(5).integers(-5, 5, (33,)).astype(F32)
    np.testing.assert_array_equal(orc.exact_dot(ints, w),
                                  (ints.astype(np.int64) @ w.astype(np.int64)).astype(F32))


# ---------------------------------------------------------------------------
# page statistics and query preparation
# ---------------------------------------------------------------------------

def _pool(rng, n_phys, hkv, page, d, integer=True):
    if integer:
        return rng.integers(-60, 60, (n_phys, 1, hkv, page, d)).astype(F32)
    return orc.bf16r(rng.standard_normal((n_phys, 1, hkv, page, d)).astype(F32))


@pytest.mark.parametrize('bs,page', [(4, 4), (4, 8), (8, 4)])
def test_page_stats_against_torch(bs, page):
    rng = np.random.default_rng(4 + bs + page)
    cfg = _cfg(bs=bs, page=page, dims=np.array([1, 3, 4, 7, 9, 12]))
    length = 37
    n_phys = 20
    k_pool = _pool(rng, n_phys, cfg.hkv, page, cfg.head_dim)
    bt = rng.permutation(n_phys).astype(np.int64)
    for kv in range(cfg.hkv):
        kmin, kmax, ksum = orc.page_stats(cfg, k_pool, bt, length, kv)
        tok = np.arange(length)
        keys = torch.from_numpy(k_pool[bt[tok // page], 0, kv, tok % page][:, cfg.dims])
        for p in range((length + bs - 1) // bs):
            blk = keys[p * bs:min(length, p * bs + bs)]
            exp_min = blk.amin(0).to(torch.bfloat16).float().numpy()
            exp_max = blk.amax(0).to(torch.bfloat16).float().numpy()
            exp_sum = blk.double().sum(0).float().to(torch.bfloat16).float().numpy()
            np.testing.assert_array_equal(kmin[p], exp_min)
            np.testing.assert_array_equal(kmax[p], exp_max)
            np.testing.assert_array_equal(ksum[p], exp_sum)


def test_page_stats_signed_zero_keeps_the_earlier_token():
    cfg = _cfg(bs=4, page=4, dims=np.array([0]), hkv=1)
    k_pool = np.zeros((1, 1, 1, 4, 16), dtype=F32)
    k_pool[0, 0, 0, :, 0] = [0.0, -0.0, -0.0, 0.0]
    kmin, kmax, _ = orc.page_stats(cfg, k_pool, np.array([0]), 4, 0)
    assert not np.signbit(kmin[0, 0]) and not np.signbit(kmax[0, 0])
    k_pool[0, 0, 0, :, 0] = [-0.0, 0.0, 0.0, -0.0]
    kmin, kmax, _ = orc.page_stats(cfg, k_pool, np.array([0]), 4, 0)
    assert np.signbit(kmin[0, 0]) and np.signbit(kmax[0, 0])


def test_query_preparation_against_torch():
    rng = np.random.default_rng(5)
    cfg = _cfg(scale=0.125, dims=np.array([0, 5, 9]), fine_dims=np.array([2, 3, 15]))
    q = rng.standard_normal((cfg.hq, cfg.head_dim)).astype(F32)
    got = orc.prepare_q(cfg, q, cfg.dims)
    exp = (torch.from_numpy(q[:, cfg.dims]) * 0.125).to(torch.bfloat16).float().numpy()
    np.testing.assert_array_equal(got, exp)
    # grouped: exact small integers, head kv*G + j belongs to kv head kv
    qi = rng.integers(-8, 8, (cfg.hq, cfg.head_dim)).astype(F32)
    cfg1 = _cfg(scale=1.0, fine_dims=np.array([2, 3, 15]))
    g = cfg1.group
    exp_g = qi[:, cfg1.fine_dims].reshape(cfg1.hkv, g, -1).sum(1)
    np.testing.assert_array_equal(orc.prepare_q_grouped(cfg1, qi), exp_g)


# ---------------------------------------------------------------------------
# L1 scores and top-k
# ---------------------------------------------------------------------------

def test_l1_page_scores_exact_integers():
    rng = np.random.default_rng(6)
    cfg = _cfg(bs=4, dims=np.arange(6))
    g = cfg.group
    n = 50
    kmin = rng.integers(-4, 2, (n, 6)).astype(F32)
    kmax = kmin + rng.integers(0, 4, (n, 6)).astype(F32)
    ksum = (4 * rng.integers(-3, 3, (n, 6))).astype(F32)   # kavg = ksum / 4 exact
    q = rng.integers(-3, 4, (g, 6)).astype(F32)
    mm, avg = orc.l1_page_scores(cfg, kmin, kmax, ksum, q)
    ql, qh = np.minimum(q, 0), np.maximum(q, 0)
    per_head = (kmin.astype(np.int64) @ ql.T.astype(np.int64)
                + kmax.astype(np.int64) @ qh.T.astype(np.int64))   # [n, g]
    exp_mm = _torch_bf16_bits(per_head.sum(1) / g)
    per_avg = (ksum.astype(np.int64) // 4) @ q.T.astype(np.int64)
    exp_avg = _torch_bf16_bits(per_avg.sum(1) / g)
    np.testing.assert_array_equal(mm.astype(np.int64), exp_mm)
    np.testing.assert_array_equal(avg.astype(np.int64), exp_avg)


def _torch_top2_reference(kavg, q_rows, bs_unused=None):
    """The reference's avg_top2 formula evaluated by torch: per-head bf16
    page means (einsum, then bf16), the top-2 values over the heads,
    their bf16 mean."""
    avg = torch.einsum('hd,td->ht', torch.from_numpy(q_rows), torch.from_numpy(kavg))
    avg = avg.to(torch.bfloat16)
    return avg.topk(2, dim=0).values.mean(dim=0)


def test_avg_top2_far_scores_match_torch():
    """avg_top2: the oracle's sequential restatement equals torch's own
    evaluation of the reference formula on inputs whose dot products are
    exact in fp32 (so the summation order cannot matter), with unrounded
    query values that bf16 cannot hold -- the score must come from the
    unrounded query -- plus pages whose rounded-query score is non-finite
    (that value stands) and all-tied heads."""
    rng = np.random.default_rng(16)
    cfg = _cfg(bs=4, dims=np.arange(8), far_method='avg_top2')
    g = cfg.group
    n = 400
    ksum = (4 * rng.integers(-15, 16, (n, 8))).astype(F32)       # kavg in [-15, 15]
    q_u = (rng.integers(-2048, 2049, (g, 8)) / 256.0).astype(F32)  # 12-bit values
    q_r = orc.bf16r(q_u)
    assert not np.array_equal(q_r, q_u)
    ksum[5] = 0.0                          # every head ties at +0
    ksum[7, 3] = np.inf                    # rounded-query score +-inf or NaN
    ksum[9, 0] = np.nan
    got = orc.l1_top2_scores(cfg, ksum, q_r, q_u).astype(np.int64)
    kavg = orc.bf16r(ksum / F32(4))
    with np.errstate(invalid='ignore'):
        exact = _torch_top2_reference(kavg, q_u)
        kernel = _torch_top2_reference(kavg, q_r)
    want = torch.where(torch.isfinite(kernel), exact, kernel)
    want_bits = want.view(torch.int16).numpy().astype(np.int64) & 0xFFFF
    nan = np.isnan(want.float().numpy())
    np.testing.assert_array_equal(got[~nan], want_bits[~nan])
    assert (got[nan] == orc.NAN_BITS).all() and nan[9]
    # the unrounded query decides: it differs from the rounded one somewhere
    assert not torch.equal(exact, kernel)
    # a planted slip (the rounded query everywhere) is caught
    slip = orc.l1_top2_scores(cfg, ksum, q_r, q_r).astype(np.int64)
    assert (slip[~nan] != want_bits[~nan]).any()


def test_top2_values_order_nan_and_signed_zero():
    v = np.array([[1.0, np.nan, 0.0, -0.0, -np.inf],
                  [3.0, 2.0, -0.0, -0.0, -np.inf],
                  [2.0, 5.0, -1.0, 0.0, -np.inf]], dtype=F32)
    t1, t2 = orc.top2_values(v)
    assert t1[0] == 3.0 and t2[0] == 2.0
    assert np.isnan(t1[1]) and t2[1] == 5.0
    assert t1[2] == 0.0 and not np.signbit(t1[2]) and t2[2] == 0.0 and np.signbit(t2[2])
    assert t1[3] == 0.0 and not np.signbit(t1[3])
    assert t1[4] == -np.inf and t2[4] == -np.inf


def test_l1_topk_brute_force():
    rng = np.random.default_rng(7)
    for trial in range(200):
        kt = int(rng.integers(1, 60))
        pool = rng.integers(0, 6, kt)      # few distinct values -> many ties
        bits = orc.bf16_bits(pool.astype(F32) - 2).astype(np.int64)
        bits[rng.random(kt) < 0.1] = orc.NEG_INF_BITS
        bits[rng.random(kt) < 0.05] = orc.NAN_BITS
        lo = int(rng.integers(0, kt))
        hi = int(rng.integers(lo, kt + 1))
        k = int(rng.integers(0, kt + 1))
        got = orc.l1_topk(bits, lo, hi, k, kt)
        eff = [int(bits[t]) if lo <= t < hi else orc.NEG_INF_BITS for t in range(kt)]
        exp = sorted(range(kt), key=lambda t: (-int(orc.ord16u(eff[t])), t))[:k]
        assert got.tolist() == exp, trial


# ---------------------------------------------------------------------------
# candidates, L2 logits and L2 selection
# ---------------------------------------------------------------------------

def test_candidate_tokens_brute_force():
    rng = np.random.default_rng(8)
    for trial in range(60):
        cfg = _cfg(bs=4, k1=6, near_pages=2, sink_tokens=int(rng.integers(0, 7)),
                   swa=int(rng.choice([4, 6, 16])), max_blocks=64)
        length = int(rng.integers(8, 200))
        kt = (length + cfg.bs - 1) // cfg.bs
        far = orc.bf16_bits(rng.standard_normal(kt).astype(F32)).astype(np.uint16)
        near = far.copy()
        far[rng.random(kt) < 0.5] = orc.NEG_INF_BITS
        near[rng.random(kt) < 0.5] = orc.NEG_INF_BITS
        i_f = orc.l1_topk(far, 0, kt, cfg.k_f, cfg.kt_cap)
        i_n = orc.l1_topk(near, 0, kt, cfg.k_n, cfg.kt_cap)
        skip = (bool(rng.random() < 0.2), bool(rng.random() < 0.2))
        lower, upper, quota = orc.l2_bounds(cfg, length, *skip)
        token, active, pack_r = orc.candidate_slots(cfg, i_f, i_n, far, near, length)
        owned = orc.owned_slots(cfg, token, active, pack_r, lower, upper)
        got = sorted(token[owned].tolist())
        # brute force: tokens of the finite-score selected pages and of the
        # kept bypass pages, inside [max(sink, lower), min(lo, L, upper))
        lo = max(0, length - cfg.swa)
        # (-inf fillers may point past kt; they never become candidates)
        pages = {int(p) for p in i_f if p < kt and far[p] != orc.NEG_INF_BITS}
        pages |= {int(p) for p in i_n if p < kt and near[p] != orc.NEG_INF_BITS}
        spl = cfg.sink_tokens // cfg.bs
        if cfg.sink_tokens % cfg.bs:
            pages.add(spl)
        byp1 = (lo % cfg.bs != 0) and (lo // cfg.bs >= spl)
        if cfg.sink_tokens % cfg.bs:
            byp1 = byp1 and lo // cfg.bs != spl
        if byp1:
            pages.add(lo // cfg.bs)
        t_lo = max(cfg.sink_tokens, lower)
        t_hi = min(lo, length, upper)
        exp = sorted(t for p in pages for t in range(p * cfg.bs, p * cfg.bs + cfg.bs)
                     if t_lo <= t < t_hi)
        assert got == exp, trial


def test_l2_logits_exact_integers():
    rng = np.random.default_rng(9)
    cfg = _cfg(fine_dims=np.array([1, 4, 6, 11]))
    k_pool = _pool(rng, 12, cfg.hkv, cfg.page, cfg.head_dim)
    bt = rng.permutation(12).astype(np.int64)
    token = rng.permutation(40)[:20].astype(np.int64)
    load = rng.random(20) < 0.7
    q = rng.integers(-3, 4, 4).astype(F32)
    for kv in range(cfg.hkv):
        got = orc.l2_logits(cfg, k_pool, bt, token, load, q, kv, quota=5)
        keys = k_pool[bt[token // cfg.page], 0, kv, token % cfg.page][:, cfg.fine_dims]
        exp = _torch_bf16_bits(keys.astype(np.int64) @ q.astype(np.int64))
        exp = np.where(load, exp, orc.NEG_INF_BITS)
        np.testing.assert_array_equal(got.astype(np.int64), exp)
        assert (orc.l2_logits(cfg, k_pool, bt, token, load, q, kv, quota=0)
                == orc.NEG_INF_BITS).all()


def test_l2_selection_brute_force():
    rng = np.random.default_rng(10)
    for trial in range(300):
        cfg = _cfg(sink_tokens=int(rng.integers(0, 6)), k2=64, max_blocks=64)
        # candidates always lie inside [low, high) (the selector builds them
        # from [max(sink, lower), min(lo, L, upper)))
        low = int(rng.integers(0, 100))
        high = int(rng.integers(low, 220))
        n = int(rng.integers(0, min(40, high - low) + 1))
        token = (low + rng.permutation(high - low)[:n]).astype(np.int64)
        bits = orc.bf16_bits(rng.integers(0, 5, n).astype(F32) - 2).astype(np.int64)
        bits[rng.random(n) < 0.2] = orc.NEG_INF_BITS
        bits[rng.random(n) < 0.05] = orc.NAN_BITS
        quota = int(rng.integers(0, min(50, high - low) + 1))
        mid, cnt = orc.l2_middle(cfg, bits.astype(np.uint16), token, 0, False, False,
                                 low, high, quota)
        valid = [i for i in range(n) if bits[i] not in (orc.NEG_INF_BITS, orc.NAN_BITS)]
        ranked = sorted(valid, key=lambda i: (-int(orc.ord16u(bits[i])), token[i]))
        chosen = [int(token[i]) for i in ranked[:quota]]
        fill = [t for t in range(low, high) if t not in chosen][:max(0, quota - len(chosen))]
        exp = sorted(t for t in chosen + fill if t >= cfg.sink_tokens)
        assert mid[:cnt].tolist() == exp, trial


# ---------------------------------------------------------------------------
# protected set, union, attention
# ---------------------------------------------------------------------------

def test_protected_ids_closed_form_and_short_context_quirk():
    cfg = _cfg(sink_tokens=4, swa=16, max_blocks=64)
    for length in range(20, 120):
        exp = list(range(4)) + list(range(length - 16, length))
        assert orc.protected_ids(cfg, length).tolist() == exp
    # below sink + swa the reference's SWA ids L - swa + aux - sink come out
    # negative and are dropped (selector:1337-1360): only the sink survives
    assert orc.protected_ids(cfg, 10).tolist() == [0, 1, 2, 3]
    # L = 19: ids 19 - 16 + aux - 4 for aux in [4, 19) -> 3..17, sink 0..3
    assert orc.protected_ids(cfg, 19).tolist() == [0, 1, 2, 3] + list(range(3, 18))


def test_final_union_brute_force():
    rng = np.random.default_rng(11)
    cfg = _cfg(sink_tokens=4, swa=16, max_blocks=64, page=4)
    for trial in range(50):
        length = int(rng.integers(20, 250))
        bt = rng.permutation(64).astype(np.int64)
        cnt = int(rng.integers(0, 30))
        middle = np.zeros(64, dtype=np.int64)
        middle[:cnt] = np.sort(rng.choice(np.arange(4, length), cnt, replace=False))
        slots, vis = orc.final_union(cfg, middle, cnt, length, bt, max_vis=40)
        ids = sorted(set(middle[:cnt].tolist()) | set(orc.protected_ids(cfg, length).tolist()))
        ids = [i for i in ids if i < cfg.s_cap]
        assert vis == len(ids)
        exp = [int(bt[i // 4]) * 4 + i % 4 for i in ids[:40]]
        assert slots.tolist() == exp


def test_sparse_attention_matches_torch_softmax():
    rng = np.random.default_rng(12)
    hkv, hq, d, page = 2, 8, 16, 4
    k_pool = rng.standard_normal((10, 1, hkv, page, d)).astype(F32)
    v_pool = rng.standard_normal((10, 1, hkv, page, d)).astype(F32)
    q = rng.standard_normal((3, hq, d)).astype(F32)
    gather = rng.integers(0, 40, (2, hkv, 12)).astype(np.int64)
    vis = np.array([[12, 5], [0, 7]])
    q2r = np.array([1, -1, 0])
    out = orc.sparse_attention(k_pool, v_pool, q, gather, vis, q2r, 0.25, page)
    kp = torch.from_numpy(k_pool).double()
    vp = torch.from_numpy(v_pool).double()
    for t, r in enumerate(q2r):
        for h in range(hq):
            kv = h // (hq // hkv)
            if r < 0 or vis[r, kv] == 0:
                assert (out[t, h] == 0).all()
                continue
            sl = torch.from_numpy(gather[r, kv, :vis[r, kv]])
            kk = kp[sl // page, 0, kv, sl % page]
            vv = vp[sl // page, 0, kv, sl % page]
            w = torch.softmax(kk @ torch.from_numpy(q[t, h]).double() * 0.25, 0)
            np.testing.assert_allclose(out[t, h], (w @ vv).numpy(), rtol=1e-9, atol=1e-12)


def test_mla_attention_equals_expanded_attention():
    """The absorbed latent attention against the torch-pinned attention
    over expanded heads (DeepseekV2Attention.expand_kv): K_h = [W_uk,h c |
    k_pe], V_h = W_uv,h c, q_h = [q_nope,h | q_pe,h]; the latent form takes
    q_lat,h = [W_uk,h^T q_nope,h | q_pe,h] and out_h = W_uv,h o_lat,h.  Equal
    in float64 up to rounding; a transposed projection, a wrong value slice
    or a dropped RoPE term fails it."""
    rng = np.random.default_rng(31)
    heads, rank, rope, nope, dv, page = 4, 16, 8, 12, 10, 4
    latent = rng.standard_normal((9, 1, 1, page, rank + rope))
    w_uk = rng.standard_normal((heads, nope, rank))
    w_uv = rng.standard_normal((heads, dv, rank))
    q_nope = rng.standard_normal((2, heads, nope))
    q_pe = rng.standard_normal((2, heads, rope))
    gather = rng.integers(0, 36, (3, heads, 10)).astype(np.int64)
    vis = rng.integers(0, 11, (3, heads))
    q2r = np.array([2, -1])
    c, k_pe = latent[..., :rank], latent[..., rank:]
    k_exp = np.concatenate([np.einsum('pabtr,hnr->pahtn', c, w_uk),
                            np.broadcast_to(k_pe, c.shape[:2] + (heads, page, rope))],
                           axis=-1)
    v_exp = np.einsum('pabtr,hvr->pahtv', c, w_uv)
    q_exp = np.concatenate([q_nope, q_pe], axis=-1)
    want = orc.sparse_attention(k_exp, v_exp, q_exp, gather, vis, q2r, 0.3, page)
    q_lat = np.concatenate([np.einsum('thn,hnr->thr', q_nope, w_uk), q_pe], axis=-1)
    o_lat = orc.mla_sparse_attention(latent, q_lat, gather, vis, q2r, 0.3, page, rank)
    got = np.einsum('thr,hvr->thv', o_lat, w_uv)
    np.testing.assert_allclose(got, want, rtol=1e-9, atol=1e-12)
    assert (got[1] == 0).all()  # the padding row


# --- 4-bit L2 keys ------------------------------------------------------------

def _torch_min_max_quant(x):
    """The reference's per-token 4-bit round trip (tia_indexer.py:22-31),
    evaluated by torch in bf16: torch rounds every op's result to bf16,
    which is what the oracle's explicit rounding points restate."""
    max_val = x.amax(dim=-1, keepdim=True)
    min_val = x.amin(dim=-1, keepdim=True)
    scales = (max_val - min_val).clamp(min=1e-9) / 15
    zeros = -min_val
    return torch.clamp(torch.round((x + zeros) / scales), 0, 15) * scales - zeros


def test_fake_quant4_matches_torch_bf16_ops():
    rng = np.random.default_rng(44)
    rows = [rng.standard_normal((4000, 32)) * s for s in (1.0, 1e-3, 37.0)]
    grid = rng.standard_normal((200, 1)) + np.arange(32)[None, :] * 0.125  # on-grid
    const = np.full((3, 32), 0.75)                                            # range 0
    ties = np.tile(np.array([0.0, 15.0] + [0.5 + k for k in range(15)] * 2)[:32],
                   (2, 1))                                                   # .5 ties
    x = np.concatenate(rows + [grid, const, ties]).astype(F32)
    xb = torch.from_numpy(x).to(torch.bfloat16)
    want = _torch_min_max_quant(xb).view(torch.int16).numpy().astype(np.int64) & 0xFFFF
    got = orc.bf16_bits(orc.fake_quant4(xb.float().numpy()))
    np.testing.assert_array_equal(got, want)
    # closed forms: a constant row is returned as is (range clamps to 1e-9);
    # codes round half to even (0.5 -> 0, 1.5 -> 2, ...)
    np.testing.assert_array_equal(orc.fake_quant4(const.astype(F32)), const)
    t = orc.fake_quant4(ties[:1].astype(F32))[0]
    assert t[0] == 0.0 and t[1] == 15.0
    assert list(t[2:6]) == [0.0, 2.0, 2.0, 4.0]


# --- disjoint-region split states and combine --------------------------------

def test_split_bounds_cover_the_row_and_every_split_works():
    # floor boundaries (not ceil-sized chunks): 10 blocks over 8 splits give
    # every split a block, and the splits tile [0, n) in order
    for n, nsplit, bt in ((10 * 128, 8, 128), (1000, 4, 128), (5, 4, 64), (0, 3, 64),
                          (129, 1, 128), (4100, 7, 64)):
        b = orc.split_bounds(n, nsplit, bt)
        assert len(b) == nsplit
        assert b[0][0] == 0 and b[-1][1] == n
        assert all(b[i][1] == b[i + 1][0] for i in range(nsplit - 1))
        nb = -(-n // bt)
        sizes = [-(-(hi - lo) // bt) for lo, hi in b]
        assert sum(sizes) == nb and max(sizes) - min(sizes) <= 1
        if nb >= nsplit:
            assert min(sizes) >= 1


def _regions_case(seed):
    rng = np.random.default_rng(seed)
    hkv, hq, d, page = 2, 8, 16, 4
    k_pool = rng.standard_normal((60, 1, hkv, page, d)).astype(F32)
    v_pool = rng.standard_normal((60, 1, hkv, page, d)).astype(F32)
    q = rng.standard_normal((3, hq, d)).astype(F32)
    # distinct slots: the two regions of a (row, kv head) are disjoint
    prot = rng.permutation(240)[:200].reshape(2, 100)
    gather_a = np.stack([prot[:, :20], prot[:, 20:40]], axis=1)  # [2, hkv, 20]
    gather_b = np.stack([prot[:, 40:70], prot[:, 70:100]], axis=1)  # [2, hkv, 30]
    gather_b[1, 0, 3] = -1  # a negative slot is skipped
    vis_a = np.array([[20, 7], [0, 13]])
    vis_b = np.array([[30, 0], [25, 30]])
    q2r = np.array([1, -1, 0])
    return k_pool, v_pool, q, (gather_a, vis_a), (gather_b, vis_b), q2r, page


@pytest.mark.parametrize('na,nb,bt', [(1, 4, 4), (2, 3, 8), (1, 1, 128), (3, 8, 2)])
def test_regions_combine_equals_attention_over_the_union(na, nb, bt):
    """Split states of two disjoint slot sets, merged, are softmax attention
    over their union: pins the partition, the per-split (m, z, acc) and the
    rescaling order together against the torch-pinned sparse_attention."""
    k_pool, v_pool, q, (ga, va), (gb, vb), q2r, page = _regions_case(5)
    pa = orc.sparse_attention_partial(k_pool, v_pool, q, ga, va, q2r, 0.3, page, na, bt)
    pb = orc.sparse_attention_partial(k_pool, v_pool, q, gb, vb, q2r, 0.3, page, nb, bt)
    got = orc.regions_combine(pa, pb)
    width = ga.shape[-1] + gb.shape[-1]
    union = np.full((2, 2, width), -1, dtype=np.int64)
    vis = np.zeros((2, 2), dtype=np.int64)
    for r in range(2):
        for kv in range(2):
            ids = np.concatenate([ga[r, kv, :va[r, kv]], gb[r, kv, :vb[r, kv]]])
            union[r, kv, :len(ids)] = ids
            vis[r, kv] = len(ids)
    want = orc.sparse_attention(k_pool, v_pool, q, union, vis, q2r, 0.3, page)
    np.testing.assert_allclose(got, want, rtol=1e-12, atol=1e-14)


def test_split_state_closed_forms():
    """One slot in a split: m is its score, z = 1, acc its value row; an
    empty split and a padding row hold (0, -inf, 0)."""
    k_pool, v_pool, q, (ga, va), _, q2r, page = _regions_case(9)
    vis = np.array([[2, 0], [1, 0]])
    acc, m, z = orc.sparse_attention_partial(k_pool, v_pool, q, ga, vis, q2r, 0.5,
                                             page, 3, 1)
    # row 1 (query 0), kv 0, one slot: floor boundaries 0, 0, 0, 1 put it in
    # split 2, splits 0-1 are empty
    assert orc.split_bounds(1, 3, 1) == [(0, 0), (0, 0), (0, 1)]
    sl = ga[1, 0, 0]
    k = k_pool[sl // page, 0, 0, sl % page].astype(np.float64)
    v = v_pool[sl // page, 0, 0, sl % page].astype(np.float64)
    for h in range(4):
        assert m[2, 0, h] == pytest.approx(float(q[0, h].astype(np.float64) @ k) * 0.5)
        assert z[2, 0, h] == 1.0
        np.testing.assert_allclose(acc[2, 0, h], v)
        assert (m[:2, 0, h] == -np.inf).all() and not z[:2, 0, h].any()
        assert not acc[:2, 0, h].any()
    assert (m[:, 1] == -np.inf).all() and not z[:, 1].any() and not acc[:, 1].any()
    # row 0 (query 2), kv 0: two slots over three splits of one-token blocks
    # -> splits 1 and 2 hold one each (floor boundaries 0, 0, 1, 2)
    assert orc.split_bounds(2, 3, 1) == [(0, 0), (0, 1), (1, 2)]
    assert z[0, 2, 0] == 0 and z[1, 2, 0] == 1.0 and z[2, 2, 0] == 1.0
    # both regions empty: the combine outputs zeros, not NaN
    empty = orc.regions_combine((acc[:, 1:2], m[:, 1:2], z[:, 1:2]),
                                (acc[:, 1:2], m[:, 1:2], z[:, 1:2]))
    assert np.isfinite(empty).all() and not empty.any()


# --- prefill region gate ---------------------------------------------------

def test_region_bounds_match_region_geometry():
    from sparse_attn.policies.region_geometry import RegionGeometry
    for sink, window, near, page in ((4, 128, 4096, 16), (0, 16, 64, 64), (128, 5, 7, 3)):
        geo = RegionGeometry(sink=sink, near=near, window=window, page=page)
        for length in list(range(0, 300)) + [4223, 4224, 4225, 131072, 131073]:
            assert orc.region_bounds(length, sink, window, near, page) == geo.bounds(length)


def test_region_profile_uniform_attention_closed_form():
    # zero queries: every visible key gets 1 / qlen
    rng = np.random.default_rng(0)
    length, rows = 300, 40
    q = np.zeros((4, length, 16))
    k = rng.standard_normal((2, length, 16))
    out = orc.region_profile(q, k, rows, 0.25, sink=4, window=16, near=64, page=16)
    for r in range(rows):
        qlen = length - rows + r + 1
        sink_hi, far_hi, near_hi = orc.region_bounds(qlen, 4, 16, 64, 16)
        np.testing.assert_allclose(out[0, :, r], (near_hi - far_hi) / qlen, rtol=1e-12)
        np.testing.assert_allclose(out[1, :, r], (far_hi - sink_hi) / qlen, rtol=1e-12)


def test_region_profile_one_hot_key():
    # one key far above the others takes all the mass of its region
    length, rows = 400, 8
    q = np.zeros((2, length, 8))
    q[:, :, 0] = 1.0
    k = np.zeros((1, length, 8))
    for j, region in ((100, 1), (350, 0)):  # far token, near token (row 399)
        k[:] = 0.0
        k[0, j, 0] = 200.0
        out = orc.region_profile(q, k, rows, 1.0, sink=4, window=16, near=64, page=16)
        assert out[region, :, -1].min() > 1 - 1e-12
        assert out[1 - region, :, -1].max() < 1e-12


def test_region_profile_matches_torch_softmax():
    rng = np.random.default_rng(1)
    length, rows, hq, hkv, d = 90, 20, 4, 2, 8
    q = rng.standard_normal((hq, length, d))
    k = rng.standard_normal((hkv, length, d))
    out = orc.region_profile(q, k, rows, 0.3, sink=2, window=8, near=16, page=4)
    qt = torch.from_numpy(q)
    kt = torch.from_numpy(k).repeat_interleave(hq // hkv, dim=0)
    s = qt @ kt.transpose(1, 2) * 0.3
    pos = torch.arange(length)
    for r in range(rows):
        row = length - rows + r
        p = torch.softmax(s[:, row].masked_fill(pos > row, float('-inf')), dim=-1)
        sink_hi, far_hi, near_hi = orc.region_bounds(row + 1, 2, 8, 16, 4)
        np.testing.assert_allclose(out[0, :, r], p[:, far_hi:near_hi].sum(-1).numpy(),
                                   rtol=1e-12, atol=1e-15)
        np.testing.assert_allclose(out[1, :, r], p[:, sink_hi:far_hi].sum(-1).numpy(),
                                   rtol=1e-12, atol=1e-15)
