"""CPU oracle for the NFA (LoDA-SA) two-level sparse decode layer.

TEST INFRASTRUCTURE ONLY.  Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import this module, and only as the
checker (or the timed CPU baseline).  The product path (``sparse_attn`` +
``libnfa_hip.so``) never imports it and has no CPU fallback.

This is a numpy restatement of the reference selector
``sparse_attn/indexer/nfa_layer_batch_selector.py`` (cited below as
``selector:<line>``) and of the sparse gather attention in
``sparse_attn/ops/paged_region_kernels.py``.  It follows the reference's own
structure: the virtual candidate slot layout, per-block owner tags, the packed
sort keys, the tiled-top-k result contract and the binary-search hole fill of
``_finish_sorted_logits_key``.  The HIP kernels use different (equivalent)
algorithms; parity tests compare the two bit for bit.

Declared arithmetic (the reference leaves fp32 reduction order to Triton, so
the order is declared here and the HIP kernels follow it exactly):

* every fp32 reduction is sequential, index ascending, starting from +0.0;
  the selector's dot products (L1 page scores, L2 logits) add each exact
  product with one rounding (``exact_dot``: a fused multiply-add per term;
  ``seq_dot``, the rounded-product order, is kept to show the difference);
* ``bf16r`` is fp32 -> bf16 round-to-nearest-even; any NaN becomes the
  canonical positive quiet NaN 0x7FC0 (NaN then ranks first, as on the
  reference GPU);
* page min/max scan tokens in ascending order with ``v < m ? v : m`` (NaN is
  ignored, ties of +-0 keep the earlier token);
* all L1 scores and L2 logits are rounded to bf16 whatever the KV/query
  dtype (the reference packs them as 16-bit keys, ``selector:1482, 688``);
  page statistics are stored in the KV dtype (``selector:120-124``).

Pinning (the reference holds no golden vectors for this path).
``tests/test_oracle_pinning.py`` checks bf16 rounding against torch, the order
key against the float order of all 65536 bf16 patterns, the declared fp32
sum order with order- and FMA-sensitive closed forms, page statistics and
query preparation against torch, L1 scores and L2 logits against exact
integer arithmetic, L1 top-k, candidate expansion + owner tags, L2
top-quota + hole fill and the final union against brute force, and the
attention against torch softmax.  ``tests/test_oracle_known_answers.py``
checks the region geometry, bounds and fixed quotas against the known
answers of the reference's own tests.  ``fake_quant4`` (the optional 4-bit
L2 keys of ``--nfa_l2_quant``, which no selector code of the reference
reads) is pinned against torch's own bf16 evaluation of the reference
formula (tia_indexer.py:22-31).
L1 page indices above 65535 use exact (score, page) order; the reference
packs the page into 16 bits (``selector:1481-1484``) and would alias there.
"""
from __future__ import annotations

import dataclasses
from typing import Optional

import numpy as np

F32 = np.float32
NEG_INF_BITS = 0xFF80
NAN_BITS = 0x7FC0


# ---------------------------------------------------------------------------
# bf16 / ordering helpers
# ---------------------------------------------------------------------------

def bf16_bits(x) -> np.ndarray:
    """fp32 -> bf16 bits, round to nearest even, canonical NaN 0x7FC0."""
    x = np.ascontiguousarray(np.asarray(x, dtype=np.float32))
    u = x.view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) & 0xFFFF
    r = r.astype(np.uint16)
    return np.where(np.isnan(x), np.uint16(NAN_BITS), r)


def bits_to_f32(bits) -> np.ndarray:
    b = np.ascontiguousarray(np.asarray(bits, dtype=np.uint16))
    return (b.astype(np.uint32) << 16).view(np.float32)


def bf16r(x) -> np.ndarray:
    """Round fp32 to the nearest bf16 value (returned as fp32)."""
    return bits_to_f32(bf16_bits(x))


def ord16u(bits) -> np.ndarray:
    """Order-preserving unsigned key of bf16 bits (``selector:1482-1485``).

    Equals the reference's ``key`` before its ``- 0x8000``: +0 ranks above
    -0, +NaN above +inf, -inf above -NaN.
    """
    b = np.asarray(bits).astype(np.int64)
    return np.where((b & 0x8000) != 0, (~b) & 0xFFFF, b | 0x8000)


def trunc_div(a, b):
    """Triton/C integer division (truncates toward zero)."""
    a = np.asarray(a, dtype=np.int64)
    q = np.abs(a) // b
    return np.where(a < 0, -q, q)


def tdiv(a: int, b: int) -> int:
    q = abs(a) // b
    return -q if a < 0 else q


def seq_dot(a, b) -> np.ndarray:
    """sum_d a[..., d] * b[..., d] in fp32, d ascending, from +0.0, no FMA."""
    a, b = np.broadcast_arrays(np.asarray(a, dtype=np.float32),
                               np.asarray(b, dtype=np.float32))
    acc = np.zeros(a.shape[:-1], dtype=np.float32)
    with np.errstate(invalid='ignore', over='ignore'):
        for d in range(a.shape[-1]):
            acc = (acc + (a[..., d] * b[..., d]).astype(F32)).astype(F32)
    return acc


_F32_OVER = float(2.0 ** 128 - 2.0 ** 103)   # fp32 overflow threshold (max + ulp/2)
_F32_MAX = float(np.finfo(np.float32).max)


def add_exact_f32(acc, p) -> np.ndarray:
    """fl32(acc + p) with one rounding: ``acc`` fp32, ``p`` an exact value
    held in float64 (the product of two fp32 values always is).  This is
    what a fused multiply-add fma(a, b, acc) computes for p = a * b.

    TwoSum gives s + e == acc + p exactly (s, e float64); fp32 rounding of
    s is the fp32 rounding of s + e unless s lies exactly on a midpoint
    between two fp32 values (midpoints are float64 numbers, and |e| is
    below half a float64 ulp of s), where the sign of e breaks the tie."""
    a = np.asarray(acc, dtype=np.float32).astype(np.float64)
    p = np.asarray(p, dtype=np.float64)
    with np.errstate(invalid='ignore', over='ignore'):
        s = a + p
        bb = s - a
        e = (a - (s - bb)) + (p - bb)
        r = s.astype(np.float32)
        fin = np.isfinite(s) & (e != 0)
        if fin.any():
            r64 = r.astype(np.float64)
            d = s - r64
            toward = np.where(d > 0, np.float32(np.inf), np.float32(-np.inf))
            n = np.nextafter(r, toward.astype(np.float32))
            mid = fin & np.isfinite(r) & (d != 0) & (2.0 * s == r64 + n.astype(np.float64))
            r = np.where(mid & (np.sign(e) == np.sign(d)), n, r)
            # s exactly on the overflow threshold: a negative e keeps the
            # result finite
            edge = fin & np.isinf(r) & (np.abs(s) == _F32_OVER) & (np.sign(e) == -np.sign(s))
            r = np.where(edge, np.sign(s).astype(np.float32) * np.float32(_F32_MAX), r)
    return np.asarray(r, dtype=np.float32)


def exact_dot(a, b) -> np.ndarray:
    """sum_d a[..., d] * b[..., d] in fp32, d ascending, from +0.0, each
    exact product added with one rounding: the fused multiply-add chain
    acc = fma(a_d, b_d, acc) of the selector's dot products.  Where the fp32
    product is already exact (always for two bf16 values in the normal
    range) this is the plain fp32 add of that product."""
    a, b = np.broadcast_arrays(np.asarray(a, dtype=np.float32),
                               np.asarray(b, dtype=np.float32))
    acc = np.zeros(a.shape[:-1], dtype=np.float32)
    with np.errstate(invalid='ignore', over='ignore'):
        for d in range(a.shape[-1]):
            x, y = a[..., d], b[..., d]
            p32 = (x * y).astype(F32)
            p64 = x.astype(np.float64) * y.astype(np.float64)
            fast = (acc + p32).astype(F32)
            ok = p32.astype(np.float64) == p64          # NaN takes the slow path
            if ok.all():
                acc = fast
            else:
                acc = np.where(ok, fast, add_exact_f32(acc, p64)).astype(F32)
    return acc


def seq_sum(values) -> np.ndarray:
    """sum over the leading axis in fp32, ascending, from +0.0."""
    acc = np.zeros(np.asarray(values).shape[1:], dtype=np.float32)
    for v in values:
        acc = (acc + np.asarray(v, dtype=np.float32)).astype(F32)
    return acc


def round_kv(x, kv_dtype: str) -> np.ndarray:
    x = np.asarray(x, dtype=np.float32)
    return bf16r(x) if kv_dtype == 'bf16' else x


# ---------------------------------------------------------------------------
# Configuration
# ---------------------------------------------------------------------------

@dataclasses.dataclass
class NfaConfig:
    """Geometry and flags of one selector call (``selector:2762-2832``).

    ``geo_*`` come from ``RegionGeometry`` (cache.geometry) and the rest from
    the ``NFAIndexer``; the reference keeps them apart and so does this.
    """
    hq: int
    hkv: int
    head_dim: int
    head_dim_v: int
    bs: int                      # tia_block_size
    page: int                    # cache.geometry.page
    max_blocks: int              # cache.max_blocks (= kt_cap)
    geo_sink: int
    geo_near: int
    geo_window: int
    sink_tokens: int             # indexer.sink_tokens
    swa: int                     # indexer.sliding_window_size
    near_len: int                # indexer.nt_near_len
    k1: int                      # tia_level1_topk
    near_pages: int              # nfa_near_pages
    k2: int                      # tia_level2_topk
    dims: np.ndarray             # L1 dims
    fine_dims: np.ndarray        # L2 dims
    scale: float
    far_method: str = 'minmax'
    near_method: str = 'avg'
    kv_dtype: str = 'bf16'
    near_tokens: Optional[int] = None   # None == 'off'
    l2_quant: bool = False

    @property
    def group(self):
        return self.hq // self.hkv

    @property
    def s_cap(self):
        return self.max_blocks * self.bs

    @property
    def kt_cap(self):
        return self.max_blocks

    @property
    def pool_near_len(self):
        return max(self.bs, int(self.near_len))

    @property
    def sink_pool_lo(self):
        return max(0, self.sink_tokens // self.bs)

    @property
    def k_n(self):
        return min(max(0, self.near_pages), self.kt_cap)

    @property
    def k_f(self):
        return min(max(0, self.k1 - max(0, self.near_pages)), self.kt_cap)


# ---------------------------------------------------------------------------
# A2: page statistics (selector:32-131)
# ---------------------------------------------------------------------------

def gather_keys(k_pool, bt_row, tokens, kv, dims, page, max_blocks):
    """K[token, kv, dims] through the block table; masked tokens read 0."""
    tokens = np.asarray(tokens, dtype=np.int64)
    lp = tokens // page
    ok = (tokens >= 0) & (lp < max_blocks)
    phys = np.where(ok, bt_row[np.clip(lp, 0, max_blocks - 1)], 0)
    off = np.where(ok, tokens % page, 0)
    vals = k_pool[phys, 0, kv, off][..., np.asarray(dims)]
    return np.where(ok[..., None], vals, 0).astype(np.float32), ok


def page_stats(cfg: NfaConfig, k_pool, bt_row, length, kv, n_pages=None):
    """Per-page min/max/sum over the visible tokens of K[:, kv, dims].

    Returns (kmin, kmax, ksum) as fp32 arrays [n_pages, Dsub] holding values
    already rounded to the KV dtype.  Tokens are scanned in ascending order
    (``selector:103-124``).
    """
    bs = cfg.bs
    if n_pages is None:
        n_pages = (length + bs - 1) // bs
    toks = np.arange(n_pages, dtype=np.int64)[:, None] * bs + np.arange(bs)
    vals, ok = gather_keys(k_pool, bt_row, toks, kv, cfg.dims, cfg.page,
                           cfg.max_blocks)
    read = ok & (toks < length)
    dsub = len(cfg.dims)
    kmin = np.full((n_pages, dsub), np.inf, dtype=np.float32)
    kmax = np.full((n_pages, dsub), -np.inf, dtype=np.float32)
    ksum = np.zeros((n_pages, dsub), dtype=np.float32)
    for i in range(bs):
        v = vals[:, i]
        r = read[:, i, None]
        kmin = np.where(r & (v < kmin), v, kmin)
        kmax = np.where(r & (v > kmax), v, kmax)
        with np.errstate(invalid='ignore'):  # inf + -inf keys sum to NaN, as on the GPU
            ksum = np.where(r, (ksum + v).astype(F32), ksum)
    return (round_kv(kmin, cfg.kv_dtype), round_kv(kmax, cfg.kv_dtype),
            round_kv(ksum, cfg.kv_dtype))


# ---------------------------------------------------------------------------
# A2/A3: query preparation (selector:943-1002)
# ---------------------------------------------------------------------------

def prepare_q(cfg: NfaConfig, q_row, dims):
    """q_full[h, d] = bf16r(f32(q[h, dims[d]]) * scale)  [HQ, len(dims)]."""
    q = np.asarray(q_row, dtype=np.float32)[:, np.asarray(dims)]
    return bf16r((q * F32(cfg.scale)).astype(F32))


def prepare_q_unrounded(cfg: NfaConfig, q_row, dims):
    """q_u[h, d] = f32(q[h, dims[d]]) * scale, not rounded: the query of the
    avg_top2 far scores (``selector:2936-2938``, ``round_bf16=False``)."""
    q = np.asarray(q_row, dtype=np.float32)[:, np.asarray(dims)]
    return (q * F32(cfg.scale)).astype(F32)


def top2_values(values):
    """The two largest of ``values`` [G, n] along axis 0 in torch.topk's
    value order (NaN above everything, +0 above -0), by the sequential
    update of ``selector:284-331`` with the comparison of ``:162-172``."""
    def greater(v, o):
        vn, on = np.isnan(v), np.isnan(o)
        pz_nz = (v == 0) & (o == 0) & ~np.signbit(v) & np.signbit(o)
        return (vn & ~on) | (~vn & ~on & ((v > o) | pz_nz))
    t1 = np.full(values.shape[1], -np.inf, dtype=np.float32)
    t2 = t1.copy()
    for v in values:
        take = greater(v, t1)
        second = np.where(take, t1, v)
        t1 = np.where(take, v, t1)
        t2 = np.where(greater(second, t2), second, t2)
    return t1, t2


def prepare_q_grouped(cfg: NfaConfig, q_row):
    """q_fine[kv, d] = sum_j bf16r(q[kv*G+j, fine_dims[d]] * scale)."""
    qf = prepare_q(cfg, q_row, cfg.fine_dims)
    g = cfg.group
    return seq_sum(np.stack([qf[j::g] for j in range(g)]))


# ---------------------------------------------------------------------------
# A4: L1 scores with pool masks (selector:175-354)
# ---------------------------------------------------------------------------

@dataclasses.dataclass
class RowGeometry:
    length: int
    kt_eff: int
    near_start: int
    swa_lo_blk: int
    far_end: int
    near_end: int


def l1_geometry(cfg: NfaConfig, length):
    bs = cfg.bs
    kt_eff = (length + bs - 1) // bs
    near_start = max(tdiv(length - cfg.geo_window - cfg.pool_near_len, bs),
                     cfg.sink_pool_lo)
    swa_lo_blk = max(near_start, kt_eff - max(1, cfg.geo_window // bs))
    return RowGeometry(length, kt_eff, near_start, swa_lo_blk,
                       min(kt_eff, near_start), swa_lo_blk)


def l1_pools(cfg: NfaConfig, length, skip_far, skip_near):
    """Boolean far/near pool masks over pages [0, kt_eff) (selector:209-262)."""
    bs, page = cfg.bs, cfg.page
    geo = l1_geometry(cfg, length)
    t = np.arange(geo.kt_eff, dtype=np.int64)
    far_on = not skip_far
    near_on = not skip_near
    sink_hi = min(cfg.geo_sink, length)
    swa_hi = max(sink_hi, length - cfg.geo_window)
    far_blk = tdiv(length - cfg.geo_window - cfg.geo_near, page)
    orig_far_hi = min(swa_hi, max(sink_hi, far_blk * page))
    block_lo = t * bs
    block_hi = block_lo + bs
    has_sink = block_lo < sink_hi
    has_far = far_on & (block_hi > sink_hi) & (block_lo < orig_far_hi)
    has_near = near_on & (block_hi > orig_far_hi) & (block_lo < swa_hi)
    has_swa = (block_hi > swa_hi) & (block_lo < length)
    block_valid = (block_lo < length) & (has_sink | has_far | has_near | has_swa)
    spl = cfg.sink_pool_lo
    swa_lo_tok = max(length - cfg.geo_window, 0)
    byp_blk = swa_lo_tok // bs
    byp_cond = (swa_lo_tok % bs != 0) and (byp_blk >= spl)
    if cfg.geo_sink % bs != 0:
        byp_cond = byp_cond and byp_blk != spl
    far_pool = (t >= spl) & (t < geo.near_start) & far_on
    near_pool = ((t >= geo.near_start) & (t < geo.swa_lo_blk) & near_on
                 & ~((t == byp_blk) & byp_cond))
    if cfg.geo_sink % bs != 0:
        far_pool &= t != spl
        near_pool &= t != spl
    return far_pool & block_valid, near_pool & block_valid, geo


def l1_top2_scores(cfg: NfaConfig, ksum, q_full_group, q_unrounded_group):
    """avg_top2 far scores (``selector:2412-2427``): per head the bf16 page
    mean against the unrounded query, the two largest heads averaged and
    rounded to bf16 -- where the same score against the bf16-rounded query
    (the score the reference's kernel writes first) is finite; elsewhere
    that value stands."""
    kavg = bf16r((ksum / F32(cfg.bs)).astype(F32))
    with np.errstate(invalid='ignore', over='ignore'):
        rounded = np.stack([bf16r(exact_dot(kavg, q[None, :])) for q in q_full_group])
        exact = np.stack([bf16r(exact_dot(kavg, q[None, :])) for q in q_unrounded_group])
        r1, r2 = top2_values(rounded)
        u1, u2 = top2_values(exact)
        kernel = bf16r(((r1 + r2).astype(F32) / F32(2)).astype(F32))
        host = bf16r(((u1 + u2).astype(F32) / F32(2)).astype(F32))
    return bf16_bits(np.where(np.isfinite(kernel), host, kernel))


def l1_page_scores(cfg: NfaConfig, kmin, kmax, ksum, q_full_group):
    """Per-page minmax and avg scores for one kv group (bf16 values as fp32).

    ``q_full_group`` is the G rows of ``prepare_q`` owned by this kv head.
    mm_j = bf16r(S- + S+) per query head, then bf16r(sum_j mm_j / G)
    (``selector:311-334``); avg uses kavg = bf16r(f32(sum)/BS)
    (``selector:305-307``).
    """
    g = cfg.group
    qlow = np.where(q_full_group < 0, q_full_group, F32(0)).astype(F32)
    qhigh = np.where(q_full_group > 0, q_full_group, F32(0)).astype(F32)
    kavg = bf16r((ksum / F32(cfg.bs)).astype(F32))
    mm_acc = np.zeros(kmin.shape[0], dtype=np.float32)
    avg_acc = np.zeros(kmin.shape[0], dtype=np.float32)
    for j in range(g):
        s_neg = exact_dot(kmin, qlow[j][None, :])
        s_pos = exact_dot(kmax, qhigh[j][None, :])
        mm_j = bf16r((s_neg + s_pos).astype(F32))
        mm_acc = (mm_acc + mm_j).astype(F32)
        avg_j = bf16r(exact_dot(kavg, q_full_group[j][None, :]))
        avg_acc = (avg_acc + avg_j).astype(F32)
    mm = bf16_bits((mm_acc / F32(g)).astype(F32))
    avg = bf16_bits((avg_acc / F32(g)).astype(F32))
    return mm, avg


def l1_scores(cfg: NfaConfig, k_pool, bt_row, length, kv, q_full,
              skip_far, skip_near, q_unrounded=None):
    """far/near bf16 score bits over pages [0, kt_eff) for one (row, kv)."""
    far_pool, near_pool, geo = l1_pools(cfg, length, skip_far, skip_near)
    kmin, kmax, ksum = page_stats(cfg, k_pool, bt_row, length, kv)
    g = cfg.group
    mm, avg = l1_page_scores(cfg, kmin, kmax, ksum, q_full[kv * g:(kv + 1) * g])
    if cfg.far_method == 'avg_top2':
        far_val = l1_top2_scores(cfg, ksum, q_full[kv * g:(kv + 1) * g],
                                 q_unrounded[kv * g:(kv + 1) * g])
    else:
        far_val = mm if cfg.far_method == 'minmax' else avg
    near_val = avg if cfg.near_method == 'avg' else mm
    far = np.where(far_pool, far_val, NEG_INF_BITS).astype(np.uint16)
    near = np.where(near_pool, near_val, NEG_INF_BITS).astype(np.uint16)
    return far, near, geo


# ---------------------------------------------------------------------------
# A5: L1 top-k (selector:1473-1497, 1766-1803)
# ---------------------------------------------------------------------------

def l1_topk(score_bits, active_lo, active_hi, k, kt):
    """Indices of the top-k pages of packed (score, -page) keys, sorted.

    Pages outside [active_lo, active_hi) (and past the written scores) count
    as -inf; ties go to the lower page.
    """
    if k <= 0:
        return np.zeros(0, dtype=np.int64)
    t = np.arange(kt, dtype=np.int64)
    s = np.full(kt, NEG_INF_BITS, dtype=np.int64)
    n = len(score_bits)
    inside = (t >= active_lo) & (t < active_hi) & (t < n)
    s[inside] = np.asarray(score_bits, dtype=np.int64)[t[inside]]
    key = ord16u(s) - 0x8000
    if kt <= 65536:
        packed = (key << 16) | ((kt - 1 - t) & 0xFFFF)
        top = np.sort(packed)[::-1][:k]
        return kt - 1 - (top & 0xFFFF)
    order = np.lexsort((t, -key))
    return t[order[:k]]


# ---------------------------------------------------------------------------
# A6: candidate expansion, owners and L2 metadata (selector:1117-1251, 1917-1986)
# ---------------------------------------------------------------------------

def l2_bounds(cfg: NfaConfig, length, skip_far, skip_near):
    """lower/upper/quota of the middle interval (selector:1160-1192)."""
    bs = cfg.bs
    lo = max(0, length - cfg.swa)
    lower = cfg.sink_pool_lo * bs
    upper = max(lower, lo)
    sink_hi = min(length, cfg.sink_tokens)
    swa_hi = max(sink_hi, length - cfg.swa)
    far_blk = (max(length - cfg.swa - cfg.geo_near, 0) // cfg.page) * cfg.page
    far_hi = min(swa_hi, max(sink_hi, far_blk))
    if skip_far:
        lower = far_hi
    if skip_near:
        upper = far_hi
    upper = max(lower, upper)
    quota = max(min(length, cfg.k2) - cfg.sink_tokens - (length - lo), 0)
    quota = min(quota, upper - lower)
    return lower, upper, quota


def candidate_slots(cfg: NfaConfig, i_f, i_n, far_bits, near_bits, length):
    """Token and active flag of every virtual candidate slot (selector:1195-1251)."""
    bs = cfg.bs
    k_f, k_n = cfg.k_f, cfg.k_n
    s_cap = cfg.s_cap
    head = min(cfg.sink_tokens, s_cap)
    tail = min(cfg.swa, s_cap)
    pack_r = (k_f + k_n + 2) * bs
    width = pack_r + head + tail
    lo = max(0, length - cfg.swa)
    kt_eff = (length + bs - 1) // bs
    spl = cfg.sink_pool_lo
    r = np.arange(width, dtype=np.int64)
    far = r < k_f * bs
    near = (r >= k_f * bs) & (r < (k_f + k_n) * bs)
    l1 = far | near
    k1w = (k_f + k_n) * bs
    byp0 = (r >= k1w) & (r < k1w + bs)
    old = r < pack_r
    i_f = np.asarray(i_f, dtype=np.int64)
    i_n = np.asarray(i_n, dtype=np.int64)
    blk_f = np.where(far, i_f[np.clip(r // bs, 0, max(k_f - 1, 0))] if k_f else 0, 0)
    blk_n = np.where(near, i_n[np.clip((r - k_f * bs) // bs, 0, max(k_n - 1, 0))]
                     if k_n else 0, 0)
    blk = np.where(far, blk_f, blk_n)
    far_bits = np.asarray(far_bits, dtype=np.int64)
    near_bits = np.asarray(near_bits, dtype=np.int64)

    def load(bits, b, mask):
        ok = mask & (b < kt_eff) & (b < len(bits))
        return np.where(ok, bits[np.clip(b, 0, max(len(bits) - 1, 0))]
                        if len(bits) else NEG_INF_BITS, NEG_INF_BITS)

    score = np.where(far, load(far_bits, blk_f, far), load(near_bits, blk_n, near))
    swa_byp_blk = lo // bs
    byp_blk = np.where(byp0, spl, swa_byp_blk)
    byp0_keep = cfg.sink_tokens % bs != 0
    byp1_keep = (lo % bs != 0) and (swa_byp_blk >= spl)
    if cfg.sink_tokens % bs != 0:
        byp1_keep = byp1_keep and swa_byp_blk != spl
    token = np.where(l1, blk * bs + r % bs, byp_blk * bs + r % bs)
    keep = np.where(l1, score != NEG_INF_BITS, np.where(byp0, byp0_keep, byp1_keep))
    active = (old & keep & (token >= cfg.sink_tokens) & (token < lo)
              & (token >= 0) & (token < length))
    is_head = (r >= pack_r) & (r < pack_r + head)
    tail_id = lo + r - pack_r - head
    new_id = np.where(is_head, r - pack_r, tail_id)
    new_valid = ((is_head & (new_id < length))
                 | ((r >= pack_r + head) & (r < pack_r + head + tail)
                    & (new_id < length) & (new_id >= cfg.sink_tokens)))
    token = np.where(old, token, new_id)
    active = np.where(old, active, new_valid)
    return token, active, pack_r


def owned_slots(cfg: NfaConfig, token, active, pack_r, lower, upper):
    """Slots that win the per-block owner tag (selector:1167-1184, 481-486).

    A block is owned by the page group with the largest slot among the active
    in-range slots mapping to it (``atomic_max`` of ``block_last_r``).
    """
    bs = cfg.bs
    r = np.arange(len(token), dtype=np.int64)
    block_last_r = (r // bs) * bs + bs - 1
    marks = active & (r < pack_r) & (token >= lower) & (token < upper)
    owner = {}
    for slot in np.nonzero(marks)[0]:
        blk = int(token[slot]) // bs
        owner[blk] = max(owner.get(blk, -1), int(block_last_r[slot]))
    in_range = active & (token >= 0) & (token < cfg.s_cap) & \
        (token >= lower) & (token < upper)
    unique = np.zeros(len(token), dtype=bool)
    for slot in np.nonzero(in_range)[0]:
        blk = int(token[slot]) // bs
        unique[slot] = owner.get(blk, -1) == int(block_last_r[slot])
    lp = np.where(unique, token, 0) // cfg.page
    return unique & (lp < cfg.max_blocks)


# ---------------------------------------------------------------------------
# A7: L2 logits (selector:423-516), optional 4-bit fake quant (tia_indexer.py:22-31)
# ---------------------------------------------------------------------------

def fake_quant4(x):
    """bf16 op-by-op ``min_max_per_token_quant`` over the last axis
    (reference indexer/tia_indexer.py:22-31): scale = bf16(bf16(max - min)
    clamped to 1e-9 / 15), zero = -min, code = clamp(round_half_even(
    bf16(bf16(x + zero) / scale)), 0, 15), result bf16(bf16(code * scale) -
    zero)."""
    x = bf16r(x)
    mx = x.max(axis=-1, keepdims=True)
    mn = x.min(axis=-1, keepdims=True)
    rng = bf16r((mx - mn).astype(F32))
    rng = np.where(rng < F32(1e-9), bf16r(F32(1e-9)), rng).astype(F32)
    scale = bf16r((rng / F32(15)).astype(F32))
    zero = (-mn).astype(F32)
    t = bf16r((x + zero).astype(F32))
    t = bf16r((t / scale).astype(F32))
    code = np.clip(np.round(t), 0, 15).astype(F32)   # np.round = half-even
    return bf16r((bf16r((code * scale).astype(F32)) - zero).astype(F32))


def l2_logits(cfg: NfaConfig, k_pool, bt_row, token, load, q_fine_kv, kv, quota):
    """bf16 logit bits per candidate slot; -inf where not scored or NaN."""
    out = np.full(len(token), NEG_INF_BITS, dtype=np.uint16)
    if quota == 0 or not load.any():
        return out
    idx = np.nonzero(load)[0]
    vals, _ = gather_keys(k_pool, bt_row, token[idx], kv, cfg.fine_dims,
                          cfg.page, cfg.max_blocks)
    if cfg.l2_quant:
        vals = fake_quant4(vals)
    logit = bf16_bits(exact_dot(vals, q_fine_kv[None, :]))
    logit = np.where(logit == NAN_BITS, NEG_INF_BITS, logit)
    out[idx] = logit
    return out


# ---------------------------------------------------------------------------
# A8: L2 filtered top-k + hole fill (selector:519-566, 569-605)
# ---------------------------------------------------------------------------

def l2_topk_keys(cfg: NfaConfig, logit_bits, token, width):
    """Sorted top-``width`` packed keys (``_nfa_filtered_topk_kernel``)."""
    s = cfg.s_cap
    tb = 32 if s >= 65536 else 16
    bits = np.asarray(logit_bits, dtype=np.int64)
    good = (bits != NEG_INF_BITS) & ~((bits & 0x7FFF) > 0x7F80)
    ordered = ord16u(bits) - 0x8000
    key = np.where(good, (ordered << tb) + (s - np.asarray(token, np.int64)),
                   -32768 << tb)
    key = np.sort(key)[::-1]
    if len(key) < width:
        key = np.concatenate([key, np.full(width - len(key), -32768 << tb)])
    return key[:width], tb


def finish_sorted_keys(cfg: NfaConfig, key, tb, low, high, quota):
    """Restatement of ``_finish_sorted_logits_key`` (selector:519-566)."""
    k = len(key)
    s = cfg.s_cap
    sink = cfg.sink_tokens
    i = np.arange(k, dtype=np.int64)
    if quota == 0:
        return np.zeros(k, dtype=np.int64), 0
    invalid = -32768 << tb
    valid = key > invalid
    mask = (1 << tb) - 1
    take = (i < quota) & valid
    chosen = np.where(take, s - (key & mask), s)
    nvalid = int(take.sum())
    if nvalid == quota:
        packed = np.sort(np.where(chosen >= sink, chosen, s))
        return np.where(packed < s, packed, 0), int((packed < s).sum())
    chosen = np.sort(chosen)
    bound = np.where(chosen < s, chosen - low - i, s)
    lo = np.zeros(k, dtype=np.int64)
    hi = np.full(k, k, dtype=np.int64)
    for _ in range(11):
        mid = lo + (hi - lo) // 2
        value = bound[np.minimum(mid, k - 1)]
        right = value <= i
        act = lo < hi
        lo = np.where(act & right, mid + 1, lo)
        hi = np.where(act & ~right, mid, hi)
    zero = low + i + lo
    zero = np.where((i < quota - nvalid) & (zero < high), zero, s)
    combined = np.concatenate([chosen, zero])
    combined = np.where(combined >= sink, combined, s)
    packed = np.sort(combined)
    out = np.where(packed[:k] < s, packed[:k], 0)
    return out, int((packed < s).sum())


def fixed_quota_regions(cfg: NfaConfig, length, skip_far, skip_near):
    """Numeric --nfa_near_tokens quotas (selector:873-920)."""
    bs = cfg.bs
    lo = max(0, length - cfg.swa)
    lower = cfg.sink_pool_lo * bs
    upper = max(lower, lo)
    sink_hi = min(length, cfg.sink_tokens)
    swa_hi = max(sink_hi, length - cfg.swa)
    far_blk = (max(length - cfg.swa - cfg.near_len, 0) // cfg.page) * cfg.page
    far_hi = min(swa_hi, max(sink_hi, far_blk))
    base = max(min(length, cfg.k2) - cfg.sink_tokens - (length - lo), 0)
    reserve = min(int(cfg.near_tokens), base)
    far_quota = max(base - reserve, 0)
    far_low = far_hi if skip_far else lower
    far_high = far_hi
    far_quota = min(far_quota, max(far_high - far_low, 0))
    near_quota = max(base - far_quota, 0)
    near_low = far_hi
    near_high = far_hi if skip_near else upper
    near_quota = min(near_quota, max(near_high - near_low, 0))
    return (far_low, far_high, far_quota), (near_low, near_high, near_quota)


def l2_middle(cfg: NfaConfig, logits, token, length, skip_far, skip_near,
              lower, upper, quota):
    """Canonical middle ids (sorted) and count for one (row, kv)."""
    width = cfg.k2
    if cfg.near_tokens is None:
        key, tb = l2_topk_keys(cfg, logits, token, width)
        return finish_sorted_keys(cfg, key, tb, lower, upper, quota)
    parts = []
    for low, high, q in fixed_quota_regions(cfg, length, skip_far, skip_near):
        tok = np.asarray(token, dtype=np.int64)
        filt = np.where((tok >= low) & (tok < high) & (q > 0),
                        logits, NEG_INF_BITS).astype(np.uint16)
        key, tb = l2_topk_keys(cfg, filt, token, width)
        ids, cnt = finish_sorted_keys(cfg, key, tb, low, high, q)
        parts.append(ids[:cnt])
    ids = np.concatenate(parts)
    out = np.zeros(width, dtype=np.int64)
    out[:len(ids)] = ids[:width]
    return out, len(ids)


# ---------------------------------------------------------------------------
# A9: protected set and final union (selector:1337-1437, 1440-1470)
# ---------------------------------------------------------------------------

def protected_ids(cfg: NfaConfig, length):
    """Sink + SWA ids exactly as ``_final_union_protected_sort_kernel``.

    For length < sink + swa some SWA ids come out negative and are dropped,
    as in the reference (``selector:1289-1298``).
    """
    s = cfg.s_cap
    prot = min(s, cfg.sink_tokens + cfg.swa)
    aux = np.arange(prot, dtype=np.int64)
    sink_count = min(length, cfg.sink_tokens)
    total = min(length, cfg.sink_tokens + cfg.swa)
    in_sink = aux < sink_count
    in_swa = (aux >= sink_count) & (aux < total)
    pid = np.where(in_sink, aux, length - cfg.swa + aux - sink_count)
    keep = (in_sink | in_swa) & (pid >= 0) & (pid < s)
    return np.sort(pid[keep])


def final_union(cfg: NfaConfig, middle, count, length, bt_row, max_vis,
                middle_only=False):
    """(physical slots written, vis_len) for one (row, kv)."""
    page = cfg.page
    mids = np.asarray(middle[:count], dtype=np.int64)
    if middle_only:
        ids = mids[:max_vis]
        slots = bt_row[ids // page].astype(np.int64) * page + ids % page
        return slots, min(count, max_vis)
    ordered = np.sort(np.concatenate([mids, protected_ids(cfg, length)]))
    ordered = ordered[ordered < cfg.s_cap]
    uniq = np.unique(ordered)
    ids = uniq[:max_vis]
    slots = bt_row[ids // page].astype(np.int64) * page + ids % page
    return slots, len(uniq)


# ---------------------------------------------------------------------------
# A1: one selector call over a batch
# ---------------------------------------------------------------------------

@dataclasses.dataclass
class RowResult:
    far: np.ndarray = None
    near: np.ndarray = None
    i_f: np.ndarray = None
    i_n: np.ndarray = None
    lower: int = 0
    upper: int = 0
    quota: int = 0
    cand_tokens: np.ndarray = None     # tokens of the scored candidate slots
    cand_logits: np.ndarray = None     # their logit bits
    middle: np.ndarray = None
    count: int = 0
    gather: np.ndarray = None
    vis_len: int = 0


def apply_decode_write(k_pool, v_pool, keys, values, slots, page):
    """K/V write of one token per row at its slot (paged_region_kernels.py:15-61).
    ``v_pool`` None writes the keys only (selection never reads V)."""
    for b, slot in enumerate(np.asarray(slots).tolist()):
        if slot < 0:
            continue
        phys, off = divmod(int(slot), page)
        k_pool[phys, 0, :, off, :] = keys[b, :, 0, :]
        if v_pool is not None:
            v_pool[phys, 0, :, off, :] = values[b, :, 0, :]


def select_row(cfg: NfaConfig, k_pool, bt_row, length, q_row, kv,
               skip_far, skip_near, max_vis, middle_only=False):
    """Everything the selector computes for one (batch row, kv head)."""
    res = RowResult()
    res.lower, res.upper, res.quota = l2_bounds(cfg, length, skip_far, skip_near)
    if length <= 0:
        res.middle = np.zeros(cfg.k2, dtype=np.int64)
        res.gather = np.zeros(0, dtype=np.int64)
        res.vis_len = 0
        return res
    q_full = prepare_q(cfg, q_row, cfg.dims)
    q_fine = prepare_q_grouped(cfg, q_row)
    q_unrounded = prepare_q_unrounded(cfg, q_row, cfg.dims)
    far, near, geo = l1_scores(cfg, k_pool, bt_row, length, kv, q_full,
                               skip_far, skip_near, q_unrounded)
    res.far, res.near = far, near
    kt = cfg.kt_cap
    res.i_f = l1_topk(far, 0, geo.far_end, cfg.k_f, kt)
    res.i_n = l1_topk(near, geo.near_start, geo.near_end, cfg.k_n, kt)
    token, active, pack_r = candidate_slots(cfg, res.i_f, res.i_n, far, near,
                                            length)
    load = owned_slots(cfg, token, active, pack_r, res.lower, res.upper)
    logits = l2_logits(cfg, k_pool, bt_row, token, load, q_fine[kv], kv,
                       res.quota)
    scored = load & (res.quota > 0)
    res.cand_tokens = token[scored]
    res.cand_logits = logits[scored]
    res.middle, res.count = l2_middle(cfg, logits, token, length, skip_far,
                                      skip_near, res.lower, res.upper,
                                      res.quota)
    res.gather, res.vis_len = final_union(cfg, res.middle, res.count, length,
                                          bt_row, max_vis, middle_only)
    return res


def select_layer(cfg: NfaConfig, k_pool, block_table, lengths, req_ids,
                 active, skip_far, skip_near, q, max_vis, middle_only=False):
    """Selector over a batch; returns results[b][kv].

    ``block_table`` is this layer's [MAX_REQ, MAX_BLOCKS]; ``skip_far`` and
    ``skip_near`` are indexed by request slot; inactive rows behave as
    length 0 (PAD rows carry planned length 0, ``paged_region_cache.py:866-872``).
    """
    out = []
    for b, req in enumerate(req_ids):
        length = int(lengths[b])
        rows = []
        for kv in range(cfg.hkv):
            rows.append(select_row(cfg, k_pool, block_table[req], length, q[b],
                                   kv, bool(skip_far[req]), bool(skip_near[req]),
                                   max_vis, middle_only))
        out.append(rows)
    return out


# ---------------------------------------------------------------------------
# A10: sparse gather attention (paged_region_kernels.py:1008-1041)
# ---------------------------------------------------------------------------

def sparse_attention(k_pool, v_pool, q, gather, vis_lens, query_to_req, scale,
                     page):
    """Textbook softmax over the gathered slots, in float64.  [T, HQ, DV]."""
    q = np.asarray(q, dtype=np.float64)
    t_total, hq, _ = q.shape
    hk = gather.shape[1]
    g = hq // hk
    dv = v_pool.shape[-1]
    max_vis = gather.shape[-1]
    out = np.zeros((t_total, hq, dv), dtype=np.float64)
    for t in range(t_total):
        req = int(query_to_req[t])
        if req < 0:
            continue
        for kh in range(hk):
            n = min(int(vis_lens[req, kh]), max_vis)
            slots = np.asarray(gather[req, kh, :n], dtype=np.int64)
            slots = slots[slots >= 0]
            if len(slots) == 0:
                continue
            phys, off = slots // page, slots % page
            k = k_pool[phys, 0, kh, off].astype(np.float64)
            v = v_pool[phys, 0, kh, off].astype(np.float64)
            s = q[t, kh * g:(kh + 1) * g] @ k.T * scale
            s = s - s.max(axis=1, keepdims=True)
            p = np.exp(s)
            p /= p.sum(axis=1, keepdims=True)
            out[t, kh * g:(kh + 1) * g] = p @ v
    return out


def mla_sparse_attention(latent_pool, q_lat, gather, vis_lens, query_to_req, scale,
                         page, value_dim):
    """Absorbed latent attention over per-head selections, in float64.

    ``latent_pool`` [P+1, 1, 1, page, D] holds one row per token, [c
    (value_dim) | k_pe]; ``q_lat`` [T, H, D] per head [W_uk,h^T q_nope,h |
    q_pe,h]; ``gather`` [rows, H, W] / ``vis_lens`` [rows, H] are each head's
    selection.  Returns [T, H, value_dim]: sum_i softmax(scale q_h . K_i)
    K_i[:value_dim] per head, before the value up-projection (0 for padding
    rows).  No reference counterpart: the algebraic form of
    ``sparse_attention`` over the expanded heads K_h = [W_uk,h c | k_pe],
    V_h = W_uv,h c, against which tests/test_oracle_pinning.py pins it."""
    q = np.asarray(q_lat, dtype=np.float64)
    t_total, heads, _ = q.shape
    max_vis = gather.shape[-1]
    out = np.zeros((t_total, heads, value_dim), dtype=np.float64)
    for t in range(t_total):
        req = int(query_to_req[t])
        if req < 0:
            continue
        for h in range(heads):
            n = min(int(vis_lens[req, h]), max_vis)
            slots = np.asarray(gather[req, h, :n], dtype=np.int64)
            slots = slots[slots >= 0]
            if len(slots) == 0:
                continue
            rows = latent_pool[slots // page, 0, 0, slots % page].astype(np.float64)
            s = rows @ q[t, h] * scale
            p = np.exp(s - s.max())
            p /= p.sum()
            out[t, h] = p @ rows[:, :value_dim]
    return out


def split_bounds(n, nsplit, block_tokens):
    """Token range [lo, hi) of each split of a row with ``n`` visible slots:
    split s takes blocks [s*nb//nsplit, (s+1)*nb//nsplit) of
    nb = ceil(n / block_tokens) (reference ops/paged_region_kernels.py:455-461)."""
    nb = -(-n // block_tokens)
    out = []
    for s in range(nsplit):
        b0, b1 = s * nb // nsplit, (s + 1) * nb // nsplit
        out.append((b0 * block_tokens, min(b1 * block_tokens, n)))
    return out


def sparse_attention_partial(k_pool, v_pool, q, gather, vis_lens, query_to_req, scale,
                             page, nsplit, block_tokens):
    """Split online-softmax states of one region's gather attention, float64
    (reference ops/paged_region_kernels.py:367-530 with WRITE_PARTIAL, host
    :727-780).  Returns acc [S, T, HQ, DV], m [S, T, HQ], z [S, T, HQ]:
    m = the split's maximum score (-inf when it holds no valid slot),
    z = sum exp(s_i - m), acc = sum exp(s_i - m) v_i; negative slots are
    skipped; padding rows hold (0, -inf, 0)."""
    q = np.asarray(q, dtype=np.float64)
    t_total, hq, _ = q.shape
    hk = gather.shape[1]
    g = hq // hk
    dv = v_pool.shape[-1]
    max_vis = gather.shape[-1]
    acc = np.zeros((nsplit, t_total, hq, dv))
    m = np.full((nsplit, t_total, hq), -np.inf)
    z = np.zeros((nsplit, t_total, hq))
    for t in range(t_total):
        req = int(query_to_req[t])
        if req < 0:
            continue
        for kh in range(hk):
            n = min(int(vis_lens[req, kh]), max_vis)
            for sp, (lo, hi) in enumerate(split_bounds(n, nsplit, block_tokens)):
                slots = np.asarray(gather[req, kh, lo:hi], dtype=np.int64)
                slots = slots[slots >= 0]
                if len(slots) == 0:
                    continue
                phys, off = slots // page, slots % page
                k = k_pool[phys, 0, kh, off].astype(np.float64)
                v = v_pool[phys, 0, kh, off].astype(np.float64)
                sc = q[t, kh * g:(kh + 1) * g] @ k.T * scale
                mx = sc.max(axis=1)
                e = np.exp(sc - mx[:, None])
                m[sp, t, kh * g:(kh + 1) * g] = mx
                z[sp, t, kh * g:(kh + 1) * g] = e.sum(axis=1)
                acc[sp, t, kh * g:(kh + 1) * g] = e @ v
    return acc, m, z


def regions_combine(parts_a, parts_b):
    """Merge two regions' split states, region a's splits first, each folded
    in with the online-softmax rescaling; acc / z, 0 where z == 0 (reference
    ops/paged_region_kernels.py:533-575).  Float64 [T, HQ, DV]."""
    acc_a = parts_a[0]
    out_acc = np.zeros(acc_a.shape[1:])
    m = np.full(acc_a.shape[1:3], -np.inf)
    z = np.zeros(acc_a.shape[1:3])
    with np.errstate(invalid='ignore'):
        for acc, pm, pz in (parts_a, parts_b):
            for sp in range(acc.shape[0]):
                new_m = np.maximum(m, pm[sp])
                safe = np.where(new_m == -np.inf, 0.0, new_m)
                alpha = np.exp(m - safe)
                beta = np.exp(pm[sp] - safe)
                out_acc = out_acc * alpha[..., None] + acc[sp] * beta[..., None]
                z = z * alpha + pz[sp] * beta
                m = new_m
    zz = np.where(z == 0.0, 1.0, z)
    return np.where((z == 0.0)[..., None], 0.0, out_acc / zz[..., None])


# ---------------------------------------------------------------------------
# prefill region gate (reference sparse_attn/policies/frozen_gate.py:45-111)
# ---------------------------------------------------------------------------

def region_bounds(length, sink, window, near, page):
    """RegionGeometry.bounds (reference policies/region_geometry.py:18-23)
    with Python floor division: (sink_hi, far_hi, near_hi)."""
    sink_hi = min(sink, length)
    near_hi = max(sink_hi, length - window)
    aligned = ((length - window - near) // page) * page
    far_hi = min(near_hi, max(sink_hi, aligned))
    return sink_hi, far_hi, near_hi


def region_profile(q, k, rows, scale, sink, window, near, page):
    """Near and far attention mass of each head and each of the last ``rows``
    query positions (``_stream_tail_profile``, frozen_gate.py:45-82): causal
    softmax of ``scale * q k^T`` over keys 0..qlen-1 in float64, summed over
    [far_hi, near_hi) and [sink_hi, far_hi) of the row's bounds.
    ``q`` [hq, L, D], ``k`` [hkv, L, D].  Returns [2, hq, rows] (near, far)."""
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    hq, length, _ = q.shape
    g = hq // k.shape[0]
    n = min(rows, length)
    out = np.zeros((2, hq, n))
    for h in range(hq):
        kk = k[h // g]
        s_all = q[h, length - n:] @ kk.T * scale
        for r in range(n):
            qlen = length - n + r + 1
            s = s_all[r, :qlen]
            p = np.exp(s - s.max())
            p /= p.sum()
            sink_hi, far_hi, near_hi = region_bounds(qlen, sink, window, near, page)
            out[0, h, r] = p[far_hi:near_hi].sum()
            out[1, h, r] = p[sink_hi:far_hi].sum()
    return out
