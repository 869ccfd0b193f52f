// NFA two-level selector for one decode layer on gfx950: one launch.
//
// Grid (batch * hkv, ntiles), 1024 threads per workgroup.
//   tile stage (workgroups whose tile holds pages of the row; a row's pages
//   spread evenly over one dispatch round of tiles, four threads per page,
//   one query head each):
//     decode K/V write of the current token (owner of the last page), page
//     min/max/sum statistics and the L2 side rows (the latest page and token,
//     or every page and token of the tile on a rebuild), L1 far/near page
//     scores.  One 16-bit score key per page (far and near pools are
//     disjoint page ranges) goes to the workspace, the high bytes of the keys
//     into a per-row, per-pool histogram (one global atomic per non-empty bin
//     and workgroup).
//   tail (the last workgroup of each (row, kv) to arrive, found with a
//     device-scope atomic counter; no workgroup ever waits on another):
//     exact top-K_F / top-K_N thresholds from the histogram plus one
//     refinement pass over the keys staged in LDS, the selected pages and
//     the sink/SWA bypass pages as an LDS bitmap (sorted and de-duplicated
//     by construction), compacted into the candidate page list; then the L2
//     logits of the candidate tokens (dense page-major slots, read from the
//     L2 side rows), the top-quota selection with the lowest-token tie-break,
//     hole fill, the sink/SWA union and the physical gather rows.
//
// Every loop a workgroup executes on the steady decode path is rolled or
// short: the code of a phase is fetched cold by nearly every workgroup, so
// executed code size is latency.
//
// Reference semantics: sparse_attn/indexer/nfa_layer_batch_selector.py
// (selector:32-131 stats, :175-354 L1, :1473-1863 L1 top-k, :1081-1251
// candidates/owners, :423-516 L2 logits, :519-848 L2 top-k, :873-940 fixed
// quota, :1337-1470 union).  Owner tags of the reference reduce to "each
// candidate token is scored once", which the candidate page bitmap gives
// directly.  Only pages with a finite L1 score become candidates
// (selector:1195-1251); the -inf fillers of I_F / I_N matter for the debug
// outputs only.
#include "nfa_common.h"

#include <atomic>
#include <type_traits>
#include <mutex>
#include <stdarg.h>
#include <stdio.h>

namespace nfa {

// ---------------------------------------------------------------------------
// LDS and workspace layouts (shared by host and device)
// ---------------------------------------------------------------------------

constexpr int SB = 1024;         // threads per selector workgroup
constexpr int SW = SB / 64;      // waves per selector workgroup
// Pages of a pass of a multi-pass tile.  Staged scores take one lane per
// page, and a pass's time grows far slower than its width (the dependent
// chain of one page's sums, then the scoring waves that share a SIMD:
// 2.4 us at 256 pages, 3.2 us at 448), so a pass is as wide as two staging
// buffers of 32-dim statistics fit in LDS beside the rest of the tile
// (seven waves score it).
constexpr int TP = 448;
constexpr int kSpanMin = NFA_SELECT_CLOCK_PAGES;  // pages per tile, at least
constexpr int kSpanMax = 448;    // pages per pass of a tile (staged in LDS)
constexpr int kPassMax = 16;     // passes per tile, at most
static_assert(kSpanMin == 64 && kSpanMax >= TP, "tile geometry");
// pages per tile, at most: kPassMax - 1 passes of TP pages and a last one of
// up to kSpanMax
constexpr int kTileMax = TP * (kPassMax - 1) + kSpanMax;
constexpr int kStatTokens = 4;   // tokens per staging round of the stats pass
constexpr int kSegMax = 1 << 17;  // keys staged in LDS at once by the tail, at most
constexpr int kQRawPerThread = 4;  // G * head_dim <= 4 * SB query elements
constexpr int kLdsMax = 160 * 1024;  // LDS per workgroup on gfx950
// Rows of more pages than this list their survivors (the tiles' own top-K
// keys) for the tail; shorter rows leave the tail every key, which costs it
// less than the listing costs the tiles.
constexpr int kSurvPages = 16384;

struct SelDims {
  int ntiles;     // L1 tiles per row at most (kernel A grid.y)
  int tcap;       // tiles per row in one dispatch round (CUs / rows)
  int clk_tiles;  // tile rows of the debug clock = ceil(max_blocks / 64)
  int seg;        // keys per segment staged in LDS by the tail
  int nseg;       // key segments per row
  int kstride;    // keys per row in the workspace = nseg * seg
  int words;      // candidate bitmap words = kstride / 32
  int np;         // candidate page capacity = k_f + k_n + 2
  int dense;      // dense candidate slots = np * bs
  int dstride;    // dense keys in LDS (multiple of 8)
  int prot;       // protected width = min(s_cap, sink + swa)
  int lds;        // LDS bytes per workgroup
  int multi;      // tiles may take several passes (second staging buffer)
  int surv;       // rows may be long enough to list survivors (multi only)
  int group;      // query heads per kv head
  int hd_sh, bs_sh, page_sh;  // log2 of head_dim, bs, page, or -1
  // LDS: a common part, then the tile part, or the tail: its candidate pages,
  // then its L1 part or (later) its L2 part
  int a_ctx;  // the row state wave 0 hands to the other waves
  int a_hist, a_tmp, a_misc, a_clk, a_qf, a_qs, a_qu, a_qg, a_fdims;
  int a_dims, a_last, a_tphys, a_stage, a_hs, a_st, a_st2;  // tile
  int a_tkeys;    // the tile's page keys over its passes (multi-pass tiles)
  int a_pages, a_pphys;                                // tail
  int sc;         // survivors the tail holds in LDS (more: every key is read)
  int a_keys, a_dbf, a_dbn, a_dsel;                    // tail, L1
  int a_dk, a_l0, a_l0x, a_l1, a_l1x, a_mid, a_mslot;  // tail, L2
  // global workspace byte offsets; counters and histograms first (they must
  // start at zero and are reset by the kernel itself)
  int64_t w_rowcnt, w_reqcnt, w_hist, w_keys, w_surv, w_scount, w_total;
};

__host__ __device__ inline int align16(int x) { return (x + 15) & ~15; }

// bf16 statistics over 32 or 64 L1 dims are staged in LDS by asynchronous
// global-to-LDS loads (32 dims double-buffered over the passes of a tile);
// other geometries are read from memory while scoring
__host__ __device__ inline bool stats_staged(const NfaSelectParams &p) {
  return (p.dsub == 32 || p.dsub == 64) && p.kv_dtype == NFA_DTYPE_BF16;
}

struct TileSplit {
  int span, tiles;  // pages per tile, tiles of the row
};

// End of the pass of a tile ending at t1 that starts at page c0: the rest of
// the tile when it fits one pass (kSpanMax pages), else one scoring round of
// TP pages.  A tile of w > kSpanMax pages takes 1 + ceil((w - kSpanMax) / TP)
// passes, all but the last of exactly TP pages.
__host__ __device__ inline int pass_end(int c0, int t1) {
  return t1 - c0 <= kSpanMax ? t1 : c0 + TP;
}

// The kt pages of a row in tiles of `span` pages: rounds of `tcap` tiles
// (one workgroup per CU over all rows of the launch), as few rounds as keep
// a tile within kTileMax pages (kPassMax passes), the pages spread evenly
// over the tiles.  A pass stages, scores and publishes the pages of one
// pass_end step; more passes per tile replace dispatch rounds of one-pass
// tiles (long rows, many rows).
__host__ __device__ inline TileSplit tile_split(int kt, int tcap) {
  TileSplit s;
  if (kt <= 0) {
    s.span = kSpanMin;
    s.tiles = 1;
    return s;
  }
  const int per_round = tcap * kTileMax;
  const int k = (kt + per_round - 1) / per_round;
  const int span = (kt + k * tcap - 1) / (k * tcap);
  s.span = span < kSpanMin ? kSpanMin : span;
  s.tiles = (kt + s.span - 1) / s.span;
  return s;
}

// LDS layout of the selector and its workspace for s.seg / s.words / s.np.
__host__ __device__ inline void sel_layout(const NfaSelectParams &p, SelDims &s) {
  const int group = p.hq / p.hkv;
  s.dense = s.np * p.bs;
  s.dstride = (s.dense + 7) & ~7;
  const int s_cap = p.max_blocks * p.bs;
  s.prot = p.sink_tokens + p.swa < s_cap ? p.sink_tokens + p.swa : s_cap;
  int o = 0;
  s.a_ctx = o;   o += align16(4 * 24);
  s.a_hist = o;  o += align16(4 * 4 * 256);
  s.a_tmp = o;   o += align16(4 * 128);
  s.a_misc = o;  o += align16(4 * 32);
  s.a_clk = o;   o += 8 * 64;  // debug timeline: tile marks, tail marks
  // query rows padded by 4 floats each
  s.a_qf = o;    o += align16(4 * group * (p.dsub + 4));
  s.a_qs = o;    o += align16(4 * group * (2 * p.dsub + 4));  // min(q,0) | max(q,0)
  s.a_qu = o;    // unrounded scaled query rows (avg_top2 far scores)
  if (p.far_method == NFA_METHOD_AVG_TOP2) o += align16(4 * group * (p.dsub + 4));
  s.a_qg = o;    o += align16(4 * p.fine_dsub);          // grouped L2 query
  s.a_fdims = o; o += align16(4 * p.fine_dsub);
  const int a_base = o;
  s.a_dims = o;  o += align16(4 * p.dsub);
  s.a_last = o;  o += align16(4 * 3 * p.dsub);
  s.a_tphys = o; o += align16(4 * kSpanMax);
  s.a_stage = o; o += align16(4 * SB * kStatTokens);
  s.a_hs = s.a_stage;  // per-head page scores, after the statistics phase
  s.a_st = o;          // bf16 32-dim statistics of the tile, staged
  if (stats_staged(p)) o += 2 * (p.dsub / 8) * kSpanMax * 16;
  s.a_st2 = o;         // the next pass's, staged while this one is scored
  if (stats_staged(p) && s.multi && p.dsub == 32) o += 2 * (32 / 8) * kSpanMax * 16;
  s.a_tkeys = o; if (s.multi) o += align16(2 * kTileMax);
  const int a_tile = o;
  o = a_base;
  s.a_pages = o; o += align16(4 * s.np);
  s.a_pphys = o; o += align16(4 * s.np);
  const int a_l12 = o;
  // the row's keys, or (instead) its survivors: pages (4 bytes) then keys
  s.sc = ((2 * s.seg) / 8) & ~15;
  if (s.sc < 8192) s.sc = 8192;
  if (s.sc > 32 * SB) s.sc = 32 * SB;  // at most 32 per thread in the selection
  s.a_keys = o;  o += align16(s.surv && 8 * s.sc > 2 * s.seg ? 8 * s.sc : 2 * s.seg);
  s.a_dbf = o;   o += align16(4 * s.words);
  s.a_dbn = o;   o += align16(4 * s.words);
  s.a_dsel = o;  o += align16(8 * (p.k_f + p.k_n + 1));
  const int a_l1 = o;
  o = a_l12;
  s.a_dk = o;    o += align16(2 * s.dstride);
  s.a_l0 = o;    o += align16(4 * p.k2);
  s.a_l0x = o;   o += align16(4 * p.k2);
  s.a_l1 = o;    o += align16(4 * p.k2);
  s.a_l1x = o;   o += align16(4 * p.k2);
  s.a_mid = o;   o += align16(4 * p.k2);
  s.a_mslot = o; o += align16(4 * p.k2);
  const int a_l2 = o;
  const int a_tail = a_l1 > a_l2 ? a_l1 : a_l2;
  s.lds = a_tile > a_tail ? a_tile : a_tail;
  // workspace
  const int rows = p.batch * p.hkv;
  int64_t w = 0;
  s.w_rowcnt = w; w += ((int64_t)4 * kArriveStride * rows + 255) & ~(int64_t)255;
  s.w_reqcnt = w; w += ((int64_t)4 * p.batch + 255) & ~(int64_t)255;
  s.w_hist = w;   w += (int64_t)4 * rows * 512;
  s.w_keys = w;   w += (((int64_t)2 * rows * s.kstride) + 255) & ~(int64_t)255;
  // survivors' pages, then keys, and the tiles' survivor counts
  s.w_surv = w;   if (s.surv) w += (int64_t)8 * rows * s.kstride;
  s.w_scount = w; if (s.surv) w += (((int64_t)4 * rows * s.ntiles) + 255) & ~(int64_t)255;
  s.w_total = w;
}

// `cus`: compute units of the device; the tile split and with it the
// workspace layout (tile counts, survivor lists) depend on it
__host__ __device__ inline SelDims sel_dims(const NfaSelectParams &p, int cus) {
  SelDims s;
  const int nrows = p.batch * p.hkv;
  auto log2_or = [](int v) {
    int sh = 0;
    while ((1 << sh) < v) ++sh;
    return v > 0 && (1 << sh) == v ? sh : -1;
  };
  s.group = p.hq / p.hkv;
  s.hd_sh = log2_or(p.head_dim);
  s.bs_sh = log2_or(p.bs);
  s.page_sh = log2_or(p.page);
  s.tcap = cus / nrows > 1 ? cus / nrows : 1;
  s.clk_tiles = (p.max_blocks + kSpanMin - 1) / kSpanMin;
  {
    // tile_split(kt).tiles <= k(kt) * tcap and <= ceil(kt / 64) for kt <= max_blocks
    const int per_round = s.tcap * kTileMax;
    const int kmax = (p.max_blocks + per_round - 1) / per_round;
    s.ntiles = kmax * s.tcap < s.clk_tiles ? kmax * s.tcap : s.clk_tiles;
  }
  const int kpad = ((p.max_blocks + TP - 1) / TP) * TP;  // keys per row
  s.np = p.k_f + p.k_n + 2;
  // a tile spans more than one pass only when a dispatch round of one-pass
  // tiles cannot cover the widest row
  s.multi = p.max_blocks > s.tcap * kSpanMax;
  s.surv = s.multi && p.max_blocks > kSurvPages && p.far_method != NFA_METHOD_AVG_TOP2;
  // keys staged per tail segment: as many as fit beside the debug bitmaps
  // (one bit per page each) in the LDS of a workgroup
  for (int seg = kpad < kSegMax ? kpad : kSegMax;; seg /= 2) {
    s.seg = seg;
    s.nseg = (kpad + s.seg - 1) / s.seg;
    s.kstride = s.nseg * s.seg;
    s.words = s.kstride / 32;
    sel_layout(p, s);
    if (s.lds <= kLdsMax || seg <= TP || seg % 16 != 0) break;
  }
  return s;
}


// ---------------------------------------------------------------------------
// per-row geometry (Appendix-A formulas of the reference, Triton integer
// division truncates toward zero exactly like C)
// ---------------------------------------------------------------------------

struct RowGeo {
  int L, kt_eff, near_start, swa_lo_blk, far_end, near_end;
  int sink_hi, swa_hi, orig_far_hi, spl, byp_blk;
  bool byp_cond, far_on, near_on, sink_unaligned;
};

__device__ __forceinline__ int imin(int a, int b) { return a < b ? a : b; }
__device__ __forceinline__ int imax(int a, int b) { return a > b ? a : b; }

// x / d with C's truncation toward zero; sh = log2(d) when d is a power of
// two (a shift instead of the division sequence), else -1
__device__ __forceinline__ int div_p2(int x, int d, int sh) {
  if (sh < 0) return x / d;
  return x >= 0 ? (x >> sh) : -((-x) >> sh);
}
// the same for x >= 0
__device__ __forceinline__ int udiv_p2(int x, int d, int sh) {
  return sh >= 0 ? (x >> sh) : x / d;
}

__device__ __forceinline__ RowGeo row_geo(const NfaSelectParams &p, const SelDims &sd,
                                          int L, bool skip_far, bool skip_near) {
  RowGeo g;
  const int bs = p.bs;
  auto dbs = [&](int x) { return div_p2(x, bs, sd.bs_sh); };
  const int pool_near_len = imax(bs, p.near_len);
  g.L = L;
  g.kt_eff = L > 0 ? dbs(L + bs - 1) : 0;
  g.spl = dbs(p.sink_tokens);
  g.near_start = imax(dbs(L - p.geo_window - pool_near_len), g.spl);
  g.swa_lo_blk = imax(g.near_start, g.kt_eff - imax(1, dbs(p.geo_window)));
  g.far_end = imin(g.kt_eff, g.near_start);
  g.near_end = g.swa_lo_blk;
  g.far_on = !skip_far;
  g.near_on = !skip_near;
  g.sink_hi = imin(p.geo_sink, L);
  g.swa_hi = imax(g.sink_hi, L - p.geo_window);
  const int far_blk = div_p2(L - p.geo_window - p.geo_near, p.page, sd.page_sh);
  g.orig_far_hi = imin(g.swa_hi, imax(g.sink_hi, far_blk * p.page));
  const int swa_lo_tok = imax(L - p.geo_window, 0);
  g.byp_blk = dbs(swa_lo_tok);
  g.sink_unaligned = (p.geo_sink - dbs(p.geo_sink) * bs) != 0;
  g.byp_cond = (swa_lo_tok - g.byp_blk * bs != 0) && (g.byp_blk >= g.spl);
  if (g.sink_unaligned) g.byp_cond = g.byp_cond && (g.byp_blk != g.spl);
  return g;
}

// The row geometry wave 0 stored at s_ctx[8..20) (int4 words 2..4), as
// wave-uniform values, with the given pool switches.
__device__ __forceinline__ RowGeo ctx_geo(const int *s_ctx, int L, bool far_on,
                                          bool near_on) {
  const int4 *c4 = reinterpret_cast<const int4 *>(s_ctx);
  const int4 e = c4[2], f = c4[3], h = c4[4];
  auto u = [](int v) { return __builtin_amdgcn_readfirstlane(v); };
  RowGeo g;
  g.L = L;
  g.kt_eff = u(e.x);
  g.near_start = u(e.y);
  g.swa_lo_blk = u(e.z);
  g.far_end = u(e.w);
  g.near_end = u(f.x);
  g.sink_hi = u(f.y);
  g.swa_hi = u(f.z);
  g.orig_far_hi = u(f.w);
  g.spl = u(h.x);
  g.byp_blk = u(h.y);
  const int fl = u(h.z);
  g.byp_cond = (fl & 1) != 0;
  g.sink_unaligned = (fl & 2) != 0;
  g.far_on = far_on;
  g.near_on = near_on;
  return g;
}

// Pool membership of page t.  Monotone in the skip flags: a page in a pool
// with skips applied is also in it without them.
__device__ __forceinline__ void pools(const NfaSelectParams &p, const RowGeo &g,
                                      int t, bool *far_pool, bool *near_pool) {
  const int bs = p.bs;
  const int block_lo = t * bs;
  const int block_hi = block_lo + bs;
  const bool has_sink = block_lo < g.sink_hi;
  const bool has_far =
      g.far_on && (block_hi > g.sink_hi) && (block_lo < g.orig_far_hi);
  const bool has_near =
      g.near_on && (block_hi > g.orig_far_hi) && (block_lo < g.swa_hi);
  const bool has_swa = (block_hi > g.swa_hi) && (block_lo < g.L);
  const bool valid =
      (block_lo < g.L) && (has_sink || has_far || has_near || has_swa);
  bool fp = (t >= g.spl) && (t < g.near_start) && g.far_on;
  bool np = (t >= g.near_start) && (t < g.swa_lo_blk) && g.near_on &&
            !((t == g.byp_blk) && g.byp_cond);
  if (g.sink_unaligned) {
    fp = fp && (t != g.spl);
    np = np && (t != g.spl);
  }
  *far_pool = fp && valid;
  *near_pool = np && valid;
}

struct L2Bounds {
  int lo, lower, upper, quota, far_hi;
};

__device__ __forceinline__ L2Bounds l2_bounds(const NfaSelectParams &p, int L,
                                              bool skip_far, bool skip_near,
                                              int near_len_for_far) {
  L2Bounds r;
  const int bs = p.bs;
  r.lo = imax(0, L - p.swa);
  int lower = (p.sink_tokens / bs) * bs;
  int upper = imax(lower, r.lo);
  const int sink_hi = imin(L, p.sink_tokens);
  const int swa_hi = imax(sink_hi, L - p.swa);
  const int far_blk = (imax(L - p.swa - near_len_for_far, 0) / p.page) * p.page;
  r.far_hi = imin(swa_hi, imax(sink_hi, far_blk));
  if (skip_far) lower = r.far_hi;
  if (skip_near) upper = r.far_hi;
  upper = imax(lower, upper);
  int quota = imax(imin(L, p.k2) - p.sink_tokens - (L - r.lo), 0);
  quota = imin(quota, upper - lower);
  r.lower = lower;
  r.upper = upper;
  r.quota = quota;
  return r;
}

// stats element index in the chunk-major layout
template <typename KV>
__device__ __forceinline__ int64_t stat_index(const NfaSelectParams &p,
                                              int64_t req, int kv, int d,
                                              int page_t, int dsub) {
  constexpr int CH = Elem<KV>::kChunk;
  return ((((req * p.kv_heads_mem + kv) * (dsub / CH) + d / CH) * (int64_t)p.max_blocks +
           page_t) *
          CH) +
         (d % CH);
}

// Block-table entries outside the arena read the PAD page (the last one).
__device__ __forceinline__ int safe_page(const NfaSelectParams &p, int phys) {
  return (phys >= 0 && phys < p.pool_pages) ? phys : p.pool_pages - 1;
}

__device__ __forceinline__ int64_t kv_offset(const NfaSelectParams &p,
                                             int phys, int kv, int off) {
  return (((int64_t)phys * p.kv_heads_mem + kv) * p.page + off) * p.head_dim;
}

// L2 side copy of one (request, kv head): per L1 page of bs tokens, when the
// L2 dims split into 16-byte chunks, chunk-major [chunk][token][CH] (a wave
// reading one chunk of consecutive tokens reads consecutive bytes), else
// token-major [token][fine_dsub].  Element d of token tok:
template <typename KV>
__device__ __forceinline__ int64_t l2_side_index(const NfaSelectParams &p,
                                                 int64_t req, int kv, int tok,
                                                 int d) {
  constexpr int CH = Elem<KV>::kChunk;
  const int64_t page = (req * p.kv_heads_mem + kv) * (int64_t)p.max_blocks + tok / p.bs;
  const int r = tok % p.bs;
  const int64_t base = page * p.bs * p.fine_dsub;
  return p.fine_dsub % CH == 0
             ? base + ((int64_t)(d / CH) * p.bs + r) * CH + d % CH
             : base + (int64_t)r * p.fine_dsub + d;
}

// 4-bit L2 side cache (--nfa_l2_quant, 32 or 64 L2 dims): per (request, kv
// head, token) fine_dsub / 2 bytes of codes -- dim d in nibble d % 2 of
// byte d / 2 -- at slot * fine_dsub / 2, and the token's bf16 scale and zero
// (scale in the low half) after every slot's codes, at slots * fine_dsub / 2
// + 4 * slot; slot = (req * hkv + kv) * max_blocks * bs + tok.
__host__ __device__ __forceinline__ bool q4_dims_ok(int fine_dsub) {
  return fine_dsub == 32 || fine_dsub == 64;
}
__device__ __forceinline__ int64_t q4_slot(const NfaSelectParams &p, int64_t req,
                                           int kv, int tok) {
  return (req * p.kv_heads_mem + kv) * (int64_t)p.max_blocks * p.bs + tok;
}
__device__ __forceinline__ int64_t q4_slots(const NfaSelectParams &p) {
  return (int64_t)p.max_req * p.kv_heads_mem * p.max_blocks * p.bs;
}

// min_max_per_token_quant (tia_indexer.py:22-31) with torch's bf16 rounding
// after every op: range = bf16(max - min) clamped to 1e-9, scale =
// bf16(range / 15), zero = -min, code = clamp(round_half_even(bf16(bf16(x +
// zero) / scale)), 0, 15).  Stores the codes and (scale, zero) of the token
// whose K row is `row` (L2 dims at fdims); the row is read twice (range,
// then codes) rather than held in registers.
template <typename KV>
__device__ __forceinline__ void q4_store(const NfaSelectParams &p, int64_t req, int kv,
                                         int tok, const KV *row, const int *fdims) {
  // eight dims per step: few registers live where the rebuild runs
  const int nd = p.fine_dsub;
  const int cb = nd / 2;  // code bytes per slot
  float mx = Elem<KV>::load(row + fdims[0]);
  float mn = mx;
#pragma unroll 1
  for (int d0 = 0; d0 < nd; d0 += 8) {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float x = Elem<KV>::load(row + fdims[d0 + e]);
      mx = fmaxf(mx, x);
      mn = fminf(mn, x);
    }
  }
  float rng = bf16r(mx - mn);
  if (rng < 1e-9f) rng = bf16r(1e-9f);
  const float scale = bf16r(rng / 15.0f);
  const float zero = -mn;
  const int64_t slot = q4_slot(p, req, kv, tok);
  unsigned char *base = (unsigned char *)p.l2_keys_l;
#pragma unroll 1
  for (int d0 = 0; d0 < nd; d0 += 8) {
    uint32_t w = 0u;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float x = Elem<KV>::load(row + fdims[d0 + e]);
      const float t = bf16r(bf16r(x + zero) / scale);
      const float c = fminf(fmaxf(rintf(t), 0.0f), 15.0f);
      w |= (uint32_t)c << (4 * e);
    }
    *reinterpret_cast<uint32_t *>(base + slot * cb + d0 / 2) = w;
  }
  *reinterpret_cast<uint32_t *>(base + q4_slots(p) * cb + slot * 4) =
      (uint32_t)bf16_bits(scale) | ((uint32_t)bf16_bits(zero) << 16);
}

// q4_store by lanes 0 .. fine_dsub - 1 of one wave, lane d holding L2 dim d
// of the token: the range by a shuffle tree over those lanes, one code per
// lane, the eight nibbles of a word OR-ed together across lanes.
__device__ __forceinline__ void q4_store_lanes(const NfaSelectParams &p, int64_t req,
                                               int kv, int tok, float x, int d) {
  const int nd = p.fine_dsub;  // 32 or 64 lanes
  float mx = x, mn = x;
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    if (off < nd) {
      mx = fmaxf(mx, __shfl_xor(mx, off, 64));
      mn = fminf(mn, __shfl_xor(mn, off, 64));
    }
  }
  float rng = bf16r(mx - mn);
  if (rng < 1e-9f) rng = bf16r(1e-9f);
  const float scale = bf16r(rng / 15.0f);
  const float zero = -mn;
  const float t = bf16r(bf16r(x + zero) / scale);
  unsigned w = (unsigned)fminf(fmaxf(rintf(t), 0.0f), 15.0f) << (4 * (d % 8));
#pragma unroll
  for (int off = 1; off < 8; off <<= 1) w |= __shfl_xor(w, off, 64);
  const int64_t slot = q4_slot(p, req, kv, tok);
  const int cb = nd / 2;
  unsigned char *base = (unsigned char *)p.l2_keys_l;
  if (d % 8 == 0) store_coherent(reinterpret_cast<uint32_t *>(base + slot * cb + d / 2), w);
  if (d == 0)
    store_coherent(reinterpret_cast<uint32_t *>(base + q4_slots(p) * cb + slot * 4),
                   (uint32_t)bf16_bits(scale) | ((uint32_t)bf16_bits(zero) << 16));
}

// ---------------------------------------------------------------------------
// page statistics of pages [pg_lo, pg_hi) for one (request, kv)
// ---------------------------------------------------------------------------

// The key row of token `new_tok` comes from `new_row` when it is non-null
// (the decode token, whose pool write is issued by this same workgroup).
__device__ __forceinline__ bool is_new(int tok, int new_tok, const void *row) {
  return row != nullptr && tok == new_tok;
}

// The page's tokens are staged through LDS in sub-batches of kStatTokens
// (all loads of a sub-batch in flight at once); each (page, dim) thread then
// scans its tokens in ascending order: v < min, v > max, sum + v.  Compact
// code: this is the path of the incremental (latest page) update.  ``s_tphys``
// (or NULL) holds the physical page of every page of the range when a page
// never straddles two physical pages.
// The stored avg statistic of one page dim: the page sum rounded to the KV
// dtype, divided by bs and rounded to bf16 -- the key the avg pools score
// with (selector:311-354), computed once when the page's statistics are
// written instead of by every query head at every decode step.
template <typename KV>
__device__ __forceinline__ KV page_mean(float sum, int bs) {
  const KV s = (KV)Elem<KV>::from_f32(sum);
  return (KV)Elem<KV>::from_f32(bf16r(Elem<KV>::load(&s) / (float)bs));
}

template <int DSUB, typename KV>
__device__ __forceinline__ void compute_stats(const NfaSelectParams &p, int64_t req, int kv,
                              int L, int pg_lo, int pg_hi, float *s_stage,
                              const int *s_dims, const int *s_tphys,
                              const KV *new_row, int new_tok, float *page_sum,
                              int sum_pg) {
  const KV *kpool = (const KV *)p.k_pool_l;
  const int32_t *bt = p.block_table_l + req * p.max_blocks;
  constexpr int PER = SB / DSUB;  // pages per pass
  const int tid = threadIdx.x;
  const int d = tid % DSUB;
  const int slot = tid / DSUB;
  KV *smin = (KV *)p.stat_min_l;
  KV *smax = (KV *)p.stat_max_l;
  KV *ssum = (KV *)p.stat_sum_l;
  for (int pg0 = pg_lo; pg0 < pg_hi; pg0 += PER) {
    const int pg = pg0 + slot;
    float mn = __uint_as_float(0x7F800000u);
    float mx = __uint_as_float(0xFF800000u);
    float sm = 0.0f;
    for (int i0 = 0; i0 < p.bs; i0 += kStatTokens) {
#pragma unroll
      for (int k = 0; k < kStatTokens; ++k) {
        const int e = tid + k * SB;  // [page slot][token][dim]
        const int dd = e % DSUB;
        const int ti = (e / DSUB) % kStatTokens;
        const int ps = e / (DSUB * kStatTokens);
        const int px = pg0 + ps;
        const int tok = px * p.bs + i0 + ti;
        const int lp = tok / p.page;
        float v = 0.0f;
        if (px < pg_hi && i0 + ti < p.bs && tok < L && lp < p.max_blocks) {
          if (is_new(tok, new_tok, new_row)) {
            v = Elem<KV>::load(new_row + s_dims[dd]);
          } else {
            const int phys = s_tphys != nullptr ? s_tphys[px - pg_lo]
                                                : safe_page(p, bt[lp]);
            v = Elem<KV>::load(kpool + kv_offset(p, phys, kv, tok % p.page) +
                               s_dims[dd]);
          }
        }
        s_stage[e] = v;
      }
      __syncthreads();
      if (pg < pg_hi) {
        for (int ti = 0; ti < kStatTokens && i0 + ti < p.bs; ++ti) {
          const int tok = pg * p.bs + i0 + ti;
          if (tok >= L || tok / p.page >= p.max_blocks) break;
          const float v = s_stage[(slot * kStatTokens + ti) * DSUB + d];
          mn = (v < mn) ? v : mn;
          mx = (v > mx) ? v : mx;
          sm = sm + v;
        }
      }
      __syncthreads();
    }
    if (pg < pg_hi) {
      const int64_t si = stat_index<KV>(p, req, kv, d, pg, DSUB);
      const KV a = (KV)Elem<KV>::from_f32(mn);
      const KV c = (KV)Elem<KV>::from_f32(mx);
      const KV s = page_mean<KV>(sm, p.bs);
      smin[si] = a;
      smax[si] = c;
      ssum[si] = s;
      if (page_sum != nullptr && pg == sum_pg) page_sum[d] = sm;
    }
  }
}

// Vector form for L1 dims made of aligned 16-byte runs: one item = (page,
// 16-byte chunk of dims); the chunk of 16 tokens is requested at once and
// each dim is then scanned over the tokens in ascending order.  ``s_coff``
// holds the element offset of every chunk, ``s_tphys`` (or NULL) the
// physical page of every page of the range when a page never straddles two
// physical pages.  ``s_last`` (or NULL) receives the stored statistics of a
// single-page range as floats.
template <int DSUB, typename KV>
__device__ __forceinline__ void compute_stats_vec(const NfaSelectParams &p, int64_t req, int kv,
                                  int L, int pg_lo, int pg_hi,
                                  const int *s_coff, const int *s_tphys,
                                  const KV *new_row, int new_tok,
                                  float *page_sum, int sum_pg) {
  constexpr int CH = Elem<KV>::kChunk;
  constexpr int NCH1 = DSUB / CH;
  constexpr int TG = 4;
  const KV *kpool = (const KV *)p.k_pool_l;
  const int32_t *bt = p.block_table_l + req * p.max_blocks;
  KV *smin = (KV *)p.stat_min_l;
  KV *smax = (KV *)p.stat_max_l;
  KV *ssum = (KV *)p.stat_sum_l;
  const int n_items = (pg_hi - pg_lo) * NCH1;
  for (int it = threadIdx.x; it < n_items; it += SB) {
    const int pg = pg_lo + it / NCH1;
    const int c = it % NCH1;
    float mn[CH], mx[CH], sm[CH];
#pragma unroll
    for (int e = 0; e < CH; ++e) {
      mn[e] = __uint_as_float(0x7F800000u);
      mx[e] = __uint_as_float(0xFF800000u);
      sm[e] = 0.0f;
    }
    for (int i0 = 0; i0 < p.bs; i0 += TG) {
      uint4 raw[TG];
      bool ok[TG];
#pragma unroll
      for (int k = 0; k < TG; ++k) {
        const int i = i0 + k;
        const int tok = pg * p.bs + i;
        const int lp = tok / p.page;
        ok[k] = i < p.bs && tok < L && lp < p.max_blocks;
        raw[k] = make_uint4(0u, 0u, 0u, 0u);
        if (ok[k]) {
          const KV *src;
          if (is_new(tok, new_tok, new_row)) {
            src = new_row;
          } else {
            const int phys = s_tphys != nullptr ? s_tphys[pg - pg_lo]
                                                : safe_page(p, bt[lp]);
            src = kpool + kv_offset(p, phys, kv, tok % p.page);
          }
          raw[k] = *reinterpret_cast<const uint4 *>(src + s_coff[c]);
        }
      }
#pragma unroll
      for (int k = 0; k < TG; ++k) {
        if (!ok[k]) continue;
        float x[CH];
        unpack_chunk<KV>(raw[k], x);
#pragma unroll
        for (int e = 0; e < CH; ++e) {
          mn[e] = (x[e] < mn[e]) ? x[e] : mn[e];
          mx[e] = (x[e] > mx[e]) ? x[e] : mx[e];
          sm[e] = sm[e] + x[e];
        }
      }
    }
    const int64_t si = stat_index<KV>(p, req, kv, c * CH, pg, DSUB);
#pragma unroll
    for (int e = 0; e < CH; ++e) {
      const KV a = (KV)Elem<KV>::from_f32(mn[e]);
      const KV b = (KV)Elem<KV>::from_f32(mx[e]);
      const KV s = page_mean<KV>(sm[e], p.bs);
      smin[si + e] = a;
      smax[si + e] = b;
      ssum[si + e] = s;
      if (page_sum != nullptr && pg == sum_pg) page_sum[c * CH + e] = sm[e];
    }
  }
}

// Statistics of the latest page (the incremental update of every decode
// step), compact: rounds of 4 * (256 / DSUB) tokens are staged through LDS by
// (token, dim) threads, four loads in flight each; thread d < DSUB then scans
// the round's tokens in ascending order.  `phys_first` is the physical page
// of the page's first token (used when a page never straddles two physical
// pages).
template <int DSUB, typename KV>
__device__ __forceinline__ void stats_latest_page(
    const NfaSelectParams &p, int64_t req, int kv, int L, int pg,
    int phys_first, const int *s_dims, float *s_stage, const KV *new_row,
    float *s_last) {
  constexpr int R = SB / DSUB;
  constexpr int RT = 4 * R;  // tokens per round
  const int tid = threadIdx.x;
  const int d = tid % DSUB;
  const int r = tid / DSUB;
  const int tok0 = pg * p.bs;
  const int nt = imin(p.bs, L - tok0);
  const bool one_phys = (p.page % p.bs) == 0;
  const int32_t *bt = p.block_table_l + req * p.max_blocks;
  const KV *kpool = (const KV *)p.k_pool_l;
  const int dim = s_dims[d];
  float mn = __uint_as_float(0x7F800000u);
  float mx = __uint_as_float(0xFF800000u);
  float sm = 0.0f;
  for (int i0 = 0; i0 < nt; i0 += RT) {
    float v[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int i = i0 + r + k * R;
      v[k] = 0.0f;
      if (i < nt) {
        const int tok = tok0 + i;
        if (new_row != nullptr && tok == L - 1) {
          v[k] = Elem<KV>::load(new_row + dim);
        } else {
          const int phys =
              one_phys ? phys_first
                       : safe_page(p, bt[imin(tok / p.page, p.max_blocks - 1)]);
          v[k] = Elem<KV>::load(kpool + kv_offset(p, phys, kv, tok % p.page) + dim);
        }
      }
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) s_stage[(r + k * R) * DSUB + d] = v[k];
    __syncthreads();
    if (tid < DSUB) {
      const int n = imin(RT, nt - i0);
      for (int i = 0; i < n; ++i) {
        const float x = s_stage[i * DSUB + d];
        mn = (x < mn) ? x : mn;
        mx = (x > mx) ? x : mx;
        sm = sm + x;
      }
    }
    __syncthreads();
  }
  if (tid < DSUB) {
    const int64_t si = stat_index<KV>(p, req, kv, d, pg, DSUB);
    const KV a = (KV)Elem<KV>::from_f32(mn);
    const KV c = (KV)Elem<KV>::from_f32(mx);
    const KV s = page_mean<KV>(sm, p.bs);
    ((KV *)p.stat_min_l)[si] = a;
    ((KV *)p.stat_max_l)[si] = c;
    ((KV *)p.stat_sum_l)[si] = s;
    s_last[d] = Elem<KV>::load(&a);
    s_last[DSUB + d] = Elem<KV>::load(&c);
    s_last[2 * DSUB + d] = Elem<KV>::load(&s);
  }
}

// LDS byte address of a pointer into the workgroup's LDS.
__device__ __forceinline__ uint32_t lds_addr(const void *ptr) {
  typedef __attribute__((address_space(3))) const void lds_cvoid;
  return (uint32_t)(uintptr_t)(lds_cvoid *)ptr;
}

// One gfx950 global_load_lds_dwordx4: lane i of the wave copies the 16 bytes
// at its src to LDS byte lds + 16 i (inactive lanes copy nothing); M0 holds
// the wave-uniform LDS base and is read one wait state after it is written.
// Written as assembly, the copy is invisible to the compiler, which
// therefore inserts no wait for it before later LDS reads of unrelated data:
// the destination may be read only after the issuing wave's vmcnt(0) wait
// followed by a workgroup barrier.
__device__ __forceinline__ void lds_dma16(const void *src, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off"
               :
               : "v"(src), "s"(lds)
               : "memory", "m0");
}

// One global_load_lds_dword: lane i copies the 4 bytes at its src to LDS
// byte lds + 4 i (inactive lanes copy nothing); the same rules as lds_dma16.
__device__ __forceinline__ void lds_dma4(const void *src, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dword %0, off"
               :
               : "v"(src), "s"(lds)
               : "memory", "m0");
}

// Asynchronous global-to-LDS copies of the bf16 statistics of pages
// [t0, t1), 32 L1 dims: s_st[slot][chunk][kSpanMax] 16-byte chunks, slot 0
// the min (minmax pools) or the sum (avg pools), slot 1 the max.  A wave
// fills 64 consecutive pages of one (slot, chunk) row per copy; pages outside
// both pools are not copied.  Complete at the issuing wave's next vmcnt(0)
// wait (see lds_dma16).
// Waves w0, w0 + 1, ... (nw of them) issue the copies.
template <int DSUB>
__device__ __forceinline__ void stage_stats_async(const NfaSelectParams &p,
                                                  const RowGeo &g, int64_t req,
                                                  int kv, int t0, int t1,
                                                  unsigned char *s_st, int w0 = 0,
                                                  int nw = SW) {
  constexpr int NC = DSUB / 8;
  const bool far_mm = p.far_method == NFA_METHOD_MINMAX;
  const bool near_mm = p.near_method == NFA_METHOD_MINMAX;
  // the statistic bases held in scalar registers: the per-lane choice of
  // base is then a register select, not a load of the kernel argument at a
  // per-lane offset (whose wait would also wait for every earlier copy)
  const uint16_t *smin = (const uint16_t *)p.stat_min_l;
  const uint16_t *ssum = (const uint16_t *)p.stat_sum_l;
  const uint16_t *smax = (const uint16_t *)p.stat_max_l;
  asm volatile("" : "+s"(smin), "+s"(ssum), "+s"(smax));
  const uint32_t lds0 = lds_addr(s_st);
  const int nblk = (t1 - t0 + 63) / 64;
  // units (chunk, 64-page block), both slots per unit
  if (wave_id() < w0) return;
  for (int u = wave_id() - w0; u < NC * nblk; u += nw) {
    const int c = u % NC;   // NC a power of two: no division
    const int blk = u / NC;
    const int t = t0 + blk * 64 + lane_id();
    bool fp = false, np = false;
    if (t < t1) pools(p, g, t, &fp, &np);
    const bool mm = (fp && far_mm) || (np && near_mm);
    const bool avg = (fp && !far_mm) || (np && !near_mm);
    const int64_t base = stat_index<uint16_t>(p, req, kv, c * 8, t, DSUB);
    const uint32_t row0 = lds0 + (uint32_t)(c * kSpanMax + blk * 64) * 16;
    if (mm || avg) lds_dma16((mm ? smin : ssum) + base, row0);
    if (mm) lds_dma16(smax + base, row0 + NC * kSpanMax * 16);
  }
}

// ---------------------------------------------------------------------------
// L1 scores of one page for one kv group (selector:311-354)
// ---------------------------------------------------------------------------

constexpr int GMAX = 8;
static_assert(GMAX * kSpanMax * 4 <= 4 * SB * kStatTokens,
              "head scores fit the stage");

// One query head of one page from the staged statistics st (chunk c at
// st[c * kSpanMax], the max slot at st[4 * kSpanMax]):
// bf16(Σ_d kmin_d·min(q_d,0) + Σ_d kmax_d·max(q_d,0)) for minmax pools, from
// the split query qs = [min(q,0) | max(q,0)], and bf16(Σ_d kmean_d·q_d)
// for avg pools (kmean_d = bf16(ksum_d / bs), the stored statistic), from
// the query qf (and, with qu, the same mean against the unrounded query into
// *un); every sum sequential in ascending d, each exact product added with
// one rounding (a fused multiply-add per term).
template <int DSUB>
__device__ __forceinline__ float l1_head_staged(const uint4 *st, const float *qs,
                                                const float *qf, const float *qu,
                                                bool need_mm, float *un) {
  constexpr int NC = DSUB / 8;
  float r, su = 0.0f;
  if (need_mm) {
    float sn = 0.0f, sp = 0.0f;
#pragma unroll (NC > 4 ? 2 : NC)
    for (int c = 0; c < NC; ++c) {
      float lo[8], hi[8], ln[8], hp[8];
      unpack_chunk<uint16_t>(st[c * kSpanMax], lo);
      unpack_chunk<uint16_t>(st[(NC + c) * kSpanMax], hi);
      load_f8(qs + c * 8, ln);
      load_f8(qs + DSUB + c * 8, hp);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        sn = __builtin_fmaf(lo[e], ln[e], sn);
        sp = __builtin_fmaf(hi[e], hp[e], sp);
      }
    }
    r = sn + sp;
  } else {
    float sa = 0.0f;
#pragma unroll (NC > 4 ? 2 : NC)
    for (int c = 0; c < NC; ++c) {
      float k[8], q[8];
      unpack_chunk<uint16_t>(st[c * kSpanMax], k);
      load_f8(qf + c * 8, q);
#pragma unroll
      for (int e = 0; e < 8; ++e) sa = __builtin_fmaf(k[e], q[e], sa);
      if (qu != nullptr) {
        load_f8(qu + c * 8, q);
#pragma unroll
        for (int e = 0; e < 8; ++e) su = __builtin_fmaf(k[e], q[e], su);
      }
    }
    r = sa;
  }
  *un = bf16r(su);
  return bf16r(r);
}

// The page's G head scores in head order, summed from +0 (the group's
// score before the division by G): the same per-head arithmetic as
// l1_head_staged, for one page per lane.  qs / qf are the first head's rows
// (strides QS / QF floats); every lane reads the same query address, so
// those reads are LDS broadcasts.
template <int QF, int QS, int DSUB>
__device__ __forceinline__ float l1_group_staged(const uint4 *st, const float *qs,
                                                 const float *qf, int G, bool need_mm) {
  constexpr int NC = DSUB / 8;
  float acc = 0.0f;
  // one head at a time, a chunk of statistics unpacked per head (few
  // registers live: the kernel sits at its register budget)
  if (need_mm) {
#pragma unroll 1
    for (int j = 0; j < G; ++j) {
      const float *q0 = qs + j * QS;
      float sn = 0.0f, sp = 0.0f;
#pragma unroll (NC > 4 ? 2 : NC)
      for (int c = 0; c < NC; ++c) {
        float lo[8], hi[8], n0[8], p0[8];
        unpack_chunk<uint16_t>(st[c * kSpanMax], lo);
        unpack_chunk<uint16_t>(st[(NC + c) * kSpanMax], hi);
        load_f8(q0 + c * 8, n0);
        load_f8(q0 + DSUB + c * 8, p0);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          sn = __builtin_fmaf(lo[e], n0[e], sn);
          sp = __builtin_fmaf(hi[e], p0[e], sp);
        }
      }
      acc = acc + bf16r(sn + sp);
    }
  } else {
#pragma unroll 1
    for (int j = 0; j < G; ++j) {
      const float *q0 = qf + j * QF;
      float sa = 0.0f;
#pragma unroll (NC > 4 ? 2 : NC)
      for (int c = 0; c < NC; ++c) {
        float k[8], v0[8];
        unpack_chunk<uint16_t>(st[c * kSpanMax], k);
        load_f8(q0 + c * 8, v0);
#pragma unroll
        for (int e = 0; e < 8; ++e) sa = __builtin_fmaf(k[e], v0[e], sa);
      }
      acc = acc + bf16r(sa);
    }
  }
  return acc;
}

// Same arithmetic with the statistics read chunk by chunk from memory (L1
// dim counts above 32, fp32 statistics) or from `s_last` (the latest page).
template <int DSUB, typename KV>
__device__ __forceinline__ void l1_head_mem(const NfaSelectParams &p,
                                            int64_t req, int kv, int t,
                                            const float *q, const float *qu,
                                            bool need_mm, bool need_avg,
                                            const float *s_last, float *mm,
                                            float *avg, float *avg_u) {
  constexpr int CH = Elem<KV>::kChunk;
  const KV *smin = (const KV *)p.stat_min_l;
  const KV *smax = (const KV *)p.stat_max_l;
  const KV *ssum = (const KV *)p.stat_sum_l;
  float sn = 0.0f, sp = 0.0f, sa = 0.0f, su = 0.0f;
  for (int c = 0; c < DSUB / CH; ++c) {
    float kmin[CH], kmax[CH], ks[CH];
    if (s_last != nullptr) {
#pragma unroll
      for (int e = 0; e < CH; ++e) {
        kmin[e] = s_last[c * CH + e];
        kmax[e] = s_last[DSUB + c * CH + e];
        ks[e] = s_last[2 * DSUB + c * CH + e];
      }
    } else {
      const int64_t base = stat_index<KV>(p, req, kv, c * CH, t, DSUB);
      if (need_mm) {
        load_chunk<KV>(smin + base, kmin);
        load_chunk<KV>(smax + base, kmax);
      }
      if (need_avg) load_chunk<KV>(ssum + base, ks);
    }
#pragma unroll
    for (int e = 0; e < CH; ++e) {
      const float qd = q[c * CH + e];
      if (need_mm) {
        const float ql = qd < 0.0f ? qd : 0.0f;
        const float qh = qd > 0.0f ? qd : 0.0f;
        sn = __builtin_fmaf(kmin[e], ql, sn);
        sp = __builtin_fmaf(kmax[e], qh, sp);
      }
      if (need_avg) {
        const float kavg = ks[e];
        sa = __builtin_fmaf(kavg, qd, sa);
        if (qu != nullptr) su = __builtin_fmaf(kavg, qu[c * CH + e], su);
      }
    }
  }
  if (need_mm) *mm = bf16r(sn + sp);
  if (need_avg) *avg = bf16r(sa);
  if (need_avg && qu != nullptr) *avg_u = bf16r(su);
}

// torch.topk's value order: NaN above everything, +0 above -0.
__device__ __forceinline__ bool score_greater(float v, float o) {
  const bool vn = v != v, on = o != o;
  const bool pz_over_nz = v == 0.0f && o == 0.0f && !signbit(v) && signbit(o);
  return (vn && !on) || (!vn && !on && (v > o || pz_over_nz));
}

// avg_top2 far score of one page (selector:2412-2427, top-2 order :162-172):
// the mean of the two largest per-head bf16 page means against the
// unrounded scaled query, used where the same mean against the bf16-rounded
// query is finite (elsewhere that value stands).  `hs` holds, per head at
// a kSpanMax stride, (rounded-query bf16 << 16) | unrounded-query bf16.
__device__ __forceinline__ uint16_t top2_far_score(const float *hs, int G) {
  const float ninf = -__builtin_inff();
  float r1 = ninf, r2 = ninf, u1 = ninf, u2 = ninf;
  for (int j = 0; j < G; ++j) {
    const uint32_t w = __float_as_uint(hs[j * kSpanMax]);
    const float r = bf16_val((uint16_t)(w >> 16));
    const float u = bf16_val((uint16_t)(w & 0xFFFFu));
    const bool tr = score_greater(r, r1);
    const float rs = tr ? r1 : r;
    r1 = tr ? r : r1;
    r2 = score_greater(rs, r2) ? rs : r2;
    const bool tu = score_greater(u, u1);
    const float us = tu ? u1 : u;
    u1 = tu ? u : u1;
    u2 = score_greater(us, u2) ? us : u2;
  }
  const float kr = bf16r((r1 + r2) / 2.0f);
  if (!isfinite(kr)) return bf16_bits(kr);
  return bf16_bits((u1 + u2) / 2.0f);
}

// ---------------------------------------------------------------------------
// tail helpers
// ---------------------------------------------------------------------------

// Final top-K rule of one pool: a key k is selected when k > T, or when
// k == T != 0 and fewer than `need` equal keys precede it in page order.
struct PoolThr {
  int T, need, nsel;
};

__device__ __forceinline__ PoolThr pool_threshold(int K, const int *coarse,
                                                  const int *fine,
                                                  const int *fine_hist) {
  PoolThr r;
  const int hb = coarse[0];
  if (K <= 0) {
    r.T = 0x10000;  // nothing
    r.need = 0;
    r.nsel = 0;
  } else if (hb < 0) {  // every valid key
    r.T = 0;
    r.need = 0;
    r.nsel = coarse[2];
  } else {
    r.T = (hb << 8) | fine[0];
    r.need = K - coarse[1] - fine[1];
    r.nsel = K;
    if (fine_hist[fine[0]] == r.need) r.need = 1 << 30;  // no tie cut
  }
  return r;
}

__device__ __forceinline__ bool tie_cut(const PoolThr &t) {
  return t.need < (1 << 30) && t.T > 0 && t.T < 0x10000;
}

// Stage keys [seg_base, seg_base + seg) of a row into LDS by asynchronous
// 16-byte copies (seg a multiple of 8 keys): readable after dma_barrier().
__device__ __forceinline__ void stage_keys(const uint16_t *g_keys, int seg_base,
                                           int seg, uint16_t *s_keys,
                                           int first_wave = 0) {
  const int n16 = seg / 8;
  const uint4 *src = reinterpret_cast<const uint4 *>(g_keys + seg_base);
  const uint32_t lds0 = lds_addr(s_keys);
  if (wave_id() < first_wave) return;
  for (int u0 = (wave_id() - first_wave) * 64; u0 < n16; u0 += (SW - first_wave) * 64) {
    const int u = u0 + lane_id();
    if (u < n16) lds_dma16(src + u, lds0 + (uint32_t)u0 * 16);
  }
}

// Completes this wave's asynchronous copies, then the workgroup's.
__device__ __forceinline__ void dma_barrier() {
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
}

// Protected sink/SWA ids as up to two disjoint intervals [u0,u1) [u2,u3),
// exactly the ids of _final_union_protected_sort_kernel (selector:1337-1360):
// aux < min(s_cap, sink+swa); sink ids aux < min(L, sink); SWA ids
// L - swa + aux - sink_count for aux < min(L, sink+swa); ids < 0 dropped.
__device__ __forceinline__ void protected_intervals(const NfaSelectParams &p,
                                                    int L, int prot, int *u0,
                                                    int *u1, int *u2, int *u3) {
  const int s_cap = p.max_blocks * p.bs;
  const int sink_count = imin(L, p.sink_tokens);
  const int total = imin(L, p.sink_tokens + p.swa);
  const int a1 = imin(imin(sink_count, prot), s_cap);
  const int aux_end = imin(total, prot);
  int b0 = L - p.swa;
  int b1 = b0 + (aux_end - sink_count);
  if (aux_end <= sink_count) b1 = b0;
  b0 = imax(b0, 0);
  b1 = imin(b1, s_cap);
  if (b1 < b0) b1 = b0;
  if (a1 <= 0) {
    *u0 = *u1 = 0;
    *u2 = b0;
    *u3 = b1;
  } else if (b1 <= b0) {
    *u0 = 0;
    *u1 = a1;
    *u2 = *u3 = a1;
  } else if (b0 <= a1) {
    *u0 = 0;
    *u1 = imax(a1, b1);
    *u2 = *u3 = *u1;
  } else {
    *u0 = 0;
    *u1 = a1;
    *u2 = b0;
    *u3 = b1;
  }
}

// (kv: the arena's kv head; no V rows when v_new is NULL, a shared latent
// arena whose values are part of the key rows)
template <typename KV>
__device__ __forceinline__ void decode_write(const NfaSelectParams &p, int b,
                                             int kv) {
  const int slot = p.slots[b];
  if (slot < 0 || slot / p.page >= p.pool_pages) return;
  const int phys = slot / p.page;
  const int off = slot % p.page;
  KV *kp = (KV *)p.k_pool_l;
  KV *vp = (KV *)p.v_pool_l;
  const KV *kn = (const KV *)p.k_new;
  const KV *vn = (const KV *)p.v_new;
  const int hm = p.kv_heads_mem;
  for (int d = threadIdx.x; d < p.head_dim; d += SB)
    kp[kv_offset(p, phys, kv, off) + d] =
        kn[((int64_t)b * hm + kv) * p.head_dim + d];
  if (vn == nullptr) return;
  for (int d = threadIdx.x; d < p.head_dim_v; d += SB)
    vp[(((int64_t)phys * hm + kv) * p.page + off) * p.head_dim_v + d] =
        vn[((int64_t)b * hm + kv) * p.head_dim_v + d];
}

// Both regions skipped (region mode 3 / disjoint protected gather): decode
// write plus the union with an empty middle; no statistics are touched.
template <typename KV>
__global__ void __launch_bounds__(SB)
    nfa_protected_kernel(const NfaSelectParams p) {
  const int row = blockIdx.x;
  const int b = row / p.hkv;
  const int kv = row % p.hkv;  // selection row of the batch row
  const int L = p.lengths[b];
  const bool active = p.active_req[b] >= 0;
  const int64_t req = p.valid_req[b];
  // a shared arena (kv_heads_mem 1) is written by selection row 0 only
  if (p.k_new != nullptr && active && kv < p.kv_heads_mem)
    decode_write<KV>(p, b, p.kv_heads_mem > 1 ? kv : 0);
  if (p.middle_only) {
    if (threadIdx.x == 0) p.vis_lens[b * p.hkv + kv] = 0;
    return;
  }
  const int s_cap = p.max_blocks * p.bs;
  const int prot = p.sink_tokens + p.swa < s_cap ? p.sink_tokens + p.swa : s_cap;
  int u0, u1, u2, u3;
  protected_intervals(p, L, prot, &u0, &u1, &u2, &u3);
  const int nu = (u1 - u0) + (u3 - u2);
  const int32_t *bt = p.block_table_l + req * p.max_blocks;
  int32_t *grow = p.gather + ((int64_t)b * p.hkv + kv) * p.max_vis;
  for (int k = threadIdx.x; k < nu && k < p.max_vis; k += SB) {
    const int x = k < (u1 - u0) ? u0 + k : u2 + (k - (u1 - u0));
    grow[k] = bt[x / p.page] * p.page + x % p.page;
  }
  if (threadIdx.x == 0) p.vis_lens[b * p.hkv + kv] = nu;
  if (p.dbg_counts != nullptr && threadIdx.x == 0) p.dbg_counts[row] = 0;
}


// ---------------------------------------------------------------------------
// L2 top-quota selection over the dense candidate slots
// ---------------------------------------------------------------------------

// Candidate tokens in the dense page-major layout: slot i belongs to page
// pages[i / bs], token pages[i / bs] * bs + i % bs.
struct DenseView {
  const uint16_t *keys;
  const int *pages;
  const int *pphys;  // raw block-table entry of every page (page_phys mode)
  const int32_t *bt;
  int n, bs, page, mb;
  bool page_phys;
  int bs_sh, page_sh;  // log2 of bs and page, or -1
  __device__ __forceinline__ int tok(int i) const {
    const int pi = udiv_p2(i, bs, bs_sh);
    return pages[pi] * bs + (i - pi * bs);
  }
  __device__ __forceinline__ int slot_of(int i, int t) const {
    const int tp = udiv_p2(t, page, page_sh);
    const int ph = page_phys ? pphys[udiv_p2(i, bs, bs_sh)] : bt[imin(tp, mb - 1)];
    return ph * page + (t - tp * page);
  }
  __device__ __forceinline__ int slot_of_token(int t) const {
    const int tp = udiv_p2(t, page, page_sh);
    return bt[imin(tp, mb - 1)] * page + (t - tp * page);
  }
};

struct RegionLists {
  int *l0, *l0x, *l1, *l1x, *mid, *mslot;
};

// One L2 region (selector:519-566): top-quota of the dense candidates whose
// token lies in [rlo, rhi) (every candidate when !masked), ties to the lower
// token, then hole fill with the smallest ids of [rlo, rhi) not chosen and
// the sink filter; appended in ascending order to mid / mslot at *mid_count.
// `hist` needs 512 ints, `tmp` 48; with `hist_ready` its first 256 bins
// already hold the high-byte histogram of the (unmasked) keys.
__device__ __forceinline__ void l2_region_dense(const DenseView &dv, bool masked,
                                                int rlo, int rhi, int quota,
                                                int sink, const RegionLists &rl,
                                                int *mid_count, int *hist,
                                                int *tmp, int64_t *clk,
                                                bool hist_ready = false) {
  if (quota <= 0) return;
  const int tid = threadIdx.x;
  // optional phase timestamps, taken right after barriers the code has anyway
  auto mark = [&](int k) {
    if (clk != nullptr && tid == 0) clk[k] = wall_clock64();
  };
  const int n = dv.n;
  auto key = [&](int i) -> uint32_t {
    uint32_t v = dv.keys[i];
    if (masked && v != 0u) {
      const int t = dv.tok(i);
      if (t < rlo || t >= rhi) v = 0u;
    }
    return v;
  };
  if (!hist_ready) {
    if (tid < 512) hist[tid] = 0;
    __syncthreads();
    mark(0);
    for (int i = tid; i < n; i += SB) {
      const uint32_t v = key(i);
      if (v) atomicAdd(&hist[v >> 8], 1);
    }
    __syncthreads();
  }
  mark(1);
  if (wave_id() == 0) wave_threshold_bin(hist, quota, tmp + 8);
  __syncthreads();
  mark(2);
  const int hb = tmp[8];
  const int above = tmp[9];
  const int total = tmp[10];
  uint32_t T = 0u;
  int need = 0;
  if (hb >= 0) {
    for (int i = tid; i < n; i += SB) {
      const uint32_t v = key(i);
      if (v != 0u && (int)(v >> 8) == hb) atomicAdd(&hist[256 + (v & 255u)], 1);
    }
    __syncthreads();
    if (wave_id() == 0) wave_threshold_bin(hist + 256, quota - above, tmp + 12, true);
    __syncthreads();
    T = ((uint32_t)hb << 8) | (uint32_t)tmp[12];
    need = quota - above - tmp[13];
  }
  mark(3);
  const int nch = total < quota ? total : quota;
  const int nfill_req = quota - nch;
  const int base_out = *mid_count;
  // no hole to fill: the chosen tokens, in order, are the region's output
  // (candidate tokens start at max(sink, lower), so the sink filter drops
  // none of them)
  const bool direct = nfill_req == 0;
  // ordered emission, one contiguous run of slots per thread
  const int per = (n + SB - 1) / SB;
  const int ia = tid * per;
  const int ib = imin(n, ia + per);
  int c[2] = {0, 0};
  for (int i = ia; i < ib; ++i) {
    const uint32_t v = key(i);
    c[0] += v > T;
    c[1] += (v == T && v != 0u);
  }
  int tot2[2];
  // (its scratch is next written after the barrier that ends the emission)
  block_scan_n<2, SW, false>(c, tmp + 32, tot2);
  mark(4);
  {
    int eq = c[1];
    int pos = c[0] + (c[1] < need ? c[1] : need);
    for (int i = ia; i < ib; ++i) {
      const uint32_t v = key(i);
      bool sel = v > T;
      if (v == T && v != 0u) {
        sel = eq < need;
        ++eq;
      }
      if (sel) {
        const int t = dv.tok(i);
        if (direct) {
          rl.mid[base_out + pos] = t;
          rl.mslot[base_out + pos] = dv.slot_of(i, t);
        } else {
          rl.l0[pos] = t;
          rl.l0x[pos] = dv.slot_of(i, t);
        }
        ++pos;
      }
    }
  }
  __syncthreads();
  mark(5);
  if (direct) {
    if (tid == 0) *mid_count = base_out + nch;
    __syncthreads();
    return;
  }
  // hole fill: the (quota - nch) smallest ids of [rlo, rhi) not chosen
  for (int i = tid; i < nfill_req; i += SB) {
    int lo = 0, hi = nch;
    while (lo < hi) {
      const int mid = (lo + hi) >> 1;
      if (rl.l0[mid] - rlo - mid <= i)
        lo = mid + 1;
      else
        hi = mid;
    }
    const int id = rlo + i + lo;
    rl.l1[i] = id < rhi ? id : 0x7FFFFFFF;
    rl.l1x[i] = id < rhi ? dv.slot_of_token(id) : 0;
  }
  __syncthreads();
  mark(6);
  // fill ids increase with i, so the valid ones form a prefix
  int nfill = 0;
  {
    int lo = 0, hi = nfill_req;
    while (lo < hi) {
      const int mid = (lo + hi) >> 1;
      if (rl.l1[mid] != 0x7FFFFFFF)
        lo = mid + 1;
      else
        hi = mid;
    }
    nfill = lo;
  }
  const int drop = lower_bound_i32(rl.l0, nch, sink) +
                   lower_bound_i32(rl.l1, nfill, sink);
  for (int j = tid; j < nch; j += SB) {
    const int v = rl.l0[j];
    if (v >= sink) {
      const int pos = base_out + j + lower_bound_i32(rl.l1, nfill, v) - drop;
      rl.mid[pos] = v;
      rl.mslot[pos] = rl.l0x[j];
    }
  }
  for (int j = tid; j < nfill; j += SB) {
    const int v = rl.l1[j];
    if (v >= sink) {
      const int pos = base_out + j + lower_bound_i32(rl.l0, nch, v) - drop;
      rl.mid[pos] = v;
      rl.mslot[pos] = rl.l1x[j];
    }
  }
  __syncthreads();
  mark(7);
  if (tid == 0) *mid_count = base_out + nch + nfill - drop;
  __syncthreads();
}

// ---------------------------------------------------------------------------
// the selector kernel: L1 tiles, then the tail (candidate pages, L2)
// ---------------------------------------------------------------------------

// A debug output of the parity tests (or the timeline), compiled into the
// DBG instances only: the production instances carry none of the debug
// stores, lists and bitmaps, whose code would otherwise sit between the hot
// blocks (the 128K instance is 77 KB with them, 68 KB without: the
// instruction cache missed on it in every workgroup; 25.4 -> 23.8 us).
#define NFA_DBGP(ptr) (DBG ? (ptr) : nullptr)

// Phase timestamp (debug timeline): every wave of the workgroup has reached
// it (memory accesses in flight stay in flight), then thread 0 keeps the
// wall clock in LDS slot k of the tile (0) or tail (32) marks; NFA_FLUSH
// copies them out at the end of the stage, so no global store of the
// timeline sits inside a measured phase.  Uniform conditions.
#define NFA_MARK(part, k)                                                 \
  do {                                                                    \
    if (NFA_COLD(NFA_DBGP(p.dbg_clock) != nullptr)) {                     \
      lds_barrier();                                                      \
      if (threadIdx.x == 0) s_clk[(part) + (k)] = wall_clock64();         \
    }                                                                     \
  } while (0)
#define NFA_FLUSH(part, slot_base)                                        \
  do {                                                                    \
    if (NFA_COLD(NFA_DBGP(p.dbg_clock) != nullptr)) {                     \
      lds_barrier();                                                      \
      if (threadIdx.x < 32 && s_clk[(part) + threadIdx.x] != 0)           \
        NFA_DBGP(p.dbg_clock)[(slot_base) + threadIdx.x] =                \
            s_clk[(part) + threadIdx.x];                                  \
    }                                                                     \
  } while (0)

// MODE 1 and 2 (MULTI): tiles may span several passes (the host picks it
// when a row can hold more pages than one pass of every tile of a dispatch
// round covers); without it every tile is a single pass and the extra-pass
// loop is absent.  MODE 2 (SURV) adds the survivor lists of rows longer than
// kSurvPages (the host picks it when the block table can hold such rows).
// TOP2: the avg_top2 far method, a separate instance so the extra query
// rows and head scores cost the default instances no registers.  DBG: the
// debug outputs compiled in (the host picks it when any is requested).  Q4:
// the L2 keys' format fixed per production instance, so the bf16 instances
// carry none of the 4-bit code and its registers (at 1M the page-list
// instance spilled two values with both: 45.5 -> 43.3 us without), and the
// L2 side copy assumed (16 ragged 51.9 -> 51.3 us); the debug instances, and
// calls without the side copy, keep both choices at run time.
template <int DSUB, typename KV, int MODE, bool TOP2, bool DBG, int Q4>
__global__ void __launch_bounds__(SB)
    nfa_select_kernel(const NfaSelectParams p, const SelDims sd) {
  // 4-bit L2 keys: fixed by the instance (0 bf16 / fp32 keys, 1 packed 4-bit
  // codes, both read from the L2 side copy), or read from the call (2: the
  // side copy may be off, the L2 dims then read from the K pool)
  const bool l2_quant = Q4 == 2 ? p.l2_quant != 0 : Q4 == 1;
  const bool l2_side = Q4 == 2 ? p.l2_keys_l != nullptr : true;
  // and the production instances (Q4 0, 1) hold only what production calls
  // take: the fp32 running sums of the latest page present, the row's keys
  // in one LDS segment, no fixed near-token quota; the host sends any other
  // call to the instances that read these from the call (Q4 2)
  const bool has_psum = Q4 == 2 ? p.page_sum_l != nullptr : true;
  const bool multi_seg = Q4 == 2 ? sd.nseg > 1 : false;
  const bool near_quota = Q4 == 2 ? p.near_tokens >= 0 : false;
  constexpr bool MULTI = MODE >= 1;
  constexpr bool SURV = MODE == 2;
  warm_kernargs<sizeof(NfaSelectParams) + sizeof(SelDims)>();
  extern __shared__ __align__(16) unsigned char smem[];
  constexpr int CH = Elem<KV>::kChunk;
  constexpr int NC = DSUB / CH;
  constexpr bool STG = (DSUB == 32 || DSUB == 64) && sizeof(KV) == 2;  // stats staged in LDS
  constexpr bool STG2 = STG && DSUB == 32;  // double-buffered over a tile's passes
  int *s_hist = (int *)(smem + sd.a_hist);  // far hi | near hi | far lo | near lo
  int *s_tmp = (int *)(smem + sd.a_tmp);
  int *s_misc = (int *)(smem + sd.a_misc);
  // query rows of the group's heads, each row padded by 16 bytes so that the
  // rows of the heads scored side by side start in different LDS banks
  constexpr int QF = DSUB + 4;      // s_qf, s_qu row stride (floats)
  constexpr int QS = 2 * DSUB + 4;  // s_qs row stride
  float *s_qf = (float *)(smem + sd.a_qf);
  float *s_qs = (float *)(smem + sd.a_qs);
  float *s_qu = (float *)(smem + sd.a_qu);
  // avg_top2 far scores (selector:2412-2427) also need the unrounded query
  constexpr bool top2 = TOP2;
  float *s_qg = (float *)(smem + sd.a_qg);
  int *s_fdims = (int *)(smem + sd.a_fdims);
  int *s_dims = (int *)(smem + sd.a_dims);
  float *s_last = (float *)(smem + sd.a_last);
  int *s_tphys = (int *)(smem + sd.a_tphys);
  float *s_stage = (float *)(smem + sd.a_stage);

  const int tid = threadIdx.x;
  // grid (kv, batch row, tile): workgroup kv + hkv * (b + batch * tile) is
  // number row + rows * tile (row = b * hkv + kv), so the first dispatch
  // round holds the low tiles of every row and a row's tiles share an XCD
  // (workgroups go round-robin over the XCDs)
  // kvq: the selection row's kv head (its query rows, gather row and
  // workspace row); kv: the arena's kv head it reads and writes, 0 for
  // every row when the rows share one arena head (kv_heads_mem 1: the
  // latent rows of an absorbed-MLA cache, one selection row per query head)
  const int kvq = blockIdx.x;
  const int kv = p.kv_heads_mem > 1 ? kvq : 0;
  const int b = blockIdx.y;
  const int tile = blockIdx.z;
  const int row = b * p.hkv + kvq;
  const int G = sd.group;
  const int bs = p.bs;
  const int mb = p.max_blocks;

  const int64_t clk_tile = ((int64_t)row * (sd.clk_tiles + 1) + tile) * 32;
  const int64_t clk_tail = ((int64_t)row * (sd.clk_tiles + 1) + sd.clk_tiles) * 32;
  int64_t *s_clk = (int64_t *)(smem + sd.a_clk);
  if (NFA_COLD(NFA_DBGP(p.dbg_clock) != nullptr) && tid < 64) s_clk[tid] = 0;
  NFA_MARK(0, 0);
  unsigned char *ws = (unsigned char *)p.workspace;
  unsigned int *row_cnt = (unsigned int *)(ws + sd.w_rowcnt);
  int *g_hist = (int *)(ws + sd.w_hist) + (int64_t)row * 512;
  uint16_t *g_keys = (uint16_t *)(ws + sd.w_keys) + (int64_t)row * sd.kstride;

  // ---- first round trip ---------------------------------------------------
  // Wave 0 alone reads the row state through the scalar cache and derives
  // the row's uniform geometry (tile split, pool boundaries), which it hands
  // to the other waves through LDS: uniform integer work executed by every
  // wave would cost each SIMD four times its issue slots.  Meanwhile every
  // wave loads its share of the query rows.
  const int dim_v = p.dims[imin(tid, DSUB - 1)];
  const int fdim_v = p.fine_dims[imin(tid, p.fine_dsub - 1)];
  // the kv group's query rows, whole (the L1 dims are gathered from LDS):
  // the aligned 32-bit word holding each element, one load for either dtype
  // (bf16 rows start at even elements, so the word stays inside the row)
  const int hd = p.head_dim;
  const int nq = G * hd;
  const int qsh = p.q_dtype == NFA_DTYPE_BF16 ? 1 : 2;  // log2 element bytes
  const int64_t qrow = (int64_t)b * p.q_stride_b + (int64_t)kvq * G * p.q_stride_h;
  uint32_t qbits[kQRawPerThread];
  int qodd[kQRawPerThread];
#pragma unroll
  for (int k = 0; k < kQRawPerThread; ++k) {
    const int i = imin(tid + k * SB, nq - 1);
    const int j = div_p2(i, hd, sd.hd_sh);
    const int64_t byte = (qrow + (int64_t)j * p.q_stride_h + (i - j * hd)) << qsh;
    qodd[k] = (int)(byte & 2);
    qbits[k] = *(const uint32_t *)((const unsigned char *)p.q + (byte & ~(int64_t)3));
  }
  int *s_ctx = (int *)(smem + sd.a_ctx);
  if (wave_id() == 0) {
    int32_t L0, slot0;
    int64_t act0, req0;
    sload_row(p.lengths + b, p.active_req + b, p.valid_req + b,
              p.k_new != nullptr ? p.slots + b : p.lengths + b, L0, act0, req0, slot0);
    if (p.k_new == nullptr) slot0 = -1;
    // pages past the block-table width are never scored (selector:205-206)
    const int kt0 = imin(L0 > 0 ? div_p2(L0 + bs - 1, bs, sd.bs_sh) : 0, mb);
    const TileSplit sp = tile_split(kt0, sd.tcap);
    // this tile's pages [t0, t1): the pages spread evenly, the first
    // kt % tiles tiles one page more (at 128K: one tile of 257 pages and 31
    // of 256, four 64-page groups per scoring round, where 257 everywhere
    // took a second round for one page)
    int t0v = 0, t1v = 0;
    if (tile < sp.tiles) {
      const int t_base = kt0 / sp.tiles;
      const int t_rem = kt0 - t_base * sp.tiles;
      t0v = tile * t_base + imin(tile, t_rem);
      t1v = t0v + t_base + (tile < t_rem ? 1 : 0);
    }
    // the pools without skip flags (a superset of the final ones): the
    // first statistics are staged from them before the flags arrive
    const RowGeo g = row_geo(p, sd, L0, false, false);
    if (lane_id() == 0) {
      int4 *c4 = reinterpret_cast<int4 *>(s_ctx);
      c4[0] = make_int4(L0, act0 >= 0 ? 1 : 0, (int)req0, (int)(req0 >> 32));
      c4[1] = make_int4(slot0, sp.tiles, t0v, t1v);
      c4[2] = make_int4(g.kt_eff, g.near_start, g.swa_lo_blk, g.far_end);
      c4[3] = make_int4(g.near_end, g.sink_hi, g.swa_hi, g.orig_far_hi);
      // (word 19: the pages the tiles split, clamped to the block-table
      // width; kt_eff at word 8 stays unclamped for the pool geometry)
      c4[4] = make_int4(g.spl, g.byp_blk,
                        (g.byp_cond ? 1 : 0) | (g.sink_unaligned ? 2 : 0), kt0);
    }
  }
  // LDS: dims, fine dims, raw query rows, histogram
  float *s_qraw = s_stage;  // until the statistics phase
  if (tid < DSUB) s_dims[tid] = dim_v;
  if (tid < p.fine_dsub) s_fdims[tid] = fdim_v;
#pragma unroll
  for (int k = 0; k < kQRawPerThread; ++k) {
    if (tid + k * SB < nq) {
      const uint32_t w = qbits[k];
      s_qraw[tid + k * SB] = qsh == 1 ? __uint_as_float(qodd[k] ? (w & 0xFFFF0000u) : (w << 16))
                                      : __uint_as_float(w);
    }
  }
  if (tid < 512) s_hist[tid] = 0;
  lds_barrier();
  NFA_MARK(0, 1);
  int32_t L, slot_b, t0, t1, kt_tiles;
  int64_t req;
  bool active;
  TileSplit split;
  {
    const int4 *c4 = reinterpret_cast<const int4 *>(s_ctx);
    const int4 a = c4[0], c = c4[1];
    auto u = [](int v) { return __builtin_amdgcn_readfirstlane(v); };
    L = u(a.x);
    active = u(a.y) != 0;
    req = (int64_t)(((uint64_t)(uint32_t)u(a.w) << 32) | (uint32_t)u(a.z));
    slot_b = u(c.x);
    split.tiles = u(c.y);
    t0 = u(c.z);
    t1 = u(c.w);
    kt_tiles = u(c4[4].w);
  }
  // tiles past the row's pages take no part, neither scores nor arrival
  if (tile >= split.tiles) return;
  const int32_t *btr = p.block_table_l + req * mb;
  const int last_blk = L > 0 ? div_p2(L - 1, bs, sd.bs_sh) : -1;
  const bool owns_last = last_blk >= t0 && last_blk < t1;

  // ---- second round trip, issued now and waited for with the first staged
  //      statistics: previous statistics length, skip flags and the physical
  //      page of the decode token.  Vector loads (a lane offset the compiler
  //      cannot prove uniform), so that the LDS accesses below wait for none
  //      of them.
  int vz = 0;
  asm volatile("" : "+v"(vz));
  const int lp_last = owns_last ? imin(div_p2(L - 1, p.page, sd.page_sh), mb - 1) : 0;
  const int prev_v = p.stats_len_l[req + vz];
  const int skf_v = p.skip_far_l[req + vz];
  const int skn_v = p.skip_near_l[req + vz];
  const int phl_v = btr[lp_last + vz];

  // the tile's first statistics, staged by asynchronous copies into LDS
  unsigned char *s_st = smem + sd.a_st;
  if constexpr (STG)
    stage_stats_async<DSUB>(p, ctx_geo(s_ctx, L, true, true), req, kv, t0, pass_end(t0, t1),
                            s_st);

  // scaled, bf16-rounded query rows of this kv group (selector:943-963), and
  // their negative and positive parts
  for (int i = tid; i < G * DSUB; i += SB) {
    const int j = i / DSUB;
    const int d = i % DSUB;
    const float qr = bf16r(s_qraw[j * hd + s_dims[d]] * p.scale);
    s_qf[j * QF + d] = qr;
    s_qs[j * QS + d] = qr < 0.0f ? qr : 0.0f;
    s_qs[j * QS + DSUB + d] = qr > 0.0f ? qr : 0.0f;
    if (top2) s_qu[j * QF + d] = s_qraw[j * hd + s_dims[d]] * p.scale;
  }
  // grouped L2 query (selector:979-1002): bf16 terms summed in head order
  for (int d = tid; d < p.fine_dsub; d += SB) {
    const int dim = s_fdims[d];
    float acc = 0.0f;
    for (int j = 0; j < G; ++j) acc = acc + bf16r(s_qraw[j * hd + dim] * p.scale);
    s_qg[d] = acc;
  }
  if (wave_id() == 0) {
    // the L2 dims as aligned 16-byte runs: their count, or 0 (element loads)
    bool ok = p.fine_dsub % CH == 0;
    for (int d = lane_id(); ok && d < p.fine_dsub; d += 64) {
      const int first = s_fdims[d - d % CH];
      ok = first % CH == 0 && first + CH <= p.head_dim && s_fdims[d] == first + d % CH;
    }
    const bool all = __ballot(!ok) == 0;
    if (lane_id() == 0) s_misc[5] = all ? p.fine_dsub / CH : 0;
  }
  // (the first pass's barrier orders these LDS writes before their reads;
  // the query rows' LDS is reused only after it)
  NFA_MARK(0, 2);

  // ---- request state ------------------------------------------------------
  const bool far_mm = p.far_method == NFA_METHOD_MINMAX;
  const bool near_mm = p.near_method == NFA_METHOD_MINMAX;
  const int32_t prev = __builtin_amdgcn_readfirstlane(prev_v);
  const bool skip_far = __builtin_amdgcn_readfirstlane(skf_v) != 0;
  const bool skip_near = __builtin_amdgcn_readfirstlane(skn_v) != 0;
  if (tid == 0) s_ctx[23] = (skip_far ? 1 : 0) | (skip_near ? 2 : 0);  // for the tail
  // ---- page statistics: latest page, or the whole tile on a rebuild -----
  const bool do_stats = active && L > 0 && !(skip_far && skip_near);
  const bool incremental = prev > 0 && L == prev + 1;
  // The decode token's physical page, and its key row, read from k_new for
  // the statistics when the fused write targets the slot of token L-1.  On
  // an incremental step with running sums only the owner's loads after the
  // first staging wait need them, so the block-table load is waited for
  // there, with the staged statistics, instead of here (the owner tile is
  // its row's last to arrive; its latest block-table entry is often a cache
  // miss)
  int32_t ph_last = 0;
  int last_phys = 0;
  const KV *new_row = nullptr;
  auto resolve_last = [&]() {
    ph_last = owns_last && active ? __builtin_amdgcn_readfirstlane(phl_v) : 0;
    last_phys = safe_page(p, ph_last);
    if (owns_last && active && p.k_new != nullptr && slot_b >= 0 &&
        slot_b / p.page < p.pool_pages && slot_b == ph_last * p.page + (L - 1) % p.page)
      new_row = (const KV *)p.k_new + ((int64_t)b * p.kv_heads_mem + kv) * p.head_dim;
  };
  const bool last_late = do_stats && incremental && has_psum;
  if (!last_late) resolve_last();
  const bool page_phys = (p.page % bs) == 0;
  const KV *kpool = (const KV *)p.k_pool_l;
  // The latest page is never in a pool (it lies in the window:
  // swa_lo_blk <= kt_eff - 1), so the decode token's statistics append, its
  // L2 side row and the decode K/V write complete after the scores, their
  // loads in flight meanwhile; only the recompute path without the fp32
  // running sums stays in front.
  // (rows sharing one arena head leave its writes to selection row 0: the
  // running sums must be continued once, and the rest are the same values)
  const bool writer = kvq < p.kv_heads_mem;
  const bool owner_late =
      do_stats && incremental && owns_last && writer && has_psum;
  if (do_stats && incremental && owns_last && writer && NFA_COLD(!has_psum)) {
    __syncthreads();  // the query preparation has read the raw rows in s_stage
    stats_latest_page<DSUB, KV>(p, req, kv, L, last_blk, last_phys, s_dims, s_stage,
                                new_row, s_last);
  }
  // The owner's decode K/V write, statistics append and L2 side row: loads
  // issued once the first pass's statistics have landed (no staging wait
  // waits for them), stores after that pass's scores.
  // (the decode write falls to the row's last tile when the last page lies
  // past the pages the tiles split: a block-table row of max_blocks pages
  // of `page` tokens can hold more than max_blocks blocks of bs < page
  // tokens, and those have no statistics to append to)
  const bool dw = p.k_new != nullptr && active && writer && last_blk >= t0 &&
                  (last_blk < t1 || t1 >= kt_tiles);
  const bool side_late =
      do_stats && incremental && owns_last && writer && l2_side;
  // (only the waves holding a written element take part: the index
  // arithmetic is uniform, and run by every wave it would cost each SIMD
  // four times its scalar issue slots.  With one lane per page the scores
  // of a pass take the first four to eight waves (64-page groups of up to
  // 448 pages), so the owner's elements go to the last waves, which score
  // nothing; owner lane o = tid - 64 * own_w0; the widest row written
  // decides how many: the last ones (a 576-dim latent row takes nine, from
  // wave 7, which also scores the eighth group of a pass that has one)
  const int own_elems = imax(imax(p.head_dim, p.head_dim_v), imax(DSUB, p.fine_dsub));
  const int own_w0 = STG && !TOP2 ? imax(SW - (own_elems + 63) / 64, 0) : 0;
  const int otid = tid - 64 * own_w0;
  const bool owner_any = (dw || owner_late || side_late) && wave_id() >= own_w0 &&
                         (wave_id() - own_w0) * 64 < own_elems;
  KV dw_k = 0, dw_v = 0, side_raw = 0;
  float ap_mn = __uint_as_float(0x7F800000u);  // a new page starts from +inf,
  float ap_mx = __uint_as_float(0xFF800000u);  // -inf and 0
  float ap_sm = 0.0f, ap_x = 0.0f;
  auto owner_finish = [&]() {
    if (dw && slot_b >= 0 && slot_b / p.page < p.pool_pages) {
      // decode write of the current token (selector:1030-1061)
      const int phys = slot_b / p.page;
      const int off = slot_b % p.page;
      if (otid < p.head_dim) store_coherent(&((KV *)p.k_pool_l)[kv_offset(p, phys, kv, off) + otid], dw_k);
      if (otid < p.head_dim_v && p.v_new != nullptr)
        ((KV *)p.v_pool_l)[(((int64_t)phys * p.kv_heads_mem + kv) * p.page + off) *
                               p.head_dim_v + otid] = dw_v;
    }
    if (owner_late && otid < DSUB) {
      // the token's dims continue the page's min / max exactly and the fp32
      // running sum sequentially (selector:32-131)
      const int64_t si = stat_index<KV>(p, req, kv, otid, last_blk, DSUB);
      const float x = ap_x;
      const float mn = (x < ap_mn) ? x : ap_mn;
      const float mx = (x > ap_mx) ? x : ap_mx;
      const float sm = ap_sm + x;
      ((KV *)p.stat_min_l)[si] = (KV)Elem<KV>::from_f32(mn);
      ((KV *)p.stat_max_l)[si] = (KV)Elem<KV>::from_f32(mx);
      ((KV *)p.stat_sum_l)[si] = page_mean<KV>(sm, p.bs);
      p.page_sum_l[(req * p.kv_heads_mem + kv) * DSUB + otid] = sm;
    }
    if (side_late && otid < p.fine_dsub) {
      // the new token's L2 side row (its 4-bit codes: lanes 0-31 of wave 0)
      if (l2_quant) {
        q4_store_lanes(p, req, kv, L - 1, Elem<KV>::load(&side_raw), otid);
      } else {
        store_coherent(&((KV *)p.l2_keys_l)[l2_side_index<KV>(p, req, kv, L - 1, otid)], side_raw);
      }
    }
  };
  auto owner_prefetch = [&]() {
    if (last_late) resolve_last();
    if (dw) {
      const int64_t nb = (int64_t)b * p.kv_heads_mem + kv;
      if (otid < p.head_dim) dw_k = ((const KV *)p.k_new)[nb * p.head_dim + otid];
      if (otid < p.head_dim_v && p.v_new != nullptr)
        dw_v = ((const KV *)p.v_new)[nb * p.head_dim_v + otid];
    }
    const KV *trow = new_row != nullptr
                         ? new_row
                         : kpool + kv_offset(p, last_phys, kv, (L - 1) % p.page);
    if (owner_late && otid < DSUB) {
      if ((L - 1) % bs != 0) {
        const int64_t si = stat_index<KV>(p, req, kv, otid, last_blk, DSUB);
        ap_mn = Elem<KV>::load((const KV *)p.stat_min_l + si);
        ap_mx = Elem<KV>::load((const KV *)p.stat_max_l + si);
        ap_sm = p.page_sum_l[(req * p.kv_heads_mem + kv) * DSUB + otid];
      }
      ap_x = Elem<KV>::load(trow + s_dims[otid]);
    }
    if (side_late && otid < p.fine_dsub) side_raw = trow[s_fdims[otid]];
  };
  const RowGeo geo = ctx_geo(s_ctx, L, !skip_far, !skip_near);
  float *s_hs = (float *)(smem + sd.a_hs);  // [head][page] bf16 head scores
  uint16_t *s_tkeys = (uint16_t *)(smem + sd.a_tkeys);  // the tile's keys
  const int lpp_log = G <= 1 ? 0 : G <= 2 ? 1 : G <= 4 ? 2 : 3;
  const int lpp = 1 << lpp_log;  // lanes per page
  const int ppw = 64 >> lpp_log;  // pages per wave and round
  // one pass scores and publishes pages [c0, c1) from the statistics staged
  // in st; the histogram accumulates in LDS over the passes of the tile.
  // The next pass's statistics, pages [n0, n1), are copied into nst while
  // this pass is scored (not on a rebuild, which restages each pass after
  // recomputing it)
  // `first` (std::true_type for the tile's first pass only) compiles the
  // owner's work into that pass alone
  auto run_pass = [&](auto first, int c0, int c1, unsigned char *st, int n0, int n1,
                      unsigned char *nst) {
    constexpr bool kFirst = decltype(first)::value;
    NFA_MARK(0, 7);
    if (NFA_COLD(do_stats && !incremental)) {
      __syncthreads();  // the query preparation has read the raw rows in s_stage
      float *psum_row = has_psum
                            ? p.page_sum_l + (req * p.kv_heads_mem + kv) * DSUB
                            : nullptr;
      int *s_coff = (int *)s_stage;  // DSUB / CH chunk offsets
      if (tid == 0) {
        bool vec = true;
        for (int c = 0; vec && c < NC; ++c) {
          const int first = s_dims[c * CH];
          vec = (first % CH) == 0;
          for (int e = 1; vec && e < CH; ++e) vec = s_dims[c * CH + e] == first + e;
          s_coff[c] = first;
        }
        s_misc[1] = vec;
      }
      if (page_phys) {
        for (int i = tid; i < c1 - c0; i += SB) {
          const int lp = imin(((c0 + i) * bs) / p.page, mb - 1);
          s_tphys[i] = safe_page(p, btr[lp]);
        }
      }
      __syncthreads();
      if (s_misc[1]) {
        compute_stats_vec<DSUB, KV>(p, req, kv, L, c0, c1, s_coff,
                                    page_phys ? s_tphys : nullptr, new_row, L - 1,
                                    psum_row, last_blk);
      } else {
        __syncthreads();
        compute_stats<DSUB, KV>(p, req, kv, L, c0, c1, s_stage, s_dims,
                                page_phys ? s_tphys : nullptr, new_row, L - 1,
                                psum_row, last_blk);
      }
      if (l2_side) {
        // L2 side rows of the tile's tokens
        const int tlo = c0 * bs;
        const int thi = imin(c1 * bs, L);
        const int nchv = s_misc[5];  // 16-byte runs of the L2 dims, 0: elements
        auto src_row = [&](int tok) -> const KV * {
          if (new_row != nullptr && tok == L - 1) return new_row;
          const int phys = page_phys ? s_tphys[tok / bs - c0]
                                     : safe_page(p, btr[imin(tok / p.page, mb - 1)]);
          return kpool + kv_offset(p, phys, kv, tok % p.page);
        };
        if (l2_quant) {
          // one thread per token: gather, quantise, store
          for (int tok = tlo + tid; tok < thi; tok += SB)
            q4_store<KV>(p, req, kv, tok, src_row(tok), s_fdims);
        } else if (nchv > 0) {
          for (int e = tid; e < (thi - tlo) * nchv; e += SB) {
            const int tok = tlo + e / nchv;
            const int c = e % nchv;
            *reinterpret_cast<uint4 *>((KV *)p.l2_keys_l +
                                       l2_side_index<KV>(p, req, kv, tok, c * CH)) =
                *reinterpret_cast<const uint4 *>(src_row(tok) + s_fdims[c * CH]);
          }
        } else {
          for (int e = tid; e < (thi - tlo) * p.fine_dsub; e += SB) {
            const int tok = tlo + e / p.fine_dsub;
            const int d = e % p.fine_dsub;
            ((KV *)p.l2_keys_l)[l2_side_index<KV>(p, req, kv, tok, d)] =
                src_row(tok)[s_fdims[d]];
          }
        }
      }
      // rebuilt statistics: complete the stores, drop cached lines, read back
      __threadfence();
      __syncthreads();
      __threadfence();
      if constexpr (STG) {
        __builtin_amdgcn_s_waitcnt(0);  // the speculative loads have landed
        // recomputed addresses: nothing of the first issue stays live across
        // the rebuild
        int t0r = c0;
        asm volatile("" : "+s"(t0r));
        stage_stats_async<DSUB>(p, geo, req, kv, t0r, c1, st);
      }
    }
    if constexpr (STG && MULTI && !STG2) {
      // one buffer: a later pass stages its own statistics now (the pass
      // before has finished reading them)
      if (!kFirst && !(do_stats && !incremental))
        stage_stats_async<DSUB>(p, geo, req, kv, c0, c1, st);
    }
    if constexpr (STG) {
      __builtin_amdgcn_s_waitcnt(0);  // this wave's staged statistics
      __syncthreads();
    }
    lds_barrier();
    NFA_MARK(0, 3);
    if (kFirst && owner_any) owner_prefetch();
    if constexpr (STG2 && MULTI) {
      // every wave has finished the previous pass, which read nst; with one
      // lane per page the copies come from waves 8-15, which score nothing
      constexpr int w0 = TOP2 ? 0 : 8;
      if (n0 < n1 && !(do_stats && !incremental))
        stage_stats_async<DSUB>(p, geo, req, kv, n0, n1, nst, w0, SW - w0);
    }

    // ---- L1 scores, group means, keys and high-byte histograms -----------
    // a page's group key: published, counted in the tile's histograms (a
    // page belongs to at most one pool: far pages lie below near_start,
    // near pages at or above it).  Multi-pass tiles keep their keys in LDS
    // and write them out after the last pass: a store issued in a pass
    // would be waited for by the next pass's staging wait (vmcnt counts
    // stores), its full write-through latency on every pass.
    auto publish = [&](int t, uint16_t far_bits, uint16_t near_bits) {
      if (NFA_COLD(NFA_DBGP(p.dbg_far) != nullptr)) {
        NFA_DBGP(p.dbg_far)[(int64_t)row * mb + t] = far_bits;
        NFA_DBGP(p.dbg_near)[(int64_t)row * mb + t] = near_bits;
      }
      const uint32_t fk = score_key(far_bits);
      const uint32_t nk = score_key(near_bits);
      if constexpr (MULTI)
        s_tkeys[t - t0] = (uint16_t)(fk ? fk : nk);
      else
        store_coherent(&g_keys[t], (uint16_t)(fk ? fk : nk));
      if (fk) atomicAdd(&s_hist[fk >> 8], 1);
      if (nk) atomicAdd(&s_hist[256 + (nk >> 8)], 1);
    };
    if constexpr (STG && !TOP2) {
      const bool g_pow2 = (G & (G - 1)) == 0;
      const float g_inv = 1.0f / (float)G;
      // One lane per page, 64 pages per wave and round: the lane reads and
      // unpacks its page's statistics once and scores the G heads in order
      // against query rows read as LDS broadcasts, so a page costs one
      // unpack, one pool test and one key instead of one per head lane.
      // The 64-page groups never straddle near_start ([c0, ns) grouped from
      // c0, [ns, c1) from ns), so no wave runs both pools' arithmetic one
      // after the other; the up to 448 pages of a pass take seven or eight
      // waves.
      const int ns = imin(imax(geo.near_start, c0), c1);
      const int nfg = (ns - c0 + 63) >> 6;
      const int ngr = nfg + ((c1 - ns + 63) >> 6);
      for (int gi = wave_id(); gi < ngr; gi += SW) {
        const int ce = gi < nfg ? ns : c1;
        const int t = (gi < nfg ? c0 + gi * 64 : ns + (gi - nfg) * 64) + lane_id();
        const int lp = t - c0;
        bool fp = false, np = false;
        if (do_stats && t < ce) pools(p, geo, t, &fp, &np);
        uint16_t far_bits = kNegInfBits, near_bits = kNegInfBits;
        if (fp || np) {
          const bool need_mm = (fp && far_mm) || (np && near_mm);
          const uint4 *su = reinterpret_cast<const uint4 *>(st) + lp;
          const float acc = l1_group_staged<QF, QS, DSUB>(su, s_qs, s_qf, G, need_mm);
          // bf16 head scores summed in head order, then the group mean (a
          // power-of-two group: the multiply by 1 / G is the same correctly
          // rounded quotient)
          const float m = g_pow2 ? acc * g_inv : acc / (float)G;
          const uint16_t mean = bf16_bits(m);
          if (fp) far_bits = mean;
          if (np) near_bits = mean;
        }
        if (t < ce) publish(t, far_bits, near_bits);
      }
    } else {
    // lpp lanes per page (one per query head of the group, padded to a
    // power of two), 64 / lpp pages per wave and round: each lane scores one
    // head of its page into s_hs, then the page's first lane combines the
    // page's head scores (written by lanes of the same wave, so in order
    // without a barrier), publishes the key and counts it in the histogram.
    // Every page of the pass gets a key (0 for pages in no pool).
    for (int base = wave_id() * ppw; base < c1 - c0; base += SW * ppw) {
      const int lp = base + (lane_id() >> lpp_log);
      const int j = lane_id() & (lpp - 1);
      const int t = c0 + lp;
      bool fp = false, np = false;
      if (do_stats && t < c1) pools(p, geo, t, &fp, &np);
      const bool need_mm = (fp && far_mm) || (np && near_mm);
      if ((fp || np) && j < G) {
        const bool need_avg = !need_mm;
        // avg_top2 far pages: the head mean against the rounded and the
        // unrounded query, packed as two bf16 patterns in the head's slot
        const bool pair = top2 && fp;
        const float *qu = pair ? s_qu + j * QF : nullptr;
        float h, u = 0.0f;
        if constexpr (STG) {
          const uint4 *su = reinterpret_cast<const uint4 *>(st) + lp;
          h = l1_head_staged<DSUB>(su, s_qs + j * QS, s_qf + j * QF, qu, need_mm, &u);
        } else {
          const bool from_lds = incremental && t == last_blk;
          float m = 0.0f, a = 0.0f;
          l1_head_mem<DSUB, KV>(p, req, kv, t, s_qf + j * QF, qu, need_mm, need_avg,
                                from_lds ? s_last : nullptr, &m, &a, &u);
          h = need_mm ? m : a;
        }
        if (pair) h = __uint_as_float(((uint32_t)bf16_bits(h) << 16) | bf16_bits(u));
        s_hs[j * kSpanMax + lp] = h;
      }
      if (j == 0 && t < c1) {
        uint16_t far_bits = kNegInfBits, near_bits = kNegInfBits;
        if (NFA_COLD(top2 && fp)) {
          far_bits = top2_far_score(s_hs + lp, G);
        } else if (fp || np) {
          // bf16 head scores summed in head order
          float acc = 0.0f;
          for (int jj = 0; jj < G; ++jj) acc = acc + s_hs[jj * kSpanMax + lp];
          const uint16_t mean = bf16_bits(acc / (float)G);
          if (fp) far_bits = mean;
          if (np) near_bits = mean;
        }
        publish(t, far_bits, near_bits);
      }
    }
    }
    // the owner's decode write, statistics append and L2 side row, once:
    // the loaded values are dead before any further pass
    if (kFirst && owner_any) owner_finish();
    lds_barrier();
    NFA_MARK(0, 5);
    NFA_MARK(0, 6);
    if (NFA_COLD(NFA_DBGP(p.dbg_clock) != nullptr) && tid == 0) {
      // per-pass durations summed over the passes: staging wait, scores, keys
      s_clk[8] += s_clk[3] - s_clk[7];
      s_clk[9] += s_clk[5] - s_clk[3];
      s_clk[10] += s_clk[6] - s_clk[5];
    }
  };
  {
    unsigned char *st = s_st;
    unsigned char *nst = STG2 ? smem + sd.a_st2 : s_st;
    int c1 = pass_end(t0, t1);
    run_pass(std::true_type{}, t0, c1, st, c1, c1 < t1 ? pass_end(c1, t1) : c1, nst);
    if constexpr (MULTI) {
      // long rows and many rows: further passes instead of dispatch rounds,
      // the staging buffers alternating
      for (int c0 = c1; c0 < t1; c0 = c1) {
        c1 = pass_end(c0, t1);
        unsigned char *tmp = st;
        st = nst;
        nst = tmp;
        run_pass(std::false_type{}, c0, c1, st, c1, c1 < t1 ? pass_end(c1, t1) : c1, nst);
      }
      // the tile's keys out to the workspace for the row's tail (the last
      // pass's barrier ordered every key's LDS write before these reads)
      for (int i = tid; i < t1 - t0; i += SB) store_coherent(&g_keys[t0 + i], s_tkeys[i]);
    }
  }
  // ---- survivors: a key below the tile's own K-th largest key (of its
  //      pool) has K keys of the tile above it, so it is not among the row's
  //      top K; the tile lists its other pages and keys, in page order, from
  //      its first page on, for the tail to read instead of every key of the
  //      row.  The tile's K-th key: the coarse bin from the tile histogram,
  //      then the low bytes of the tile's keys in that bin.
  if (SURV && kt_tiles > kSurvPages) {
    if (wave_id() == 0) wave_threshold_bin(s_hist, p.k_f, s_tmp + 40);
    if (wave_id() == 1) wave_threshold_bin(s_hist + 256, p.k_n, s_tmp + 44);
    int *s_lo = (int *)(smem + sd.a_stage);  // low-byte histograms (far | near)
    if (tid < 512) s_lo[tid] = 0;
    lds_barrier();
    NFA_MARK(0, 11);
    const int hb_f = s_tmp[40], hb_n = s_tmp[44];
    const int npg = t1 - t0;
    const int ppt = (npg + SB - 1) / SB;
    const int pa = imin(tid * ppt, npg);
    const int pb = imin(pa + ppt, npg);
    // keys >= thr survive: every valid key when the pool's keys all fit K
    int thr_f = 1, thr_n = 1;
    if (hb_f >= 0 || hb_n >= 0) {
      for (int i = pa; i < pb; ++i) {
        const uint32_t key = s_tkeys[i];
        const bool near = t0 + i >= geo.near_start;
        if (key != 0u && (int)(key >> 8) == (near ? hb_n : hb_f))
          atomicAdd(&s_lo[(near ? 256 : 0) + (key & 255u)], 1);
      }
      lds_barrier();
      NFA_MARK(0, 12);
      if (wave_id() == 0 && hb_f >= 0)
        wave_threshold_bin(s_lo, p.k_f - s_tmp[41], s_tmp + 48, true);
      if (wave_id() == 1 && hb_n >= 0)
        wave_threshold_bin(s_lo + 256, p.k_n - s_tmp[45], s_tmp + 52, true);
      lds_barrier();
      // (a fine bin of -1: the whole coarse bin is taken, down to its
      // lowest key)
      if (hb_f >= 0) thr_f = (hb_f << 8) | imax(s_tmp[48], 0);
      if (hb_n >= 0) thr_n = (hb_n << 8) | imax(s_tmp[52], 0);
    }
    auto survives = [&](int i, uint32_t key) {
      return key != 0u && (int)key >= (t0 + i >= geo.near_start ? thr_n : thr_f);
    };
    int c = 0;
    for (int i = pa; i < pb; ++i) c += survives(i, s_tkeys[i]) ? 1 : 0;
    NFA_MARK(0, 13);
    int total;
    int pos = block_scan_exclusive<SW>(c, s_tmp, &total);
    NFA_MARK(0, 14);
    int *sv_page = (int *)(ws + sd.w_surv) + (int64_t)row * 2 * sd.kstride + t0;
    uint32_t *sv_key = (uint32_t *)(sv_page + sd.kstride);
    for (int i = pa; i < pb; ++i) {
      const uint32_t key = s_tkeys[i];
      if (survives(i, key)) {
        store_coherent(&sv_page[pos], t0 + i);
        store_coherent(&sv_key[pos], key);
        ++pos;
      }
    }
    if (tid == 0) store_coherent(&((int *)(ws + sd.w_scount))[(int64_t)row * sd.ntiles + tile], total);
    NFA_MARK(0, 15);
  }
  if (tid < 256) {
    const int hf = s_hist[tid];
    const int hn = s_hist[256 + tid];
    if (hf) atomicAdd(&g_hist[tid], hf);
    if (hn) atomicAdd(&g_hist[256 + tid], hn);
  }
  NFA_MARK(0, 4);
  NFA_FLUSH(0, clk_tile);

  // ---- arrival; the last workgroup of the row runs the tail --------------
  // What the tail reads of this workgroup's writes -- keys, page lists, the
  // decode token's K row and L2 side row -- went out through coherent
  // stores and the histogram through atomics; only a rebuild's side rows
  // and statistics are plain stores that need the L2 writeback.
  NFA_MARK(32, 27);
  if (!arrive_last(&row_cnt[row * kArriveStride], (unsigned int)split.tiles, &s_misc[0],
                   do_stats && !incremental))
    return;

  // =========================== tail ======================================
  // The tail re-derives its state: the kernel arguments read again through
  // a pointer the compiler cannot fold into the tile stage's copies, the row
  // state from what wave 0 left in LDS.  Nothing of the tile stage stays live
  // across the arrival (scalar registers are the scarce resource of this
  // kernel: every value held across it is spilled and reloaded in the tail).
  {
  typedef __attribute__((address_space(4))) const NfaSelectParams ParamsK;
  typedef __attribute__((address_space(4))) const SelDims DimsK;
  ParamsK *pk = (ParamsK *)__builtin_amdgcn_kernarg_segment_ptr();
  asm volatile("" : "+s"(pk));
  constexpr size_t kSdOff =
      (sizeof(NfaSelectParams) + alignof(SelDims) - 1) / alignof(SelDims) * alignof(SelDims);
  DimsK *dk = (DimsK *)((__attribute__((address_space(4))) const char *)pk + kSdOff);
  // generic pointers cast from the hidden constant-space ones: after
  // inlining, the loads are scalar loads from the kernel argument segment
  const NfaSelectParams &p = *(const NfaSelectParams *)pk;
  const SelDims &sd = *(const SelDims *)dk;
  const int tid = threadIdx.x;
  const int kvq = blockIdx.x;  // selection row, as in the tile stage
  const int kv = p.kv_heads_mem > 1 ? kvq : 0;  // the arena's kv head
  const int b = blockIdx.y;
  const int row = b * p.hkv + kvq;
  const int bs = p.bs;
  const int mb = p.max_blocks;
  const int *s_ctx = (const int *)(smem + sd.a_ctx);
  const int L = __builtin_amdgcn_readfirstlane(s_ctx[0]);
  const int64_t req = (int64_t)(((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane(s_ctx[3]) << 32) |
                                (uint32_t)__builtin_amdgcn_readfirstlane(s_ctx[2]));
  // the pages the tiles split and keyed: ceil(L / bs) clamped to the
  // block-table width (pages past it are never scored, selector:205-206);
  // the survivor offsets and the key scans cover exactly these
  const int kt_tiles = __builtin_amdgcn_readfirstlane(s_ctx[19]);
  const int skf = __builtin_amdgcn_readfirstlane(s_ctx[23]);
  const bool skip_far = (skf & 1) != 0;
  const bool skip_near = (skf & 2) != 0;
  const RowGeo geo = ctx_geo(s_ctx, L, !skip_far, !skip_near);
  const int32_t *btr = p.block_table_l + req * mb;
  const bool page_phys = (p.page % bs) == 0;
  const KV *kpool = (const KV *)p.k_pool_l;
  unsigned char *ws = (unsigned char *)p.workspace;
  // Every workgroup of the request has read its statistics length once the
  // tails of all its kv rows have started; the last of them records the new
  // length (the counter's answer is read after the key staging below waited
  // for every load anyway).
  unsigned int *req_cnt = (unsigned int *)(ws + sd.w_reqcnt);
  // (through a lane offset the compiler cannot prove uniform: a uniform
  // address lets the atomic optimizer rewrite the ticket into a wave
  // reduction that waits for the answer on the spot)
  unsigned int req_rank = 0u;
  int t_vz = 0;
  asm volatile("" : "+v"(t_vz));
  if (tid == 0)
    req_rank = __hip_atomic_fetch_add(&req_cnt[b + t_vz], 1u, __ATOMIC_RELAXED,
                                      __HIP_MEMORY_SCOPE_AGENT);
  int *g_hist = (int *)(ws + sd.w_hist) + (int64_t)row * 512;
  uint16_t *g_keys = (uint16_t *)(ws + sd.w_keys) + (int64_t)row * sd.kstride;
  int *s_hist = (int *)(smem + sd.a_hist);
  int *s_tmp = (int *)(smem + sd.a_tmp);
  int *s_misc = (int *)(smem + sd.a_misc);
  float *s_qg = (float *)(smem + sd.a_qg);
  int *s_fdims = (int *)(smem + sd.a_fdims);
  int64_t *s_clk = (int64_t *)(smem + sd.a_clk);
  const int64_t clk_tail = ((int64_t)row * (sd.clk_tiles + 1) + sd.clk_tiles) * 32;
  // (its LDS overlaps the tile stage's private part, no longer used)
  uint16_t *s_keys = (uint16_t *)(smem + sd.a_keys);
  const bool dbg = NFA_DBGP(p.dbg_i_f) != nullptr;
  uint32_t *s_dbf = (uint32_t *)(smem + sd.a_dbf);
  uint32_t *s_dbn = (uint32_t *)(smem + sd.a_dbn);
  uint64_t *s_dsel = (uint64_t *)(smem + sd.a_dsel);
  NFA_MARK(32, 0);

  const L2Bounds lb = l2_bounds(p, L, skip_far, skip_near, p.geo_near);
  if (NFA_COLD(NFA_DBGP(p.dbg_bounds) != nullptr) && kvq == 0 && tid == 0) {
    NFA_DBGP(p.dbg_bounds)[b * 3 + 0] = lb.lower;
    NFA_DBGP(p.dbg_bounds)[b * 3 + 1] = lb.upper;
    NFA_DBGP(p.dbg_bounds)[b * 3 + 2] = lb.quota;
  }
  // candidate tokens lie in [tok_lo, tok_hi) and exist only when quota > 0;
  // below S_cap = max_blocks * bs too (selector:1167-1184): a bypass page
  // past it (a block-table row of bs < page holds more blocks than that)
  // is no candidate
  const int tok_lo = imax(p.sink_tokens, lb.lower);
  const int tok_hi = imin(imin(imin(lb.lo, L), lb.upper), mb * bs);
  const bool any_cand = lb.quota > 0 && tok_hi > tok_lo;
  const int near_start = geo.near_start;

  // row histograms into LDS, reset for the next launch: wave 0 takes the
  // far pool's 256 bins and wave 1 the near pool's (four a lane, as their
  // threshold scans read them), so each can find its coarse threshold bin
  // while the other waves copy the keys
  if (wave_id() < 2) {
    const int base = wave_id() * 256 + 4 * lane_id();
    int h[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) h[k] = atomicExch(&g_hist[base + k], 0);
#pragma unroll
    for (int k = 0; k < 4; ++k) s_hist[base + k] = h[k];
  } else if (tid < 128 + 512) {
    s_hist[512 + (tid - 128)] = 0;
  }
  if (NFA_COLD(dbg)) {
    for (int w = tid; w < sd.words; w += SB) {
      s_dbf[w] = 0u;
      s_dbn[w] = 0u;
    }
  }
  if (tid == 0) {
    s_misc[3] = 0;  // debug selection list lengths (far, near)
    s_misc[4] = 0;
  }
  // The row's survivors (every tile listed them at its first page, in page
  // order) are read instead of every key when the row has at most 64 tiles
  // and they fit the LDS; their counts come first.
  const int ntile = __builtin_amdgcn_readfirstlane(s_ctx[5]);
  int *s_spre = s_tmp + 64;  // survivors of the tiles before tile t
  const bool surv_on = SURV && kt_tiles > kSurvPages;
  if (surv_on && wave_id() == 0) {
    const int lane = lane_id();
    const int cnt = lane < ntile && ntile <= 64
                        ? ((const int *)(ws + sd.w_scount))[(int64_t)row * sd.ntiles + lane]
                        : 0;
    const int inc = wave_incl_sum(cnt);
    s_spre[lane] = inc - cnt;
    if (lane == 63) s_misc[8] = inc;
  }
  if (surv_on) lds_barrier();
  const int n_surv = surv_on ? __builtin_amdgcn_readfirstlane(s_misc[8]) : 0;
  const bool surv_path = surv_on && ntile <= 64 && n_surv <= sd.sc;
  int *s_spage = (int *)(smem + sd.a_keys);               // survivors' pages
  uint32_t *s_skey = (uint32_t *)(s_spage + sd.sc);       // and keys
  if (surv_path) {
    // each tile's list in runs of 64 entries, copied straight into LDS
    const int t_base = kt_tiles / ntile;
    const int t_rem = kt_tiles - t_base * ntile;
    const int *sv_page = (const int *)(ws + sd.w_surv) + (int64_t)row * 2 * sd.kstride;
    const uint32_t *sv_key = (const uint32_t *)(sv_page + sd.kstride);
    for (int t = wave_id(); t < ntile; t += SW) {
      const int tt0 = t * t_base + imin(t, t_rem);
      const int pre = s_spre[t];
      const int cnt = (t + 1 < ntile ? s_spre[t + 1] : n_surv) - pre;
      for (int e0 = 0; e0 < cnt; e0 += 64) {
        if (e0 + lane_id() < cnt) {
          lds_dma4(sv_page + tt0 + e0 + lane_id(), lds_addr(s_spage + pre + e0));
          lds_dma4(sv_key + tt0 + e0 + lane_id(), lds_addr(s_skey + pre + e0));
        }
      }
    }
  } else if (!multi_seg) {
    stage_keys(g_keys, 0, sd.seg, s_keys, 2);
  }
  // coarse threshold bins: wave 0 the far pool, wave 1 the near pool
  if (wave_id() == 0) wave_threshold_bin(s_hist, p.k_f, s_tmp + 8);
  if (wave_id() == 1) wave_threshold_bin(s_hist + 256, p.k_n, s_tmp + 12);
  dma_barrier();
  if (tid == 0 && req_rank == (unsigned int)(p.hkv - 1)) {
    const bool active = __builtin_amdgcn_readfirstlane(s_ctx[1]) != 0;
    if (active && L > 0 && !(skip_far && skip_near)) p.stats_len_l[req] = L;
    __hip_atomic_store(&req_cnt[b], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  NFA_MARK(32, 24);
  NFA_MARK(32, 25);
  const int hbf = s_tmp[8], hbn = s_tmp[12];
  if ((hbf >= 0 || hbn >= 0) && surv_path) {
    // refinement over the survivors (every key of a threshold bin is one)
    for (int i = tid; i < n_surv; i += SB) {
      const uint32_t k = s_skey[i];
      const bool near = s_spage[i] >= near_start;
      if ((int)(k >> 8) == (near ? hbn : hbf))
        atomicAdd(&s_hist[(near ? 768 : 512) + (k & 255u)], 1);
    }
  }
  if ((hbf >= 0 || hbn >= 0) && !surv_path) {
    // refinement: low-byte histograms of the keys in the threshold bins
    for (int sg = 0; sg < sd.nseg; ++sg) {
      const int seg_base = sg * sd.seg;
      if (NFA_COLD(multi_seg)) {
        __syncthreads();
        stage_keys(g_keys, seg_base, sd.seg, s_keys);
        dma_barrier();
      }
      const int n = imin(sd.seg, kt_tiles - seg_base);
      // sixteen keys per thread from two 16-byte reads (the segment holds a
      // multiple of 16 keys): one round of the block up to 16384 pages
      for (int v = tid; v < (n + 15) / 16; v += SB) {
        const uint4 wa = reinterpret_cast<const uint4 *>(s_keys)[2 * v];
        const uint4 wb = reinterpret_cast<const uint4 *>(s_keys)[2 * v + 1];
        const uint32_t ws[8] = {wa.x, wa.y, wa.z, wa.w, wb.x, wb.y, wb.z, wb.w};
#pragma unroll
        for (int j = 0; j < 16; ++j) {
          const uint32_t k = (ws[j >> 1] >> (16 * (j & 1))) & 0xFFFFu;
          const int i = v * 16 + j;
          const bool near = seg_base + i >= near_start;
          const int hb = near ? hbn : hbf;
          if (i < n && k != 0u && (int)(k >> 8) == hb)
            atomicAdd(&s_hist[(near ? 768 : 512) + (k & 255u)], 1);
        }
      }
    }
  }
  if (hbf >= 0 || hbn >= 0) {
    __syncthreads();
    NFA_MARK(32, 26);
    if (wave_id() == 0 && hbf >= 0)
      wave_threshold_bin(s_hist + 512, p.k_f - s_tmp[9], s_tmp + 16, true);
    if (wave_id() == 1 && hbn >= 0)
      wave_threshold_bin(s_hist + 768, p.k_n - s_tmp[13], s_tmp + 20, true);
    __syncthreads();
  }
  const PoolThr tf = pool_threshold(p.k_f, s_tmp + 8, s_tmp + 16, s_hist + 512);
  const PoolThr tn = pool_threshold(p.k_n, s_tmp + 12, s_tmp + 20, s_hist + 768);
  NFA_MARK(32, 1);

  // ---- selected pages -> sorted candidate page list ----------------------
  // L1 selection of the debug outputs: per-pool lists and page bitmaps
  auto dbg_select = [&](int page, uint32_t k, bool near) {
    const int pos = atomicAdd(&s_misc[near ? 4 : 3], 1);
    s_dsel[(near ? p.k_f : 0) + pos] = ((uint64_t)k << 32) | (uint32_t)page;
    atomicOr(near ? &s_dbn[page >> 5] : &s_dbf[page >> 5], 1u << (page & 31));
  };
  auto in_cand = [&](int page) {
    return any_cand && page * bs < tok_hi && page * bs + bs > tok_lo;
  };
  // the same as a page range [cp_lo, cp_hi) (tok_lo >= 0)
  const int cp_lo = any_cand ? tok_lo / bs : 0;
  const int cp_hi = any_cand ? (tok_hi + bs - 1) / bs : 0;
  // sink and SWA bypass pages (selector:1195-1251)
  int bp0 = -1, bp1 = -1;
  {
    const int spl = p.sink_tokens / bs;
    const bool byp0_keep = (p.sink_tokens % bs) != 0;
    bool byp1_keep = (lb.lo % bs != 0) && (lb.lo / bs >= spl);
    if (p.sink_tokens % bs != 0) byp1_keep = byp1_keep && (lb.lo / bs != spl);
    if (byp0_keep && in_cand(spl)) bp0 = spl;
    if (byp1_keep && in_cand(lb.lo / bs)) bp1 = lb.lo / bs;
  }
  // Sixteen pages per thread, in page order over the threads (one round of
  // the block for up to 16384 pages): keys above the
  // threshold are selected, keys equal to it too unless only some of them
  // are (then the first `need` tied pages of the pool in page order, ranked
  // by a block scan); a second scan places the candidates, so the list is
  // sorted and free of duplicates by construction.
  int *s_pages = (int *)(smem + sd.a_pages);
  // bit j set for pages pg0 + j in [lo, hi), j < 16
  auto range16 = [](int pg0, int lo, int hi) -> uint32_t {
    const int a = imin(imax(lo - pg0, 0), 16);
    const int b = imin(imax(hi - pg0, 0), 16);
    return ((1u << b) - 1u) & ~((1u << a) - 1u);
  };
  int np_u = 0;          // candidates so far (uniform)
  int tfb = 0, tnb = 0;  // tied far / near pages so far (uniform)
  if (surv_path) {
    // The survivors in page order, a contiguous run per thread: the tied
    // keys ranked by a first scan, candidate positions by a second, the
    // bypass pages (in no pool, so never survivors unless the two
    // geometries disagree) placed among them.
    const int per = (n_surv + SB - 1) / SB;  // <= 32
    const int ia = imin(tid * per, n_surv);
    const int ib = imin(ia + per, n_surv);
    const bool all_f = tf.need == (1 << 30);
    const bool all_n = tn.need == (1 << 30);
    int rf = 0, rn = 0;
    if (tie_cut(tf) || tie_cut(tn)) {
      int c2[2] = {0, 0}, tot2[2];
      for (int i = ia; i < ib; ++i) {
        const bool near = s_spage[i] >= near_start;
        if (s_skey[i] == (uint32_t)(near ? tn.T : tf.T) && !(near ? all_n : all_f))
          ++c2[near ? 1 : 0];
      }
      block_scan_n<2, SW>(c2, s_tmp + 32, tot2);
      rf = c2[0];
      rn = c2[1];
    }
    int c5[5] = {0, 0, 0, 0, 0}, tot5[5];
    uint32_t candm = 0u;
    for (int i = ia; i < ib; ++i) {
      const int page = s_spage[i];
      const uint32_t k = s_skey[i];
      const bool near = page >= near_start;
      const uint32_t T = (uint32_t)(near ? tn.T : tf.T);
      bool sel = k > T;
      if (k == T) sel = (near ? all_n : all_f) || (near ? rn++ < tn.need : rf++ < tf.need);
      if (!sel) continue;
      if (NFA_COLD(dbg)) dbg_select(page, k, near);
      if (page >= cp_lo && page < cp_hi) {
        candm |= 1u << (i - ia);
        ++c5[0];
        c5[1] += page < bp0 ? 1 : 0;
        c5[2] += page < bp1 ? 1 : 0;
        c5[3] += page == bp0 ? 1 : 0;
        c5[4] += page == bp1 ? 1 : 0;
      }
    }
    block_scan_n<5, SW>(c5, s_tmp + 32, tot5);
    const bool ins0 = bp0 >= 0 && tot5[3] == 0;
    const bool ins1 = bp1 >= 0 && bp1 != bp0 && tot5[4] == 0;
    int pos = c5[0];
    for (uint32_t bits = candm; bits; bits &= bits - 1u) {
      const int page = s_spage[ia + __ffs(bits) - 1];
      const int dest = pos + (ins0 && page > bp0 ? 1 : 0) + (ins1 && page > bp1 ? 1 : 0);
      if (dest < sd.np) s_pages[dest] = page;
      ++pos;
    }
    if (tid == 0) {
      if (ins0) {
        const int r0 = tot5[1] + (ins1 && bp1 < bp0 ? 1 : 0);
        if (r0 < sd.np) s_pages[r0] = bp0;
      }
      if (ins1) {
        const int r1 = tot5[2] + (ins0 && bp0 < bp1 ? 1 : 0);
        if (r1 < sd.np) s_pages[r1] = bp1;
      }
    }
    np_u = tot5[0] + (ins0 ? 1 : 0) + (ins1 ? 1 : 0);
  }
  for (int sg = 0; sg < (surv_path ? 0 : sd.nseg); ++sg) {
    const int seg_base = sg * sd.seg;
    if (NFA_COLD(multi_seg)) {
      __syncthreads();
      stage_keys(g_keys, seg_base, sd.seg, s_keys);
      dma_barrier();
    }
    const int n = imin(sd.seg, kt_tiles - seg_base);
    const int n16 = (n + 15) / 16;  // the segment holds a multiple of 16 keys
    for (int v0 = 0; v0 < n16; v0 += SB) {  // uniform trip count
      const int v = v0 + tid;
      const int pg0 = seg_base + v * 16;
      uint32_t cand = 0u, tief = 0u, tien = 0u;
      if (v < n16) {
        const uint4 wa = reinterpret_cast<const uint4 *>(s_keys)[2 * v];
        const uint4 wb = reinterpret_cast<const uint4 *>(s_keys)[2 * v + 1];
        const uint32_t ws[8] = {wa.x, wa.y, wa.z, wa.w, wb.x, wb.y, wb.z, wb.w};
        // masks over the sixteen pages: in range, near pool, candidate range
        const uint32_t valid = range16(pg0, pg0, seg_base + n);
        const uint32_t nearm = range16(pg0, near_start, 0x7FFFFFFF);
        const uint32_t candm = range16(pg0, cp_lo, cp_hi);
        auto byp16 = [&](int bp) -> uint32_t {
          return bp >= pg0 && bp < pg0 + 16 ? 1u << (bp - pg0) : 0u;
        };
        uint32_t gt = 0u, eq = 0u;
#pragma unroll
        for (int j = 0; j < 16; ++j) {
          const uint32_t k = (ws[j >> 1] >> (16 * (j & 1))) & 0xFFFFu;
          const uint32_t T = ((nearm >> j) & 1u) ? (uint32_t)tn.T : (uint32_t)tf.T;
          gt |= (k > T ? 1u : 0u) << j;
          eq |= (k == T ? 1u : 0u) << j;
        }
        gt &= valid;
        eq &= valid;
        // keys equal to the threshold: all selected, or tied (zero keys equal
        // a threshold of 0 only when every valid key is selected: no tie cut)
        const uint32_t all_eq = (tf.need == (1 << 30) ? ~nearm : 0u) |
                                (tn.need == (1 << 30) ? nearm : 0u);
        const uint32_t sel = gt | (eq & all_eq);
        tief = eq & ~all_eq & ~nearm;
        tien = eq & ~all_eq & nearm;
        cand = (sel & candm) | byp16(bp0) | byp16(bp1);
        if (NFA_COLD(dbg)) {
          for (uint32_t bits = sel; bits; bits &= bits - 1u) {
            const int j = __ffs(bits) - 1;
            const uint32_t k = (ws[j >> 1] >> (16 * (j & 1))) & 0xFFFFu;
            dbg_select(pg0 + j, k, ((nearm >> j) & 1u) != 0u);
          }
        }
      }
      if (tie_cut(tf) || tie_cut(tn)) {
        int c2[2] = {(int)__popc(tief), (int)__popc(tien)}, tot2[2];
        // (the position scan below, on other scratch, holds the barriers
        // before this scratch is written again)
        block_scan_n<2, SW, false>(c2, s_tmp + 32, tot2);
        int rf = tfb + c2[0], rn = tnb + c2[1];
        for (uint32_t bits = tief; bits; bits &= bits - 1u) {
          const int j = __ffs(bits) - 1;
          if (rf++ < tf.need) {
            if (in_cand(pg0 + j)) cand |= 1u << j;
            if (NFA_COLD(dbg)) dbg_select(pg0 + j, (uint32_t)tf.T, false);
          }
        }
        for (uint32_t bits = tien; bits; bits &= bits - 1u) {
          const int j = __ffs(bits) - 1;
          if (rn++ < tn.need) {
            if (in_cand(pg0 + j)) cand |= 1u << j;
            if (NFA_COLD(dbg)) dbg_select(pg0 + j, (uint32_t)tn.T, true);
          }
        }
        tfb += tot2[0];
        tnb += tot2[1];
      }
      int ctot;
      int pos = np_u + block_scan_exclusive<SW>(__popc(cand), s_tmp, &ctot);
      for (uint32_t bits = cand; bits; bits &= bits - 1u) {
        if (pos < sd.np) s_pages[pos] = pg0 + __ffs(bits) - 1;
        ++pos;
      }
      np_u += ctot;
    }
  }
  NFA_MARK(32, 2);
  // word ranges of the debug outputs
  const int wpt = (sd.words + SB - 1) / SB;
  const int w0 = tid * wpt;
  const int w1 = imin(w0 + wpt, sd.words);
  NFA_MARK(32, 3);
  __syncthreads();
  np_u = imin(np_u, sd.np);
  // protected ids; the gather slots of the first SB are fetched now
  int u0, u1, u2, u3;
  protected_intervals(p, L, sd.prot, &u0, &u1, &u2, &u3);
  const int nu = (u1 - u0) + (u3 - u2);
  int pre_slot = 0;
  if (!p.middle_only && tid < nu) {
    const int x = tid < (u1 - u0) ? u0 + tid : u2 + (tid - (u1 - u0));
    const int xp = udiv_p2(x, p.page, sd.page_sh);
    pre_slot = btr[imin(xp, mb - 1)] * p.page + (x - xp * p.page);
  }
  // physical pages of the candidates: with the L2 side copy nothing reads
  // them before the L2 top-quota, so their loads stay in flight through the
  // logits (held in a register, stored to LDS after them)
  int *s_pphys = (int *)(smem + sd.a_pphys);
  const bool pphys_late = l2_side && np_u <= SB;
  int pphys_reg = 0;
  if (pphys_late) {
    if (tid < np_u)
      pphys_reg = btr[imin(udiv_p2(s_pages[tid] * bs, p.page, sd.page_sh), mb - 1)];
  } else {
    for (int i = tid; i < np_u; i += SB)
      s_pphys[i] = btr[imin(udiv_p2(s_pages[i] * bs, p.page, sd.page_sh), mb - 1)];
  }
  if (tid == 0 && NFA_DBGP(p.dbg_cand_count) != nullptr)
    NFA_DBGP(p.dbg_cand_count)[row] = imin(np_u * bs, p.dbg_cand_cap);
  NFA_MARK(32, 4);
  // L1 debug outputs: I_F / I_N (selector:1766-1803 order: valid pages by
  // (score desc, page asc), then -inf fillers by ascending page)
  if (NFA_COLD(dbg)) {
    for (int pool = 0; pool < 2; ++pool) {
      const int K = pool == 0 ? p.k_f : p.k_n;
      const int nsel = pool == 0 ? tf.nsel : tn.nsel;
      const uint64_t *sel = s_dsel + (pool == 0 ? 0 : p.k_f);
      const uint32_t *bm = pool == 0 ? s_dbf : s_dbn;
      int32_t *out = (pool == 0 ? NFA_DBGP(p.dbg_i_f) + (int64_t)row * p.k_f
                                : NFA_DBGP(p.dbg_i_n) + (int64_t)row * p.k_n);
      for (int i = tid; i < nsel; i += SB) {
        const uint64_t ki = sel[i];
        const uint32_t vi = (uint32_t)(ki >> 32), ti = (uint32_t)ki;
        int rank = 0;
        for (int j = 0; j < nsel; ++j) {
          const uint64_t kj = sel[j];
          const uint32_t vj = (uint32_t)(kj >> 32), tj = (uint32_t)kj;
          rank += (vj > vi) || (vj == vi && tj < ti);
        }
        out[rank] = (int)ti;
      }
      const int nfill = K - nsel;  // uniform
      if (nfill > 0) {
        int z = 0;
        for (int w = w0; w < w1; ++w) z += 32 - __popc(bm[w]);
        int tz;
        int r = block_scan_exclusive<SW>(z, s_tmp, &tz);
        for (int w = w0; w < w1 && r < nfill; ++w) {
          uint32_t zeros = ~bm[w];
          while (zeros && r < nfill) {
            out[nsel + r++] = w * 32 + __ffs(zeros) - 1;
            zeros &= zeros - 1u;
          }
        }
      }
    }
  }
  if (tid == 0) s_misc[2] = 0;  // middle count
  // bf16/fp32 side copy in 16-byte runs: this thread's first L2 slot's row is
  // requested now, ahead of the barrier below (the logits loop starts from it)
  const int nchs = p.fine_dsub % CH == 0 ? p.fine_dsub / CH : 0;
  const bool l2_pre = l2_side && !l2_quant && nchs > 0 && nchs <= 4;
  // the side copy of this (request, kv head): page pg's token r starts at
  // side0 + pg * bs * fine_dsub + r * (CH, chunk-major, or fine_dsub)
  const KV *side0 = l2_side
                        ? (const KV *)p.l2_keys_l + l2_side_index<KV>(p, req, kv, 0, 0)
                        : nullptr;
  int tk_pre = -1;
  const KV *kr_pre = nullptr;
  uint4 r_pre[4];
  if (l2_pre) {
    if (tid < np_u * bs) {
      const int pi = udiv_p2(tid, bs, sd.bs_sh);
      const int r = tid - pi * bs;
      const int pg = s_pages[pi];
      const int tk = pg * bs + r;
      if (tk >= tok_lo && tk < tok_hi) {
        tk_pre = tk;
        kr_pre = side0 + (int64_t)pg * (bs * p.fine_dsub) + r * CH;
      }
    }
#pragma unroll
    for (int c = 0; c < 4; ++c)
      r_pre[c] = kr_pre != nullptr && c < nchs
                     ? *reinterpret_cast<const uint4 *>(kr_pre + c * bs * CH)
                     : make_uint4(0u, 0u, 0u, 0u);
  }
  // the same for the 4-bit side cache: the first slot's codes (one or two
  // 16-byte runs for 32 or 64 L2 dims) and (scale, zero)
  int64_t sl_pre = -1;
  uint4 cw_pre = make_uint4(0u, 0u, 0u, 0u), cw2_pre = make_uint4(0u, 0u, 0u, 0u);
  uint32_t pw_pre = 0u;
  if (l2_quant) {
    if (tid < np_u * bs) {
      const int pi = udiv_p2(tid, bs, sd.bs_sh);
      const int tk = s_pages[pi] * bs + (tid - pi * bs);
      if (tk >= tok_lo && tk < tok_hi) {
        tk_pre = tk;
        sl_pre = q4_slot(p, req, kv, tk);
      }
    }
    if (sl_pre >= 0) {
      const unsigned char *qb = (const unsigned char *)p.l2_keys_l;
      const int cb = p.fine_dsub / 2;
      cw_pre = *reinterpret_cast<const uint4 *>(qb + sl_pre * cb);
      if (cb > 16) cw2_pre = *reinterpret_cast<const uint4 *>(qb + sl_pre * cb + 16);
      pw_pre = *reinterpret_cast<const uint32_t *>(qb + q4_slots(p) * cb + sl_pre * 4);
    }
  }
  // one unmasked L2 region: its high-byte key histogram accumulates while
  // the logits are computed (the L1 histograms are dead here)
  const bool hist_fused = lb.quota > 0 && !near_quota;
  if (hist_fused && tid < 512) s_hist[tid] = 0;
  __syncthreads();  // the L1 part of the tail LDS is dead from here
  NFA_MARK(32, 6);

  // ---- L2 logits (selector:423-516): fp32 dot over the L2 dims in order --
  //      (a fused multiply-add per dim), the dense slots of the candidate
  //      pages, SPT per thread in flight
  uint16_t *s_dk = (uint16_t *)(smem + sd.a_dk);
  const int n_dense = np_u * bs;
  {
    const float *s_qg = (const float *)(smem + sd.a_qg);
    // the L2 dims of a slot: its side row (dense, in order) or its K row
    const bool side = l2_side;
    const int nch = side ? (p.fine_dsub % CH == 0 ? p.fine_dsub / CH : 0)
                         : s_misc[5];  // 16-byte runs, 0: element loads
    // side copy: kr = element 0 of the token, chunk c at c * bs * CH (chunk-
    // major) or element d at d (token-major); K pool: the L2 dims' offsets
    auto choff = [&](int c) { return side ? c * bs * CH : s_fdims[c * CH]; };
    auto eoff = [&](int d) { return side ? d : s_fdims[d]; };
    const int side_pg = bs * p.fine_dsub;
    const int side_tk = p.fine_dsub % CH == 0 ? CH : p.fine_dsub;
    // slot i: its token and L2 row (null outside the candidate range)
    auto slot_row = [&](int i, int &tk) -> const KV * {
      const int pi = div_p2(i, bs, sd.bs_sh);
      const int r = i - pi * bs;
      const int pg = s_pages[pi];
      tk = pg * bs + r;
      if (tk < tok_lo || tk >= tok_hi) return nullptr;
      if (side) return side0 + (int64_t)pg * side_pg + r * side_tk;
      const int phys =
          safe_page(p, page_phys ? s_pphys[pi] : btr[imin(tk / p.page, mb - 1)]);
      return kpool + kv_offset(p, phys, kv, tk % p.page);
    };
    // logit key of dense slot i (and the parity-test record)
    const bool dbg_cand = NFA_COLD(NFA_DBGP(p.dbg_cand_tok) != nullptr);
    auto emit = [&](int i, int tk, bool scored, float acc) {
      uint16_t key = 0;
      if (scored) {
        const uint16_t bits = bf16_bits(acc);
        key = bits == kNanBits ? 0 : (uint16_t)score_key(bits);
        if (NFA_COLD(dbg_cand) && i < p.dbg_cand_cap) {
          NFA_DBGP(p.dbg_cand_tok)[(int64_t)row * p.dbg_cand_cap + i] = tk;
          NFA_DBGP(p.dbg_cand_logit)[(int64_t)row * p.dbg_cand_cap + i] =
              bits == kNanBits ? kNegInfBits : bits;
        }
      } else if (NFA_COLD(dbg_cand) && i < p.dbg_cand_cap) {
        NFA_DBGP(p.dbg_cand_tok)[(int64_t)row * p.dbg_cand_cap + i] = -1;
      }
      s_dk[i] = key;
      if (hist_fused && key != 0) atomicAdd(&s_hist[key >> 8], 1);
    };
    if (l2_quant) {
      // 4-bit side cache: 16 bytes of codes and 4 of (scale, zero) per
      // slot, dequantised in registers as bf16(bf16(code * scale) - zero)
      const unsigned char *qb = (const unsigned char *)p.l2_keys_l;
      const int cb = p.fine_dsub / 2;  // 16 or 32 code bytes per slot
      const bool two = cb > 16;
      const int64_t poff = q4_slots(p) * cb;
      auto q4_of = [&](int i, int &tk) -> int64_t {
        const int pi = udiv_p2(i, bs, sd.bs_sh);
        tk = s_pages[pi] * bs + (i - pi * bs);
        if (tk < tok_lo || tk >= tok_hi) return -1;
        return q4_slot(p, req, kv, tk);
      };
      // 32 dims of dequantised keys from one 16-byte run of codes, dotted
      // with the grouped query from dim d0 on, in dim order
      // (two dims per conversion; a code's byte from the nibbles spread
      // into bytes, even and odd nibbles apart)
      auto dot32 = [&](const uint4 &cw, float sc, float zr, int d0, float acc) {
        const uint32_t w4[4] = {cw.x, cw.y, cw.z, cw.w};
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const uint32_t ev = w4[k] & 0x0F0F0F0Fu;         // dims 0, 2, 4, 6
          const uint32_t od = (w4[k] >> 4) & 0x0F0F0F0Fu;  // dims 1, 3, 5, 7
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const float c0 = (float)((ev >> (8 * j)) & 0xFFu);
            const float c1 = (float)((od >> (8 * j)) & 0xFFu);
            float a, b;
            bf16r_hw2(c0 * sc, c1 * sc, a, b);
            // a NaN here (non-finite keys) still ends as a NaN logit
            bf16r_hw2(a - zr, b - zr, a, b);
            acc = __builtin_fmaf(a, s_qg[d0 + 8 * k + 2 * j], acc);
            acc = __builtin_fmaf(b, s_qg[d0 + 8 * k + 2 * j + 1], acc);
          }
        }
        return acc;
      };
      // the first slot's loads were issued before the L1 LDS was released
      int tk = tk_pre;
      int64_t sl = sl_pre;
      uint4 cw = cw_pre, cw2 = cw2_pre;
      uint32_t pw = pw_pre;
#pragma unroll 1
      for (int i = tid; i < n_dense; i += SB) {
        int tkn = -1;
        const int64_t sln = i + SB < n_dense ? q4_of(i + SB, tkn) : -1;
        uint4 cwn = make_uint4(0u, 0u, 0u, 0u), cwn2 = make_uint4(0u, 0u, 0u, 0u);
        uint32_t pwn = 0u;
        if (sln >= 0) {
          cwn = *reinterpret_cast<const uint4 *>(qb + sln * cb);
          if (two) cwn2 = *reinterpret_cast<const uint4 *>(qb + sln * cb + 16);
          pwn = *reinterpret_cast<const uint32_t *>(qb + poff + sln * 4);
        }
        float acc = 0.0f;
        if (sl >= 0) {
          const float sc = bf16_val((uint16_t)(pw & 0xFFFFu));
          const float zr = bf16_val((uint16_t)(pw >> 16));
          acc = dot32(cw, sc, zr, 0, acc);
          if (two) acc = dot32(cw2, sc, zr, 32, acc);
        }
        emit(i, tk, sl >= 0, acc);
        tk = tkn;
        sl = sln;
        cw = cwn;
        cw2 = cwn2;
        pw = pwn;
      }
    } else {
    const bool vec4 = nch > 0 && nch <= 4;  // the L2 row in at most 4 loads
    auto fetch = [&](const KV *kr, uint4 (&r)[4]) {
#pragma unroll
      for (int c = 0; c < 4; ++c)
        r[c] = kr != nullptr && c < nch
                   ? *reinterpret_cast<const uint4 *>(kr + choff(c))
                   : make_uint4(0u, 0u, 0u, 0u);
    };
    // slots tid, tid + SB, ...: the next slot's loads are in flight while
    // the current slot's dot product runs (rolled: compact code)
    // the grouped L2 query in registers (the loop's LDS stores would keep
    // the compiler from hoisting its reads)
    float qv[4 * CH];
#pragma unroll
    for (int e = 0; e < 4 * CH; ++e) qv[e] = vec4 && e < nch * CH ? s_qg[e] : 0.0f;
    int tk = -1;
    const KV *kr = nullptr;
    uint4 r[4];
    if (l2_pre) {
      tk = tk_pre;
      kr = kr_pre;
#pragma unroll
      for (int c = 0; c < 4; ++c) r[c] = r_pre[c];
    } else {
      if (tid < n_dense) kr = slot_row(tid, tk);
      if (vec4) fetch(kr, r);
    }
#pragma unroll 1
    for (int i = tid; i < n_dense; i += SB) {
      int tkn = -1;
      const KV *krn = nullptr;
      uint4 rn[4];
      if (i + SB < n_dense) krn = slot_row(i + SB, tkn);
      if (vec4) fetch(krn, rn);
      float acc = 0.0f;
      if (kr != nullptr) {
        if (vec4) {
#pragma unroll
          for (int c = 0; c < 4; ++c) {
            if (c >= nch) continue;
            float x[CH];
            unpack_chunk<KV>(r[c], x);
#pragma unroll
            for (int e = 0; e < CH; ++e) {
              acc = __builtin_fmaf(x[e], qv[c * CH + e], acc);
            }
          }
        } else if (nch > 0) {
          for (int c = 0; c < nch; ++c) {
            float x[CH];
            load_chunk<KV>(kr + choff(c), x);
            for (int e = 0; e < CH; ++e) {
              acc = __builtin_fmaf(x[e], s_qg[c * CH + e], acc);
            }
          }
        } else {
          for (int d = 0; d < p.fine_dsub; ++d) {
            acc = __builtin_fmaf(Elem<KV>::load(kr + eoff(d)), s_qg[d], acc);
          }
        }
      }
      emit(i, tk, kr != nullptr, acc);
      tk = tkn;
      kr = krn;
#pragma unroll
      for (int c = 0; c < 4; ++c) r[c] = rn[c];
    }
    }
  }
  if (pphys_late && tid < np_u) s_pphys[tid] = pphys_reg;
  __syncthreads();
  NFA_MARK(32, 9);

  // ---- L2 top-quota + hole fill (+ fixed near quota), selector:519-566,
  //      873-940 -------------------------------------------------------------
  const RegionLists rl{(int *)(smem + sd.a_l0), (int *)(smem + sd.a_l0x),
                       (int *)(smem + sd.a_l1), (int *)(smem + sd.a_l1x),
                       (int *)(smem + sd.a_mid), (int *)(smem + sd.a_mslot)};
  const DenseView dv{s_dk, s_pages, s_pphys, btr, n_dense, bs, p.page, mb,
                     page_phys, sd.bs_sh, sd.page_sh};
  if (lb.quota > 0) {
    int nreg = 1;
    bool masked = false;
    int r_lo[2] = {lb.lower, 0}, r_hi[2] = {lb.upper, 0}, r_q[2] = {lb.quota, 0};
    if (NFA_COLD(near_quota)) {
      // far quota first, the remainder goes to near (selector:873-920)
      const L2Bounds fb = l2_bounds(p, L, false, false, p.near_len);
      const int base = imax(imin(L, p.k2) - p.sink_tokens - (L - fb.lo), 0);
      const int reserve = imin(p.near_tokens, base);
      const int lower0 = (p.sink_tokens / bs) * bs;
      const int upper0 = imax(lower0, fb.lo);
      int far_quota = imax(base - reserve, 0);
      const int far_low = skip_far ? fb.far_hi : lower0;
      const int far_high = fb.far_hi;
      far_quota = imin(far_quota, imax(far_high - far_low, 0));
      int near_quota = imax(base - far_quota, 0);
      const int near_low = fb.far_hi;
      const int near_high = skip_near ? fb.far_hi : upper0;
      near_quota = imin(near_quota, imax(near_high - near_low, 0));
      nreg = 2;
      masked = true;
      r_lo[0] = far_low;
      r_hi[0] = imax(far_low, far_high);
      r_q[0] = far_quota;
      r_lo[1] = near_low;
      r_hi[1] = imax(near_low, near_high);
      r_q[1] = near_quota;
    }
    int64_t *rclk = NFA_DBGP(p.dbg_clock) != nullptr ? s_clk + 32 + 16 : nullptr;
    for (int r = 0; r < nreg; ++r)
      l2_region_dense(dv, masked, r_lo[r], r_hi[r], r_q[r], p.sink_tokens, rl,
                      &s_misc[2], s_hist, s_tmp, rclk, hist_fused);
  }
  __syncthreads();
  NFA_MARK(32, 12);
  int mcount = s_misc[2];
  if (mcount > p.k2) mcount = p.k2;
  const int *s_mid = rl.mid;
  const int *s_mslot = rl.mslot;
  if (NFA_COLD(NFA_DBGP(p.dbg_middle) != nullptr)) {
    for (int k = tid; k < p.k2; k += SB)
      NFA_DBGP(p.dbg_middle)[(int64_t)row * p.k2 + k] = k < mcount ? s_mid[k] : 0;
    if (tid == 0) NFA_DBGP(p.dbg_counts)[row] = mcount;
  }

  // ---- final union with the protected sink/SWA ids (selector:1337-1437) --
  int32_t *grow = p.gather + (int64_t)row * p.max_vis;
  if (NFA_COLD(p.middle_only)) {
    const int n = imin(mcount, p.max_vis);
    for (int k = tid; k < n; k += SB) grow[k] = s_mslot[k];
    if (tid == 0) p.vis_lens[row] = n;
    NFA_MARK(32, 13);
    NFA_FLUSH(32, clk_tail);
    return;
  }
  const int n0 = u1 - u0;  // protected ids of the first interval
  if (__builtin_expect(u0 == 0 && (mcount == 0 || (s_mid[0] >= u1 && s_mid[mcount - 1] < u2)), 1)) {
    // the usual case: the middle lies between the sink and the SWA ids, so
    // the union is [0, u1) ++ middle ++ [u2, u3) with no duplicates
    for (int k = tid; k < mcount; k += SB)
      if (n0 + k < p.max_vis) grow[n0 + k] = s_mslot[k];
    for (int k = tid; k < nu; k += SB) {
      const int x = k < n0 ? u0 + k : u2 + (k - n0);
      const int dest = k < n0 ? k : k + mcount;
      const int slot = k == tid ? pre_slot
                                : btr[imin(x / p.page, mb - 1)] * p.page + x % p.page;
      if (dest < p.max_vis) grow[dest] = slot;
    }
    if (tid == 0) p.vis_lens[row] = mcount + nu;
    NFA_MARK(32, 13);
    NFA_FLUSH(32, clk_tail);
    return;
  }
  auto in_u = [&](int x) { return (x >= u0 && x < u1) || (x >= u2 && x < u3); };
  auto below_u = [&](int x) {  // |U ∩ [0, x)|
    return imax(0, imin(x, u1) - u0) + imax(0, imin(x, u3) - u2);
  };
  // middle entries inside U are duplicates; the rest keep their order
  int nkeep;
  {
    const int per = (mcount + SB - 1) / SB;
    const int ia = tid * per;
    const int ib = imin(mcount, ia + per);
    int c = 0;
    for (int k = ia; k < ib; ++k) c += !in_u(s_mid[k]);
    int r = block_scan_exclusive<SW>(c, s_tmp, &nkeep);
    for (int k = ia; k < ib; ++k) {
      const int x = s_mid[k];
      if (in_u(x)) continue;
      const int dest = r + below_u(x);
      if (dest < p.max_vis) grow[dest] = s_mslot[k];
      ++r;
    }
  }
  // kept-middle entries below x: lower_bound over s_mid minus duplicates
  auto kept_below = [&](int x) {
    const int lbx = lower_bound_i32(s_mid, mcount, x);
    const int d0 = lower_bound_i32(s_mid, mcount, imin(imax(x, u0), u1)) -
                   lower_bound_i32(s_mid, mcount, u0);
    const int d1 = lower_bound_i32(s_mid, mcount, imin(imax(x, u2), u3)) -
                   lower_bound_i32(s_mid, mcount, u2);
    return lbx - d0 - d1;
  };
  for (int k = tid; k < nu; k += SB) {
    const int x = k < (u1 - u0) ? u0 + k : u2 + (k - (u1 - u0));
    const int dest = k + kept_below(x);
    const int slot = k == tid ? pre_slot
                              : btr[imin(x / p.page, mb - 1)] * p.page + x % p.page;
    if (dest < p.max_vis) grow[dest] = slot;
  }
  if (tid == 0) p.vis_lens[row] = nkeep + nu;
  NFA_MARK(32, 13);
  NFA_FLUSH(32, clk_tail);
  }  // tail
}



}  // namespace nfa

// ---------------------------------------------------------------------------
// host entry
// ---------------------------------------------------------------------------

using nfa::SelDims;

// compute units of the current device, cached per device

// The parameters with defaults filled in (kv_heads_mem 0 = hkv).
static NfaSelectParams select_normalized(const NfaSelectParams &p) {
  NfaSelectParams q = p;
  if (q.kv_heads_mem == 0) q.kv_heads_mem = q.hkv;
  return q;
}

static int select_check(const NfaSelectParams *p, bool need_workspace) {
  if (p == nullptr) {
    nfa_set_error("nfa_select_layer: null params");
    return NFA_EINVAL;
  }
  if (p->abi_version != NFA_ABI_VERSION ||
      p->struct_size != (int32_t)sizeof(NfaSelectParams)) {
    nfa_set_error("nfa_select_layer: ABI mismatch (version %d size %d, expected %d/%d)",
                  p->abi_version, p->struct_size, NFA_ABI_VERSION,
                  (int)sizeof(NfaSelectParams));
    return NFA_EINVAL;
  }
  if (p->batch <= 0 || p->hkv <= 0 || p->hq % p->hkv != 0 ||
      p->hq / p->hkv > nfa::GMAX) {
    nfa_set_error("nfa_select_layer: unsupported heads hq=%d hkv=%d", p->hq, p->hkv);
    return NFA_EINVAL;
  }
  if (p->kv_heads_mem != 0 && p->kv_heads_mem != p->hkv && p->kv_heads_mem != 1) {
    nfa_set_error("nfa_select_layer: kv_heads_mem %d must be hkv (%d) or 1",
                  p->kv_heads_mem, p->hkv);
    return NFA_EINVAL;
  }
  if (p->far_method < NFA_METHOD_MINMAX || p->far_method > NFA_METHOD_AVG_TOP2 ||
      p->near_method < NFA_METHOD_MINMAX || p->near_method > NFA_METHOD_AVG ||
      (p->far_method == NFA_METHOD_AVG_TOP2 && p->hq / p->hkv < 2)) {
    nfa_set_error("nfa_select_layer: unsupported L1 methods far=%d near=%d "
                  "(avg_top2 needs 2+ query heads per kv head)",
                  p->far_method, p->near_method);
    return NFA_EINVAL;
  }
  if (!(p->dsub == 32 || p->dsub == 64 || p->dsub == 128)) {
    nfa_set_error("nfa_select_layer: unsupported L1 dim count %d", p->dsub);
    return NFA_EINVAL;
  }
  if (p->fine_dsub <= 0 || p->fine_dsub > p->head_dim) {
    nfa_set_error("nfa_select_layer: bad L2 dim count %d", p->fine_dsub);
    return NFA_EINVAL;
  }
  if (p->l2_quant && (p->l2_keys_l == nullptr || !nfa::q4_dims_ok(p->fine_dsub) ||
                      p->kv_dtype != NFA_DTYPE_BF16)) {
    nfa_set_error("nfa_select_layer: 4-bit L2 keys need the L2 side cache, 32 or 64 "
                  "L2 dims and bf16 KV (got %d dims, kv dtype %d)",
                  p->fine_dsub, p->kv_dtype);
    return NFA_EINVAL;
  }
  if (p->bs <= 0 || p->page <= 0 || p->max_blocks <= 0 || p->k2 <= 0 ||
      p->k2 > 2048 || p->k_f < 0 || p->k_n < 0 || p->k_f > 1024 ||
      p->k_n > 1024 || p->k_f > p->max_blocks || p->k_n > p->max_blocks) {
    nfa_set_error("nfa_select_layer: unsupported budgets bs=%d k_f=%d k_n=%d k2=%d",
                  p->bs, p->k_f, p->k_n, p->k2);
    return NFA_EINVAL;
  }
  if (p->kv_dtype != NFA_DTYPE_BF16 && p->kv_dtype != NFA_DTYPE_F32) {
    nfa_set_error("nfa_select_layer: unsupported kv dtype %d", p->kv_dtype);
    return NFA_EINVAL;
  }
  if (p->max_vis <= 0) {
    nfa_set_error("nfa_select_layer: max_vis must be positive");
    return NFA_EINVAL;
  }
  if (p->pool_pages <= 0) {
    nfa_set_error("nfa_select_layer: pool_pages must be positive");
    return NFA_EINVAL;
  }
  const SelDims sd = nfa::sel_dims(*p, nfa::device_cus());
  if (sd.lds > nfa::kLdsMax) {
    nfa_set_error("nfa_select_layer: geometry needs %d bytes of LDS (> %d)", sd.lds,
                  nfa::kLdsMax);
    return NFA_EINVAL;
  }
  if ((p->hq / p->hkv) * p->head_dim > nfa::kQRawPerThread * nfa::SB) {
    nfa_set_error("nfa_select_layer: query group of %d x %d elements is too wide",
                  p->hq / p->hkv, p->head_dim);
    return NFA_EINVAL;
  }
  if (p->k_new != nullptr && (p->head_dim > nfa::SB || p->head_dim_v > nfa::SB)) {
    // one element per thread of the workgroup in the fused decode write
    nfa_set_error("nfa_select_layer: the fused decode write takes rows of at most %d "
                  "elements (K %d, V %d)", nfa::SB, p->head_dim, p->head_dim_v);
    return NFA_EINVAL;
  }
  if (sd.ntiles > 65535) {
    nfa_set_error("nfa_select_layer: max_blocks %d exceeds the grid limit", p->max_blocks);
    return NFA_EINVAL;
  }
  if (need_workspace && (p->workspace == nullptr || p->workspace_bytes < sd.w_total)) {
    nfa_set_error("nfa_select_layer: workspace %lld < %lld bytes",
                  (long long)p->workspace_bytes, (long long)sd.w_total);
    return NFA_EWORKSPACE;
  }
  if (!p->k_pool_l || !p->block_table_l || !p->lengths || !p->active_req ||
      !p->valid_req || !p->skip_far_l || !p->skip_near_l || !p->dims ||
      !p->fine_dims || !p->q || !p->stat_min_l || !p->stat_max_l ||
      !p->stat_sum_l || !p->stats_len_l || !p->gather || !p->vis_lens) {
    nfa_set_error("nfa_select_layer: null device pointer");
    return NFA_EINVAL;
  }
  // (a shared arena head may take keys only: its values are part of them)
  const bool shared = p->kv_heads_mem != 0 && p->kv_heads_mem < p->hkv;
  if (p->k_new != nullptr &&
      ((p->v_new == nullptr && !shared) || p->slots == nullptr ||
       (p->v_new != nullptr && p->v_pool_l == nullptr))) {
    nfa_set_error("nfa_select_layer: decode write needs k, v, slots and v pool");
    return NFA_EINVAL;
  }
  if (p->dbg_far != nullptr &&
      (!p->dbg_near || !p->dbg_i_f || !p->dbg_i_n || !p->dbg_middle ||
       !p->dbg_counts || !p->dbg_bounds)) {
    nfa_set_error("nfa_select_layer: partial debug buffers");
    return NFA_EINVAL;
  }
  return NFA_OK;
}

extern "C" int64_t nfa_select_workspace_bytes(const NfaSelectParams *p) {
  if (p == nullptr || p->batch <= 0 || p->hkv <= 0) return 0;
  // the same CU count as the launch: the tile split (tiles per row, passes,
  // page lists) and so the workspace layout depend on it
  return nfa::sel_dims(*p, nfa::device_cus()).w_total;
}

// The launch plan of a checked call: which kernel instance runs and how a
// row of max_blocks pages is tiled (parity tests assert the instance).
extern "C" int32_t nfa_select_plan(const NfaSelectParams *p, int32_t *out, int32_t n) {
  const int rc = select_check(p, false);
  if (rc != NFA_OK) return rc;
  if (out == nullptr || n < 0) {
    nfa_set_error("nfa_select_plan: null output");
    return NFA_EINVAL;
  }
  const SelDims sd = nfa::sel_dims(*p, nfa::device_cus());
  const nfa::TileSplit sp = nfa::tile_split(p->max_blocks, sd.tcap);
  const int passes =
      sp.span <= nfa::kSpanMax ? 1 : 1 + (sp.span - nfa::kSpanMax + nfa::TP - 1) / nfa::TP;
  const int32_t v[8] = {p->protected_only ? -1 : (sd.multi ? (sd.surv ? 2 : 1) : 0),
                        sd.tcap, sd.ntiles, sp.tiles, passes, sd.lds, sd.nseg,
                        (int32_t)(sd.w_total < INT32_MAX ? sd.w_total : INT32_MAX)};
  for (int i = 0; i < n && i < 8; ++i) out[i] = v[i];
  return NFA_OK;
}

// Lets `kernel` take up to kLdsMax bytes of dynamic LDS on the current
// device (the default cap is 64 KiB); `done` remembers the devices already
// set, one bit each.
static hipError_t lds_optin(const void *kernel, std::atomic<uint64_t> &done) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  const uint64_t bit = 1ull << (dev & 63);
  if (done.load(std::memory_order_acquire) & bit) return hipSuccess;
  e = hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                          nfa::kLdsMax);
  if (e == hipSuccess) done.fetch_or(bit, std::memory_order_acq_rel);
  return e;
}

template <int DSUB, typename KV>
static hipError_t launch_select(const NfaSelectParams &p, const SelDims &sd,
                                hipStream_t stream) {
  // one pass per tile whenever a dispatch round of single-pass tiles covers
  // the widest possible row; several passes stage the next pass's statistics
  // in a second LDS buffer (beyond 64 KiB); rows that may be long list their
  // survivors
  const int mode = sd.multi ? (sd.surv ? 2 : 1) : 0;
  const bool top2 = p.far_method == NFA_METHOD_AVG_TOP2;
  const bool dbg = p.dbg_far != nullptr || p.dbg_i_f != nullptr ||
                   p.dbg_counts != nullptr || p.dbg_bounds != nullptr ||
                   p.dbg_cand_tok != nullptr || p.dbg_clock != nullptr;
  const dim3 grid(p.hkv, p.batch, sd.ntiles);
  // instances by (mode, top2): 0/false, 0/true, 1/false, 1/true, 2/false;
  // production ones with bf16 L2 keys, then with 4-bit keys (both from the
  // L2 side copy), then the debug ones (the key format, the side copy and the
  // other options read at run time; they also serve production calls that
  // take one of those options)
#define NFA_SEL_K5(d, q)                                                          \
  reinterpret_cast<const void *>(&nfa::nfa_select_kernel<DSUB, KV, 0, false, d, q>), \
      reinterpret_cast<const void *>(&nfa::nfa_select_kernel<DSUB, KV, 0, true, d, q>), \
      reinterpret_cast<const void *>(&nfa::nfa_select_kernel<DSUB, KV, 1, false, d, q>), \
      reinterpret_cast<const void *>(&nfa::nfa_select_kernel<DSUB, KV, 1, true, d, q>), \
      reinterpret_cast<const void *>(&nfa::nfa_select_kernel<DSUB, KV, 2, false, d, q>)
  const void *k[15] = {NFA_SEL_K5(false, 0), NFA_SEL_K5(false, 1), NFA_SEL_K5(true, 2)};
#undef NFA_SEL_K5
  // what only the run-time instances hold
  const bool rt = dbg || p.l2_keys_l == nullptr || p.page_sum_l == nullptr ||
                  sd.nseg > 1 || p.near_tokens >= 0;
  const int i = (mode == 2 ? 4 : 2 * mode + (int)top2) + (rt ? 10 : p.l2_quant ? 5 : 0);
  if (sd.lds > 64 * 1024) {
    static std::atomic<uint64_t> optin[15];
    const hipError_t e = lds_optin(k[i], optin[i]);
    if (e != hipSuccess) return e;
  }
  // the kernel's arguments as the launch API takes them
  NfaSelectParams pa = p;
  SelDims sa = sd;
  void *args[] = {&pa, &sa};
  const hipError_t le = hipLaunchKernel(k[i], grid, dim3(nfa::SB), args, sd.lds, stream);
  if (le != hipSuccess) return le;
  return hipGetLastError();
}

// Launches the selector (or the protected-only union) of a checked call
// with the workspace layout `sd`.
static int32_t select_launch(const NfaSelectParams &p, const SelDims &sd,
                             hipStream_t s, const char *who) {
  hipError_t err;
  const bool bf = p.kv_dtype == NFA_DTYPE_BF16;
  if (p.protected_only) {
    dim3 grid(p.batch * p.hkv);
    if (bf)
      hipLaunchKernelGGL(nfa::nfa_protected_kernel<uint16_t>, grid,
                         dim3(nfa::SB), 0, s, p);
    else
      hipLaunchKernelGGL(nfa::nfa_protected_kernel<float>, grid, dim3(nfa::SB),
                         0, s, p);
    err = hipGetLastError();
  } else {
    switch (p.dsub) {
      case 32:
        err = bf ? launch_select<32, uint16_t>(p, sd, s)
                 : launch_select<32, float>(p, sd, s);
        break;
      case 64:
        err = bf ? launch_select<64, uint16_t>(p, sd, s)
                 : launch_select<64, float>(p, sd, s);
        break;
      default:
        err = bf ? launch_select<128, uint16_t>(p, sd, s)
                 : launch_select<128, float>(p, sd, s);
        break;
    }
  }
  if (err != hipSuccess) {
    nfa_set_error("%s: launch failed: %s", who, hipGetErrorString(err));
    return NFA_ELAUNCH;
  }
  return NFA_OK;
}

extern "C" int32_t nfa_select_layer(const NfaSelectParams *p, void *stream) {
  const int rc = select_check(p, true);
  if (rc != NFA_OK) return rc;
  const NfaSelectParams q = select_normalized(*p);
  const SelDims sd = nfa::sel_dims(q, nfa::device_cus());
  return select_launch(q, sd, (hipStream_t)stream, "nfa_select_layer");
}

// ---------------------------------------------------------------------------
// allocation-free entry: the workspace is a static device array
// ---------------------------------------------------------------------------

// Fixed layout, so that calls of different batch shapes never place one
// call's keys over another's counters: row arrival counters, request
// counters, per-row histograms for the maximum row count, then the keys.
// The kernel leaves the counters and histograms at zero when it ends, so
// they are cleared once per device, at the first call.
constexpr int64_t kScratchRowCnt = 0;
constexpr int64_t kScratchReqCnt = (int64_t)4 * nfa::kArriveStride * NFA_SELECT_SCRATCH_ROWS;
constexpr int64_t kScratchHist = kScratchReqCnt + 4 * NFA_SELECT_SCRATCH_ROWS;
constexpr int64_t kScratchKeys = kScratchHist + (int64_t)4 * 512 * NFA_SELECT_SCRATCH_ROWS;
static_assert(kScratchKeys % 256 == 0 && kScratchKeys < NFA_SELECT_SCRATCH_BYTES,
              "scratch layout");

static __device__ __align__(256) unsigned char scratch[NFA_SELECT_SCRATCH_BYTES];

__global__ void __launch_bounds__(256) nfa_scratch_clear_kernel(uint4 *dst, int64_t n16) {
  const uint4 z = make_uint4(0u, 0u, 0u, 0u);
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n16;
       i += (int64_t)gridDim.x * blockDim.x)
    dst[i] = z;
}

static std::mutex g_scratch_mu;
static void *g_scratch_ptr[64];

// This device's copy of `scratch` (its address differs per device), with the
// counters and histograms cleared; set up at the device's first call.
static int32_t scratch_for_device(hipStream_t s, void **out) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) {
    nfa_set_error("nfa_select_layer_noalloc: no current device");
    return NFA_EINVAL;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] != nullptr) {
    *out = g_scratch_ptr[dev];
    return NFA_OK;
  }
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(s, &cap) != hipSuccess || cap != hipStreamCaptureStatusNone) {
    nfa_set_error("nfa_select_layer_noalloc: the first call on a device sets up "
                  "its scratch array and must not be captured");
    return NFA_EINVAL;
  }
  void *ptr = nullptr;
  hipError_t err = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
  if (err != hipSuccess || ptr == nullptr) {
    nfa_set_error("nfa_select_layer_noalloc: hipGetSymbolAddress failed: %s",
                  hipGetErrorString(err));
    return NFA_ELAUNCH;
  }
  hipLaunchKernelGGL(nfa_scratch_clear_kernel, dim3(256), dim3(256), 0, s,
                     (uint4 *)ptr, kScratchKeys / 16);
  err = hipGetLastError();
  if (err == hipSuccess) err = hipStreamSynchronize(s);
  if (err != hipSuccess) {
    nfa_set_error("nfa_select_layer_noalloc: scratch clear failed: %s",
                  hipGetErrorString(err));
    return NFA_ELAUNCH;
  }
  g_scratch_ptr[dev] = ptr;
  *out = ptr;
  return NFA_OK;
}

extern "C" int32_t nfa_select_layer_noalloc(const NfaSelectParams *p, void *stream) {
  int rc = select_check(p, false);
  if (rc != NFA_OK) return rc;
  SelDims sd = nfa::sel_dims(*p, nfa::device_cus());
  const int64_t rows = (int64_t)p->batch * p->hkv;
  // per row: keys (2 bytes a page), survivors (8 bytes a page), tile counts
  const int64_t keys = (((int64_t)2 * rows * sd.kstride) + 255) & ~(int64_t)255;
  const int64_t surv = sd.surv ? (int64_t)8 * rows * sd.kstride : 0;
  const int64_t scnt = sd.surv ? (((int64_t)4 * rows * sd.ntiles) + 255) & ~(int64_t)255 : 0;
  const int64_t need = kScratchKeys + keys + surv + scnt;
  if (rows > NFA_SELECT_SCRATCH_ROWS || need > NFA_SELECT_SCRATCH_BYTES) {
    nfa_set_error("nfa_select_layer_noalloc: %lld rows (batch x kv heads) of %d "
                  "pages need %lld scratch bytes; the static array holds %lld "
                  "bytes and %d rows",
                  (long long)rows, p->max_blocks, (long long)need,
                  (long long)NFA_SELECT_SCRATCH_BYTES, NFA_SELECT_SCRATCH_ROWS);
    return NFA_EWORKSPACE;
  }
  hipStream_t s = (hipStream_t)stream;
  void *ptr = nullptr;
  rc = scratch_for_device(s, &ptr);
  if (rc != NFA_OK) return rc;
  sd.w_rowcnt = kScratchRowCnt;
  sd.w_reqcnt = kScratchReqCnt;
  sd.w_hist = kScratchHist;
  sd.w_keys = kScratchKeys;
  sd.w_surv = kScratchKeys + keys;
  sd.w_scount = sd.w_surv + surv;
  sd.w_total = need;
  NfaSelectParams q = select_normalized(*p);
  q.workspace = ptr;
  q.workspace_bytes = NFA_SELECT_SCRATCH_BYTES;
  return select_launch(q, sd, s, "nfa_select_layer_noalloc");
}
