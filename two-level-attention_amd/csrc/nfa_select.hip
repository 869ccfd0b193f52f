// NFA two-level selector for one decode layer on gfx950.
//
// One launch, grid (ntiles, batch * hkv), 256 threads per workgroup:
//
//   tile stage (every workgroup, 256 pages = one page per thread):
//     decode K/V write of the current token (owner of the last page),
//     page min/max/sum statistics (latest page, or every page of the tile on
//     a rebuild), L1 far/near page scores, and the exact top-K_F / top-K_N
//     of the tile written to scratch in page order.
//   tail stage (the last workgroup of each (row, kv) to arrive, found with a
//     device-scope atomic counter; no workgroup ever waits on another):
//     merge of the tile top-k lists into I_F / I_N, candidate pages, L2
//     logits over the L2 dims, top-quota selection with lowest-token
//     tie-break, hole fill, sink/SWA union and the physical gather rows.
//
// Reference semantics: sparse_attn/indexer/nfa_layer_batch_selector.py
// (selector:32-131 stats, :175-354 L1, :1473-1863 L1 top-k, :1081-1251
// candidates/owners, :423-516 L2 logits, :519-848 L2 top-k, :873-940 fixed
// quota, :1337-1470 union).  Owner tags of the reference reduce to "each
// candidate token is scored once", which the sorted, de-duplicated candidate
// page list gives directly.
#include "nfa_common.h"

#include <stdarg.h>
#include <stdio.h>

namespace nfa {

// ---------------------------------------------------------------------------
// scratch layouts (shared by host and device)
// ---------------------------------------------------------------------------

struct SelDims {
  int ntiles;      // L1 tiles per row
  int np;          // candidate page slots = k_f + k_n + 2
  int cand_cap;    // np * bs
  int prot;        // protected width = min(s_cap, sink + swa)
  int n_merge;     // keys merged per L1 pool: ntiles * max(k_f, k_n)
  bool merge_lds;  // merge keys fit the LDS union
  int lds_bytes;   // dynamic LDS of the launch
  // LDS byte offsets: common part, then the tile and tail parts overlap
  int o_hist, o_tmp;
  int o_qf, o_key, o_dims, o_stage;                       // tile stage
  int o_fp, o_np, o_sel, o_qg, o_choff, o_fdims, o_pages, o_pgoff, o_pphys,
      o_sp, o_rank, o_union, o_cand, o_l0, o_l1, o_mid;  // tail stage
  // global workspace byte offsets
  int64_t w_rowcnt, w_reqcnt, w_far, w_near, w_total;
};

__host__ __device__ inline int align16(int x) { return (x + 15) & ~15; }

// Tokens per staging sub-batch of the page-statistics pass.
constexpr int kStatTokens = 16;

__host__ __device__ inline SelDims sel_dims(const NfaSelectParams &p) {
  SelDims s;
  const int group = p.hq / p.hkv;
  s.ntiles = (p.max_blocks + NFA_BLOCK - 1) / NFA_BLOCK;
  s.np = p.k_f + p.k_n + 2;
  s.cand_cap = s.np * p.bs;
  const int s_cap = p.max_blocks * p.bs;
  s.prot = p.sink_tokens + p.swa < s_cap ? p.sink_tokens + p.swa : s_cap;
  const int kmax = p.k_f > p.k_n ? p.k_f : p.k_n;
  s.n_merge = s.ntiles * (kmax > 0 ? kmax : 1);
  int o = 0;
  s.o_hist = o;  o += align16(4 * 256);
  s.o_tmp = o;   o += align16(4 * 32);
  const int base = o;
  // tile stage
  s.o_qf = o;    o += align16(4 * group * p.dsub);
  s.o_key = o;   o += align16(4 * NFA_BLOCK);
  s.o_dims = o;  o += align16(4 * p.dsub);
  s.o_stage = o; o += align16(4 * NFA_BLOCK * kStatTokens);
  const int tile_end = o;
  // tail stage
  o = base;
  s.o_fp = o;    o += align16(4 * (p.k_f > 0 ? p.k_f : 1));
  s.o_np = o;    o += align16(4 * (p.k_n > 0 ? p.k_n : 1));
  s.o_sel = o;   o += align16(8 * (kmax > 0 ? kmax : 1));
  s.o_qg = o;    o += align16(4 * p.fine_dsub);
  s.o_choff = o; o += align16(4 * 64);
  s.o_fdims = o; o += align16(4 * p.fine_dsub);
  s.o_pages = o; o += align16(4 * s.np);
  s.o_pgoff = o; o += align16(4 * (s.np + 1));
  s.o_pphys = o; o += align16(4 * s.np);
  s.o_sp = o;    o += align16(4 * s.np);
  s.o_rank = o;  o += align16(4 * s.np);
  s.o_union = o;
  // union: merge keys (u16) | candidates + lists
  s.o_cand = o;  o += align16(2 * s.cand_cap);
  s.o_l0 = o;    o += align16(4 * p.k2);
  s.o_l1 = o;    o += align16(4 * p.k2);
  s.o_mid = o;   o += align16(4 * p.k2);
  int tail_end = o;
  const int merge_end = s.o_union + align16(2 * s.n_merge);
  s.merge_lds = merge_end <= 60 * 1024;
  if (s.merge_lds && merge_end > tail_end) tail_end = merge_end;
  s.lds_bytes = tile_end > tail_end ? tile_end : tail_end;
  const int rows = p.batch * p.hkv;
  int64_t w = 0;
  s.w_rowcnt = w; w += ((int64_t)4 * rows + 255) & ~(int64_t)255;
  s.w_reqcnt = w; w += ((int64_t)4 * p.batch + 255) & ~(int64_t)255;
  s.w_far = w;    w += (int64_t)8 * rows * s.ntiles * (p.k_f > 0 ? p.k_f : 1);
  s.w_near = w;   w += (int64_t)8 * rows * s.ntiles * (p.k_n > 0 ? p.k_n : 1);
  s.w_total = w;
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

__device__ __forceinline__ RowGeo row_geo(const NfaSelectParams &p, int L,
                                          bool skip_far, bool skip_near) {
  RowGeo g;
  const int bs = p.bs;
  const int pool_near_len = imax(bs, p.near_len);
  g.L = L;
  g.kt_eff = L > 0 ? (L + bs - 1) / bs : 0;
  g.spl = p.sink_tokens / bs;
  g.near_start = imax((L - p.geo_window - pool_near_len) / bs, g.spl);
  g.swa_lo_blk = imax(g.near_start, g.kt_eff - imax(1, p.geo_window / bs));
  g.far_end = imin(g.kt_eff, g.near_start);
  g.near_end = g.swa_lo_blk;
  g.far_on = !skip_far;
  g.near_on = !skip_near;
  g.sink_hi = imin(p.geo_sink, L);
  g.swa_hi = imax(g.sink_hi, L - p.geo_window);
  const int far_blk = (L - p.geo_window - p.geo_near) / p.page;
  g.orig_far_hi = imin(g.swa_hi, imax(g.sink_hi, far_blk * p.page));
  const int swa_lo_tok = imax(L - p.geo_window, 0);
  g.byp_blk = swa_lo_tok / bs;
  g.sink_unaligned = (p.geo_sink % bs) != 0;
  g.byp_cond = (swa_lo_tok % bs != 0) && (g.byp_blk >= g.spl);
  if (g.sink_unaligned) g.byp_cond = g.byp_cond && (g.byp_blk != g.spl);
  return g;
}

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
  return ((((req * p.hkv + kv) * (dsub / CH) + d / CH) * (int64_t)p.max_blocks +
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
  return (((int64_t)phys * p.hkv + kv) * p.page + off) * p.head_dim;
}

// ---------------------------------------------------------------------------
// page statistics of pages [pg_lo, pg_hi) for one (request, kv)
// ---------------------------------------------------------------------------

// The page's tokens are staged through LDS in sub-batches of kStatTokens
// (all loads of a sub-batch in flight at once); each (page, dim) thread then
// scans its tokens in ascending order: v < min, v > max, sum + v.
template <int DSUB, typename KV>
__device__ void compute_stats(const NfaSelectParams &p, int64_t req, int kv,
                              int L, int pg_lo, int pg_hi, float *s_stage,
                              const int *s_dims) {
  const KV *kpool = (const KV *)p.k_pool_l;
  const int32_t *bt = p.block_table_l + req * p.max_blocks;
  constexpr int PER = NFA_BLOCK / DSUB;  // pages per pass
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
        const int e = tid + k * NFA_BLOCK;  // [page slot][token][dim]
        const int dd = e % DSUB;
        const int ti = (e / DSUB) % kStatTokens;
        const int ps = e / (DSUB * kStatTokens);
        const int px = pg0 + ps;
        const int tok = px * p.bs + i0 + ti;
        const int lp = tok / p.page;
        float v = 0.0f;
        if (px < pg_hi && i0 + ti < p.bs && tok < L && lp < p.max_blocks) {
          const int phys = safe_page(p, bt[lp]);
          v = Elem<KV>::load(kpool + kv_offset(p, phys, kv, tok % p.page) +
                             s_dims[dd]);
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
      smin[si] = (KV)Elem<KV>::from_f32(mn);
      smax[si] = (KV)Elem<KV>::from_f32(mx);
      ssum[si] = (KV)Elem<KV>::from_f32(sm);
    }
  }
}

// Vector form for L1 dims made of aligned 16-byte runs: one item = (page,
// 16-byte chunk of dims); the chunk of 16 tokens is requested at once and
// each dim is then scanned over the tokens in ascending order.  ``s_coff``
// holds the element offset of every chunk, ``s_tphys`` (or NULL) the
// physical page of every page of the range when a page never straddles two
// physical pages.
template <int DSUB, typename KV>
__device__ void compute_stats_vec(const NfaSelectParams &p, int64_t req, int kv,
                                  int L, int pg_lo, int pg_hi,
                                  const int *s_coff, const int *s_tphys) {
  constexpr int CH = Elem<KV>::kChunk;
  constexpr int NCH1 = DSUB / CH;
  constexpr int TG = 16;
  const KV *kpool = (const KV *)p.k_pool_l;
  const int32_t *bt = p.block_table_l + req * p.max_blocks;
  KV *smin = (KV *)p.stat_min_l;
  KV *smax = (KV *)p.stat_max_l;
  KV *ssum = (KV *)p.stat_sum_l;
  const int n_items = (pg_hi - pg_lo) * NCH1;
  for (int it = threadIdx.x; it < n_items; it += NFA_BLOCK) {
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
          const int phys = s_tphys != nullptr ? s_tphys[pg - pg_lo]
                                              : safe_page(p, bt[lp]);
          raw[k] = *reinterpret_cast<const uint4 *>(
              kpool + kv_offset(p, phys, kv, tok % p.page) + s_coff[c]);
        }
      }
#pragma unroll
      for (int k = 0; k < TG; ++k) {
        if (!ok[k]) continue;
        float x[CH];
        load_chunk<KV>(reinterpret_cast<const KV *>(&raw[k]), x);
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
      smin[si + e] = (KV)Elem<KV>::from_f32(mn[e]);
      smax[si + e] = (KV)Elem<KV>::from_f32(mx[e]);
      ssum[si + e] = (KV)Elem<KV>::from_f32(sm[e]);
    }
  }
}

// ---------------------------------------------------------------------------
// L1 scores of one page for one kv group (selector:311-354)
// ---------------------------------------------------------------------------

constexpr int GMAX = 8;

template <int DSUB, typename KV>
__device__ __forceinline__ void l1_page_scores(const NfaSelectParams &p,
                                               int64_t req, int kv, int t,
                                               int G, const float *qf,
                                               bool need_mm, bool need_avg,
                                               uint16_t *mm_bits,
                                               uint16_t *avg_bits) {
  constexpr int CH = Elem<KV>::kChunk;
  const KV *smin = (const KV *)p.stat_min_l;
  const KV *smax = (const KV *)p.stat_max_l;
  const KV *ssum = (const KV *)p.stat_sum_l;
  float sneg[GMAX], spos[GMAX], savg[GMAX];
#pragma unroll
  for (int j = 0; j < GMAX; ++j) {
    sneg[j] = 0.0f;
    spos[j] = 0.0f;
    savg[j] = 0.0f;
  }
  const float inv_bs = (float)p.bs;
#pragma unroll
  for (int c = 0; c < DSUB / CH; ++c) {
    const int64_t base = stat_index<KV>(p, req, kv, c * CH, t, DSUB);
    float kmin[CH], kmax[CH], kavg[CH];
    if (need_mm) {
      load_chunk<KV>(smin + base, kmin);
      load_chunk<KV>(smax + base, kmax);
    }
    if (need_avg) {
      float ks[CH];
      load_chunk<KV>(ssum + base, ks);
#pragma unroll
      for (int e = 0; e < CH; ++e) kavg[e] = bf16r(ks[e] / inv_bs);
    }
#pragma unroll
    for (int e = 0; e < CH; ++e) {
      const int d = c * CH + e;
#pragma unroll
      for (int j = 0; j < GMAX; ++j) {
        if (j < G) {
          const float q = qf[j * DSUB + d];
          if (need_mm) {
            const float ql = q < 0.0f ? q : 0.0f;
            const float qh = q > 0.0f ? q : 0.0f;
            const float a = kmin[e] * ql;
            const float b = kmax[e] * qh;
            sneg[j] = sneg[j] + a;
            spos[j] = spos[j] + b;
          }
          if (need_avg) {
            const float a = kavg[e] * q;
            savg[j] = savg[j] + a;
          }
        }
      }
    }
  }
  float mm_acc = 0.0f, avg_acc = 0.0f;
#pragma unroll
  for (int j = 0; j < GMAX; ++j) {
    if (j < G) {
      mm_acc = mm_acc + bf16r(sneg[j] + spos[j]);
      avg_acc = avg_acc + bf16r(savg[j]);
    }
  }
  *mm_bits = bf16_bits(mm_acc / (float)G);
  *avg_bits = bf16_bits(avg_acc / (float)G);
}

// ---------------------------------------------------------------------------
// tile top-k: select the best K of the block's 256 keys (one per thread,
// 0 = invalid) and write them in thread (= page) order, padded with zeros.
// ---------------------------------------------------------------------------

__device__ void tile_topk(uint32_t key, int t, int K, uint64_t *out,
                          uint32_t *s_key, int *hist, int *tmp) {
  if (K <= 0) return;
  const int tid = threadIdx.x;
  s_key[tid] = key;
  __syncthreads();
  int *thr = tmp + 16;
  topk_threshold16([&](int i) { return s_key[i]; }, NFA_BLOCK, K, hist, tmp,
                   thr);
  const uint32_t T = (uint32_t)thr[0];
  const int need = thr[1];
  int tot;
  const bool eq = key != 0 && key == T;
  const int r_eq = block_count_exclusive(eq, tmp, &tot);
  const bool sel = key > T || (eq && r_eq < need);
  const int pos = block_count_exclusive(sel, tmp, &tot);
  if (sel && pos < K) out[pos] = ((uint64_t)key << 32) | (uint32_t)t;
  for (int i = tot + tid; i < K; i += NFA_BLOCK) out[i] = 0;
}

// ---------------------------------------------------------------------------
// tail: merge of tile lists into the sorted L1 top-K page list
// (selector:1766-1803 contract: valid pages by (score desc, page asc), then
// -inf pages by ascending index)
// ---------------------------------------------------------------------------

__device__ int merge_l1(const uint64_t *part, int n, int K, int *out_pages,
                        uint64_t *s_sel, uint16_t *s_m16, int *hist,
                        int *tmp) {
  const int tid = threadIdx.x;
  int *thr = tmp + 16;
  if (s_m16 != nullptr) {
    // stage the 16-bit score keys, four loads in flight per thread
    for (int i0 = tid; i0 < n; i0 += 4 * NFA_BLOCK) {
      uint64_t k[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int i = i0 + u * NFA_BLOCK;
        k[u] = i < n ? part[i] : 0ull;
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int i = i0 + u * NFA_BLOCK;
        if (i < n) s_m16[i] = (uint16_t)(k[u] >> 32);
      }
    }
    __syncthreads();
    topk_threshold16([&](int i) { return (uint32_t)s_m16[i]; }, n, K, hist,
                     tmp, thr);
  } else {
    topk_threshold16([&](int i) { return (uint32_t)(part[i] >> 32); }, n, K,
                     hist, tmp, thr);
  }
  const uint32_t T = (uint32_t)thr[0];
  const int need = thr[1];
  const int nvalid = thr[2] < K ? thr[2] : K;
  int carry_eq = 0, carry_sel = 0;
  for (int base = 0; base < n; base += NFA_BLOCK) {
    const int i = base + tid;
    uint32_t v = 0;
    if (i < n) v = s_m16 != nullptr ? (uint32_t)s_m16[i] : (uint32_t)(part[i] >> 32);
    const bool eq = v != 0 && v == T;
    int tot_eq, tot_sel;
    const int r_eq = block_count_exclusive(eq, tmp, &tot_eq) + carry_eq;
    const bool sel = v > T || (eq && r_eq < need);
    const int pos = block_count_exclusive(sel, tmp, &tot_sel) + carry_sel;
    if (sel && pos < K) ((int *)s_sel)[pos] = i;  // index now, key below
    carry_eq += tot_eq;
    carry_sel += tot_sel;
  }
  __syncthreads();
  {
    // fetch the selected keys: all loads in flight, no barrier in between
    int idx[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int pos = tid + u * NFA_BLOCK;
      idx[u] = pos < nvalid ? ((const int *)s_sel)[pos] : 0;
    }
    uint64_t key[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int pos = tid + u * NFA_BLOCK;
      key[u] = pos < nvalid ? part[idx[u]] : 0ull;
    }
    __syncthreads();
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int pos = tid + u * NFA_BLOCK;
      if (pos < nvalid) s_sel[pos] = key[u];
    }
    __syncthreads();
  }
  // order the selection by (score desc, page asc)
  for (int i = tid; i < nvalid; i += NFA_BLOCK) {
    const uint64_t ki = s_sel[i];
    const uint32_t vi = (uint32_t)(ki >> 32);
    const uint32_t ti = (uint32_t)ki;
    int rank = 0;
    for (int j = 0; j < nvalid; ++j) {
      const uint64_t kj = s_sel[j];
      const uint32_t vj = (uint32_t)(kj >> 32);
      const uint32_t tj = (uint32_t)kj;
      rank += (vj > vi) || (vj == vi && tj < ti);
    }
    out_pages[rank] = (int)ti;
  }
  __syncthreads();
  if (nvalid < K) {
    // -inf fillers: the lowest page indices that are not valid pages.
    // s_sel is reused to hold the valid pages sorted ascending as ints.
    int *vt = (int *)s_sel;
    int vtmp[4];
    int cnt = 0;
    for (int i = tid; i < nvalid && cnt < 4; i += NFA_BLOCK) {
      const int ti = out_pages[i];
      int rank = 0;
      for (int j = 0; j < nvalid; ++j) rank += out_pages[j] < ti;
      vtmp[cnt++] = rank;
    }
    __syncthreads();
    cnt = 0;
    for (int i = tid; i < nvalid && cnt < 4; i += NFA_BLOCK) {
      vt[vtmp[cnt++]] = out_pages[i];
    }
    __syncthreads();
    // boundary b[j] = vt[j] - j counts non-valid pages below vt[j]
    for (int i = tid; i < K - nvalid; i += NFA_BLOCK) {
      int lo = 0, hi = nvalid;
      while (lo < hi) {
        const int mid = (lo + hi) >> 1;
        if (vt[mid] - mid <= i)
          lo = mid + 1;
        else
          hi = mid;
      }
      out_pages[nvalid + i] = i + lo;
    }
    __syncthreads();
  }
  return nvalid;
}

// ---------------------------------------------------------------------------
// tail: L2 logits of the candidate tokens (selector:459-516).  One token per
// thread, the fp32 dot product runs over the L2 dims in order.  When the L2
// dims form aligned 16-byte runs (tail, rope, nope, full) each token's keys
// come in NCH vector loads with U tokens in flight per thread.
// ---------------------------------------------------------------------------

struct CandView {
  const int *pages;   // sorted unique candidate pages
  const int *pgoff;   // exclusive offsets, np_u + 1 entries
  int np_u;
  int tok_lo;         // first token of every page is max(page*bs, tok_lo)
  int bs;
  __device__ __forceinline__ int page_index(int i) const {
    return upper_bound_i32(pgoff, np_u + 1, i) - 1;
  }
  __device__ __forceinline__ int token_at(int pi, int i) const {
    const int first = pages[pi] * bs > tok_lo ? pages[pi] * bs : tok_lo;
    return first + (i - pgoff[pi]);
  }
  __device__ __forceinline__ int token(int i) const {
    return token_at(page_index(i), i);
  }
};

template <typename KV>
__device__ __forceinline__ uint16_t logit_key(const NfaSelectParams &p,
                                              float acc, int row, int i,
                                              int tok) {
  const uint16_t bits = bf16_bits(acc);
  if (p.dbg_cand_tok != nullptr && i < p.dbg_cand_cap) {
    p.dbg_cand_tok[(int64_t)row * p.dbg_cand_cap + i] = tok;
    p.dbg_cand_logit[(int64_t)row * p.dbg_cand_cap + i] =
        bits == kNanBits ? kNegInfBits : bits;
  }
  return bits == kNanBits ? 0 : (uint16_t)score_key(bits);
}

template <typename KV, int NCH>
__device__ void l2_logits_vec(const NfaSelectParams &p, const CandView &cv,
                              int n_cand, int kv, int row, const int *s_pphys,
                              const int *s_choff, const float *s_qg,
                              uint16_t *s_cand) {
  constexpr int CH = Elem<KV>::kChunk;
  constexpr int U = NCH <= 4 ? 4 : (NCH <= 8 ? 2 : 1);
  const KV *kpool = (const KV *)p.k_pool_l;
  const int32_t *bt = p.block_table_l + p.valid_req[row / p.hkv] * p.max_blocks;
  const bool page_phys = (p.page % p.bs) == 0;
  for (int i0 = threadIdx.x; i0 < n_cand; i0 += U * NFA_BLOCK) {
    uint4 raw[U][NCH];
    int tok[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int i = i0 + u * NFA_BLOCK;
      tok[u] = 0;
      if (i < n_cand) {
        const int pi = cv.page_index(i);
        tok[u] = cv.token_at(pi, i);
        const int phys =
            page_phys ? s_pphys[pi] : safe_page(p, bt[tok[u] / p.page]);
        const KV *kr = kpool + kv_offset(p, phys, kv, tok[u] % p.page);
#pragma unroll
        for (int c = 0; c < NCH; ++c)
          raw[u][c] = *reinterpret_cast<const uint4 *>(kr + s_choff[c]);
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int i = i0 + u * NFA_BLOCK;
      if (i < n_cand) {
        float acc = 0.0f;
#pragma unroll
        for (int c = 0; c < NCH; ++c) {
          float x[CH];
          load_chunk<KV>(reinterpret_cast<const KV *>(&raw[u][c]), x);
#pragma unroll
          for (int e = 0; e < CH; ++e) {
            const float prod = x[e] * s_qg[c * CH + e];
            acc = acc + prod;
          }
        }
        s_cand[i] = logit_key<KV>(p, acc, row, i, tok[u]);
      }
    }
  }
}

template <typename KV>
__device__ void l2_logits_scalar(const NfaSelectParams &p, const CandView &cv,
                                 int n_cand, int kv, int row,
                                 const int *s_pphys, const int *s_fdims,
                                 const float *s_qg, uint16_t *s_cand) {
  const KV *kpool = (const KV *)p.k_pool_l;
  const int32_t *bt = p.block_table_l + p.valid_req[row / p.hkv] * p.max_blocks;
  const bool page_phys = (p.page % p.bs) == 0;
  for (int i = threadIdx.x; i < n_cand; i += NFA_BLOCK) {
    const int pi = cv.page_index(i);
    const int tok = cv.token_at(pi, i);
    const int phys = page_phys ? s_pphys[pi] : safe_page(p, bt[tok / p.page]);
    const KV *kr = kpool + kv_offset(p, phys, kv, tok % p.page);
    float acc = 0.0f;
    for (int d0 = 0; d0 < p.fine_dsub; d0 += 8) {
      float x[8];
#pragma unroll
      for (int e = 0; e < 8; ++e)
        x[e] = d0 + e < p.fine_dsub ? Elem<KV>::load(kr + s_fdims[d0 + e]) : 0.0f;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        if (d0 + e < p.fine_dsub) {
          const float prod = x[e] * s_qg[d0 + e];
          acc = acc + prod;
        }
      }
    }
    s_cand[i] = logit_key<KV>(p, acc, row, i, tok);
  }
}

// ---------------------------------------------------------------------------
// tail: one L2 region -- top-quota of the candidates in index range [ia, ib),
// hole fill inside [rlo, rhi), sink filter; appended to s_mid at *mid_count.
// ---------------------------------------------------------------------------

__device__ void l2_region(const CandView &cv, const uint16_t *s_cand, int ia,
                          int ib, int rlo, int rhi, int quota, int sink,
                          int *s_l0, int *s_l1, int *s_mid, int *mid_count,
                          int *hist, int *tmp) {
  const int tid = threadIdx.x;
  if (quota <= 0) return;
  const int n = ib > ia ? ib - ia : 0;
  int *thr = tmp + 16;
  topk_threshold16([&](int i) { return (uint32_t)s_cand[ia + i]; }, n, quota,
                   hist, tmp, thr);
  const uint32_t T = (uint32_t)thr[0];
  const int need = thr[1];
  const int nvalid = thr[2];
  const int nch = nvalid < quota ? nvalid : quota;
  int carry_eq = 0, carry_sel = 0;
  for (int base = 0; base < n; base += NFA_BLOCK) {
    const int i = base + tid;
    const uint32_t v = i < n ? (uint32_t)s_cand[ia + i] : 0u;
    const bool eq = v != 0 && v == T;
    int tot_eq, tot_sel;
    const int r_eq = block_count_exclusive(eq, tmp, &tot_eq) + carry_eq;
    const bool sel = v > T || (eq && r_eq < need);
    const int pos = block_count_exclusive(sel, tmp, &tot_sel) + carry_sel;
    if (sel && pos < quota) s_l0[pos] = cv.token(ia + i);
    carry_eq += tot_eq;
    carry_sel += tot_sel;
  }
  __syncthreads();
  // hole fill: the (quota - nch) smallest ids of [rlo, rhi) not chosen
  const int nfill_req = quota - nch;
  for (int i = tid; i < nfill_req; i += NFA_BLOCK) {
    int lo = 0, hi = nch;
    while (lo < hi) {
      const int mid = (lo + hi) >> 1;
      if (s_l0[mid] - rlo - mid <= i)
        lo = mid + 1;
      else
        hi = mid;
    }
    const int id = rlo + i + lo;
    s_l1[i] = id < rhi ? id : 0x7FFFFFFF;
  }
  __syncthreads();
  // fill ids increase with i, so the valid ones form a prefix
  int nfill = 0;
  {
    int lo = 0, hi = nfill_req;
    while (lo < hi) {
      const int mid = (lo + hi) >> 1;
      if (s_l1[mid] != 0x7FFFFFFF)
        lo = mid + 1;
      else
        hi = mid;
    }
    nfill = lo;
  }
  const int drop = lower_bound_i32(s_l0, nch, sink) +
                   lower_bound_i32(s_l1, nfill, sink);
  const int base_out = *mid_count;
  for (int j = tid; j < nch; j += NFA_BLOCK) {
    const int v = s_l0[j];
    if (v >= sink) {
      const int pos = j + lower_bound_i32(s_l1, nfill, v) - drop;
      s_mid[base_out + pos] = v;
    }
  }
  for (int j = tid; j < nfill; j += NFA_BLOCK) {
    const int v = s_l1[j];
    if (v >= sink) {
      const int pos = j + lower_bound_i32(s_l0, nch, v) - drop;
      s_mid[base_out + pos] = v;
    }
  }
  __syncthreads();
  if (tid == 0) *mid_count = base_out + nch + nfill - drop;
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
  for (int d = threadIdx.x; d < p.head_dim; d += NFA_BLOCK)
    kp[kv_offset(p, phys, kv, off) + d] =
        kn[((int64_t)b * p.hkv + kv) * p.head_dim + d];
  for (int d = threadIdx.x; d < p.head_dim_v; d += NFA_BLOCK)
    vp[(((int64_t)phys * p.hkv + kv) * p.page + off) * p.head_dim_v + d] =
        vn[((int64_t)b * p.hkv + kv) * p.head_dim_v + d];
}

// Both regions skipped (region mode 3 / disjoint protected gather): decode
// write plus the union with an empty middle; no statistics are touched.
template <typename KV>
__global__ void __launch_bounds__(NFA_BLOCK)
    nfa_protected_kernel(const NfaSelectParams p) {
  const int row = blockIdx.x;
  const int b = row / p.hkv;
  const int kv = row % p.hkv;
  const int L = p.lengths[b];
  const bool active = p.active_req[b] >= 0;
  const int64_t req = p.valid_req[b];
  if (p.k_new != nullptr && active) decode_write<KV>(p, b, kv);
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
  for (int k = threadIdx.x; k < nu && k < p.max_vis; k += NFA_BLOCK) {
    const int x = k < (u1 - u0) ? u0 + k : u2 + (k - (u1 - u0));
    grow[k] = bt[x / p.page] * p.page + x % p.page;
  }
  if (threadIdx.x == 0) p.vis_lens[b * p.hkv + kv] = nu;
  if (p.dbg_counts != nullptr && threadIdx.x == 0) p.dbg_counts[row] = 0;
}

// ---------------------------------------------------------------------------
// the kernel
// ---------------------------------------------------------------------------

// Phase timestamp (debug timeline): completes the phase for the whole
// workgroup, then thread 0 stores the wall clock.  Uniform condition.
#define NFA_MARK(slot_base, k)                                        \
  do {                                                                \
    if (p.dbg_clock != nullptr) {                                     \
      __syncthreads();                                                \
      if (threadIdx.x == 0) p.dbg_clock[(slot_base) + (k)] = wall_clock64(); \
    }                                                                 \
  } while (0)

template <int DSUB, typename KV>
__global__ void __launch_bounds__(NFA_BLOCK)
    nfa_select_kernel(const NfaSelectParams p) {
  extern __shared__ __align__(16) unsigned char smem[];
  const SelDims sd = sel_dims(p);
  int *s_hist = (int *)(smem + sd.o_hist);
  int *s_tmp = (int *)(smem + sd.o_tmp);
  float *s_qf = (float *)(smem + sd.o_qf);
  uint32_t *s_key = (uint32_t *)(smem + sd.o_key);
  int *s_dims = (int *)(smem + sd.o_dims);
  float *s_stage = (float *)(smem + sd.o_stage);

  const int tid = threadIdx.x;
  const int tile = blockIdx.x;
  const int ntiles = gridDim.x;
  const int row = blockIdx.y;
  const int b = row / p.hkv;
  const int kv = row % p.hkv;
  const int G = p.hq / p.hkv;
  const int L = p.lengths[b];
  const bool active = p.active_req[b] >= 0;
  const int64_t req = p.valid_req[b];
  const bool skip_far = p.skip_far_l[req] != 0;
  const bool skip_near = p.skip_near_l[req] != 0;
  const int bs = p.bs;
  const int t0 = tile * NFA_BLOCK;
  // pages past the block-table width are never scored (selector:205-206)
  const int kt_eff = imin(L > 0 ? (L + bs - 1) / bs : 0, p.max_blocks);
  const int last_blk = L > 0 ? (L - 1) / bs : -1;
  const bool owns_last = last_blk >= t0 && last_blk < t0 + NFA_BLOCK &&
                         last_blk < p.max_blocks;

  const int64_t clk_tile = ((int64_t)row * (ntiles + 1) + tile) * 16;
  const int64_t clk_tail = ((int64_t)row * (ntiles + 1) + ntiles) * 16;
  NFA_MARK(clk_tile, 0);
  unsigned char *ws = (unsigned char *)p.workspace;
  unsigned int *row_cnt = (unsigned int *)(ws + sd.w_rowcnt);
  unsigned int *req_cnt = (unsigned int *)(ws + sd.w_reqcnt);
  uint64_t *part_far = (uint64_t *)(ws + sd.w_far);
  uint64_t *part_near = (uint64_t *)(ws + sd.w_near);

  // 1. decode write of the current token (selector:1030-1061)
  if (p.k_new != nullptr && active && owns_last) decode_write<KV>(p, b, kv);
  for (int i = tid; i < DSUB; i += NFA_BLOCK) s_dims[i] = p.dims[i];
  __syncthreads();

  NFA_MARK(clk_tile, 1);
  // 2. page statistics: latest page, or the whole tile on a rebuild
  const int prev = p.stats_len_l[req];
  const bool do_stats = active && L > 0 && !(skip_far && skip_near);
  const bool incremental = prev > 0 && L == prev + 1;
  if (do_stats && (!incremental || owns_last)) {
    const int pg_lo = incremental ? last_blk : t0;
    const int pg_hi = incremental ? last_blk + 1 : imin(t0 + NFA_BLOCK, kt_eff);
    // aligned 16-byte runs of L1 dims -> vector path
    constexpr int CH = Elem<KV>::kChunk;
    int *s_coff = (int *)s_stage;              // DSUB / CH chunk offsets
    int *s_tphys = s_coff + 32;                // physical page per page
    __shared__ int s_vec;
    if (tid == 0) {
      bool vec = true;
      for (int c = 0; vec && c < DSUB / CH; ++c) {
        const int first = s_dims[c * CH];
        vec = (first % CH) == 0;
        for (int e = 1; vec && e < CH; ++e) vec = s_dims[c * CH + e] == first + e;
        s_coff[c] = first;
      }
      s_vec = vec;
    }
    const bool page_phys = (p.page % bs) == 0;
    if (page_phys) {
      const int32_t *btr = p.block_table_l + req * p.max_blocks;
      for (int i = tid; i < pg_hi - pg_lo; i += NFA_BLOCK) {
        const int lp = imin(((pg_lo + i) * bs) / p.page, p.max_blocks - 1);
        s_tphys[i] = safe_page(p, btr[lp]);
      }
    }
    __syncthreads();
    if (s_vec) {
      compute_stats_vec<DSUB, KV>(p, req, kv, L, pg_lo, pg_hi, s_coff,
                                  page_phys ? s_tphys : nullptr);
    } else {
      __syncthreads();
      compute_stats<DSUB, KV>(p, req, kv, L, pg_lo, pg_hi, s_stage, s_dims);
    }
  }
  NFA_MARK(clk_tile, 2);

  // 3. scaled, bf16-rounded query rows of this kv group (selector:943-963)
  for (int i = tid; i < G * DSUB; i += NFA_BLOCK) {
    const int j = i / DSUB;
    const int d = i % DSUB;
    const int64_t qi = (int64_t)b * p.q_stride_b +
                       (int64_t)(kv * G + j) * p.q_stride_h + s_dims[d];
    const float qv = load_any(p.q, qi, p.q_dtype);
    s_qf[i] = bf16r(qv * p.scale);
  }
  __syncthreads();
  NFA_MARK(clk_tile, 3);

  // 4. L1 scores, one page per thread
  const RowGeo geo = row_geo(p, L, skip_far, skip_near);
  const int t = t0 + tid;
  uint16_t far_bits = kNegInfBits, near_bits = kNegInfBits;
  if (do_stats && t < kt_eff) {
    bool fp, np;
    pools(p, geo, t, &fp, &np);
    if (fp || np) {
      const bool far_mm = p.far_method == NFA_METHOD_MINMAX;
      const bool near_mm = p.near_method == NFA_METHOD_MINMAX;
      const bool need_mm = (fp && far_mm) || (np && near_mm);
      const bool need_avg = (fp && !far_mm) || (np && !near_mm);
      uint16_t mm, avg;
      l1_page_scores<DSUB, KV>(p, req, kv, t, G, s_qf, need_mm, need_avg, &mm,
                               &avg);
      if (fp) far_bits = far_mm ? mm : avg;
      if (np) near_bits = near_mm ? mm : avg;
    }
  }
  if (p.dbg_far != nullptr && t < kt_eff) {
    p.dbg_far[(int64_t)row * p.max_blocks + t] = far_bits;
    p.dbg_near[(int64_t)row * p.max_blocks + t] = near_bits;
  }

  NFA_MARK(clk_tile, 4);
  // 5. exact top-k of this tile
  tile_topk(score_key(far_bits), t, p.k_f,
            part_far + ((int64_t)row * ntiles + tile) * p.k_f, s_key, s_hist,
            s_tmp);
  tile_topk(score_key(near_bits), t, p.k_n,
            part_near + ((int64_t)row * ntiles + tile) * p.k_n, s_key, s_hist,
            s_tmp);

  NFA_MARK(clk_tile, 5);
  // 6. arrival; the last workgroup of the row runs the tail
  __syncthreads();
  if (tid == 0) {
    __threadfence();
    const unsigned int before = atomicAdd(&row_cnt[row], 1u);
    s_tmp[0] = before == (unsigned int)(ntiles - 1);
    const unsigned int rb = atomicAdd(&req_cnt[b], 1u);
    if (rb == (unsigned int)(ntiles * p.hkv - 1)) {
      // every workgroup of this request has read stats_len
      if (do_stats) p.stats_len_l[req] = L;
      atomicExch(&req_cnt[b], 0u);
    }
  }
  __syncthreads();
  if (!s_tmp[0]) return;
  __threadfence();
  if (tid == 0) atomicExch(&row_cnt[row], 0u);

  // =========================== tail stage ================================
  // (its LDS overlaps the tile stage's, which is no longer used)
  int *s_pages = (int *)(smem + sd.o_pages);
  int *s_pgoff = (int *)(smem + sd.o_pgoff);
  int *s_pphys = (int *)(smem + sd.o_pphys);
  uint16_t *s_cand = (uint16_t *)(smem + sd.o_cand);
  int *s_l0 = (int *)(smem + sd.o_l0);
  int *s_l1 = (int *)(smem + sd.o_l1);
  int *s_mid = (int *)(smem + sd.o_mid);
  uint64_t *s_sel = (uint64_t *)(smem + sd.o_sel);
  int *s_fp = (int *)(smem + sd.o_fp);
  int *s_np = (int *)(smem + sd.o_np);
  float *s_qg = (float *)(smem + sd.o_qg);
  int *s_choff = (int *)(smem + sd.o_choff);
  int *s_fdims = (int *)(smem + sd.o_fdims);
  uint16_t *s_m16 = sd.merge_lds ? (uint16_t *)(smem + sd.o_union) : nullptr;
  __shared__ int s_misc[8];
  __syncthreads();
  NFA_MARK(clk_tail, 0);

  const L2Bounds lb = l2_bounds(p, L, skip_far, skip_near, p.geo_near);
  if (p.dbg_bounds != nullptr && kv == 0 && tid == 0) {
    p.dbg_bounds[b * 3 + 0] = lb.lower;
    p.dbg_bounds[b * 3 + 1] = lb.upper;
    p.dbg_bounds[b * 3 + 2] = lb.quota;
  }

  // L1 merge (skipped pools give 0..K-1, which the filler rule reproduces)
  int nfv = 0, nnv = 0;
  if (p.k_f > 0)
    nfv = merge_l1(part_far + (int64_t)row * ntiles * p.k_f, ntiles * p.k_f,
                   p.k_f, s_fp, s_sel, s_m16, s_hist, s_tmp);
  if (p.k_n > 0)
    nnv = merge_l1(part_near + (int64_t)row * ntiles * p.k_n, ntiles * p.k_n,
                   p.k_n, s_np, s_sel, s_m16, s_hist, s_tmp);
  __syncthreads();
  NFA_MARK(clk_tail, 1);
  if (p.dbg_i_f != nullptr) {
    for (int i = tid; i < p.k_f; i += NFA_BLOCK)
      p.dbg_i_f[(int64_t)row * p.k_f + i] = s_fp[i];
    for (int i = tid; i < p.k_n; i += NFA_BLOCK)
      p.dbg_i_n[(int64_t)row * p.k_n + i] = s_np[i];
  }

  // candidate pages in slot order: far | near | sink bypass | SWA bypass
  const int spl = p.sink_tokens / bs;
  const bool byp0_keep = (p.sink_tokens % bs) != 0;
  bool byp1_keep = (lb.lo % bs != 0) && (lb.lo / bs >= spl);
  if (p.sink_tokens % bs != 0) byp1_keep = byp1_keep && (lb.lo / bs != spl);
  const int np_all = sd.np;
  auto slot_page = [&](int s) -> int {
    if (s < p.k_f) return s < nfv ? s_fp[s] : -1;
    s -= p.k_f;
    if (s < p.k_n) return s < nnv ? s_np[s] : -1;
    s -= p.k_n;
    if (s == 0) return byp0_keep ? spl : -1;
    return byp1_keep ? lb.lo / bs : -1;
  };
  // unique pages sorted ascending; candidates only exist when quota > 0
  const int tok_lo = imax(p.sink_tokens, lb.lower);
  const int tok_hi = imin(imin(lb.lo, L), lb.upper);
  int *s_sp = (int *)(smem + sd.o_sp);
  int *s_rank = (int *)(smem + sd.o_rank);
  for (int s = tid; s < np_all; s += NFA_BLOCK)
    s_sp[s] = lb.quota > 0 ? slot_page(s) : -1;
  __syncthreads();
  for (int s = tid; s < np_all; s += NFA_BLOCK) {
    const int pg = s_sp[s];
    bool first = pg >= 0;
    for (int j = 0; j < s && first; ++j) first = s_sp[j] != pg;
    s_rank[s] = first ? 0 : -1;
  }
  __syncthreads();
  int np_u;
  {
    int cnt = 0;
    for (int s = tid; s < np_all; s += NFA_BLOCK) {
      if (s_rank[s] < 0) continue;
      ++cnt;
    }
    block_scan_exclusive(cnt, s_tmp, &np_u);
  }
  for (int s = tid; s < np_all; s += NFA_BLOCK) {
    if (s_rank[s] < 0) continue;
    const int pg = s_sp[s];
    int r = 0;
    for (int j = 0; j < np_all; ++j) r += (s_rank[j] >= 0) && (s_sp[j] < pg);
    s_pages[r] = pg;
  }
  __syncthreads();
  // token counts per page and exclusive offsets
  int n_cand;
  {
    // np_u <= np_all; process in chunks of the block
    int carry = 0;
    for (int base = 0; base < np_u; base += NFA_BLOCK) {
      const int i = base + tid;
      int c = 0;
      if (i < np_u) {
        const int pg = s_pages[i];
        const int a = imax(pg * bs, tok_lo);
        const int e = imin(pg * bs + bs, tok_hi);
        c = e > a ? e - a : 0;
      }
      int tot;
      const int ex = block_scan_exclusive(c, s_tmp, &tot);
      if (i < np_u) s_pgoff[i] = carry + ex;
      carry += tot;
    }
    if (tid == 0) s_pgoff[np_u] = carry;
    n_cand = carry;
  }
  // pages that contribute no token keep offset == next offset; harmless
  __syncthreads();

  NFA_MARK(clk_tail, 2);
  // physical page of every candidate page (one lookup per page when a
  // statistics block never straddles a physical page)
  {
    const int32_t *btr = p.block_table_l + req * p.max_blocks;
    for (int i = tid; i < np_u; i += NFA_BLOCK) {
      const int lp = imin((s_pages[i] * bs) / p.page, p.max_blocks - 1);
      s_pphys[i] = safe_page(p, btr[lp]);
    }
  }
  // grouped query over the L2 dims (selector:979-1002)
  for (int d = tid; d < p.fine_dsub; d += NFA_BLOCK) {
    const int dim = p.fine_dims[d];
    s_fdims[d] = dim;
    float acc = 0.0f;
    for (int j = 0; j < G; ++j) {
      const int64_t qi = (int64_t)b * p.q_stride_b +
                         (int64_t)(kv * G + j) * p.q_stride_h + dim;
      acc = acc + bf16r(load_any(p.q, qi, p.q_dtype) * p.scale);
    }
    s_qg[d] = acc;
  }
  __syncthreads();
  // vector path when the L2 dims are aligned runs of 16 bytes
  constexpr int CH = Elem<KV>::kChunk;
  const int nch = p.fine_dsub / CH;
  if (tid == 0) {
    bool vec = (p.fine_dsub % CH == 0) && (nch == 4 || nch == 8 || nch == 16);
    for (int c = 0; vec && c < nch; ++c) {
      const int first = s_fdims[c * CH];
      vec = (first % CH) == 0;
      for (int e = 1; vec && e < CH; ++e) vec = s_fdims[c * CH + e] == first + e;
      s_choff[c] = first;
    }
    s_misc[1] = vec;
  }
  __syncthreads();

  NFA_MARK(clk_tail, 3);
  // L2 logits (selector:459-516)
  CandView cv{s_pages, s_pgoff, np_u, tok_lo, bs};
  if (s_misc[1]) {
    if (nch == 4)
      l2_logits_vec<KV, 4>(p, cv, n_cand, kv, row, s_pphys, s_choff, s_qg, s_cand);
    else if (nch == 8)
      l2_logits_vec<KV, 8>(p, cv, n_cand, kv, row, s_pphys, s_choff, s_qg, s_cand);
    else
      l2_logits_vec<KV, 16>(p, cv, n_cand, kv, row, s_pphys, s_choff, s_qg, s_cand);
  } else {
    l2_logits_scalar<KV>(p, cv, n_cand, kv, row, s_pphys, s_fdims, s_qg, s_cand);
  }
  if (p.dbg_cand_count != nullptr && tid == 0) p.dbg_cand_count[row] = n_cand;
  __syncthreads();

  NFA_MARK(clk_tail, 4);
  // L2 top-quota + hole fill (+ fixed near quota), selector:519-566, 873-940
  if (tid == 0) s_misc[0] = 0;
  __syncthreads();
  auto index_of_token = [&](int x) {  // first candidate index with token >= x
    int lo = 0, hi = n_cand;
    while (lo < hi) {
      const int mid = (lo + hi) >> 1;
      if (cv.token(mid) < x)
        lo = mid + 1;
      else
        hi = mid;
    }
    return lo;
  };
  if (lb.quota > 0) {
    if (p.near_tokens < 0) {
      l2_region(cv, s_cand, 0, n_cand, lb.lower, lb.upper, lb.quota,
                p.sink_tokens, s_l0, s_l1, s_mid, &s_misc[0], s_hist, s_tmp);
    } else {
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
      const int fa = index_of_token(far_low), fz = index_of_token(far_high);
      l2_region(cv, s_cand, fa, imax(fa, fz), far_low, far_high, far_quota,
                p.sink_tokens, s_l0, s_l1, s_mid, &s_misc[0], s_hist, s_tmp);
      const int na = index_of_token(near_low), nz = index_of_token(near_high);
      l2_region(cv, s_cand, na, imax(na, nz), near_low, near_high, near_quota,
                p.sink_tokens, s_l0, s_l1, s_mid, &s_misc[0], s_hist, s_tmp);
    }
  }
  __syncthreads();
  NFA_MARK(clk_tail, 5);
  int mcount = s_misc[0];
  if (mcount > p.k2) mcount = p.k2;
  if (p.dbg_middle != nullptr) {
    for (int i = tid; i < p.k2; i += NFA_BLOCK)
      p.dbg_middle[(int64_t)row * p.k2 + i] = i < mcount ? s_mid[i] : 0;
    if (tid == 0) p.dbg_counts[row] = mcount;
  }

  // final union with the protected sink/SWA ids (selector:1337-1437)
  const int32_t *bt = p.block_table_l + req * p.max_blocks;
  int32_t *grow = p.gather + ((int64_t)b * p.hkv + kv) * p.max_vis;
  auto phys_slot = [&](int id) {
    return bt[imin(id / p.page, p.max_blocks - 1)] * p.page + id % p.page;
  };
  if (p.middle_only) {
    const int n = imin(mcount, p.max_vis);
    for (int i = tid; i < n; i += NFA_BLOCK) grow[i] = phys_slot(s_mid[i]);
    if (tid == 0) p.vis_lens[b * p.hkv + kv] = n;
    return;
  }
  int u0, u1, u2, u3;
  protected_intervals(p, L, sd.prot, &u0, &u1, &u2, &u3);
  auto in_u = [&](int x) { return (x >= u0 && x < u1) || (x >= u2 && x < u3); };
  auto below_u = [&](int x) {  // |U ∩ [0, x)|
    return imax(0, imin(x, u1) - u0) + imax(0, imin(x, u3) - u2);
  };
  const int nu = (u1 - u0) + (u3 - u2);
  // middle entries inside U are duplicates; the rest keep their order.
  // Destinations first (barrier loop, LDS only), then one mapping pass.
  int carry = 0;
  for (int base = 0; base < mcount; base += NFA_BLOCK) {
    const int i = base + tid;
    const int x = i < mcount ? s_mid[i] : 0;
    const bool keep = i < mcount && !in_u(x);
    int tot;
    const int r = block_count_exclusive(keep, s_tmp, &tot) + carry;
    if (i < mcount) s_l0[i] = keep ? r + below_u(x) : -1;
    carry += tot;
  }
  const int nkeep = carry;
  __syncthreads();
  for (int i = tid; i < mcount; i += NFA_BLOCK) {
    const int dest = s_l0[i];
    if (dest >= 0 && dest < p.max_vis) grow[dest] = phys_slot(s_mid[i]);
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
  for (int k = tid; k < nu; k += NFA_BLOCK) {
    const int x = k < (u1 - u0) ? u0 + k : u2 + (k - (u1 - u0));
    const int dest = k + kept_below(x);
    if (dest < p.max_vis) grow[dest] = phys_slot(x);
  }
  if (tid == 0) p.vis_lens[b * p.hkv + kv] = nkeep + nu;
  NFA_MARK(clk_tail, 6);
}

}  // namespace nfa

// ---------------------------------------------------------------------------
// host entry
// ---------------------------------------------------------------------------

using nfa::SelDims;

static int select_check(const NfaSelectParams *p) {
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
  if (!(p->dsub == 32 || p->dsub == 64 || p->dsub == 128)) {
    nfa_set_error("nfa_select_layer: unsupported L1 dim count %d", p->dsub);
    return NFA_EINVAL;
  }
  if (p->fine_dsub <= 0 || p->fine_dsub > p->head_dim) {
    nfa_set_error("nfa_select_layer: bad L2 dim count %d", p->fine_dsub);
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
  const SelDims sd = nfa::sel_dims(*p);
  if (sd.lds_bytes > 64 * 1024) {
    nfa_set_error("nfa_select_layer: geometry needs %d bytes of LDS (> 64 KiB)",
                  sd.lds_bytes);
    return NFA_EINVAL;
  }
  if (p->workspace == nullptr || p->workspace_bytes < sd.w_total) {
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
  if (p->k_new != nullptr && (p->v_new == nullptr || p->slots == nullptr ||
                              p->v_pool_l == nullptr)) {
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
  return nfa::sel_dims(*p).w_total;
}

template <int DSUB, typename KV>
static hipError_t launch_select(const NfaSelectParams &p, hipStream_t stream) {
  const SelDims sd = nfa::sel_dims(p);
  dim3 grid(sd.ntiles, p.batch * p.hkv);
  hipLaunchKernelGGL((nfa::nfa_select_kernel<DSUB, KV>), grid, dim3(NFA_BLOCK),
                     sd.lds_bytes, stream, p);
  return hipGetLastError();
}

extern "C" int32_t nfa_select_layer(const NfaSelectParams *p, void *stream) {
  const int rc = select_check(p);
  if (rc != NFA_OK) return rc;
  hipStream_t s = (hipStream_t)stream;
  hipError_t err;
  const bool bf = p->kv_dtype == NFA_DTYPE_BF16;
  if (p->protected_only) {
    dim3 grid(p->batch * p->hkv);
    if (bf)
      hipLaunchKernelGGL(nfa::nfa_protected_kernel<uint16_t>, grid,
                         dim3(NFA_BLOCK), 0, s, *p);
    else
      hipLaunchKernelGGL(nfa::nfa_protected_kernel<float>, grid, dim3(NFA_BLOCK),
                         0, s, *p);
    err = hipGetLastError();
    if (err != hipSuccess) {
      nfa_set_error("nfa_select_layer: launch failed: %s", hipGetErrorString(err));
      return NFA_ELAUNCH;
    }
    return NFA_OK;
  }
  switch (p->dsub) {
    case 32:
      err = bf ? launch_select<32, uint16_t>(*p, s) : launch_select<32, float>(*p, s);
      break;
    case 64:
      err = bf ? launch_select<64, uint16_t>(*p, s) : launch_select<64, float>(*p, s);
      break;
    default:
      err = bf ? launch_select<128, uint16_t>(*p, s) : launch_select<128, float>(*p, s);
      break;
  }
  if (err != hipSuccess) {
    nfa_set_error("nfa_select_layer: launch failed: %s", hipGetErrorString(err));
    return NFA_ELAUNCH;
  }
  return NFA_OK;
}
