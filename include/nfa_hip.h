/*
 * nfa_hip.h -- C ABI of libnfa_hip.so, the MI355X (gfx950) implementation of
 * the NFA / LoDA-SA two-level sparse-attention decode path.
 *
 * Every entry point takes plain device pointers, sizes and a hipStream_t
 * (passed as void*), launches asynchronously on that stream, allocates no
 * memory and never synchronises, so calls can be captured into a hipGraph.
 * Outputs and persistent state live in caller-owned buffers.
 *
 * Return value: 0 on success, a negative NFA_E* code on a rejected argument
 * or a failed launch; nfa_last_error() then describes the problem.  Argument
 * checks run before any launch or KV mutation, as the reference's host checks
 * do before its kernels run.
 *
 * Reference interfaces replaced (Chosen-David/two-level-attention):
 *   nfa_select_layer        <- sparse_attn/indexer/nfa_layer_batch_selector.py:2649-2720
 *                              (select_topk_for_layer_batched; kernels :29-2028)
 *   nfa_sparse_attn_decode  <- sparse_attn/ops/paged_region_kernels.py:800-1006
 *                              (sparse_paged_attention_gather; kernel :251-363)
 *   nfa_sparse_attn_partial <- sparse_attn/ops/paged_region_kernels.py:727-780
 *   nfa_attn_regions_combine <- sparse_attn/ops/paged_region_kernels.py:783-797
 *   nfa_paged_write_decode  <- sparse_attn/ops/paged_region_kernels.py:665-724
 *   nfa_paged_write_prefill <- sparse_attn/ops/paged_region_kernels.py:610-662
 */
#ifndef NFA_HIP_H
#define NFA_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define NFA_ABI_VERSION 1

/* sizes the dbg_clock timeline: a selector workgroup scores at least this
   many pages, so a row has at most ceil(max_blocks / 64) tiles */
#define NFA_SELECT_CLOCK_PAGES 64

/* error codes */
#define NFA_OK 0
#define NFA_EINVAL (-1)    /* bad geometry / flags / pointer */
#define NFA_ELAUNCH (-2)   /* hipLaunch failed */
#define NFA_EWORKSPACE (-3) /* workspace too small */

/* dtypes of KV pools, queries and outputs */
#define NFA_DTYPE_BF16 0
#define NFA_DTYPE_F32 1

/* L1 score sources (--nfa_far_method / --nfa_near_method) */
#define NFA_METHOD_MINMAX 0
#define NFA_METHOD_AVG 1
#define NFA_METHOD_AVG_TOP2 2   /* far pool only: mean of the two largest
                                   per-head page means (needs a GQA group of
                                   at least 2) */

/*
 * One selector call over B batch rows for one layer.  Mirrors the arguments
 * of select_topk_for_layer_batched after its host-side geometry resolution
 * (selector:2762-2832).  Pointers with a _l suffix point at this layer's slice.
 */
typedef struct NfaSelectParams {
  int32_t abi_version;        /* = NFA_ABI_VERSION */
  int32_t struct_size;        /* = sizeof(NfaSelectParams) */

  /* geometry */
  int32_t batch;              /* B selector rows (visible bucket rows) */
  int32_t hq, hkv;            /* query heads, kv heads */
  int32_t head_dim, head_dim_v;
  int32_t bs;                 /* --tia_block_size (L1 statistics block) */
  int32_t page;               /* physical KV page size */
  int32_t max_blocks;         /* block-table width = kt_cap */
  int32_t max_req;            /* request slots */
  int32_t geo_sink, geo_near, geo_window;   /* RegionGeometry */
  int32_t sink_tokens, swa;   /* --nfa_sink_tokens, --nfa_swa_size */
  int32_t near_len;           /* --nfa_near_len */
  int32_t k_f, k_n;           /* far / near L1 page budgets */
  int32_t k2;                 /* --tia_level2_topk */
  int32_t near_tokens;        /* --nfa_near_tokens, -1 == off */
  int32_t far_method, near_method;
  int32_t dsub, fine_dsub;    /* number of L1 / L2 dims */
  int32_t kv_dtype, q_dtype;
  int32_t max_vis;            /* gather row width */
  int32_t middle_only;        /* write only the middle selection */
  int32_t pool_pages;         /* pages in the KV arena (P + 1); block-table
                                 entries outside [0, pool_pages) read the
                                 last (PAD) page */
  int32_t protected_only;     /* sink/SWA union with an empty middle only
                                 (both regions skipped); no statistics */
  float scale;                /* attention.scaling */
  int32_t l2_quant;           /* --nfa_l2_quant: L2 logits over 4-bit keys
                                 (min_max_per_token_quant, tia_indexer.py:
                                 22-31) from the packed side cache; needs
                                 l2_keys_l, 32 or 64 L2 dims and bf16 KV */
  int32_t kv_heads_mem;       /* kv heads of the KV arena, the statistics,
                                 the side cache, k_new and v_new: hkv (or 0,
                                 read as hkv), or 1
                                 when every selection row reads one shared
                                 arena head (an absorbed-MLA latent cache:
                                 hkv = hq selection rows of one query head
                                 each; only selection row 0 writes the
                                 shared state, and v_new may then be NULL:
                                 the values are part of the key rows) */

  /* cache state (device pointers) */
  void *k_pool_l, *v_pool_l;          /* [P+1,1,kv_heads_mem,page,D] of this layer */
  const int32_t *block_table_l;       /* [max_req, max_blocks] */
  const int32_t *lengths;             /* [batch] planned lengths */
  const int64_t *active_req;          /* [batch] request id or -1 */
  const int64_t *valid_req;           /* [batch] request id (PAD rows -> 0) */
  const int32_t *skip_far_l;          /* [max_req] */
  const int32_t *skip_near_l;         /* [max_req] */
  const int32_t *dims;                /* [dsub] */
  const int32_t *fine_dims;           /* [fine_dsub] */
  const void *q;                      /* [batch, hq, head_dim] rows */
  int64_t q_stride_b, q_stride_h;     /* element strides */

  /* decode write fused into the selector; k_new == NULL disables it */
  const void *k_new, *v_new;          /* [batch, kv_heads_mem, 1, D] contiguous */
  const int32_t *slots;               /* [batch] physical slot or -1 */

  /* persistent page statistics of this layer, KV dtype,
     [max_req, kv_heads_mem, dsub/chunk, max_blocks, chunk], chunk = 16B/elem:
     per page dim the min, the max and the mean bf16(KV(sum) / bs) (the avg
     pools' key; the fp32 running sum of the newest page is page_sum_l) */
  void *stat_min_l, *stat_max_l, *stat_sum_l;
  int32_t *stats_len_l;               /* [max_req] */
  /* optional L2 side copy of this layer, KV dtype: the L2 dims of every
     visible token in fine_dims order, [max_req, hkv, max_blocks * bs,
     fine_dsub]; valid with the statistics (written by the same rebuild and
     incremental update).  NULL: the L2 logits read the K pool.  With
     l2_quant: fine_dsub / 2 + 4 bytes per (request, kv head, token) slot
     instead -- the fine_dsub / 2 bytes of 4-bit codes of all slots (dim d in
     nibble d % 2 of byte d / 2), then the 4 bytes of (bf16 scale, bf16
     zero) of all slots, slot = (req * hkv + kv) * max_blocks * bs + token. */
  void *l2_keys_l;
  /* optional fp32 running sums of each request's last (partial) L1 page,
     [max_req, hkv, dsub], valid with the statistics: with them a decode step
     updates the last page's statistics from the new token alone.  NULL: the
     last page is re-read. */
  float *page_sum_l;

  /* outputs */
  int32_t *gather;                    /* [rows >= batch, hkv, max_vis] */
  int32_t *vis_lens;                  /* [rows >= batch, hkv] */

  /* scratch: nfa_select_workspace_bytes() bytes, zero-filled once; the
     kernels leave their counters and histograms at zero, so calls need no
     clearing in between.  Calls that share a workspace must not overlap. */
  void *workspace;
  int64_t workspace_bytes;

  /* optional intermediate outputs for parity tests (NULL = off) */
  uint16_t *dbg_far, *dbg_near;       /* [batch, hkv, max_blocks] bf16 bits */
  int32_t *dbg_i_f, *dbg_i_n;         /* [batch, hkv, k_f] / [.., k_n] */
  int32_t *dbg_middle, *dbg_counts;   /* [batch, hkv, k2] / [batch, hkv] */
  int64_t *dbg_bounds;                /* [batch, 3] lower, upper, quota */
  int32_t *dbg_cand_tok;              /* [batch, hkv, dbg_cand_cap] scored tokens */
  uint16_t *dbg_cand_logit;           /* their bf16 logit bits */
  int32_t *dbg_cand_count;            /* [batch, hkv] */
  int64_t dbg_cand_cap;
  int64_t *dbg_clock;                 /* [batch*hkv, ntiles + 1, 32] phase
                                         timestamps (wall clock), or NULL;
                                         ntiles = ceil(max_blocks /
                                         NFA_SELECT_CLOCK_PAGES): tile rows,
                                         then the tail row */
} NfaSelectParams;

typedef struct NfaAttnParams {
  int32_t abi_version;
  int32_t struct_size;
  int32_t total_q;            /* T query rows */
  int32_t hq, hkv, head_dim, head_dim_v, page;  /* K and V row widths, each
                                 8, 16, 24 or 32 chunks of 16 bytes (bf16:
                                 64/128/192/256 dims; fp32: 32 to 128) */
  int32_t gather_rows;        /* rows of gather / vis_lens */
  int32_t max_vis;
  int32_t kv_dtype, q_dtype;  /* output dtype == q dtype */
  int32_t tokens_per_split;   /* 0 = automatic */
  int32_t pool_pages;         /* pages in the KV arena; slots beyond are
                                 skipped like negative slots */
  float scale;
  float pad1;
  const void *q;              /* [T, hq, head_dim] contiguous */
  const void *k_pool, *v_pool;
  const int32_t *gather;      /* [gather_rows, hkv, max_vis] physical slots */
  const int32_t *vis_lens;    /* [gather_rows, hkv] */
  const int32_t *query_to_req;/* [T] */
  void *out;                  /* [T, hq, head_dim_v] */
  /* scratch: nfa_attn_workspace_bytes() bytes, zero-filled once; the kernel
     leaves its counters at zero, so calls need no clearing in between */
  void *workspace;
  int64_t workspace_bytes;
} NfaAttnParams;

/*
 * Absorbed multi-head latent attention decode (DeepSeek-V2 MLA): one latent
 * row per token, [kv_a_layernorm(c) (value_dim) | RoPE'd k_pe (latent_dim -
 * value_dim)], shared by every head (a KV arena of one kv head); each query
 * head attends over its own gather row (its selection, from nfa_select_layer
 * with kv_heads_mem 1 and one selection row per head).
 */
typedef struct NfaMlaAttnParams {
  int32_t abi_version;
  int32_t struct_size;
  int32_t total_q;            /* T query rows */
  int32_t heads;              /* query heads = gather rows per query row */
  int32_t latent_dim;         /* latent row width = value_dim + 64 */
  int32_t value_dim;          /* 64, 128, 256 or 512: the row's first dims */
  int32_t page;
  int32_t gather_rows;        /* rows of gather / vis_lens */
  int32_t max_vis;
  int32_t kv_dtype;           /* NFA_DTYPE_BF16 */
  int32_t q_dtype, out_dtype; /* NFA_DTYPE_BF16 or NFA_DTYPE_F32 */
  int32_t pool_pages;         /* pages in the arena; slots beyond are skipped */
  float scale;
  const void *q;              /* [T, heads, latent_dim]: per head
                                 [W_uk,h^T q_nope,h | q_pe,h] */
  const void *kv_pool;        /* [P+1, 1, 1, page, latent_dim] */
  const int32_t *gather;      /* [gather_rows, heads, max_vis] physical slots */
  const int32_t *vis_lens;    /* [gather_rows, heads] */
  const int32_t *query_to_req;/* [T] */
  const void *w_uv;           /* optional [heads, out_dim, value_dim] bf16: each
                                 head's value up-projection (kv_b_proj's value
                                 rows), applied to the head's result */
  int32_t out_dim;            /* rows of each head's w_uv (e.g. v_head_dim) */
  int32_t pad0;
  void *out;                  /* [T, heads, out_dim] = W_uv,h (sum_i p_i c_i)
                                 with w_uv, else [T, heads, value_dim] */
  void *workspace;            /* nfa_mla_attn_workspace_bytes(), zero-filled
                                 once; counters are left at zero */
  int64_t workspace_bytes;
} NfaMlaAttnParams;

/* Decode-step dense layers around the sparse attention (bf16 only). */
#define NFA_EPI_PLAIN 0      /* y_s = x W_s^T for each segment s */
#define NFA_EPI_RESIDUAL 1   /* y = residual + x W^T (one segment) */
#define NFA_EPI_SILU_GATE 2  /* y = silu(x W_gate^T) * (x W_up^T), segments
                                gate (0) and up (1) of equal rows */

typedef struct NfaLinearParams {
  int32_t abi_version;
  int32_t struct_size;
  int32_t m;                  /* activation rows (decode batch), 1..4 */
  int32_t k;                  /* input features, multiple of 8; m*k*2 <= 48 KiB */
  int32_t nseg;               /* weight segments sharing x, 1..3 */
  int32_t epilogue;           /* NFA_EPI_* */
  const void *x;              /* [m, k] bf16, rows x_stride elements apart */
  int64_t x_stride;
  const void *norm_weight;    /* [k] bf16, or NULL: when set, x is first
                                 RMS-normalised as HF's RMSNorm */
  float norm_eps;
  float pad0;
  const void *w[3];           /* [n_s, k] bf16 row-major (nn.Linear weight) */
  int32_t n[3];
  int32_t pad1;
  void *y[3];                 /* [m, n_s] bf16, rows y_stride[s] apart */
  int64_t y_stride[3];
  const void *residual;       /* [m, n_0] bf16 (NFA_EPI_RESIDUAL) */
  int64_t residual_stride;
} NfaLinearParams;

typedef struct NfaRopeParams {
  int32_t abi_version;
  int32_t struct_size;
  int32_t batch, hq, hkv, head_dim;
  const void *q;              /* [batch, hq*head_dim] bf16 rows (projection out) */
  int64_t q_stride_b;
  const void *k;              /* [batch, hkv*head_dim] bf16 rows */
  int64_t k_stride_b;
  const void *q_weight;       /* [head_dim] bf16 per-head RMSNorm weights, or */
  const void *k_weight;       /*   both NULL (no q/k norm, e.g. Llama) */
  float eps;
  float pad0;
  const void *cos, *sin;      /* [batch, head_dim] bf16 */
  int64_t cs_stride_b;
  void *q_out;                /* [batch, hq, head_dim] bf16 */
  void *k_out;                /* [batch, hkv, head_dim] bf16 */
} NfaRopeParams;

typedef struct NfaGateParams {
  int32_t abi_version;
  int32_t struct_size;
  int32_t hq, hkv, head_dim;  /* GQA group hq/hkv divides 64; head_dim <= 128 */
  int32_t length;             /* prompt tokens */
  int32_t rows;               /* profiled query rows: the last `rows` */
  int32_t sink, window, near, page;  /* RegionGeometry of the request */
  int32_t q_dtype;            /* q and k dtype: NFA_DTYPE_BF16 */
  float scale;
  int32_t pad0;
  const void *q;              /* [hq, length, head_dim] post-RoPE, strides in */
  int64_t q_stride_h, q_stride_l;  /* elements, head_dim contiguous */
  const void *k;              /* [hkv, length, head_dim] post-RoPE */
  int64_t k_stride_h, k_stride_l;
  float *out;                 /* [2, hq, rows] fp32: near mass, then far mass */
} NfaGateParams;

/* ABI / diagnostics */
int32_t nfa_abi_version(void);
int32_t nfa_gate_params_size(void);
int32_t nfa_linear_params_size(void);
int32_t nfa_rope_params_size(void);
int32_t nfa_wall_clock_khz(void);   /* rate of the dbg_clock timestamps */
int32_t nfa_select_params_size(void);
int32_t nfa_attn_params_size(void);
int32_t nfa_attn_partial_size(void);
int32_t nfa_attn_combine_params_size(void);
const char *nfa_last_error(void);

/* Scratch bytes a call with these parameters needs (0 on bad params). */
int64_t nfa_select_workspace_bytes(const NfaSelectParams *p);
int64_t nfa_attn_workspace_bytes(const NfaAttnParams *p);

/* A1-A9: decode write + page statistics + L1 + L2 + union for one layer. */
int32_t nfa_select_layer(const NfaSelectParams *p, void *stream);

/* No counterpart in the reference (its Triton launches have no instances to
   choose): diagnostics of the launch plan of nfa_select_layer for these
   parameters, for tests and benchmarks.  Writes up to n of: [0] kernel
   instance (0 single-pass tiles, 1 multi-pass tiles, 2 multi-pass tiles that
   list their top-K pages for the tail, -1 protected-only union), [1] tiles
   per row in one dispatch round, [2] grid tiles, [3] tiles of a row of
   max_blocks pages, [4] their passes, [5] LDS bytes per workgroup, [6] key
   segments of the tail, [7] workspace bytes (clamped to int32).  Launches
   nothing. */
int32_t nfa_select_plan(const NfaSelectParams *p, int32_t *out, int32_t n);

/* No counterpart in the reference.  nfa_select_layer for callers that cannot
   allocate device memory (code under hipGraph capture, tight serving loops,
   harnesses that forbid hipMalloc): the same kernels and results, but the
   scratch is a static device array of NFA_SELECT_SCRATCH_BYTES per GPU
   (held until the process ends) instead of p->workspace, which is ignored.
   Calls with more than NFA_SELECT_SCRATCH_ROWS rows (batch x kv heads), or
   whose page keys (2 bytes per page slot and row; 10 bytes plus 4 per tile
   when the block table can hold rows of more than 16384 pages, whose tiles
   then list their pages for the tail) do not fit beside the fixed counters
   and histograms, fail with NFA_EWORKSPACE.  The first call on a
   device takes the array's address and clears its counters (it synchronises
   the stream once and must not be captured); later calls allocate, clear
   and synchronise nothing.  All calls on one GPU share the array, so calls
   that overlap on one GPU race: serialise them (one stream, or events). */
#define NFA_SELECT_SCRATCH_BYTES (16 << 20)
#define NFA_SELECT_SCRATCH_ROWS 256
int32_t nfa_select_layer_noalloc(const NfaSelectParams *p, void *stream);

/* A10: sparse gather attention, out[t,h] = softmax(scale q k^T) v. */
int32_t nfa_sparse_attn_decode(const NfaAttnParams *p, void *stream);

/* No counterpart in the reference, whose DeepSeek-V2 and GLM patches expand
   the latent per head first (v1 tree sparse_attn/patches/
   deepseek_v2_attn_patch.py; sparse_attn/patches/glm4_moe_lite_attn_patch.py:
   36-59) and run sparse_paged_attention_gather on the expanded heads: the
   absorbed form of that attention over a latent arena, per head
   out_h = softmax(scale q_h K^T) K[:, :value_dim] over the head's gather
   row (equal to the expanded attention up to rounding). */
int32_t nfa_mla_attn_decode(const NfaMlaAttnParams *p, void *stream);
int64_t nfa_mla_attn_workspace_bytes(const NfaMlaAttnParams *p);
int32_t nfa_mla_attn_params_size(void);

/* Per-split online-softmax state of one region's gather attention. */
typedef struct NfaAttnPartial {
  int32_t abi_version;
  int32_t struct_size;
  int32_t nsplit;             /* splits per (query row, kv head), >= 1 */
  int32_t block_tokens;       /* split s of a row with n visible slots takes
                                 the blocks [s*nb/nsplit, (s+1)*nb/nsplit) of
                                 nb = ceil(n / block_tokens) blocks */
  float *acc;                 /* [nsplit, T, hq, head_dim_v]: sum_i e_i v_i */
  float *m;                   /* [nsplit, T, hq]: max score (-inf if none) */
  float *z;                   /* [nsplit, T, hq]: sum_i e_i, e_i = exp(s_i - m) */
} NfaAttnPartial;

/* Disjoint-region attention (protected and middle sets attended apart, then
   merged).  The partial replaces sparse_paged_attention_gather_partial,
   sparse_attn/ops/paged_region_kernels.py:727-780 (kernel :367-530 with
   WRITE_PARTIAL): p->out is unused, p->workspace holds
   nfa_attn_partial_workspace_bytes() bytes (zero-filled once, counters left
   at zero); padding rows store (0, -inf, 0).  The combine replaces
   sparse_paged_attention_regions_combine, :783-797 (kernel :533-575): the
   splits of region a, then those of region b, merge in split order. */
int32_t nfa_sparse_attn_partial(const NfaAttnParams *p, const NfaAttnPartial *pt,
                                void *stream);
int64_t nfa_attn_partial_workspace_bytes(const NfaAttnParams *p, const NfaAttnPartial *pt);

typedef struct NfaAttnCombineParams {
  int32_t abi_version;
  int32_t struct_size;
  int32_t total_q, hq, head_dim_v;
  int32_t out_dtype;          /* NFA_DTYPE_BF16 or NFA_DTYPE_F32 */
  int32_t nsplit_a, nsplit_b; /* splits of each region's state (0 = absent) */
  const float *acc_a, *m_a, *z_a;   /* NfaAttnPartial layouts */
  const float *acc_b, *m_b, *z_b;
  void *out;                  /* [T, hq, head_dim_v], acc / z (0 where z == 0) */
} NfaAttnCombineParams;

int32_t nfa_attn_regions_combine(const NfaAttnCombineParams *c, void *stream);

/* A11: one decode token per row; slot < 0 writes nothing.  head_dim_v 0
   writes the keys only (values and v_pool may be NULL), for a latent arena
   whose values are part of the key rows; the same holds for the prefill. */
int32_t nfa_paged_write_decode(const void *keys, const void *values,
                               const int32_t *slots, int32_t batch,
                               int32_t hkv, int32_t head_dim,
                               int32_t head_dim_v, int32_t page,
                               int32_t kv_dtype, void *k_pool, void *v_pool,
                               void *stream);

/* K13: prefill of n tokens of one request through its block-table row. */
int32_t nfa_paged_write_prefill(const void *keys, const void *values,
                                int64_t n, const int32_t *block_table_row,
                                int32_t hkv, int32_t head_dim,
                                int32_t head_dim_v, int32_t page,
                                int32_t kv_dtype, void *k_pool, void *v_pool,
                                void *stream);

/* Decode linear layer (batch <= 4) with optional RMSNorm prologue and a
   residual or SiLU-gate epilogue.  Replaces the decode-step projection
   chain of HF's Qwen3/Llama decoder layer that the reference runs as vendor
   GEMMs plus the fused RMSNorm of sparse_attn/ops/qwen3_rmsnorm_triton.py:
   240-300 and the SiLU*up of sparse_attn/ops/qwen3_mlp_silu_triton.py:
   102-130 (wired in by patches/qwen3_rmsnorm_patch.py:48 and
   patches/qwen3_mlp_silu_patch.py:59). */
int32_t nfa_decode_linear(const NfaLinearParams *p, void *stream);

/* Per-head q/k RMSNorm (optional) and rotate-half RoPE of one decode token
   per row.  Replaces qwen3_decode_rope, sparse_attn/ops/qwen3_rope_triton.py:
   118-160, together with the q_norm/k_norm calls before it
   (patches/qwen3_attn_patch.py:46-50). */
int32_t nfa_qk_norm_rope_decode(const NfaRopeParams *p, void *stream);

/* HF RMSNorm of `rows` rows of `dim` bf16 elements.  Replaces
   fused_rmsnorm_decode, sparse_attn/ops/qwen3_rmsnorm_triton.py:240-300. */
int32_t nfa_rmsnorm_decode(const void *x, int64_t x_stride, const void *weight,
                           void *out, int64_t out_stride, int32_t rows,
                           int32_t dim, float eps, void *stream);

/* Prefill region gate: per head and profiled row, the attention mass of
   the far and near regions (online softmax over keys 0..qlen-1).  Replaces
   fused_region_profile, sparse_attn/ops/frozen_gate_triton.py:84-111, behind
   profile_regions, sparse_attn/policies/frozen_gate.py:99-111. */
int32_t nfa_region_profile(const NfaGateParams *p, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* NFA_HIP_H */
