// Sparse gather decode attention over selected physical slots (gfx950).
//
// Reference: sparse_paged_attention_gather / _gather_attend_grouped_kernel,
// sparse_attn/ops/paged_region_kernels.py:251-363 and :800-1006.
//
// Grid nsplit x T * hkv (rows padded to a multiple of 8, one dimension, in
// an XCD-aware order), 256 threads.  Each workgroup owns one (query row,
// kv head) and the chunks split, split + nsplit, ... of at most 64 selected
// slots (one chunk per workgroup at decode widths; any visible width is
// covered with at most 256 workgroups per row), handles the G query heads of
// the group together (K/V rows are read once per group), and writes an
// online-softmax partial (m, z, acc).  The last workgroup of
// the (row, kv) to arrive -- device-scope atomic counter, no waiting --
// merges the partials and writes the output in the query dtype.
//
// Row layout: kTpr = 8 threads share a K/V row, each holding CK 16-byte
// chunks of the K row and CV of the V row (K and V widths are independent:
// 64 to 256 dims, e.g. 192 / 128 for DeepSeek-V2's expanded heads), so a
// pass of the 256 threads covers 32 rows and every K and V chunk of the
// split is requested before the first one is used.  Scores reduce over the
// 8 threads with lane shuffles; V rows are staged in LDS and P.V runs with
// one thread per (head, dim pair).  All loops are rolled or short: the code
// a workgroup executes stays a few KB, so instruction fetch does not become
// the latency of the launch.
#include "nfa_common.h"

namespace nfa {

constexpr int AGMAX = 8;         // query heads per kv head
constexpr int kTpr = 8;          // threads per K/V row
constexpr int kXcds = 8;         // XCDs of the device (MI355X), for the block order
constexpr int kSplitMax = 64;    // tokens per workgroup
constexpr int kMaxSplits = 256;  // splits merged in LDS

struct AttnDims {
  int split;    // tokens per split
  int nsplit;
  int rows;     // T * hkv
  int64_t w_cnt, w_part, w_total;
  int part_stride;  // floats per (row, split): G * (DV + 2)
};

// `cus`: compute units of the device.  Rows get as many split workgroups as
// keep about four workgroups per CU busy (every split workgroup costs a
// partial write and an arrival; a row with one split writes its output
// directly): a workgroup's chunks run one after another, each a chain of
// scores, softmax and P.V with its barriers, which the other workgroups of
// the CU overlap (16 ragged requests: 28.7 us at two per CU, 25.8 at three,
// 23.6 at four, 24.9 at five).
// `mult` caller splits per (query row, kv head), each spanning at most
// `span` slots (1 and max_vis for the plain decode call).
__host__ __device__ inline AttnDims attn_dims(const NfaAttnParams &p, int cus,
                                              int mult = 1, int span = -1) {
  AttnDims a;
  a.rows = p.total_q * p.hkv * mult;
  int split = p.tokens_per_split;
  if (split <= 0) split = kSplitMax;  // fewer, longer splits: a cheaper merge
  a.split = split;
  const int G = p.hq / p.hkv;
  // at most kMaxSplits workgroups per row; a workgroup takes every
  // nsplit-th chunk of the row
  int cap = kMaxSplits;
  const int want = a.rows > 0 ? (4 * cus + a.rows - 1) / a.rows : 1;
  if (want < cap) cap = want;
  a.nsplit = ((span >= 0 ? span : p.max_vis) + split - 1) / split;
  if (a.nsplit > cap) a.nsplit = cap;
  if (a.nsplit < 1) a.nsplit = 1;
  a.part_stride = G * (p.head_dim_v + 2);
  int64_t w = 0;
  a.w_cnt = w;  w += ((int64_t)4 * kArriveStride * a.rows + 255) & ~(int64_t)255;
  a.w_part = w; w += (int64_t)4 * a.rows * a.nsplit * a.part_stride;
  a.w_total = w;
  return a;
}

// Most slots one caller split of a partial call can hold: ceil(nb / nsplit)
// blocks of the nb = ceil(max_vis / block_tokens).
__host__ __device__ inline int part_span(const NfaAttnParams &p, const NfaAttnPartial &pt) {
  const int nb = (p.max_vis + pt.block_tokens - 1) / pt.block_tokens;
  const int64_t span = (int64_t)((nb + pt.nsplit - 1) / pt.nsplit) * pt.block_tokens;
  return span < p.max_vis ? (int)span : p.max_vis;
}

// Two adjacent KV elements of an LDS row as floats.
__device__ __forceinline__ void lds_pair(const uint16_t *v, int d, float *a,
                                         float *b) {
  const uint32_t x = *reinterpret_cast<const uint32_t *>(v + d);
  *a = __uint_as_float(x << 16);
  *b = __uint_as_float(x & 0xFFFF0000u);
}
__device__ __forceinline__ void lds_pair(const float *v, int d, float *a,
                                         float *b) {
  const float2 x = *reinterpret_cast<const float2 *>(v + d);
  *a = x.x;
  *b = x.y;
}

// LOOP: a workgroup may own several chunks (rows wider than nsplit chunks);
// without it every workgroup owns at most one and nothing is carried.
// PART: grid row y is (query row, kv head, caller split cs) and covers the
// caller's split -- blocks [cs * nb / nsplit, (cs + 1) * nb / nsplit) of the
// row's nb = ceil(n / block_tokens) token blocks -- with its own chunks and
// split workgroups; the merge stores the unnormalised state (acc, m, z)
// into the caller's buffers instead of the output.
template <typename KV, int CK, int CV, bool LOOP, bool PART = false>
__global__ void __launch_bounds__(NFA_BLOCK)
    nfa_attn_kernel(const NfaAttnParams p, int cus, const NfaAttnPartial pt) {
  constexpr int CH = Elem<KV>::kChunk;  // dims per 16-byte chunk
  constexpr int DK = kTpr * CK * CH;    // K head dim
  constexpr int D = kTpr * CV * CH;     // V head dim
  constexpr int RPP = NFA_BLOCK / kTpr; // rows per pass
  constexpr int PMAX = kSplitMax / RPP; // passes per split
  const AttnDims ad = PART ? attn_dims(p, cus, pt.nsplit, part_span(p, pt))
                           : attn_dims(p, cus);
  const int tid = threadIdx.x;
  const int lane = lane_id();
  const int w = wave_id();
  // XCD-aware order: workgroups are dispatched round-robin over the XCDs
  // in linear id order, so ids congruent mod kXcds share an XCD (and its
  // L2).  Rows go in groups of kXcds, row r of a group taking the ids
  // congruent to r: all splits of a row run on one XCD, and the merge reads
  // their partials from that XCD's L2.  Rows past the last one (the padding
  // of the final group) exit at once.
  const int linear = blockIdx.x;
  const int group = linear / (kXcds * ad.nsplit);
  const int within = linear % (kXcds * ad.nsplit);
  const int vrow = group * kXcds + within % kXcds;  // arrival counter and staging row
  const int split = within / kXcds;
  if (vrow >= ad.rows) return;
  const int row = PART ? vrow / pt.nsplit : vrow;
  const int cs = PART ? vrow % pt.nsplit : 0;
  const int t = row / p.hkv;
  const int kh = row % p.hkv;
  const int G = p.hq / p.hkv;
  const float kNegInf = __uint_as_float(0xFF800000u);

  __shared__ __align__(16) float s_q[AGMAX * DK];
  __shared__ __align__(16) float s_p[AGMAX * kSplitMax];  // scores, then exp weights
  __shared__ int s_slot[kSplitMax];
  __shared__ __align__(16) KV s_v[kSplitMax * D];
  __shared__ float s_m[AGMAX], s_z[AGMAX], s_f[AGMAX];
  __shared__ int s_last;

  unsigned char *ws = (unsigned char *)p.workspace;
  unsigned int *cnt = (unsigned int *)(ws + ad.w_cnt);
  float *part = (float *)(ws + ad.w_part) +
                ((int64_t)vrow * ad.nsplit + split) * ad.part_stride;

  // the query rows of the group, requested first (they depend on nothing;
  // stored to LDS once the row's metadata is in)
  constexpr int QPT = (AGMAX * DK + NFA_BLOCK - 1) / NFA_BLOCK;
  float qv[QPT];
#pragma unroll
  for (int k = 0; k < QPT; ++k) {
    const int i = tid + k * NFA_BLOCK;
    qv[k] = i < G * DK ? load_any(p.q, ((int64_t)t * p.hq + kh * G) * DK + i, p.q_dtype)
                       : 0.0f;
  }
  // Query row t usually reads gather row t (query_to_req is the identity at
  // decode): that row's visible length and this thread's slot of the first
  // chunk are loaded together with query_to_req, and used when it agrees,
  // instead of three dependent round trips.
  const int spec = !PART && t < p.gather_rows ? t : -1;
  const int spec_i = split * ad.split + tid;  // first chunk's slot of this thread
  int spec_n = 0, spec_slot = -1;
  if (spec >= 0) {
    spec_n = p.vis_lens[spec * p.hkv + kh];
    if (tid < ad.split && spec_i < p.max_vis)
      spec_slot = p.gather[((int64_t)spec * p.hkv + kh) * p.max_vis + spec_i];
  }
  int req = p.query_to_req[t];
  if (req >= p.gather_rows) req = -1;  // out-of-range rows act as padding
  const bool spec_ok = spec >= 0 && req == spec;
  int n = 0;
  if (req >= 0) {
    n = spec_ok ? spec_n : p.vis_lens[req * p.hkv + kh];
    if (n > p.max_vis) n = p.max_vis;
  }
  // chunks split, split + nsplit, ... of ad.split slots each; the running
  // (max, denominator, P.V) of the workgroup carries from chunk to chunk
  int lo = 0, c_end = n;
  if constexpr (PART) {
    // the caller's split of the row
    const int bt = pt.block_tokens;
    const int nb = (n + bt - 1) / bt;
    lo = (int)((int64_t)cs * nb / pt.nsplit) * bt;
    const int b_end = (int)((int64_t)(cs + 1) * nb / pt.nsplit);
    c_end = b_end * bt < n ? b_end * bt : n;
  }
  const int c_first = lo + split * ad.split;
  const int c_step = ad.nsplit * ad.split;
  if (c_first < c_end) {
#pragma unroll
    for (int k = 0; k < QPT; ++k) {
      const int i = tid + k * NFA_BLOCK;
      if (i < G * DK) s_q[i] = qv[k];
    }
  }
  if (tid < G) {
    s_m[tid] = kNegInf;
    s_z[tid] = 0.0f;
  }
  constexpr int OPT = (AGMAX * (D / 2) + NFA_BLOCK - 1) / NFA_BLOCK;  // outputs per thread
  float acc0[OPT], acc1[OPT];
#pragma unroll
  for (int k = 0; k < OPT; ++k) acc0[k] = acc1[k] = 0.0f;

  const int32_t *grow = req >= 0 ? p.gather + ((int64_t)req * p.hkv + kh) * p.max_vis
                                 : nullptr;
  // slots outside the arena are skipped like negative ones
  const int max_slot = p.pool_pages * p.page;
  const int sc = tid % kTpr;  // this thread's chunks of the row: sc, sc + 8, ...
  const int rr = tid / kTpr;  // row within a pass
  const KV *kpool = (const KV *)p.k_pool;
  const KV *vpool = (const KV *)p.v_pool;
  for (int c0 = c_first; c0 < c_end; c0 += c_step) {
    const int cn = c_end - c0 < ad.split ? c_end - c0 : ad.split;
    if (LOOP && c0 != c_first) __syncthreads();  // the previous chunk's readers are done
    for (int i = tid; i < cn; i += NFA_BLOCK) {
      const int sl = spec_ok && c0 == c_first ? spec_slot : grow[c0 + i];
      s_slot[i] = sl < max_slot ? sl : -1;
    }
    __syncthreads();

    // every K and V chunk of the split in flight at once
    uint4 kr[PMAX][CK], vr[PMAX][CV];
#pragma unroll
    for (int pp = 0; pp < PMAX; ++pp) {
      const int j = pp * RPP + rr;
      const int slot = j < cn ? s_slot[j] : -1;
#pragma unroll
      for (int c = 0; c < CK; ++c) kr[pp][c] = make_uint4(0u, 0u, 0u, 0u);
#pragma unroll
      for (int c = 0; c < CV; ++c) vr[pp][c] = make_uint4(0u, 0u, 0u, 0u);
      if (slot >= 0) {
        const int64_t cell = ((int64_t)(slot / p.page) * p.hkv + kh) * p.page + slot % p.page;
#pragma unroll
        for (int c = 0; c < CK; ++c)
          kr[pp][c] = *reinterpret_cast<const uint4 *>(kpool + cell * DK + (c * kTpr + sc) * CH);
#pragma unroll
        for (int c = 0; c < CV; ++c)
          vr[pp][c] = *reinterpret_cast<const uint4 *>(vpool + cell * D + (c * kTpr + sc) * CH);
      }
    }
    // scores: partial dot over the thread's chunks, then a shuffle
    // reduction over the 8 threads of the row
#pragma unroll
    for (int pp = 0; pp < PMAX; ++pp) {
      if (pp * RPP >= cn) break;
      const int j = pp * RPP + rr;
      float x[CK][CH];
#pragma unroll
      for (int c = 0; c < CK; ++c) unpack_chunk<KV>(kr[pp][c], x[c]);
      for (int g = 0; g < G; ++g) {
        float part_s = 0.0f;
#pragma unroll
        for (int c = 0; c < CK; ++c) {
          const float *q = s_q + g * DK + (c * kTpr + sc) * CH;
#pragma unroll
          for (int e = 0; e < CH; ++e) part_s = fmaf(q[e], x[c][e], part_s);
        }
        part_s = sum8(part_s);  // the 8 threads of the row (kTpr == 8)
        if (sc == 0 && j < cn)
          s_p[g * kSplitMax + j] = s_slot[j] >= 0 ? part_s * p.scale : kNegInf;
      }
    }
    // stage V rows for P.V
#pragma unroll
    for (int pp = 0; pp < PMAX; ++pp) {
      const int j = pp * RPP + rr;
      if (j < cn) {
#pragma unroll
        for (int c = 0; c < CV; ++c)
          *reinterpret_cast<uint4 *>(s_v + j * D + (c * kTpr + sc) * CH) = vr[pp][c];
      }
    }
    __syncthreads();

    // online softmax per head (one wave per head): new running max, the
    // factor for what was accumulated so far, weights of this chunk
    for (int g = w; g < G; g += NFA_WAVES) {
      // one score per lane (a chunk holds at most 64 = kSplitMax slots)
      const float sl = lane < cn ? s_p[g * kSplitMax + lane] : kNegInf;
      const float m = wave_max_dpp(sl);
      const float m_old = s_m[g];
      const float m_new = fmaxf(m_old, m);
      const float e = (m_new == kNegInf || lane >= cn) ? 0.0f : __expf(sl - m_new);
      if (lane < cn) s_p[g * kSplitMax + lane] = e;
      const float z = wave_sum_dpp(e);
      if (lane == 0) {
        const float f = m_old == kNegInf ? 0.0f : __expf(m_old - m_new);
        s_f[g] = f;
        s_m[g] = m_new;
        s_z[g] = s_z[g] * f + z;
      }
    }
    __syncthreads();

    // P.V, one thread per (head, dim pair)
#pragma unroll
    for (int k = 0; k < OPT; ++k) {
      const int o = tid + k * NFA_BLOCK;
      if (o >= G * (D / 2)) break;
      const int g = o / (D / 2);
      const int d = 2 * (o % (D / 2));
      const float f = LOOP ? s_f[g] : 0.0f;
      // four weights per 16-byte LDS read, two independent chains per output
      // (weights past cn are 0 and their V rows are never staged: skipped)
      float a0 = 0.0f, a1 = 0.0f, b0 = 0.0f, b1 = 0.0f;
      const float4 *pw = reinterpret_cast<const float4 *>(s_p + g * kSplitMax);
      if (cn == kSplitMax) {
        // a full chunk: sixteen slots' weights and V pairs requested before
        // their multiply-adds (one LDS round trip per sixteen slots, not per
        // four), the same two chains in the same order as below
#pragma unroll
        for (int j0 = 0; j0 < kSplitMax; j0 += 16) {
          float4 w4[4];
          float va[16], vb[16];
#pragma unroll
          for (int u = 0; u < 4; ++u) w4[u] = pw[j0 / 4 + u];
#pragma unroll
          for (int u = 0; u < 16; ++u) lds_pair(s_v + (j0 + u) * D, d, &va[u], &vb[u]);
#pragma unroll
          for (int u = 0; u < 4; ++u) {
            a0 = fmaf(w4[u].x, va[4 * u], a0);
            a1 = fmaf(w4[u].x, vb[4 * u], a1);
            b0 = fmaf(w4[u].y, va[4 * u + 1], b0);
            b1 = fmaf(w4[u].y, vb[4 * u + 1], b1);
            a0 = fmaf(w4[u].z, va[4 * u + 2], a0);
            a1 = fmaf(w4[u].z, vb[4 * u + 2], a1);
            b0 = fmaf(w4[u].w, va[4 * u + 3], b0);
            b1 = fmaf(w4[u].w, vb[4 * u + 3], b1);
          }
        }
      } else
      for (int j = 0; j < cn; j += 4) {
        const float4 w4 = pw[j / 4];
        float v0, v1, u0, u1;
        lds_pair(s_v + j * D, d, &v0, &v1);
        a0 = fmaf(w4.x, v0, a0);
        a1 = fmaf(w4.x, v1, a1);
        if (j + 1 < cn) {
          lds_pair(s_v + (j + 1) * D, d, &u0, &u1);
          b0 = fmaf(w4.y, u0, b0);
          b1 = fmaf(w4.y, u1, b1);
        }
        if (j + 2 < cn) {
          lds_pair(s_v + (j + 2) * D, d, &v0, &v1);
          a0 = fmaf(w4.z, v0, a0);
          a1 = fmaf(w4.z, v1, a1);
        }
        if (j + 3 < cn) {
          lds_pair(s_v + (j + 3) * D, d, &u0, &u1);
          b0 = fmaf(w4.w, u0, b0);
          b1 = fmaf(w4.w, u1, b1);
        }
      }
      a0 = a0 + b0;
      a1 = a1 + b1;
      if (LOOP) {
        acc0[k] = acc0[k] * f + a0;
        acc1[k] = acc1[k] * f + a1;
      } else {
        store_coherent(&part[g * (D + 2) + 2 + d], a0);
        store_coherent(&part[g * (D + 2) + 3 + d], a1);
      }
    }
    if (!LOOP) break;
  }
  // s_m / s_z of a head were last written before the barrier that precedes
  // the P.V step (or, with no chunk, by the same thread that reads them)
  // caller state [cs][t][head]; acc rows of head_dim_v floats
  const int64_t pb = ((int64_t)cs * p.total_q + t) * p.hq + kh * G;
  if (PART && LOOP && ad.nsplit == 1) {
    // the whole caller split in this workgroup: its state as accumulated
#pragma unroll
    for (int k = 0; k < OPT; ++k) {
      const int o = tid + k * NFA_BLOCK;
      if (o >= G * (D / 2)) break;
      const int g = o / (D / 2);
      const int d = 2 * (o % (D / 2));
      pt.acc[(pb + g) * D + d] = acc0[k];
      pt.acc[(pb + g) * D + d + 1] = acc1[k];
    }
    if (tid < G) {
      pt.m[pb + tid] = s_m[tid];
      pt.z[pb + tid] = s_z[tid];
    }
    return;
  }
  if (LOOP && ad.nsplit == 1) {
    // the whole row in this workgroup: normalise and write the output
#pragma unroll
    for (int k = 0; k < OPT; ++k) {
      const int o = tid + k * NFA_BLOCK;
      if (o >= G * (D / 2)) break;
      const int g = o / (D / 2);
      const int d = 2 * (o % (D / 2));
      const float z = s_z[g];
      const float o0 = z == 0.0f ? 0.0f : acc0[k] / z;
      const float o1 = z == 0.0f ? 0.0f : acc1[k] / z;
      const int64_t oi = ((int64_t)t * p.hq + kh * G + g) * D + d;
      if (p.q_dtype == NFA_DTYPE_BF16) {
        ((uint16_t *)p.out)[oi] = bf16_bits(o0);
        ((uint16_t *)p.out)[oi + 1] = bf16_bits(o1);
      } else {
        ((float *)p.out)[oi] = o0;
        ((float *)p.out)[oi + 1] = o1;
      }
    }
    return;
  }
  // (a single-chunk workgroup stored its P.V above; one with no chunk
  // stores zeros here)
  const bool store_acc = LOOP || c_first >= c_end;
#pragma unroll
  for (int k = 0; k < OPT; ++k) {
    const int o = tid + k * NFA_BLOCK;
    if (!store_acc || o >= G * (D / 2)) break;
    const int g = o / (D / 2);
    const int d = 2 * (o % (D / 2));
    store_coherent(&part[g * (D + 2) + 2 + d], acc0[k]);
    store_coherent(&part[g * (D + 2) + 3 + d], acc1[k]);
  }
  if (tid < G) {
    store_coherent(&part[tid * (D + 2) + 0], s_m[tid]);
    store_coherent(&part[tid * (D + 2) + 1], s_z[tid]);
  }

  // arrival; the last split of the (row, kv) merges (the partials went out
  // through coherent stores: no L2 writeback)
  if (!arrive_last(&cnt[vrow * kArriveStride], (unsigned int)ad.nsplit, &s_last, false)) return;

  const float *base = (const float *)(ws + ad.w_part) +
                      (int64_t)vrow * ad.nsplit * ad.part_stride;
  // two adjacent outputs per thread; each split's (max, denominator, P.V
  // pair) for them requested in one round (they come from the other split
  // workgroups of this row, through this XCD's L2), merged as a stream:
  // rescale what is held to the new maximum, add the batch
  const int ns = ad.nsplit;
  constexpr int kMergeBatch = 16;
  for (int i = tid; i < G * (D / 2); i += NFA_BLOCK) {
    const int g = i / (D / 2), d = 2 * (i % (D / 2));
    const float *pg = base + g * (D + 2);
    float M = kNegInf, Z = 0.0f, O0 = 0.0f, O1 = 0.0f;
    for (int s0 = 0; s0 < ns; s0 += kMergeBatch) {
      float2 mz[kMergeBatch], av[kMergeBatch];
#pragma unroll
      for (int k = 0; k < kMergeBatch; ++k) {
        const int sp = s0 + k < ns ? s0 + k : ns - 1;  // clamped, unconditional
        const float *ps = pg + (int64_t)sp * ad.part_stride;
        mz[k] = *reinterpret_cast<const float2 *>(ps);          // 8-byte aligned:
        av[k] = *reinterpret_cast<const float2 *>(ps + 2 + d);  // D + 2, d even
      }
      float mb = M;
#pragma unroll
      for (int k = 0; k < kMergeBatch; ++k)
        if (s0 + k < ns) mb = fmaxf(mb, mz[k].x);
      if (mb == kNegInf) continue;  // nothing valid yet
      const float fo = M == kNegInf ? 0.0f : __expf(M - mb);
      Z *= fo;
      O0 *= fo;
      O1 *= fo;
#pragma unroll
      for (int k = 0; k < kMergeBatch; ++k) {
        // splits past ns (clamped loads) and empty splits weigh zero
        const float f = (s0 + k < ns && mz[k].x != kNegInf) ? __expf(mz[k].x - mb) : 0.0f;
        Z += mz[k].y * f;
        O0 += av[k].x * f;
        O1 += av[k].y * f;
      }
      M = mb;
    }
    if constexpr (PART) {
      pt.acc[(pb + g) * D + d] = O0;
      pt.acc[(pb + g) * D + d + 1] = O1;
      if (d == 0) {
        pt.m[pb + g] = M;
        pt.z[pb + g] = Z;
      }
      continue;
    }
    const float o0 = Z == 0.0f ? 0.0f : O0 / Z;
    const float o1 = Z == 0.0f ? 0.0f : O1 / Z;
    const int64_t oi = ((int64_t)t * p.hq + kh * G + g) * D + d;
    if (p.q_dtype == NFA_DTYPE_BF16) {
      ((uint16_t *)p.out)[oi] = bf16_bits(o0);
      ((uint16_t *)p.out)[oi + 1] = bf16_bits(o1);
    } else {
      ((float *)p.out)[oi] = o0;
      ((float *)p.out)[oi + 1] = o1;
    }
  }
}

// Regions combine: one thread per output element (t, head, dim).  The
// states of up to kCombineRegs splits load in one round (they were written
// by other kernels, possibly through another XCD's L2, so each dependent
// load would cost a full memory latency); then the maximum over every split
// of both regions, and each split's denominator and P.V scaled by
// exp(m_s - M): the softmax over the union, as the sequential rescaling
// region a then region b gives it.
constexpr int kCombineRegs = 16;
__global__ void __launch_bounds__(NFA_BLOCK)
    nfa_regions_combine_kernel(const NfaAttnCombineParams c) {
  const int64_t i = (int64_t)blockIdx.x * NFA_BLOCK + threadIdx.x;
  const int64_t heads = (int64_t)c.total_q * c.hq;
  if (i >= heads * c.head_dim_v) return;
  const int64_t th = i / c.head_dim_v;
  const int d = (int)(i % c.head_dim_v);
  const float kNegInf = __uint_as_float(0xFF800000u);
  const int ns = c.nsplit_a + c.nsplit_b;
  float M = kNegInf, z = 0.0f, acc = 0.0f;
  for (int s0 = 0; s0 < ns; s0 += kCombineRegs) {
    float rm[kCombineRegs], rz[kCombineRegs], ra[kCombineRegs];
#pragma unroll
    for (int k = 0; k < kCombineRegs; ++k) {
      const int sp = s0 + k;
      rm[k] = kNegInf;
      rz[k] = ra[k] = 0.0f;
      if (sp < ns) {
        const bool in_a = sp < c.nsplit_a;
        const int64_t e = (in_a ? sp : sp - c.nsplit_a) * heads + th;
        rm[k] = (in_a ? c.m_a : c.m_b)[e];
        rz[k] = (in_a ? c.z_a : c.z_b)[e];
        ra[k] = (in_a ? c.acc_a : c.acc_b)[e * c.head_dim_v + d];
      }
    }
    float m_new = M;
#pragma unroll
    for (int k = 0; k < kCombineRegs; ++k) m_new = fmaxf(m_new, rm[k]);
    if (m_new == kNegInf) continue;  // nothing valid so far
    const float f_old = M == kNegInf ? 0.0f : __expf(M - m_new);
    z *= f_old;
    acc *= f_old;
#pragma unroll
    for (int k = 0; k < kCombineRegs; ++k) {
      const float f = rm[k] == kNegInf ? 0.0f : __expf(rm[k] - m_new);
      z += rz[k] * f;
      acc += ra[k] * f;
    }
    M = m_new;
  }
  const float o = z == 0.0f ? 0.0f : acc / z;
  if (c.out_dtype == NFA_DTYPE_BF16)
    ((uint16_t *)c.out)[i] = bf16_bits(o);
  else
    ((float *)c.out)[i] = o;
}

}  // namespace nfa

extern "C" int64_t nfa_attn_workspace_bytes(const NfaAttnParams *p) {
  if (p == nullptr || p->total_q <= 0 || p->hkv <= 0) return 0;
  return nfa::attn_dims(*p, nfa::device_cus()).w_total;
}

// Shared argument checks of the gather attention entry points; `tpr` gets
// the threads per K/V row.  The output pointer is checked by the caller.
static int32_t check_attn(const NfaAttnParams *p, const char *fn, int *tpr_out) {
  // *tpr_out = 4 * (K chunks per thread - 1) + (V chunks per thread - 1)
  if (p == nullptr || p->abi_version != NFA_ABI_VERSION ||
      p->struct_size != (int32_t)sizeof(NfaAttnParams)) {
    nfa_set_error("%s: ABI mismatch", fn);
    return NFA_EINVAL;
  }
  if (p->hkv <= 0 || p->hq % p->hkv != 0 || p->hq / p->hkv > nfa::AGMAX) {
    nfa_set_error("%s: unsupported heads hq=%d hkv=%d", fn, p->hq, p->hkv);
    return NFA_EINVAL;
  }
  // K and V rows: 8, 16, 24 or 32 chunks of 16 bytes each (64 to 256 bf16
  // dims, 32 to 128 fp32 dims), independently
  const int chunk = p->kv_dtype == NFA_DTYPE_BF16 ? 8 : 4;
  const int ck = p->head_dim / (chunk * nfa::kTpr);
  const int cv = p->head_dim_v / (chunk * nfa::kTpr);
  if (p->head_dim % (chunk * nfa::kTpr) != 0 || p->head_dim_v % (chunk * nfa::kTpr) != 0 ||
      ck < 1 || ck > 4 || cv < 1 || cv > 4) {
    nfa_set_error("%s: unsupported head dims %d/%d "
                  "(K and V rows must each span 8, 16, 24 or 32 chunks of 16 bytes)",
                  fn, p->head_dim, p->head_dim_v);
    return NFA_EINVAL;
  }
  if (p->kv_dtype != NFA_DTYPE_BF16 && p->kv_dtype != NFA_DTYPE_F32) {
    nfa_set_error("%s: unsupported kv dtype %d", fn, p->kv_dtype);
    return NFA_EINVAL;
  }
  if (p->max_vis <= 0 || p->page <= 0 || p->pool_pages <= 0 ||
      p->gather_rows <= 0) {
    nfa_set_error("%s: bad max_vis/page/pool/rows", fn);
    return NFA_EINVAL;
  }
  if (p->tokens_per_split < 0 || p->tokens_per_split > nfa::kSplitMax) {
    nfa_set_error("%s: tokens_per_split must be in [0,64]", fn);
    return NFA_EINVAL;
  }
  if (!p->q || !p->k_pool || !p->v_pool || !p->gather || !p->vis_lens ||
      !p->query_to_req) {
    nfa_set_error("%s: null device pointer", fn);
    return NFA_EINVAL;
  }
  *tpr_out = 4 * (ck - 1) + (cv - 1);
  return NFA_OK;
}

// The kernel instance of a (K chunks, V chunks) per thread pair: `shape` =
// 4 * (ck - 1) + (cv - 1), as check_attn reports it.
template <typename KV, bool PART, int CK, int CV>
static void launch_attn_cv(bool loop, dim3 grid, hipStream_t s, const NfaAttnParams &p,
                           int cus, const NfaAttnPartial &pt) {
  if (loop)
    hipLaunchKernelGGL((nfa::nfa_attn_kernel<KV, CK, CV, true, PART>), grid,
                       dim3(NFA_BLOCK), 0, s, p, cus, pt);
  else
    hipLaunchKernelGGL((nfa::nfa_attn_kernel<KV, CK, CV, false, PART>), grid,
                       dim3(NFA_BLOCK), 0, s, p, cus, pt);
}

template <typename KV, bool PART, int CK>
static void launch_attn_ck(int cv, bool loop, dim3 grid, hipStream_t s,
                           const NfaAttnParams &p, int cus, const NfaAttnPartial &pt) {
  switch (cv) {
    case 1: launch_attn_cv<KV, PART, CK, 1>(loop, grid, s, p, cus, pt); break;
    case 2: launch_attn_cv<KV, PART, CK, 2>(loop, grid, s, p, cus, pt); break;
    case 3: launch_attn_cv<KV, PART, CK, 3>(loop, grid, s, p, cus, pt); break;
    default: launch_attn_cv<KV, PART, CK, 4>(loop, grid, s, p, cus, pt); break;
  }
}

template <typename KV, bool PART>
static void launch_attn(int shape, bool loop, dim3 grid, hipStream_t s,
                        const NfaAttnParams &p, int cus, const NfaAttnPartial &pt) {
  const int cv = shape % 4 + 1;
  switch (shape / 4 + 1) {
    case 1: launch_attn_ck<KV, PART, 1>(cv, loop, grid, s, p, cus, pt); break;
    case 2: launch_attn_ck<KV, PART, 2>(cv, loop, grid, s, p, cus, pt); break;
    case 3: launch_attn_ck<KV, PART, 3>(cv, loop, grid, s, p, cus, pt); break;
    default: launch_attn_ck<KV, PART, 4>(cv, loop, grid, s, p, cus, pt); break;
  }
}

extern "C" int32_t nfa_sparse_attn_decode(const NfaAttnParams *p, void *stream) {
  if (p != nullptr && p->abi_version == NFA_ABI_VERSION &&
      p->struct_size == (int32_t)sizeof(NfaAttnParams) && p->total_q <= 0)
    return NFA_OK;
  int tpr = 0;
  const int32_t rc = check_attn(p, "nfa_sparse_attn_decode", &tpr);
  if (rc != NFA_OK) return rc;
  if (!p->out) {
    nfa_set_error("nfa_sparse_attn_decode: null device pointer");
    return NFA_EINVAL;
  }
  const NfaAttnPartial none{};
  const int cus = nfa::device_cus();
  const nfa::AttnDims ad = nfa::attn_dims(*p, cus);
  if (p->workspace == nullptr || p->workspace_bytes < ad.w_total) {
    nfa_set_error("nfa_sparse_attn_decode: workspace %lld < %lld bytes",
                  (long long)p->workspace_bytes, (long long)ad.w_total);
    return NFA_EWORKSPACE;
  }
  dim3 grid((unsigned)(((ad.rows + nfa::kXcds - 1) / nfa::kXcds) * nfa::kXcds * ad.nsplit));
  hipStream_t s = (hipStream_t)stream;
  const bool bf = p->kv_dtype == NFA_DTYPE_BF16;
  const bool loop = (int64_t)ad.nsplit * ad.split < p->max_vis;
  if (bf)
    launch_attn<uint16_t, false>(tpr, loop, grid, s, *p, cus, none);
  else
    launch_attn<float, false>(tpr, loop, grid, s, *p, cus, none);
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess) {
    nfa_set_error("nfa_sparse_attn_decode: launch failed: %s", hipGetErrorString(err));
    return NFA_ELAUNCH;
  }
  return NFA_OK;
}

extern "C" int32_t nfa_sparse_attn_partial(const NfaAttnParams *p,
                                           const NfaAttnPartial *pt, void *stream) {
  if (pt == nullptr || pt->abi_version != NFA_ABI_VERSION ||
      pt->struct_size != (int32_t)sizeof(NfaAttnPartial)) {
    nfa_set_error("nfa_sparse_attn_partial: ABI mismatch");
    return NFA_EINVAL;
  }
  if (p != nullptr && p->abi_version == NFA_ABI_VERSION &&
      p->struct_size == (int32_t)sizeof(NfaAttnParams) && p->total_q <= 0)
    return NFA_OK;
  int tpr = 0;
  const int32_t rc = check_attn(p, "nfa_sparse_attn_partial", &tpr);
  if (rc != NFA_OK) return rc;
  if (pt->nsplit < 1 || pt->nsplit > 65535 || pt->block_tokens < 1) {
    nfa_set_error("nfa_sparse_attn_partial: nsplit %d / block_tokens %d out of range",
                  pt->nsplit, pt->block_tokens);
    return NFA_EINVAL;
  }
  if (!pt->acc || !pt->m || !pt->z) {
    nfa_set_error("nfa_sparse_attn_partial: null state pointer");
    return NFA_EINVAL;
  }
  const int cus = nfa::device_cus();
  const int span = nfa::part_span(*p, *pt);
  const nfa::AttnDims ad = nfa::attn_dims(*p, cus, pt->nsplit, span);
  if (p->workspace == nullptr || p->workspace_bytes < ad.w_total) {
    nfa_set_error("nfa_sparse_attn_partial: workspace %lld < %lld bytes",
                  (long long)p->workspace_bytes, (long long)ad.w_total);
    return NFA_EWORKSPACE;
  }
  dim3 grid((unsigned)(((ad.rows + nfa::kXcds - 1) / nfa::kXcds) * nfa::kXcds * ad.nsplit));
  hipStream_t s = (hipStream_t)stream;
  const bool bf = p->kv_dtype == NFA_DTYPE_BF16;
  const bool loop = (int64_t)ad.nsplit * ad.split < span;
  if (bf)
    launch_attn<uint16_t, true>(tpr, loop, grid, s, *p, cus, *pt);
  else
    launch_attn<float, true>(tpr, loop, grid, s, *p, cus, *pt);
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess) {
    nfa_set_error("nfa_sparse_attn_partial: launch failed: %s", hipGetErrorString(err));
    return NFA_ELAUNCH;
  }
  return NFA_OK;
}

extern "C" int32_t nfa_attn_regions_combine(const NfaAttnCombineParams *c, void *stream) {
  if (c == nullptr || c->abi_version != NFA_ABI_VERSION ||
      c->struct_size != (int32_t)sizeof(NfaAttnCombineParams)) {
    nfa_set_error("nfa_attn_regions_combine: ABI mismatch");
    return NFA_EINVAL;
  }
  if (c->total_q <= 0) return NFA_OK;
  if (c->hq <= 0 || c->head_dim_v <= 0 || c->nsplit_a < 0 || c->nsplit_b < 0 ||
      (c->out_dtype != NFA_DTYPE_BF16 && c->out_dtype != NFA_DTYPE_F32)) {
    nfa_set_error("nfa_attn_regions_combine: bad shape or dtype");
    return NFA_EINVAL;
  }
  if (!c->out || (c->nsplit_a > 0 && (!c->acc_a || !c->m_a || !c->z_a)) ||
      (c->nsplit_b > 0 && (!c->acc_b || !c->m_b || !c->z_b))) {
    nfa_set_error("nfa_attn_regions_combine: null device pointer");
    return NFA_EINVAL;
  }
  const int64_t n = (int64_t)c->total_q * c->hq * c->head_dim_v;
  const int64_t blocks = (n + NFA_BLOCK - 1) / NFA_BLOCK;
  if (blocks > 0x7FFFFFFF) {
    nfa_set_error("nfa_attn_regions_combine: too many outputs");
    return NFA_EINVAL;
  }
  hipLaunchKernelGGL(nfa::nfa_regions_combine_kernel, dim3((unsigned)blocks),
                     dim3(NFA_BLOCK), 0, (hipStream_t)stream, *c);
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess) {
    nfa_set_error("nfa_attn_regions_combine: launch failed: %s", hipGetErrorString(err));
    return NFA_ELAUNCH;
  }
  return NFA_OK;
}

extern "C" int64_t nfa_attn_partial_workspace_bytes(const NfaAttnParams *p,
                                                     const NfaAttnPartial *pt) {
  if (p == nullptr || pt == nullptr || p->total_q <= 0 || p->hkv <= 0 ||
      pt->nsplit < 1 || pt->block_tokens < 1 || p->max_vis <= 0)
    return 0;
  return nfa::attn_dims(*p, nfa::device_cus(), pt->nsplit, nfa::part_span(*p, *pt)).w_total;
}

extern "C" int32_t nfa_attn_partial_size(void) { return (int32_t)sizeof(NfaAttnPartial); }
extern "C" int32_t nfa_attn_combine_params_size(void) {
  return (int32_t)sizeof(NfaAttnCombineParams);
}
