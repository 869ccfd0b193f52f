// Absorbed multi-head latent attention decode over selected latent rows
// (gfx950).
//
// The latent arena holds one row per token, shared by every head:
// K = [kv_a_layernorm(c) (value_dim) | RoPE'd k_pe (latent_dim - value_dim)].
// Query head h of query row t attends over its own gather row (the head's
// selection):
//   s_i = scale * (q_h . K_i),  q_h = [W_uk,h^T q_nope,h | q_pe,h]
//   o_h = sum_i softmax(s)_i * K_i[0 : value_dim]
// and, given w_uv, the head's value up-projection W_uv,h o_h is written
// instead of o_h (fused into the merge: no second launch).  The
// same attention as DeepseekV2Attention over its expanded heads (reference
// v1 tree sparse_attn/patches/deepseek_v2_attn_patch.py, transformers'
// expand_kv): q_nope . (W_uk c) = (W_uk^T q_nope) . c and
// sum_i p_i (W_uv c_i) = W_uv (sum_i p_i c_i), up to rounding.
//
// Grid nsplit x rows (rows = T * heads, one gather row per head).  Workgroups
// go round-robin over the XCDs in linear id order; each XCD takes a
// contiguous block of rows (query-row major), so a row's splits, and the
// heads of one query row, which share their sink / window rows and part of
// their middles, run on one XCD and share its L2.
// A workgroup takes the chunks split, split + nsplit, ... of 32 selected
// slots; 8 threads share a latent row, each holding CK 16-byte chunks of it
// (its first CV chunks are value dims), so one read of the row serves the
// score and the value; the value dims are staged in LDS for P.V (one thread
// per dim pair).  Online-softmax partials (m, z, acc) are merged by the last
// split of the row to arrive (device-scope counter, nothing waits).
#include "nfa_common.h"

namespace nfa {

constexpr int kMlaTpr = 8;         // threads per latent row
constexpr int kMlaSplit = 32;      // slots per chunk: one pass of 256 threads
constexpr int kMlaMaxSplits = 256;
constexpr int kMlaXcds = 8;

struct MlaDims {
  int nsplit, rows, part_stride;
  int64_t w_cnt, w_part, w_total;
};

// Rows get as many split workgroups as keep about four workgroups per CU
// busy (35 KB of LDS each at 576-dim rows).
__host__ __device__ inline MlaDims mla_dims(const NfaMlaAttnParams &p, int cus) {
  MlaDims a;
  a.rows = p.total_q * p.heads;
  int cap = kMlaMaxSplits;
  const int want = a.rows > 0 ? (4 * cus + a.rows - 1) / a.rows : 1;
  if (want < cap) cap = want;
  a.nsplit = (p.max_vis + kMlaSplit - 1) / kMlaSplit;
  if (a.nsplit > cap) a.nsplit = cap;
  if (a.nsplit < 1) a.nsplit = 1;
  a.part_stride = p.value_dim + 2;
  int64_t w = 0;
  a.w_cnt = w;  w += ((int64_t)4 * kArriveStride * a.rows + 255) & ~(int64_t)255;
  a.w_part = w; w += (int64_t)4 * a.rows * a.nsplit * a.part_stride;
  a.w_total = w;
  return a;
}

__device__ __forceinline__ void store_out(const NfaMlaAttnParams &p, int64_t i, float v) {
  if (p.out_dtype == NFA_DTYPE_BF16)
    ((uint16_t *)p.out)[i] = bf16_bits(v);
  else
    ((float *)p.out)[i] = v;
}

// The head's output from its DV-dim result in LDS: W_uv,h s_o (out_dim
// values) with the up-projection, else s_o itself.  8 lanes share a weight
// row (lane sc takes the row's 16-byte chunks sc, sc + 8, ..., so one load
// of the 8 lanes is one whole 128-byte line), U rows in flight per lane;
// the 8 partial sums meet in sum8.
template <int DV>
__device__ __forceinline__ void mla_write_out(const NfaMlaAttnParams &p, int t, int h,
                                              const float *s_o) {
  if (p.w_uv == nullptr) {
    for (int d = threadIdx.x; d < DV; d += NFA_BLOCK)
      store_out(p, ((int64_t)t * p.heads + h) * DV + d, s_o[d]);
    return;
  }
  constexpr int CH = 8;                          // bf16 per 16-byte chunk
  constexpr int CV = DV / (CH * kMlaTpr);        // chunks per lane and row
  constexpr int U = CV >= 8 ? 1 : 4;             // rows in flight per lane
  constexpr int RPP = NFA_BLOCK / kMlaTpr;       // rows per pass of the block
  const int sc = threadIdx.x % kMlaTpr;
  const int rr = threadIdx.x / kMlaTpr;
  const int od = p.out_dim;
  const uint16_t *w = (const uint16_t *)p.w_uv + (int64_t)h * od * DV;
  const int64_t ob = ((int64_t)t * p.heads + h) * od;
  // (rr is uniform over the 8 lanes of a group, so sum8 sees whole groups)
  for (int o0 = rr; o0 < od; o0 += U * RPP) {
    uint4 wr[U][CV];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int o = o0 + u * RPP;
#pragma unroll
      for (int c = 0; c < CV; ++c)
        wr[u][c] = o < od ? *reinterpret_cast<const uint4 *>(w + (int64_t)o * DV +
                                                             (c * kMlaTpr + sc) * CH)
                          : make_uint4(0u, 0u, 0u, 0u);
    }
    float acc[U];
#pragma unroll
    for (int u = 0; u < U; ++u) acc[u] = 0.0f;
#pragma unroll
    for (int c = 0; c < CV; ++c) {
      const float4 x0 = *reinterpret_cast<const float4 *>(s_o + (c * kMlaTpr + sc) * CH);
      const float4 x1 = *reinterpret_cast<const float4 *>(s_o + (c * kMlaTpr + sc) * CH + 4);
      const float x[CH] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
      for (int u = 0; u < U; ++u) {
        float w8[CH];
        unpack_chunk<uint16_t>(wr[u][c], w8);
#pragma unroll
        for (int e = 0; e < CH; ++e) acc[u] = fmaf(w8[e], x[e], acc[u]);
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const float v = sum8(acc[u]);
      const int o = o0 + u * RPP;
      if (sc == 0 && o < od) store_out(p, ob + o, v);
    }
  }
}

// LOOP: a workgroup may own several chunks (rows wider than nsplit chunks).
template <int CK, int CV, bool LOOP>
__global__ void __launch_bounds__(NFA_BLOCK)
    nfa_mla_attn_kernel(const NfaMlaAttnParams p, int cus) {
  constexpr int CH = 8;                    // bf16 per 16-byte chunk
  constexpr int DK = kMlaTpr * CK * CH;    // latent row width
  constexpr int DV = kMlaTpr * CV * CH;    // value dims (the row's first DV)
  constexpr int OPT = (DV / 2 + NFA_BLOCK - 1) / NFA_BLOCK;  // dim pairs per thread
  const MlaDims ad = mla_dims(p, cus);
  const int tid = threadIdx.x;
  const int lane = lane_id();
  // XCD x = linear % 8 takes rows [x * r8, (x + 1) * r8)
  const int linear = blockIdx.x;
  const int r8 = (ad.rows + kMlaXcds - 1) / kMlaXcds;
  const int j = linear / kMlaXcds;
  const int row = (linear % kMlaXcds) * r8 + j / ad.nsplit;
  const int split = j % ad.nsplit;
  if (j / ad.nsplit >= r8 || row >= ad.rows) return;
  const int t = row / p.heads;
  const int h = row % p.heads;
  const float kNegInf = __uint_as_float(0xFF800000u);

  __shared__ __align__(16) float s_q[DK];
  __shared__ __align__(16) float s_p[kMlaSplit];  // scores, then exp weights
  __shared__ int s_slot[kMlaSplit];
  __shared__ __align__(16) uint16_t s_v[kMlaSplit * DV];
  __shared__ float s_m, s_z, s_f;
  __shared__ int s_last;

  unsigned char *ws = (unsigned char *)p.workspace;
  unsigned int *cnt = (unsigned int *)(ws + ad.w_cnt);
  float *part = (float *)(ws + ad.w_part) + ((int64_t)row * ad.nsplit + split) * ad.part_stride;

  for (int i = tid; i < DK; i += NFA_BLOCK)
    s_q[i] = load_any(p.q, ((int64_t)t * p.heads + h) * DK + i, p.q_dtype);
  int req = p.query_to_req[t];
  if (req >= p.gather_rows) req = -1;  // out-of-range rows act as padding
  int n = 0;
  if (req >= 0) {
    n = p.vis_lens[(int64_t)req * p.heads + h];
    if (n > p.max_vis) n = p.max_vis;
  }
  if (tid == 0) {
    s_m = kNegInf;
    s_z = 0.0f;
  }
  float acc0[OPT], acc1[OPT];
#pragma unroll
  for (int k = 0; k < OPT; ++k) acc0[k] = acc1[k] = 0.0f;
  const int32_t *grow = req >= 0 ? p.gather + ((int64_t)req * p.heads + h) * p.max_vis : nullptr;
  const int max_slot = p.pool_pages * p.page;  // slots beyond are skipped
  const int sc = tid % kMlaTpr;  // this thread's chunks of the row: sc, sc + 8, ...
  const int rr = tid / kMlaTpr;  // its row of the chunk
  const uint16_t *pool = (const uint16_t *)p.kv_pool;
  const int c_first = split * kMlaSplit;
  const int c_step = ad.nsplit * kMlaSplit;
  __syncthreads();  // the query row
  for (int c0 = c_first; c0 < n; c0 += c_step) {
    const int cn = n - c0 < kMlaSplit ? n - c0 : kMlaSplit;
    if (LOOP && c0 != c_first) __syncthreads();  // the previous chunk's readers are done
    if (tid < cn) {
      const int sl = grow[c0 + tid];
      s_slot[tid] = sl < max_slot ? sl : -1;
    }
    __syncthreads();
    const int slot = rr < cn ? s_slot[rr] : -1;
    uint4 kr[CK];
#pragma unroll
    for (int c = 0; c < CK; ++c) kr[c] = make_uint4(0u, 0u, 0u, 0u);
    if (slot >= 0) {
      const int64_t cell = (int64_t)(slot / p.page) * p.page + slot % p.page;
#pragma unroll
      for (int c = 0; c < CK; ++c)
        kr[c] = *reinterpret_cast<const uint4 *>(pool + cell * DK + (c * kMlaTpr + sc) * CH);
    }
    // score: the thread's chunks, then the 8 threads of the row
    float ps = 0.0f;
#pragma unroll
    for (int c = 0; c < CK; ++c) {
      float x[CH];
      unpack_chunk<uint16_t>(kr[c], x);
      const float *q = s_q + (c * kMlaTpr + sc) * CH;
#pragma unroll
      for (int e = 0; e < CH; ++e) ps = fmaf(q[e], x[e], ps);
    }
    ps = sum8(ps);
    if (sc == 0 && rr < cn) s_p[rr] = slot >= 0 ? ps * p.scale : kNegInf;
    // the value dims of the row for P.V
    if (rr < cn) {
#pragma unroll
      for (int c = 0; c < CV; ++c)
        *reinterpret_cast<uint4 *>(s_v + rr * DV + (c * kMlaTpr + sc) * CH) = kr[c];
    }
    __syncthreads();
    // online softmax (wave 0, one score per lane)
    if (wave_id() == 0) {
      const float sl = lane < cn ? s_p[lane] : kNegInf;
      const float m = wave_max_dpp(sl);
      const float m_old = s_m;
      const float m_new = fmaxf(m_old, m);
      const float e = (m_new == kNegInf || lane >= cn) ? 0.0f : __expf(sl - m_new);
      if (lane < cn) s_p[lane] = e;
      const float z = wave_sum_dpp(e);
      if (lane == 0) {
        const float f = m_old == kNegInf ? 0.0f : __expf(m_old - m_new);
        s_f = f;
        s_m = m_new;
        s_z = s_z * f + z;
      }
    }
    __syncthreads();
    // P.V, one thread per dim pair, two chains of alternate slots
#pragma unroll
    for (int k = 0; k < OPT; ++k) {
      const int o = tid + k * NFA_BLOCK;
      if (o >= DV / 2) break;
      const int d = 2 * o;
      float a0 = 0.0f, a1 = 0.0f, b0 = 0.0f, b1 = 0.0f;
      for (int j = 0; j < cn; j += 2) {
        const uint32_t va = *reinterpret_cast<const uint32_t *>(s_v + j * DV + d);
        a0 = fmaf(s_p[j], __uint_as_float(va << 16), a0);
        a1 = fmaf(s_p[j], __uint_as_float(va & 0xFFFF0000u), a1);
        if (j + 1 < cn) {
          const uint32_t vb = *reinterpret_cast<const uint32_t *>(s_v + (j + 1) * DV + d);
          b0 = fmaf(s_p[j + 1], __uint_as_float(vb << 16), b0);
          b1 = fmaf(s_p[j + 1], __uint_as_float(vb & 0xFFFF0000u), b1);
        }
      }
      a0 = a0 + b0;
      a1 = a1 + b1;
      if (LOOP) {
        const float f = s_f;
        acc0[k] = acc0[k] * f + a0;
        acc1[k] = acc1[k] * f + a1;
      } else {
        store_coherent(&part[2 + d], a0);
        store_coherent(&part[3 + d], a1);
      }
    }
    if (!LOOP) break;
  }
  // (s_m / s_z were last written before the barrier ahead of P.V, or with
  // no chunk by thread 0 before the first barrier)
  float *s_o = reinterpret_cast<float *>(s_v);  // the head's result (P.V is done)
  if (LOOP && ad.nsplit == 1) {
    // the whole row in this workgroup: normalise and write the output
    __syncthreads();  // every thread's P.V reads of s_v are done
#pragma unroll
    for (int k = 0; k < OPT; ++k) {
      const int o = tid + k * NFA_BLOCK;
      if (o >= DV / 2) break;
      const int d = 2 * o;
      const float z = s_z;
      s_o[d] = z == 0.0f ? 0.0f : acc0[k] / z;
      s_o[d + 1] = z == 0.0f ? 0.0f : acc1[k] / z;
    }
    __syncthreads();
    mla_write_out<DV>(p, t, h, s_o);
    return;
  }
  // (a single-chunk workgroup stored its P.V above; one with no chunk
  // stores zeros here)
  const bool store_acc = LOOP || c_first >= n;
#pragma unroll
  for (int k = 0; k < OPT; ++k) {
    const int o = tid + k * NFA_BLOCK;
    if (!store_acc || o >= DV / 2) break;
    store_coherent(&part[2 + 2 * o], acc0[k]);
    store_coherent(&part[3 + 2 * o], acc1[k]);
  }
  if (tid == 0) {
    store_coherent(&part[0], s_m);
    store_coherent(&part[1], s_z);
  }
  // arrival; the last split of the row merges (the partials went out through
  // coherent stores: no L2 writeback)
  if (!arrive_last(&cnt[row * kArriveStride], (unsigned int)ad.nsplit, &s_last, false)) return;
  const float *base = (const float *)(ws + ad.w_part) + (int64_t)row * ad.nsplit * ad.part_stride;
  const int ns = ad.nsplit;
  constexpr int kBatch = 16;
  for (int i = tid; i < DV / 2; i += NFA_BLOCK) {
    const int d = 2 * i;
    float M = kNegInf, Z = 0.0f, O0 = 0.0f, O1 = 0.0f;
    for (int s0 = 0; s0 < ns; s0 += kBatch) {
      float2 mz[kBatch], av[kBatch];
#pragma unroll
      for (int k = 0; k < kBatch; ++k) {
        const int sp = s0 + k < ns ? s0 + k : ns - 1;  // clamped, unconditional
        const float *ps = base + (int64_t)sp * ad.part_stride;
        mz[k] = *reinterpret_cast<const float2 *>(ps);
        av[k] = *reinterpret_cast<const float2 *>(ps + 2 + d);
      }
      float mb = M;
#pragma unroll
      for (int k = 0; k < kBatch; ++k)
        if (s0 + k < ns) mb = fmaxf(mb, mz[k].x);
      if (mb == kNegInf) continue;  // nothing valid yet
      const float fo = M == kNegInf ? 0.0f : __expf(M - mb);
      Z *= fo;
      O0 *= fo;
      O1 *= fo;
#pragma unroll
      for (int k = 0; k < kBatch; ++k) {
        const float f = (s0 + k < ns && mz[k].x != kNegInf) ? __expf(mz[k].x - mb) : 0.0f;
        Z += mz[k].y * f;
        O0 += av[k].x * f;
        O1 += av[k].y * f;
      }
      M = mb;
    }
    s_o[d] = Z == 0.0f ? 0.0f : O0 / Z;
    s_o[d + 1] = Z == 0.0f ? 0.0f : O1 / Z;
  }
  __syncthreads();
  mla_write_out<DV>(p, t, h, s_o);
}

}  // namespace nfa

extern "C" int32_t nfa_mla_attn_params_size(void) { return (int32_t)sizeof(NfaMlaAttnParams); }

static int32_t check_mla(const NfaMlaAttnParams *p, int *cv_out) {
  if (p == nullptr || p->abi_version != NFA_ABI_VERSION ||
      p->struct_size != (int32_t)sizeof(NfaMlaAttnParams)) {
    nfa_set_error("nfa_mla_attn_decode: ABI mismatch");
    return NFA_EINVAL;
  }
  // value rows of 64, 128, 256 or 512 bf16 dims, the latent row 64 wider
  // (the RoPE dims): 8 threads per row hold CV and CV + 1 16-byte chunks
  const int cv = p->value_dim / (8 * nfa::kMlaTpr);
  if (p->value_dim % (8 * nfa::kMlaTpr) != 0 || !(cv == 1 || cv == 2 || cv == 4 || cv == 8) ||
      p->latent_dim != p->value_dim + 8 * nfa::kMlaTpr) {
    nfa_set_error("nfa_mla_attn_decode: unsupported latent %d / value %d dims "
                  "(value 64, 128, 256 or 512 bf16 dims, latent = value + 64)",
                  p->latent_dim, p->value_dim);
    return NFA_EINVAL;
  }
  if (p->kv_dtype != NFA_DTYPE_BF16 ||
      (p->q_dtype != NFA_DTYPE_BF16 && p->q_dtype != NFA_DTYPE_F32) ||
      (p->out_dtype != NFA_DTYPE_BF16 && p->out_dtype != NFA_DTYPE_F32)) {
    nfa_set_error("nfa_mla_attn_decode: unsupported dtypes kv %d q %d out %d "
                  "(bf16 latent rows)", p->kv_dtype, p->q_dtype, p->out_dtype);
    return NFA_EINVAL;
  }
  if (p->heads <= 0 || p->max_vis <= 0 || p->page <= 0 || p->pool_pages <= 0 ||
      p->gather_rows <= 0) {
    nfa_set_error("nfa_mla_attn_decode: bad heads/max_vis/page/pool/rows");
    return NFA_EINVAL;
  }
  if (!p->q || !p->kv_pool || !p->gather || !p->vis_lens || !p->query_to_req || !p->out) {
    nfa_set_error("nfa_mla_attn_decode: null device pointer");
    return NFA_EINVAL;
  }
  if (p->w_uv != nullptr && (p->out_dim <= 0 || p->out_dim > 4096)) {
    nfa_set_error("nfa_mla_attn_decode: out_dim %d out of range", p->out_dim);
    return NFA_EINVAL;
  }
  *cv_out = cv;
  return NFA_OK;
}

extern "C" int64_t nfa_mla_attn_workspace_bytes(const NfaMlaAttnParams *p) {
  if (p == nullptr || p->total_q <= 0 || p->heads <= 0 || p->max_vis <= 0) return 0;
  return nfa::mla_dims(*p, nfa::device_cus()).w_total;
}

template <int CV>
static void launch_mla(bool loop, dim3 grid, hipStream_t s, const NfaMlaAttnParams &p,
                       int cus) {
  if (loop)
    hipLaunchKernelGGL((nfa::nfa_mla_attn_kernel<CV + 1, CV, true>), grid, dim3(NFA_BLOCK),
                       0, s, p, cus);
  else
    hipLaunchKernelGGL((nfa::nfa_mla_attn_kernel<CV + 1, CV, false>), grid, dim3(NFA_BLOCK),
                       0, s, p, cus);
}

extern "C" int32_t nfa_mla_attn_decode(const NfaMlaAttnParams *p, void *stream) {
  if (p != nullptr && p->abi_version == NFA_ABI_VERSION &&
      p->struct_size == (int32_t)sizeof(NfaMlaAttnParams) && p->total_q <= 0)
    return NFA_OK;
  int cv = 0;
  const int32_t rc = check_mla(p, &cv);
  if (rc != NFA_OK) return rc;
  const int cus = nfa::device_cus();
  const nfa::MlaDims ad = nfa::mla_dims(*p, cus);
  if (p->workspace == nullptr || p->workspace_bytes < ad.w_total) {
    nfa_set_error("nfa_mla_attn_decode: workspace %lld < %lld bytes",
                  (long long)p->workspace_bytes, (long long)ad.w_total);
    return NFA_EWORKSPACE;
  }
  const dim3 grid((unsigned)(((ad.rows + nfa::kMlaXcds - 1) / nfa::kMlaXcds) * nfa::kMlaXcds *
                             ad.nsplit));
  const bool loop = (int64_t)ad.nsplit * nfa::kMlaSplit < p->max_vis;
  hipStream_t s = (hipStream_t)stream;
  switch (cv) {
    case 1: launch_mla<1>(loop, grid, s, *p, cus); break;
    case 2: launch_mla<2>(loop, grid, s, *p, cus); break;
    case 4: launch_mla<4>(loop, grid, s, *p, cus); break;
    default: launch_mla<8>(loop, grid, s, *p, cus); break;
  }
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess) {
    nfa_set_error("nfa_mla_attn_decode: launch failed: %s", hipGetErrorString(err));
    return NFA_ELAUNCH;
  }
  return NFA_OK;
}
