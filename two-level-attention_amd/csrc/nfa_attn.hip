// Sparse gather decode attention over selected physical slots (gfx950).
//
// Reference: sparse_paged_attention_gather / _gather_attend_grouped_kernel,
// sparse_attn/ops/paged_region_kernels.py:251-363 and :800-1006.
//
// Grid (nsplit, T * hkv), 256 threads.  Each workgroup owns one (query row,
// kv head) and a contiguous chunk of the selected slots, handles the G query
// heads of the group together (K/V rows are read once per group, not once per
// query head), and writes an online-softmax partial (m, z, acc).  The last
// workgroup of the (row, kv) to arrive -- device-scope atomic counter, no
// waiting -- merges the partials and writes the output in the query dtype.
// Selected rows are 256-byte K/V rows: each wave reads a whole row per
// instruction (lane = 2 dims), the 4 waves stream different rows.
#include "nfa_common.h"

namespace nfa {

constexpr int AGMAX = 8;     // query heads per kv head
constexpr int ADMAX = 256;   // head dim
constexpr int kSplitMax = 64;                    // tokens per workgroup
constexpr int kTpw = kSplitMax / NFA_WAVES;      // tokens per wave
constexpr int kMaxSplits = 256;                  // splits merged in LDS

// Two adjacent elements of a K/V row as one load.
template <typename T> struct PairOf;
template <> struct PairOf<uint16_t> {
  using type = uint32_t;
  static __device__ __forceinline__ type zero() { return 0u; }
  static __device__ __forceinline__ void unpack(type v, float *a, float *b) {
    *a = __uint_as_float(v << 16);
    *b = __uint_as_float(v & 0xFFFF0000u);
  }
};
template <> struct PairOf<float> {
  using type = float2;
  static __device__ __forceinline__ type zero() { return make_float2(0.f, 0.f); }
  static __device__ __forceinline__ void unpack(type v, float *a, float *b) {
    *a = v.x;
    *b = v.y;
  }
};

struct AttnDims {
  int split;    // tokens per split
  int nsplit;
  int rows;     // T * hkv
  int64_t w_cnt, w_part, w_total;
  int part_stride;  // floats per (row, split): G * (DV + 2)
};

__host__ __device__ inline AttnDims attn_dims(const NfaAttnParams &p) {
  AttnDims a;
  a.rows = p.total_q * p.hkv;
  int split = p.tokens_per_split;
  if (split <= 0) split = a.rows <= 16 ? 32 : 64;
  a.split = split;
  a.nsplit = (p.max_vis + split - 1) / split;
  if (a.nsplit < 1) a.nsplit = 1;
  const int G = p.hq / p.hkv;
  a.part_stride = G * (p.head_dim_v + 2);
  int64_t w = 0;
  a.w_cnt = w;  w += ((int64_t)4 * a.rows + 255) & ~(int64_t)255;
  a.w_part = w; w += (int64_t)4 * a.rows * a.nsplit * a.part_stride;
  a.w_total = w;
  return a;
}

template <typename KV>
__global__ void __launch_bounds__(NFA_BLOCK)
    nfa_attn_kernel(const NfaAttnParams p) {
  const AttnDims ad = attn_dims(p);
  const int tid = threadIdx.x;
  const int lane = lane_id();
  const int w = wave_id();
  const int split = blockIdx.x;
  const int row = blockIdx.y;
  const int t = row / p.hkv;
  const int kh = row % p.hkv;
  const int G = p.hq / p.hkv;
  const int D = p.head_dim;
  const int DV = p.head_dim_v;

  __shared__ float s_q[AGMAX * ADMAX];
  __shared__ float s_p[AGMAX * kSplitMax];    // probabilities [G][split]
  __shared__ int s_slot[kSplitMax];
  __shared__ float s_red[NFA_WAVES * AGMAX * ADMAX];
  __shared__ float s_m[AGMAX], s_z[AGMAX];
  __shared__ int s_last;

  unsigned char *ws = (unsigned char *)p.workspace;
  unsigned int *cnt = (unsigned int *)(ws + ad.w_cnt);
  float *part = (float *)(ws + ad.w_part) +
                ((int64_t)row * ad.nsplit + split) * ad.part_stride;

  int req = p.query_to_req[t];
  if (req >= p.gather_rows) req = -1;  // out-of-range rows act as padding
  int n = 0;
  if (req >= 0) {
    n = p.vis_lens[req * p.hkv + kh];
    if (n > p.max_vis) n = p.max_vis;
  }
  const int c0 = split * ad.split;
  int c1 = c0 + ad.split;
  if (c1 > n) c1 = n;
  const int cn = c1 > c0 ? c1 - c0 : 0;

  if (cn > 0) {
    for (int i = tid; i < G * D; i += NFA_BLOCK) {
      const int g = i / D, d = i % D;
      s_q[g * ADMAX + d] =
          load_any(p.q, ((int64_t)t * p.hq + kh * G + g) * D + d, p.q_dtype);
    }
    const int32_t *grow = p.gather + ((int64_t)req * p.hkv + kh) * p.max_vis;
    // slots outside the arena are skipped like negative ones
    const int max_slot = p.pool_pages * p.page;
    for (int i = tid; i < cn; i += NFA_BLOCK) {
      const int sl = grow[c0 + i];
      s_slot[i] = sl < max_slot ? sl : -1;
    }
  }
  __syncthreads();

  const KV *kpool = (const KV *)p.k_pool;
  const KV *vpool = (const KV *)p.v_pool;
  // Raw row pieces: lane holds dims 2*lane + 128*h (h < 2); every row this
  // wave needs is requested before the first one is used.
  using Pair = typename PairOf<KV>::type;
  constexpr int H = ADMAX / 128;
  // scores: wave w takes tokens w, w+4, ... (at most kTpw of them)
  Pair kraw[kTpw][H];
#pragma unroll
  for (int t = 0; t < kTpw; ++t) {
    const int i = w + t * NFA_WAVES;
    const int slot = i < cn ? s_slot[i] : -1;
#pragma unroll
    for (int h = 0; h < H; ++h) {
      kraw[t][h] = PairOf<KV>::zero();
      const int d = 2 * lane + 128 * h;
      if (slot >= 0 && d < D) {
        const int phys = slot / p.page, off = slot % p.page;
        kraw[t][h] = *reinterpret_cast<const Pair *>(
            kpool + (((int64_t)phys * p.hkv + kh) * p.page + off) * D + d);
      }
    }
  }
#pragma unroll
  for (int t = 0; t < kTpw; ++t) {
    const int i = w + t * NFA_WAVES;
    if (i >= cn) break;
    const int slot = s_slot[i];
    float part_s[AGMAX];
#pragma unroll
    for (int g = 0; g < AGMAX; ++g) part_s[g] = 0.0f;
#pragma unroll
    for (int h = 0; h < H; ++h) {
      const int d = 2 * lane + 128 * h;
      if (d < D) {
        float k0, k1;
        PairOf<KV>::unpack(kraw[t][h], &k0, &k1);
#pragma unroll
        for (int g = 0; g < AGMAX; ++g) {
          if (g < G) {
            part_s[g] = fmaf(s_q[g * ADMAX + d], k0, part_s[g]);
            part_s[g] = fmaf(s_q[g * ADMAX + d + 1], k1, part_s[g]);
          }
        }
      }
    }
#pragma unroll
    for (int g = 0; g < AGMAX; ++g) {
      if (g < G) {
        float x = part_s[g];
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) x += __shfl_xor(x, off, 64);
        if (lane == 0)
          s_p[g * kSplitMax + i] =
              slot >= 0 ? x * p.scale : __uint_as_float(0xFF800000u);
      }
    }
  }
  __syncthreads();

  // softmax partial per head (one wave per head)
  for (int g = w; g < G; g += NFA_WAVES) {
    float m = __uint_as_float(0xFF800000u);
    for (int i = lane; i < cn; i += 64) m = fmaxf(m, s_p[g * kSplitMax + i]);
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
    float z = 0.0f;
    for (int i = lane; i < cn; i += 64) {
      const float sc = s_p[g * kSplitMax + i];
      const float e = (m == __uint_as_float(0xFF800000u)) ? 0.0f : __expf(sc - m);
      s_p[g * kSplitMax + i] = e;
      z += e;
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) z += __shfl_xor(z, off, 64);
    if (lane == 0) {
      s_m[g] = m;
      s_z[g] = z;
    }
  }
  __syncthreads();

  // P V with the same token assignment; V rows requested up front
  Pair vraw[kTpw][H];
#pragma unroll
  for (int t = 0; t < kTpw; ++t) {
    const int i = w + t * NFA_WAVES;
    const int slot = i < cn ? s_slot[i] : -1;
#pragma unroll
    for (int h = 0; h < H; ++h) {
      vraw[t][h] = PairOf<KV>::zero();
      const int d = 2 * lane + 128 * h;
      if (slot >= 0 && d < DV) {
        const int phys = slot / p.page, off = slot % p.page;
        vraw[t][h] = *reinterpret_cast<const Pair *>(
            vpool + (((int64_t)phys * p.hkv + kh) * p.page + off) * DV + d);
      }
    }
  }
  float acc[AGMAX][H * 2];
#pragma unroll
  for (int g = 0; g < AGMAX; ++g)
#pragma unroll
    for (int e = 0; e < H * 2; ++e) acc[g][e] = 0.0f;
#pragma unroll
  for (int t = 0; t < kTpw; ++t) {
    const int i = w + t * NFA_WAVES;
    if (i >= cn) break;
    if (s_slot[i] < 0) continue;
#pragma unroll
    for (int h = 0; h < H; ++h) {
      const int d = 2 * lane + 128 * h;
      if (d < DV) {
        float v0, v1;
        PairOf<KV>::unpack(vraw[t][h], &v0, &v1);
#pragma unroll
        for (int g = 0; g < AGMAX; ++g) {
          if (g < G) {
            const float pr = s_p[g * kSplitMax + i];
            acc[g][2 * h] = fmaf(pr, v0, acc[g][2 * h]);
            acc[g][2 * h + 1] = fmaf(pr, v1, acc[g][2 * h + 1]);
          }
        }
      }
    }
  }
#pragma unroll
  for (int g = 0; g < AGMAX; ++g) {
    if (g < G) {
#pragma unroll
      for (int k = 0; k < ADMAX / 128; ++k) {
        const int d = 2 * lane + 128 * k;
        if (d < DV) {
          s_red[(w * AGMAX + g) * ADMAX + d] = acc[g][2 * k];
          s_red[(w * AGMAX + g) * ADMAX + d + 1] = acc[g][2 * k + 1];
        }
      }
    }
  }
  __syncthreads();
  for (int i = tid; i < G * DV; i += NFA_BLOCK) {
    const int g = i / DV, d = i % DV;
    float s = 0.0f;
#pragma unroll
    for (int ww = 0; ww < NFA_WAVES; ++ww) s += s_red[(ww * AGMAX + g) * ADMAX + d];
    part[g * (DV + 2) + 2 + d] = s;
  }
  if (tid < G) {
    part[tid * (DV + 2) + 0] = cn > 0 ? s_m[tid] : __uint_as_float(0xFF800000u);
    part[tid * (DV + 2) + 1] = cn > 0 ? s_z[tid] : 0.0f;
  }

  // arrival; the last split of the (row, kv) merges
  __syncthreads();
  if (tid == 0) {
    __threadfence();
    const unsigned int before = atomicAdd(&cnt[row], 1u);
    s_last = before == (unsigned int)(ad.nsplit - 1);
  }
  __syncthreads();
  if (!s_last) return;
  __threadfence();
  if (tid == 0) atomicExch(&cnt[row], 0u);

  const float *base = (const float *)(ws + ad.w_part) +
                      (int64_t)row * ad.nsplit * ad.part_stride;
  // split maxima and denominators -> LDS (one round of loads)
  float *s_ms = s_red;                         // [G][kMaxSplits]
  float *s_zs = s_red + AGMAX * kMaxSplits;    // [G][kMaxSplits]
  for (int i = tid; i < G * ad.nsplit; i += NFA_BLOCK) {
    const int g = i / ad.nsplit, sp = i % ad.nsplit;
    const float *ps = base + (int64_t)sp * ad.part_stride + g * (DV + 2);
    s_ms[g * kMaxSplits + sp] = ps[0];
    s_zs[g * kMaxSplits + sp] = ps[1];
  }
  __syncthreads();
  for (int i = tid; i < G * DV; i += NFA_BLOCK) {
    const int g = i / DV, d = i % DV;
    float M = __uint_as_float(0xFF800000u);
    for (int sp = 0; sp < ad.nsplit; ++sp) M = fmaxf(M, s_ms[g * kMaxSplits + sp]);
    float Z = 0.0f, O = 0.0f;
    if (M != __uint_as_float(0xFF800000u)) {
      for (int s0 = 0; s0 < ad.nsplit; s0 += 8) {
        float a[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          const int sp = s0 + u;
          a[u] = sp < ad.nsplit
                     ? base[(int64_t)sp * ad.part_stride + g * (DV + 2) + 2 + d]
                     : 0.0f;
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          const int sp = s0 + u;
          if (sp >= ad.nsplit) break;
          const float ms = s_ms[g * kMaxSplits + sp];
          if (ms == __uint_as_float(0xFF800000u)) continue;
          const float f = __expf(ms - M);
          Z += s_zs[g * kMaxSplits + sp] * f;
          O += a[u] * f;
        }
      }
    }
    const float o = Z == 0.0f ? 0.0f : O / Z;
    const int64_t oi = ((int64_t)t * p.hq + kh * G + g) * DV + d;
    if (p.q_dtype == NFA_DTYPE_BF16)
      ((uint16_t *)p.out)[oi] = bf16_bits(o);
    else
      ((float *)p.out)[oi] = o;
  }
}

}  // namespace nfa

extern "C" int64_t nfa_attn_workspace_bytes(const NfaAttnParams *p) {
  if (p == nullptr || p->total_q <= 0 || p->hkv <= 0) return 0;
  return nfa::attn_dims(*p).w_total;
}

extern "C" int32_t nfa_sparse_attn_decode(const NfaAttnParams *p, void *stream) {
  if (p == nullptr || p->abi_version != NFA_ABI_VERSION ||
      p->struct_size != (int32_t)sizeof(NfaAttnParams)) {
    nfa_set_error("nfa_sparse_attn_decode: ABI mismatch");
    return NFA_EINVAL;
  }
  if (p->total_q <= 0) return NFA_OK;
  if (p->hkv <= 0 || p->hq % p->hkv != 0 || p->hq / p->hkv > nfa::AGMAX) {
    nfa_set_error("nfa_sparse_attn_decode: unsupported heads hq=%d hkv=%d",
                  p->hq, p->hkv);
    return NFA_EINVAL;
  }
  if (p->head_dim <= 0 || p->head_dim > nfa::ADMAX || (p->head_dim & 1) ||
      p->head_dim_v <= 0 || p->head_dim_v > nfa::ADMAX || (p->head_dim_v & 1)) {
    nfa_set_error("nfa_sparse_attn_decode: unsupported head dims %d/%d",
                  p->head_dim, p->head_dim_v);
    return NFA_EINVAL;
  }
  if (p->max_vis <= 0 || p->page <= 0 || p->pool_pages <= 0 ||
      p->gather_rows <= 0) {
    nfa_set_error("nfa_sparse_attn_decode: bad max_vis/page/pool/rows");
    return NFA_EINVAL;
  }
  if (p->tokens_per_split < 0 || p->tokens_per_split > nfa::kSplitMax) {
    nfa_set_error("nfa_sparse_attn_decode: tokens_per_split must be in [0,64]");
    return NFA_EINVAL;
  }
  if (nfa::attn_dims(*p).nsplit > nfa::kMaxSplits) {
    nfa_set_error("nfa_sparse_attn_decode: %d splits exceed %d",
                  nfa::attn_dims(*p).nsplit, nfa::kMaxSplits);
    return NFA_EINVAL;
  }
  if (!p->q || !p->k_pool || !p->v_pool || !p->gather || !p->vis_lens ||
      !p->query_to_req || !p->out) {
    nfa_set_error("nfa_sparse_attn_decode: null device pointer");
    return NFA_EINVAL;
  }
  const nfa::AttnDims ad = nfa::attn_dims(*p);
  if (p->workspace == nullptr || p->workspace_bytes < ad.w_total) {
    nfa_set_error("nfa_sparse_attn_decode: workspace %lld < %lld bytes",
                  (long long)p->workspace_bytes, (long long)ad.w_total);
    return NFA_EWORKSPACE;
  }
  dim3 grid(ad.nsplit, ad.rows);
  hipStream_t s = (hipStream_t)stream;
  if (p->kv_dtype == NFA_DTYPE_BF16)
    hipLaunchKernelGGL(nfa::nfa_attn_kernel<uint16_t>, grid, dim3(NFA_BLOCK), 0, s, *p);
  else
    hipLaunchKernelGGL(nfa::nfa_attn_kernel<float>, grid, dim3(NFA_BLOCK), 0, s, *p);
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess) {
    nfa_set_error("nfa_sparse_attn_decode: launch failed: %s", hipGetErrorString(err));
    return NFA_ELAUNCH;
  }
  return NFA_OK;
}
