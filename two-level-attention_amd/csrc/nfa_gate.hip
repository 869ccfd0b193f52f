// Prefill region gate: near / far attention mass of the last prompt rows
// (gfx950).
//
// Reference: profile_regions / fused_region_profile,
// sparse_attn/policies/frozen_gate.py:99-111 and
// sparse_attn/ops/frozen_gate_triton.py:7-111.  For each query head and each
// of the last `rows` prompt positions, one pass over the keys 0..qlen-1
// keeps an online softmax (running max, total, far and near sums, all
// rescaled together) and returns far / total and near / total; the regions
// follow RegionGeometry.bounds at qlen (sink_hi = min(qlen, sink),
// near_hi = max(sink_hi, qlen - window), far_hi = min(near_hi,
// max(sink_hi, floor((qlen - window - near) / page) * page))).
//
// Grid (ceil(rows / (64 / G)), hkv), 256 threads.  A workgroup holds 64
// query vectors (64 / G prompt rows x the G heads of one kv head) in LDS as
// fp32 and streams 64-key tiles of K through LDS (the next tile's loads in
// flight during the current tile's dots).  Thread (qb, kb) = (tid / 16,
// tid % 16) owns the four heads of one row and keys kb + 16 i, i < 4: a 4x4
// block of fp32 dot products per 4-dim step; row reductions run over the 16
// lanes of a row.  Vector FMA, not MFMA: a 128K prompt costs about 2 ms per
// layer, once per request.
#include "nfa_common.h"

namespace nfa {

constexpr int GQ = 64;        // query vectors per workgroup
constexpr int GK = 64;        // keys per tile
constexpr int GDMAX = 128;    // largest head dim
constexpr int GQP = GDMAX + 4;  // fp32 query row pitch in LDS
constexpr int GKP = GDMAX + 8;  // bf16 key row pitch in LDS

__device__ __forceinline__ int gmin(int a, int b) { return a < b ? a : b; }

__device__ __forceinline__ int floordiv(int a, int b) {
  const int q = a / b;
  return (a % b != 0 && ((a < 0) != (b < 0))) ? q - 1 : q;
}

__device__ __forceinline__ float row16_max(float v) {
#pragma unroll
  for (int off = 1; off < 16; off <<= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
  return v;
}
__device__ __forceinline__ float row16_sum(float v) {
#pragma unroll
  for (int off = 1; off < 16; off <<= 1) v += __shfl_xor(v, off, 64);
  return v;
}

__global__ void __launch_bounds__(NFA_BLOCK) gate_kernel(const NfaGateParams p) {
  __shared__ __align__(16) float s_q[GQ * GQP];
  __shared__ __align__(16) uint16_t s_k[GK * GKP];
  const int tid = threadIdx.x;
  const int G = p.hq / p.hkv;
  const int rows_wg = GQ / G;
  const int kvh = blockIdx.y;
  const int r0 = blockIdx.x * rows_wg;
  const int start = p.length - p.rows;  // absolute position of profiled row 0
  const int D = p.head_dim;
  const int dch = D / 8;                // 16-byte chunks per row
  const float kNegInf = __uint_as_float(0xFF800000u);

  // query vectors v = row_local * G + g, fp32 in LDS (zeros past the rows)
  for (int i = tid; i < GQ * dch; i += NFA_BLOCK) {
    const int v = i / dch, c = i % dch;
    const int r = r0 + v / G;
    uint4 x = make_uint4(0u, 0u, 0u, 0u);
    if (r < p.rows) {
      const uint16_t *src = (const uint16_t *)p.q + (int64_t)(kvh * G + v % G) * p.q_stride_h +
                            (int64_t)(start + r) * p.q_stride_l + c * 8;
      x = *reinterpret_cast<const uint4 *>(src);
    }
    float *dst = s_q + v * GQP + c * 8;
    const uint32_t w[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      dst[2 * e] = __uint_as_float(w[e] << 16);
      dst[2 * e + 1] = __uint_as_float(w[e] & 0xFFFF0000u);
    }
  }

  // this thread: query vectors 4 qb .. 4 qb + 3, keys kb + 16 i of a tile
  const int qb = tid >> 4, kb = tid & 15;
  // row of each of the four vectors, its qlen and region bounds
  int qlen[4], sink_hi[4], far_hi[4], near_hi[4];
  bool live[4];
#pragma unroll
  for (int a = 0; a < 4; ++a) {
    const int v = qb * 4 + a;
    const int r = r0 + v / G;
    live[a] = v < GQ && r < p.rows;
    const int ql = start + r + 1;
    qlen[a] = ql;
    sink_hi[a] = gmin(ql, p.sink);
    near_hi[a] = sink_hi[a] > ql - p.window ? sink_hi[a] : ql - p.window;
    const int fb = floordiv(ql - p.window - p.near, p.page) * p.page;
    const int fh = sink_hi[a] > fb ? sink_hi[a] : fb;
    far_hi[a] = gmin(near_hi[a], fh);
  }
  const int last_row = gmin(r0 + rows_wg, p.rows) - 1;
  const int key_end = last_row >= 0 ? start + last_row + 1 : 0;  // keys any row sees
  const int ntiles = (key_end + GK - 1) / GK;

  float m[4], tot[4], far[4], near[4];
#pragma unroll
  for (int a = 0; a < 4; ++a) {
    m[a] = kNegInf;
    tot[a] = far[a] = near[a] = 0.0f;
  }
  // K tile loads: 64 keys x dch chunks, at most 4 per thread
  uint4 kr[4];
  auto load_tile = [&](int t) {
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int i = tid + u * NFA_BLOCK;
      const int key = t * GK + i / dch, c = i % dch;
      kr[u] = make_uint4(0u, 0u, 0u, 0u);
      if (i < GK * dch && key < key_end)
        kr[u] = *reinterpret_cast<const uint4 *>(
            (const uint16_t *)p.k + (int64_t)kvh * p.k_stride_h +
            (int64_t)key * p.k_stride_l + c * 8);
    }
  };
  if (ntiles > 0) load_tile(0);
  for (int t = 0; t < ntiles; ++t) {
    __syncthreads();  // previous tile's readers are done (and the queries landed)
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int i = tid + u * NFA_BLOCK;
      if (i < GK * dch)
        *reinterpret_cast<uint4 *>(s_k + (i / dch) * GKP + (i % dch) * 8) = kr[u];
    }
    __syncthreads();
    if (t + 1 < ntiles) load_tile(t + 1);

    float s[4][4];
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
      for (int i = 0; i < 4; ++i) s[a][i] = 0.0f;
    const float *qp = s_q + (qb * 4) * GQP;
    for (int d = 0; d < D; d += 4) {
      float4 qv[4];
#pragma unroll
      for (int a = 0; a < 4; ++a) qv[a] = *reinterpret_cast<const float4 *>(qp + a * GQP + d);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint2 kw = *reinterpret_cast<const uint2 *>(s_k + (kb + 16 * i) * GKP + d);
        const float k0 = __uint_as_float(kw.x << 16), k1 = __uint_as_float(kw.x & 0xFFFF0000u);
        const float k2 = __uint_as_float(kw.y << 16), k3 = __uint_as_float(kw.y & 0xFFFF0000u);
#pragma unroll
        for (int a = 0; a < 4; ++a) {
          float acc = s[a][i];
          acc = fmaf(qv[a].x, k0, acc);
          acc = fmaf(qv[a].y, k1, acc);
          acc = fmaf(qv[a].z, k2, acc);
          acc = fmaf(qv[a].w, k3, acc);
          s[a][i] = acc;
        }
      }
    }
    // online softmax over this tile's keys, per query vector
#pragma unroll
    for (int a = 0; a < 4; ++a) {
      float tmax = kNegInf;
      bool ok[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int j = t * GK + kb + 16 * i;
        ok[i] = live[a] && j < qlen[a];
        s[a][i] = ok[i] ? s[a][i] * p.scale : kNegInf;
        tmax = fmaxf(tmax, s[a][i]);
      }
      tmax = row16_max(tmax);
      const float m_new = fmaxf(m[a], tmax);
      if (m_new == kNegInf) continue;  // nothing visible yet (uniform per row)
      const float alpha = m[a] == kNegInf ? 0.0f : __expf(m[a] - m_new);
      float ts = 0.0f, tf = 0.0f, tn = 0.0f;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int j = t * GK + kb + 16 * i;
        const float e = ok[i] ? __expf(s[a][i] - m_new) : 0.0f;
        ts += e;
        if (j >= sink_hi[a] && j < far_hi[a]) tf += e;
        if (j >= far_hi[a] && j < near_hi[a]) tn += e;
      }
      ts = row16_sum(ts);
      tf = row16_sum(tf);
      tn = row16_sum(tn);
      tot[a] = tot[a] * alpha + ts;
      far[a] = far[a] * alpha + tf;
      near[a] = near[a] * alpha + tn;
      m[a] = m_new;
    }
  }
  if (kb == 0) {
#pragma unroll
    for (int a = 0; a < 4; ++a) {
      if (!live[a]) continue;
      const int v = qb * 4 + a;
      const int head = kvh * G + v % G;
      const int r = r0 + v / G;
      const float inv = tot[a] > 0.0f ? 1.0f / tot[a] : 0.0f;
      p.out[(int64_t)head * p.rows + r] = near[a] * inv;
      p.out[((int64_t)p.hq + head) * p.rows + r] = far[a] * inv;
    }
  }
}

}  // namespace nfa

extern "C" int32_t nfa_gate_params_size(void) { return (int32_t)sizeof(NfaGateParams); }

extern "C" int32_t nfa_region_profile(const NfaGateParams *p, void *stream) {
  if (p == nullptr || p->abi_version != NFA_ABI_VERSION ||
      p->struct_size != (int32_t)sizeof(NfaGateParams)) {
    nfa_set_error("nfa_region_profile: ABI mismatch");
    return NFA_EINVAL;
  }
  if (p->hkv < 1 || p->hq % p->hkv != 0 || nfa::GQ % (p->hq / p->hkv) != 0) {
    nfa_set_error("nfa_region_profile: unsupported heads hq=%d hkv=%d", p->hq, p->hkv);
    return NFA_EINVAL;
  }
  if (p->head_dim < 8 || p->head_dim > nfa::GDMAX || p->head_dim % 8 != 0 ||
      p->q_dtype != NFA_DTYPE_BF16) {
    nfa_set_error("nfa_region_profile: head_dim %d / dtype %d unsupported "
                  "(bf16, multiple of 8, at most 128)", p->head_dim, p->q_dtype);
    return NFA_EINVAL;
  }
  if (p->length < 1 || p->rows < 1 || p->rows > p->length || p->page < 1 ||
      p->sink < 0 || p->window < 0 || p->near < 0) {
    nfa_set_error("nfa_region_profile: bad length %d rows %d or geometry",
                  p->length, p->rows);
    return NFA_EINVAL;
  }
  if (!p->q || !p->k || !p->out || ((uintptr_t)p->q & 15) || ((uintptr_t)p->k & 15) ||
      p->q_stride_l % 8 || p->q_stride_h % 8 || p->k_stride_l % 8 || p->k_stride_h % 8) {
    nfa_set_error("nfa_region_profile: null or unaligned q/k/out");
    return NFA_EINVAL;
  }
  const int G = p->hq / p->hkv;
  const int rows_wg = nfa::GQ / G;
  dim3 grid((unsigned)((p->rows + rows_wg - 1) / rows_wg), (unsigned)p->hkv);
  hipLaunchKernelGGL(nfa::gate_kernel, grid, dim3(NFA_BLOCK), 0, (hipStream_t)stream, *p);
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess) {
    nfa_set_error("nfa_region_profile: launch failed: %s", hipGetErrorString(err));
    return NFA_ELAUNCH;
  }
  return NFA_OK;
}
