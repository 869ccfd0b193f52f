// Fused decode-step kernels of the dense model parts around the sparse
// attention (gfx950): skinny linear layers with RMSNorm prologue and
// residual / SiLU-gate epilogues, per-head q/k RMSNorm + RoPE, and RMSNorm.
//
// Reference: the decode patches sparse_attn/patches/qwen3_rmsnorm_patch.py,
// qwen3_mlp_silu_patch.py and ops/qwen3_rope_triton.py:118-160 fuse the
// RMSNorm, SiLU*up and q/k RoPE chains of HF's Qwen3 decoder layer; the
// reference leaves the projections to the vendor GEMM.  Here a decode layer
// is seven launches: [norm + qkv] -> [q/k norm + RoPE] -> selector ->
// attention -> [o_proj + residual] -> [norm + gate/up + SiLU*up] ->
// [down_proj + residual].
//
// Rounding follows HF's bf16 op chain (fp32 opmath, one bf16 rounding per HF
// op); the RMSNorm mean and the dot products sum in this file's own order,
// so results agree with HF's to bf16 rounding, not bit for bit.
//
// Linear layers at decode batch M <= 4 are HBM-bound matrix-vector products:
// each wave streams two weight rows in 16-byte chunks (8 chunks of each row
// in flight per lane), the activations sit in LDS (staged, and normalised
// when a norm weight is given, by every workgroup), and a 64-lane butterfly
// reduces each row.  No MFMA: one multiply-add per weight element.
#include "nfa_common.h"

namespace nfa {

constexpr int LIN_WAVES = 4;
constexpr int LIN_CPI = 8;                     // chunks per lane per iteration
constexpr int LIN_MMAX = 4;
constexpr int LIN_LDS_BYTES = 48 * 1024;

__device__ __forceinline__ float bf_lo(uint32_t u) { return __uint_as_float(u << 16); }
__device__ __forceinline__ float bf_hi(uint32_t u) {
  return __uint_as_float(u & 0xFFFF0000u);
}

__device__ __forceinline__ float dot8(const uint4 &w, const uint4 &x, float acc) {
  acc = fmaf(bf_lo(w.x), bf_lo(x.x), acc);
  acc = fmaf(bf_hi(w.x), bf_hi(x.x), acc);
  acc = fmaf(bf_lo(w.y), bf_lo(x.y), acc);
  acc = fmaf(bf_hi(w.y), bf_hi(x.y), acc);
  acc = fmaf(bf_lo(w.z), bf_lo(x.z), acc);
  acc = fmaf(bf_hi(w.z), bf_hi(x.z), acc);
  acc = fmaf(bf_lo(w.w), bf_lo(x.w), acc);
  acc = fmaf(bf_hi(w.w), bf_hi(x.w), acc);
  return acc;
}

__device__ __forceinline__ float sumsq8(const uint4 &x, float acc) {
  const uint32_t v[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float a = bf_lo(v[i]), b = bf_hi(v[i]);
    acc = acc + a * a;
    acc = acc + b * b;
  }
  return acc;
}

__device__ __forceinline__ uint32_t pack2(float lo, float hi) {
  return (uint32_t)bf16_bits(lo) | ((uint32_t)bf16_bits(hi) << 16);
}

// HF RMSNorm of 8 elements: bf16(w * bf16(x * rstd)).
__device__ __forceinline__ uint4 norm8(const uint4 &x, const uint4 &w, float rstd) {
  const uint32_t xv[4] = {x.x, x.y, x.z, x.w};
  const uint32_t wv[4] = {w.x, w.y, w.z, w.w};
  uint32_t o[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float a = bf16r(bf_lo(xv[i]) * rstd), b = bf16r(bf_hi(xv[i]) * rstd);
    o[i] = pack2(bf_lo(wv[i]) * a, bf_hi(wv[i]) * b);
  }
  return make_uint4(o[0], o[1], o[2], o[3]);
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

// Sum of squares of one row over the workgroup, then rstd = rsqrt(mean + eps)
// (mean = sum * (1/K), as torch's mean).
__device__ float block_rstd(float ss, int k, float eps, float *s_red) {
  ss = wave_sum(ss);
  const int w = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) s_red[w] = ss;
  __syncthreads();
  float t = 0.0f;
  for (int i = 0; i < (int)(blockDim.x >> 6); ++i) t = t + s_red[i];
  return rsqrtf(t * (1.0f / (float)k) + eps);
}

// Stage x [m][k] into LDS as 16-byte chunks, RMS-normalised when NORM.
template <bool NORM>
__device__ void stage_x(const NfaLinearParams &p, int nch, uint4 *s_x, float *s_red) {
  for (int m = 0; m < p.m; ++m) {
    const uint4 *xr = reinterpret_cast<const uint4 *>(
        (const uint16_t *)p.x + (int64_t)m * p.x_stride);
    float ss = 0.0f;
    for (int c = threadIdx.x; c < nch; c += blockDim.x) {
      const uint4 v = xr[c];
      s_x[m * nch + c] = v;
      if (NORM) ss = sumsq8(v, ss);
    }
    if (NORM) {
      const float rstd = block_rstd(ss, p.k, p.norm_eps, s_red);
      const uint4 *wr = reinterpret_cast<const uint4 *>(p.norm_weight);
      for (int c = threadIdx.x; c < nch; c += blockDim.x)
        s_x[m * nch + c] = norm8(s_x[m * nch + c], wr[c], rstd);
    }
  }
  __syncthreads();
}

// Weight row `row` of the concatenated segments: its base pointer, or null.
__device__ __forceinline__ const uint4 *seg_row(const NfaLinearParams &p, int row,
                                                int *seg, int *local) {
  int r = row;
#pragma unroll
  for (int s = 0; s < 3; ++s) {
    if (s < p.nseg && r < p.n[s]) {
      *seg = s;
      *local = r;
      return reinterpret_cast<const uint4 *>((const uint16_t *)p.w[s] +
                                             (int64_t)r * p.k);
    }
    if (s < p.nseg) r -= p.n[s];
  }
  *seg = -1;
  *local = 0;
  return nullptr;
}

// v when keep, else zeros (component-wise selects: a select of the whole
// vector is lowered through scratch memory)
__device__ __forceinline__ uint4 keep4(bool keep, const uint4 &v) {
  return make_uint4(keep ? v.x : 0u, keep ? v.y : 0u, keep ? v.z : 0u, keep ? v.w : 0u);
}

// One iteration's weight chunks of two rows: chunk base + 64 j + lane of
// each row, zeros past the row end or for a missing second row.  The loads
// themselves are unconditional (clamped to the row's last chunk) so that all
// of them are in flight before the first is waited for.  w0 is not null.
template <int CPI>
__device__ __forceinline__ void load_iter(const uint4 *w0, const uint4 *w1, int base,
                                          int nch, uint4 (&a)[CPI], uint4 (&b)[CPI]) {
  const int lane = threadIdx.x & 63;
  const uint4 *p1 = w1 ? w1 : w0;
#pragma unroll
  for (int j = 0; j < CPI; ++j) {
    const int c = base + j * 64 + lane;
    const int cc = c < nch ? c : nch - 1;
    a[j] = w0[cc];
    b[j] = p1[cc];
  }
#pragma unroll
  for (int j = 0; j < CPI; ++j) {
    const bool in = base + j * 64 + lane < nch;
    a[j] = keep4(in, a[j]);
    b[j] = keep4(in && w1, b[j]);
  }
}

// Multiply-add one iteration's chunks with every x row: acc[r][m] per lane.
template <int MM, int CPI>
__device__ __forceinline__ void dot_iter(const uint4 (&a)[CPI], const uint4 (&b)[CPI],
                                         int base, int nch, const uint4 *s_x,
                                         float (&acc)[2][LIN_MMAX]) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int j = 0; j < CPI; ++j) {
    const int c = base + j * 64 + lane;
    if (c >= nch) break;
#pragma unroll
    for (int m = 0; m < MM; ++m) {
      const uint4 xv = s_x[m * nch + c];
      acc[0][m] = dot8(a[j], xv, acc[0][m]);
      acc[1][m] = dot8(b[j], xv, acc[1][m]);
    }
  }
}

__device__ __forceinline__ uint16_t ld_bf(const void *base, int64_t i) {
  return ((const uint16_t *)base)[i];
}

// PRO: 0 no norm, 1 norm then the first weight loads, 2 the first weight
// loads in flight through the norm (for grids that fit on the device at
// once: holding those registers through the prologue costs occupancy).
template <int EPI, int PRO, int MM>
__global__ void __launch_bounds__(NFA_BLOCK)
    linear_kernel(const NfaLinearParams p) {
  constexpr bool NORM = PRO != 0;
  extern __shared__ uint4 s_x[];
  __shared__ float s_red[NFA_WAVES];
  const int nch = p.k / 8;
  const int lane = threadIdx.x & 63;
  const int unit = blockIdx.x * LIN_WAVES + (threadIdx.x >> 6);  // wave's work

  // the wave's two weight rows: gate and up row `unit` (SiLU gate), else rows
  // 2 unit and 2 unit + 1 of the concatenated segments
  const uint4 *w0 = nullptr, *w1 = nullptr;
  int seg[2] = {-1, -1}, loc[2] = {0, 0};
  if (EPI == NFA_EPI_SILU_GATE) {
    if (unit < p.n[0]) {
      w0 = reinterpret_cast<const uint4 *>((const uint16_t *)p.w[0] + (int64_t)unit * p.k);
      w1 = reinterpret_cast<const uint4 *>((const uint16_t *)p.w[1] + (int64_t)unit * p.k);
    }
  } else {
    w0 = seg_row(p, unit * 2, &seg[0], &loc[0]);
    w1 = seg_row(p, unit * 2 + 1, &seg[1], &loc[1]);
  }
  // Two buffers of half an iteration each: the next half's loads are in
  // flight while the current half is multiplied.  The first weight chunks
  // are in flight while the activations are staged, unless a norm prologue
  // would hold them at the cost of occupancy (PRO 1).
  constexpr int HC = LIN_CPI / 2;
  constexpr int STEP = 64 * HC;
  uint4 a0[HC], b0[HC], a1[HC], b1[HC];
  if (PRO != 1 && w0) {
    load_iter<HC>(w0, w1, 0, nch, a0, b0);
    load_iter<HC>(w0, w1, STEP, nch, a1, b1);
  }
  stage_x<NORM>(p, nch, s_x, s_red);
  if (!w0) return;
  if (PRO == 1) {
    load_iter<HC>(w0, w1, 0, nch, a0, b0);
    load_iter<HC>(w0, w1, STEP, nch, a1, b1);
  }

  float acc[2][LIN_MMAX];
#pragma unroll
  for (int r = 0; r < 2; ++r)
#pragma unroll
    for (int m = 0; m < LIN_MMAX; ++m) acc[r][m] = 0.0f;
  for (int base = 0; base < nch; base += 2 * STEP) {
    dot_iter<MM, HC>(a0, b0, base, nch, s_x, acc);
    if (base + 2 * STEP < nch) load_iter<HC>(w0, w1, base + 2 * STEP, nch, a0, b0);
    if (base + STEP < nch) dot_iter<MM, HC>(a1, b1, base + STEP, nch, s_x, acc);
    if (base + 3 * STEP < nch) load_iter<HC>(w0, w1, base + 3 * STEP, nch, a1, b1);
  }

  if (EPI == NFA_EPI_SILU_GATE) {
#pragma unroll
    for (int m = 0; m < MM; ++m) {
      const float g = bf16r(wave_sum(acc[0][m]));
      const float u = bf16r(wave_sum(acc[1][m]));
      if (lane == m) {
        const float act = bf16r(g / (1.0f + expf(-g)));
        ((uint16_t *)p.y[0])[(int64_t)m * p.y_stride[0] + unit] = bf16_bits(act * u);
      }
    }
    return;
  }
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    if (seg[r] < 0) break;
#pragma unroll
    for (int m = 0; m < MM; ++m) {
      const float s = bf16r(wave_sum(acc[r][m]));
      if (lane == m) {
        float out = s;
        if (EPI == NFA_EPI_RESIDUAL)
          out = bf16_val(ld_bf(p.residual, (int64_t)m * p.residual_stride + loc[r])) + s;
        ((uint16_t *)p.y[seg[r]])[(int64_t)m * p.y_stride[seg[r]] + loc[r]] =
            bf16_bits(out);
      }
    }
  }
}

// Per-head q/k RMSNorm (optional) and rotate-half RoPE, one wave per head.
// out[i] = bf16(bf16(x[i] cos[i]) + bf16(-x[i+P] sin[i])), i < P = D/2, and
// out[i+P] = bf16(bf16(x[i+P] cos[i+P]) + bf16(x[i] sin[i+P])): HF's
// apply_rotary_pos_emb with each bf16 op rounded.
__global__ void __launch_bounds__(NFA_BLOCK)
    qk_rope_kernel(const NfaRopeParams p) {
  const int lane = threadIdx.x & 63;
  const int head = blockIdx.x * NFA_WAVES + (threadIdx.x >> 6);
  const int heads = p.hq + p.hkv;
  if (head >= p.batch * heads) return;
  const int b = head / heads, h = head % heads;
  const bool is_q = h < p.hq;
  const int hh = is_q ? h : h - p.hq;
  const uint16_t *x = (const uint16_t *)(is_q ? p.q : p.k) +
                      (int64_t)b * (is_q ? p.q_stride_b : p.k_stride_b) +
                      (int64_t)hh * p.head_dim;
  const uint16_t *wt = (const uint16_t *)(is_q ? p.q_weight : p.k_weight);
  uint16_t *out = (uint16_t *)(is_q ? p.q_out : p.k_out) +
                  ((int64_t)b * (is_q ? p.hq : p.hkv) + hh) * p.head_dim;
  const uint16_t *cs = (const uint16_t *)p.cos + (int64_t)b * p.cs_stride_b;
  const uint16_t *sn = (const uint16_t *)p.sin + (int64_t)b * p.cs_stride_b;
  const int P = p.head_dim / 2;
  // lane owns pairs (i, i + P) for i = lane, lane + 64
  float lo[2], hi[2];
  float ss = 0.0f;
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int i = lane + 64 * j;
    lo[j] = hi[j] = 0.0f;
    if (i < P) {
      lo[j] = bf16_val(x[i]);
      hi[j] = bf16_val(x[i + P]);
      ss = ss + lo[j] * lo[j];
      ss = ss + hi[j] * hi[j];
    }
  }
  if (wt) {
    const float rstd = rsqrtf(wave_sum(ss) * (1.0f / (float)p.head_dim) + p.eps);
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int i = lane + 64 * j;
      if (i < P) {
        lo[j] = bf16r(bf16_val(wt[i]) * bf16r(lo[j] * rstd));
        hi[j] = bf16r(bf16_val(wt[i + P]) * bf16r(hi[j] * rstd));
      }
    }
  }
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int i = lane + 64 * j;
    if (i < P) {
      const float c0 = bf16_val(cs[i]), s0 = bf16_val(sn[i]);
      const float c1 = bf16_val(cs[i + P]), s1 = bf16_val(sn[i + P]);
      out[i] = bf16_bits(bf16r(lo[j] * c0) + bf16r(-hi[j] * s0));
      out[i + P] = bf16_bits(bf16r(hi[j] * c1) + bf16r(lo[j] * s1));
    }
  }
}

// HF RMSNorm of each row: one workgroup per row.
__global__ void __launch_bounds__(NFA_BLOCK)
    rmsnorm_kernel(const void *x, int64_t x_stride, const void *weight, void *out,
                   int64_t out_stride, int dim, float eps) {
  __shared__ float s_red[NFA_WAVES];
  const int nch = dim / 8;
  const uint4 *xr = reinterpret_cast<const uint4 *>((const uint16_t *)x +
                                                    (int64_t)blockIdx.x * x_stride);
  uint4 *orow = reinterpret_cast<uint4 *>((uint16_t *)out +
                                          (int64_t)blockIdx.x * out_stride);
  const uint4 *wr = reinterpret_cast<const uint4 *>(weight);
  float ss = 0.0f;
  for (int c = threadIdx.x; c < nch; c += blockDim.x) ss = sumsq8(xr[c], ss);
  const float rstd = block_rstd(ss, dim, eps, s_red);
  for (int c = threadIdx.x; c < nch; c += blockDim.x)
    orow[c] = norm8(xr[c], wr[c], rstd);
}

}  // namespace nfa

namespace {

bool aligned16(const void *ptr) { return ((uintptr_t)ptr & 15u) == 0; }

}  // namespace

extern "C" int32_t nfa_linear_params_size(void) { return (int32_t)sizeof(NfaLinearParams); }
extern "C" int32_t nfa_rope_params_size(void) { return (int32_t)sizeof(NfaRopeParams); }

extern "C" int32_t nfa_decode_linear(const NfaLinearParams *p, void *stream) {
  if (p == nullptr || p->abi_version != NFA_ABI_VERSION ||
      p->struct_size != (int32_t)sizeof(NfaLinearParams)) {
    nfa_set_error("nfa_decode_linear: ABI mismatch");
    return NFA_EINVAL;
  }
  if (p->m < 1 || p->m > nfa::LIN_MMAX || p->k < 8 || p->k % 8 != 0 ||
      (int64_t)p->m * p->k * 2 > nfa::LIN_LDS_BYTES) {
    nfa_set_error("nfa_decode_linear: unsupported m=%d k=%d (m <= 4, k %% 8 == 0, "
                  "m*k*2 <= %d bytes)", p->m, p->k, nfa::LIN_LDS_BYTES);
    return NFA_EINVAL;
  }
  if (p->nseg < 1 || p->nseg > 3 || !p->x || !aligned16(p->x) || p->x_stride % 8 != 0 ||
      (p->m > 1 && p->x_stride < p->k) ||
      (p->norm_weight && !aligned16(p->norm_weight))) {
    nfa_set_error("nfa_decode_linear: bad segments or activation layout");
    return NFA_EINVAL;
  }
  int64_t rows = 0;
  for (int s = 0; s < p->nseg; ++s) {
    if (!p->w[s] || !aligned16(p->w[s]) || !p->y[s] || p->n[s] < 1 ||
        p->y_stride[s] < p->n[s]) {
      nfa_set_error("nfa_decode_linear: bad weight/output segment %d", s);
      return NFA_EINVAL;
    }
    rows += p->n[s];
  }
  int64_t units;
  if (p->epilogue == NFA_EPI_SILU_GATE) {
    if (p->nseg != 2 || p->n[0] != p->n[1]) {
      nfa_set_error("nfa_decode_linear: SiLU gate needs gate and up of equal rows");
      return NFA_EINVAL;
    }
    units = p->n[0];
  } else if (p->epilogue == NFA_EPI_PLAIN || p->epilogue == NFA_EPI_RESIDUAL) {
    if (p->epilogue == NFA_EPI_RESIDUAL && (p->nseg != 1 || !p->residual)) {
      nfa_set_error("nfa_decode_linear: residual epilogue needs one segment");
      return NFA_EINVAL;
    }
    units = (rows + 1) / 2;
  } else {
    nfa_set_error("nfa_decode_linear: unknown epilogue %d", p->epilogue);
    return NFA_EINVAL;
  }
  const int64_t blocks = (units + nfa::LIN_WAVES - 1) / nfa::LIN_WAVES;
  if (blocks > 0x7FFFFFFF) {
    nfa_set_error("nfa_decode_linear: too many rows");
    return NFA_EINVAL;
  }
  const size_t lds = (size_t)p->m * p->k * 2;
  hipStream_t s = (hipStream_t)stream;
  const bool norm = p->norm_weight != nullptr;
  // a grid of at most four workgroups (16 waves) per CU runs in one round:
  // its first weight loads can be in flight through the norm prologue
  const bool early = blocks <= (int64_t)4 * nfa::device_cus();
#define NFA_LIN(E, N, M)                                                          \
  hipLaunchKernelGGL((nfa::linear_kernel<E, N, M>), dim3((unsigned)blocks),    \
                     dim3(NFA_BLOCK), lds, s, *p)
#define NFA_LIN_M(E, N)                                            \
  switch (p->m) {                                                  \
    case 1: NFA_LIN(E, N, 1); break;                               \
    case 2: NFA_LIN(E, N, 2); break;                               \
    case 3: NFA_LIN(E, N, 3); break;                               \
    default: NFA_LIN(E, N, 4); break;                              \
  }
#define NFA_LIN_P(E)                                                              \
  if (!norm) { NFA_LIN_M(E, 0) } else if (early) { NFA_LIN_M(E, 2) } else { NFA_LIN_M(E, 1) }
  if (p->epilogue == NFA_EPI_SILU_GATE) {
    NFA_LIN_P(NFA_EPI_SILU_GATE)
  } else if (p->epilogue == NFA_EPI_RESIDUAL) {
    NFA_LIN_P(NFA_EPI_RESIDUAL)
  } else {
    NFA_LIN_P(NFA_EPI_PLAIN)
  }
#undef NFA_LIN_P
#undef NFA_LIN_M
#undef NFA_LIN
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess) {
    nfa_set_error("nfa_decode_linear: launch failed: %s", hipGetErrorString(err));
    return NFA_ELAUNCH;
  }
  return NFA_OK;
}

extern "C" int32_t nfa_qk_norm_rope_decode(const NfaRopeParams *p, void *stream) {
  if (p == nullptr || p->abi_version != NFA_ABI_VERSION ||
      p->struct_size != (int32_t)sizeof(NfaRopeParams)) {
    nfa_set_error("nfa_qk_norm_rope_decode: ABI mismatch");
    return NFA_EINVAL;
  }
  if (p->batch < 0 || p->hq < 1 || p->hkv < 1 || p->head_dim < 2 ||
      p->head_dim % 2 != 0 || p->head_dim > 256) {
    nfa_set_error("nfa_qk_norm_rope_decode: unsupported heads %d/%d dim %d",
                  p->hq, p->hkv, p->head_dim);
    return NFA_EINVAL;
  }
  if (p->batch == 0) return NFA_OK;
  if (!p->q || !p->k || !p->cos || !p->sin || !p->q_out || !p->k_out ||
      (!p->q_weight) != (!p->k_weight)) {
    nfa_set_error("nfa_qk_norm_rope_decode: null pointer");
    return NFA_EINVAL;
  }
  const int64_t heads = (int64_t)p->batch * (p->hq + p->hkv);
  const unsigned blocks = (unsigned)((heads + NFA_WAVES - 1) / NFA_WAVES);
  hipLaunchKernelGGL(nfa::qk_rope_kernel, dim3(blocks), dim3(NFA_BLOCK), 0,
                     (hipStream_t)stream, *p);
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess) {
    nfa_set_error("nfa_qk_norm_rope_decode: launch failed: %s", hipGetErrorString(err));
    return NFA_ELAUNCH;
  }
  return NFA_OK;
}

extern "C" int32_t nfa_rmsnorm_decode(const void *x, int64_t x_stride, const void *weight,
                                      void *out, int64_t out_stride, int32_t rows,
                                      int32_t dim, float eps, void *stream) {
  if (rows < 0 || dim < 8 || dim % 8 != 0 || x_stride % 8 != 0 || out_stride % 8 != 0) {
    nfa_set_error("nfa_rmsnorm_decode: unsupported rows=%d dim=%d", rows, dim);
    return NFA_EINVAL;
  }
  if (rows == 0) return NFA_OK;
  if (!x || !weight || !out || !aligned16(x) || !aligned16(weight) || !aligned16(out)) {
    nfa_set_error("nfa_rmsnorm_decode: null or unaligned pointer");
    return NFA_EINVAL;
  }
  hipLaunchKernelGGL(nfa::rmsnorm_kernel, dim3((unsigned)rows), dim3(NFA_BLOCK), 0,
                     (hipStream_t)stream, x, x_stride, weight, out, out_stride, dim, eps);
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess) {
    nfa_set_error("nfa_rmsnorm_decode: launch failed: %s", hipGetErrorString(err));
    return NFA_ELAUNCH;
  }
  return NFA_OK;
}
