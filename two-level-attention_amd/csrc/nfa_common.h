// Device helpers shared by the NFA selector and attention kernels (gfx950).
//
// Arithmetic contract (shared with the CPU oracle): fp32 reductions are
// sequential, index ascending, from +0.0, with separately rounded multiply and
// add.  This file is compiled with -ffp-contract=off and additionally turns
// contraction off with a pragma so no FMA is formed behind our back.
#pragma once
#pragma clang fp contract(off)

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/nfa_hip.h"

#define NFA_BLOCK 256
#define NFA_WAVES (NFA_BLOCK / 64)

namespace nfa {

// ---------------------------------------------------------------------------
// bf16 and ordering
// ---------------------------------------------------------------------------

// fp32 -> bf16 bits, round to nearest even; any NaN -> 0x7FC0.
__device__ __forceinline__ uint16_t bf16_bits(float x) {
  uint32_t u = __float_as_uint(x);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return 0x7FC0u;
  u += 0x7FFFu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

__device__ __forceinline__ float bf16_val(uint16_t b) {
  return __uint_as_float(((uint32_t)b) << 16);
}

__device__ __forceinline__ float bf16r(float x) { return bf16_val(bf16_bits(x)); }

// Order-preserving 16-bit key of bf16 bits: +0 > -0, +NaN highest.
__device__ __forceinline__ uint32_t ord16u(uint32_t b) {
  return (b & 0x8000u) ? ((~b) & 0xFFFFu) : (b | 0x8000u);
}

constexpr uint16_t kNegInfBits = 0xFF80u;
constexpr uint16_t kNanBits = 0x7FC0u;

// Valid-score key: 0 marks -inf (never selected as a scored entry).  With
// canonical NaN nothing ranks below -inf, so every other score maps to > 0.
__device__ __forceinline__ uint32_t score_key(uint16_t bits) {
  return bits == kNegInfBits ? 0u : ord16u(bits);
}

// ---------------------------------------------------------------------------
// typed loads of KV / query elements
// ---------------------------------------------------------------------------

template <typename T> struct Elem;
template <> struct Elem<uint16_t> {  // bf16 storage
  static __device__ __forceinline__ float load(const uint16_t *p) {
    return bf16_val(*p);
  }
  static __device__ __forceinline__ uint16_t from_f32(float x) {
    return bf16_bits(x);
  }
  static constexpr int kChunk = 8;  // elements per 16 bytes
};
template <> struct Elem<float> {
  static __device__ __forceinline__ float load(const float *p) { return *p; }
  static __device__ __forceinline__ float from_f32(float x) { return x; }
  static constexpr int kChunk = 4;
};

__device__ __forceinline__ float load_any(const void *base, int64_t idx,
                                          int dtype) {
  if (dtype == NFA_DTYPE_BF16)
    return bf16_val(((const uint16_t *)base)[idx]);
  return ((const float *)base)[idx];
}

// 16-byte vector load of one chunk of T elements into floats.
template <typename T>
__device__ __forceinline__ void load_chunk(const T *p, float *out) {
  const uint4 v = *reinterpret_cast<const uint4 *>(p);
  if constexpr (sizeof(T) == 2) {
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      out[2 * i] = __uint_as_float(w[i] << 16);
      out[2 * i + 1] = __uint_as_float(w[i] & 0xFFFF0000u);
    }
  } else {
    out[0] = __uint_as_float(v.x);
    out[1] = __uint_as_float(v.y);
    out[2] = __uint_as_float(v.z);
    out[3] = __uint_as_float(v.w);
  }
}

// ---------------------------------------------------------------------------
// block-level (256 threads) scans and reductions
// ---------------------------------------------------------------------------

__device__ __forceinline__ int lane_id() { return threadIdx.x & 63; }
__device__ __forceinline__ int wave_id() { return threadIdx.x >> 6; }

// Exclusive count of `pred` over the block in thread order; *total receives
// the block total.  `scratch` needs NFA_WAVES ints.  Contains two barriers.
__device__ __forceinline__ int block_count_exclusive(bool pred, int *scratch,
                                                     int *total) {
  const unsigned long long mask = __ballot(pred);
  const int lane = lane_id();
  const int w = wave_id();
  const unsigned long long below = lane ? (mask & ((1ull << lane) - 1ull)) : 0ull;
  const int in_wave = __popcll(below);
  if (lane == 0) scratch[w] = __popcll(mask);
  __syncthreads();
  int before = 0, sum = 0;
#pragma unroll
  for (int i = 0; i < NFA_WAVES; ++i) {
    const int c = scratch[i];
    if (i < w) before += c;
    sum += c;
  }
  __syncthreads();
  *total = sum;
  return before + in_wave;
}

// Exclusive prefix sum of an int over the block; two barriers.
__device__ __forceinline__ int block_scan_exclusive(int v, int *scratch,
                                                    int *total) {
  const int lane = lane_id();
  const int w = wave_id();
  int x = v;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int y = __shfl_up(x, off, 64);
    if (lane >= off) x += y;
  }
  if (lane == 63) scratch[w] = x;
  __syncthreads();
  int before = 0, sum = 0;
#pragma unroll
  for (int i = 0; i < NFA_WAVES; ++i) {
    const int c = scratch[i];
    if (i < w) before += c;
    sum += c;
  }
  __syncthreads();
  *total = sum;
  return before + x - v;
}

// Given a 256-bin histogram in LDS and K >= 1, find the bin b with
// above(b) < K <= above(b) + hist[b], where above(b) counts entries in bins
// greater than b.  Executed by wave 0; results land in out[0] (bin) and
// out[1] (above).  Requires K <= total count.  Caller syncs afterwards.
__device__ __forceinline__ void find_threshold_bin(const int *hist, int K,
                                                   int *out) {
  if (wave_id() != 0) return;
  const int lane = lane_id();
  const int h0 = hist[4 * lane + 0], h1 = hist[4 * lane + 1];
  const int h2 = hist[4 * lane + 2], h3 = hist[4 * lane + 3];
  const int s = h0 + h1 + h2 + h3;
  // inclusive suffix sum over lanes (lane l sums lanes l..63)
  int x = s;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int y = __shfl_down(x, off, 64);
    if (lane + off < 64) x += y;
  }
  int above = x - s;  // entries in lanes > lane
  // bins in descending order within the lane: 3, 2, 1, 0
  const int hb[4] = {h3, h2, h1, h0};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    if (above < K && K <= above + hb[i]) {
      out[0] = 4 * lane + 3 - i;
      out[1] = above;
    }
    above += hb[i];
  }
}

// Threshold of the top-K among `n` 16-bit keys (0 = invalid) supplied by
// `get(i)`.  Returns via out: out[0] = threshold key T, out[1] = number of
// entries equal to T that are selected (the lowest-index ones), out[2] =
// number of valid entries.  If valid <= K every valid entry is selected and
// out[0] = 1, out[1] = large.  `hist` needs 256 ints, `tmp` 8 ints.
template <typename Get>
__device__ void topk_threshold16(Get get, int n, int K, int *hist, int *tmp,
                                 int *out) {
  const int tid = threadIdx.x;
  for (int i = tid; i < 256; i += NFA_BLOCK) hist[i] = 0;
  __syncthreads();
  int local_valid = 0;
  for (int i = tid; i < n; i += NFA_BLOCK) {
    const uint32_t v = get(i);
    if (v) {
      atomicAdd(&hist[v >> 8], 1);
      ++local_valid;
    }
  }
  int total_valid;
  block_scan_exclusive(local_valid, tmp, &total_valid);
  if (total_valid <= K) {
    if (tid == 0) {
      out[0] = 1;
      out[1] = 1 << 30;
      out[2] = total_valid;
    }
    __syncthreads();
    return;
  }
  find_threshold_bin(hist, K, tmp + 4);
  __syncthreads();
  const int hb = tmp[4];
  const int above_hb = tmp[5];
  __syncthreads();
  for (int i = tid; i < 256; i += NFA_BLOCK) hist[i] = 0;
  __syncthreads();
  for (int i = tid; i < n; i += NFA_BLOCK) {
    const uint32_t v = get(i);
    if (v && (int)(v >> 8) == hb) atomicAdd(&hist[v & 255u], 1);
  }
  __syncthreads();
  find_threshold_bin(hist, K - above_hb, tmp + 4);
  __syncthreads();
  if (tid == 0) {
    const int lb = tmp[4];
    const int above_lb = tmp[5];
    out[0] = (hb << 8) | lb;
    out[1] = K - above_hb - above_lb;
    out[2] = total_valid;
  }
  __syncthreads();
}

// Upper bound: first index in sorted a[0..n) with a[idx] > x.
__device__ __forceinline__ int upper_bound_i32(const int *a, int n, int x) {
  int lo = 0, hi = n;
  while (lo < hi) {
    const int mid = (lo + hi) >> 1;
    if (a[mid] <= x)
      lo = mid + 1;
    else
      hi = mid;
  }
  return lo;
}

// Lower bound: first index with a[idx] >= x.
__device__ __forceinline__ int lower_bound_i32(const int *a, int n, int x) {
  int lo = 0, hi = n;
  while (lo < hi) {
    const int mid = (lo + hi) >> 1;
    if (a[mid] < x)
      lo = mid + 1;
    else
      hi = mid;
  }
  return lo;
}

}  // namespace nfa

// error reporting shared by the entry points (defined in nfa_capi.hip)
extern "C" void nfa_set_error(const char *fmt, ...);
