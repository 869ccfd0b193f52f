// Device helpers shared by the NFA selector and attention kernels (gfx950).
//
// Arithmetic contract (shared with the CPU oracle): fp32 reductions are
// sequential, index ascending, from +0.0.  The selector's dot products (L1
// page scores, L2 logits) add each exact product with one rounding, an
// explicit fused multiply-add per term; every other product is rounded
// before its add.  This file is compiled with -ffp-contract=off and
// additionally turns contraction off with a pragma, so the only FMAs are the
// explicit ones.
#pragma once
#pragma clang fp contract(off)

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/nfa_hip.h"

// Branch hint for paths the steady decode step does not take (debug
// outputs, rebuilds, rare geometries): the compiler lays them out after the
// hot code, which keeps the executed instruction stream contiguous.
#define NFA_COLD(x) __builtin_expect(!!(x), 0)

#define NFA_BLOCK 256
#define NFA_WAVES (NFA_BLOCK / 64)

namespace nfa {

// Compute units of the current device (cached per device; 256 when the
// runtime cannot tell).
inline int device_cus() {
  static int cached[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  int v = __atomic_load_n(&cached[dev], __ATOMIC_RELAXED);
  if (v <= 0) {
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) !=
            hipSuccess ||
        v <= 0)
      v = 256;
    __atomic_store_n(&cached[dev], v, __ATOMIC_RELAXED);
  }
  return v;
}

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

// bf16r through gfx950's conversion instruction (v_cvt_pk_bf16_f32, round
// to nearest even with denormals kept): the same value as bf16r for every
// non-NaN fp32 input -- compared over all 2^32 bit patterns on the device
// -- in two instructions; a NaN input gives a NaN of another payload.
__device__ __forceinline__ float bf16r_hw(float x) { return (float)(__bf16)x; }

// Two roundings in one conversion (the same round-to-nearest-even per value).
typedef __bf16 nfa_bf16x2 __attribute__((ext_vector_type(2)));
typedef float nfa_f32x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ void bf16r_hw2(float a, float b, float &ra, float &rb) {
  const nfa_f32x2 v = {a, b};
  const nfa_bf16x2 h = __builtin_convertvector(v, nfa_bf16x2);
  ra = (float)h.x;
  rb = (float)h.y;
}

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

// 16 bytes of KV elements (already in registers) as floats.
template <typename KV>
__device__ __forceinline__ void unpack_chunk(const uint4 &raw, float *out) {
  load_chunk<KV>(reinterpret_cast<const KV *>(&raw), out);
}

// Touches every 64-byte line of the kernel arguments (BYTES explicit bytes,
// at most 12 lines) with independent scalar loads and one wait: the compiler
// reads the arguments where it needs them, one dependent scalar-cache miss
// per line, which at kernel start costs several memory latencies in a row.
// The loads and the wait are one asm statement, so no load is in flight when
// it ends; lines past the last one repeat it.
template <int BYTES>
__device__ __forceinline__ void warm_kernargs() {
  static_assert(BYTES > 0 && BYTES <= 12 * 64, "at most 12 argument lines");
  constexpr int last = (BYTES - 1) / 64;
  auto k = __builtin_amdgcn_kernarg_segment_ptr();
  uint32_t d0, d1, d2, d3, d4, d5, d6, d7, d8, d9, d10, d11;
  asm volatile(
      "s_load_dword %0, %12, %13\n"
      "s_load_dword %1, %12, %14\n"
      "s_load_dword %2, %12, %15\n"
      "s_load_dword %3, %12, %16\n"
      "s_load_dword %4, %12, %17\n"
      "s_load_dword %5, %12, %18\n"
      "s_load_dword %6, %12, %19\n"
      "s_load_dword %7, %12, %20\n"
      "s_load_dword %8, %12, %21\n"
      "s_load_dword %9, %12, %22\n"
      "s_load_dword %10, %12, %23\n"
      "s_load_dword %11, %12, %24\n"
      "s_waitcnt lgkmcnt(0)"
      : "=&s"(d0), "=&s"(d1), "=&s"(d2), "=&s"(d3), "=&s"(d4), "=&s"(d5),
        "=&s"(d6), "=&s"(d7), "=&s"(d8), "=&s"(d9), "=&s"(d10), "=&s"(d11)
      : "s"(k), "i"(0), "i"((1 < last ? 1 : last) * 64),
        "i"((2 < last ? 2 : last) * 64), "i"((3 < last ? 3 : last) * 64),
        "i"((4 < last ? 4 : last) * 64), "i"((5 < last ? 5 : last) * 64),
        "i"((6 < last ? 6 : last) * 64), "i"((7 < last ? 7 : last) * 64),
        "i"((8 < last ? 8 : last) * 64), "i"((9 < last ? 9 : last) * 64),
        "i"((10 < last ? 10 : last) * 64), "i"((11 < last ? 11 : last) * 64));
}

// Wave-uniform values read through the scalar cache, all loads issued
// together and awaited once inside the asm statement (nothing is in flight
// when it ends; vector loads issued before it stay in flight).  The data was
// written before the kernel started or is not written by it.
__device__ __forceinline__ void sload_i32x4(const int32_t *pa, const int32_t *pb,
                                            const int32_t *pc, const int32_t *pd,
                                            int32_t &a, int32_t &b, int32_t &c,
                                            int32_t &d) {
  asm volatile(
      "s_load_dword %0, %4, 0x0\n"
      "s_load_dword %1, %5, 0x0\n"
      "s_load_dword %2, %6, 0x0\n"
      "s_load_dword %3, %7, 0x0\n"
      "s_waitcnt lgkmcnt(0)"
      : "=&s"(a), "=&s"(b), "=&s"(c), "=&s"(d)
      : "s"(pa), "s"(pb), "s"(pc), "s"(pd));
}

__device__ __forceinline__ void sload_row(const int32_t *pl, const int64_t *pa,
                                          const int64_t *pr, const int32_t *ps,
                                          int32_t &l, int64_t &a, int64_t &r,
                                          int32_t &s) {
  asm volatile(
      "s_load_dword %0, %4, 0x0\n"
      "s_load_dwordx2 %1, %5, 0x0\n"
      "s_load_dwordx2 %2, %6, 0x0\n"
      "s_load_dword %3, %7, 0x0\n"
      "s_waitcnt lgkmcnt(0)"
      : "=&s"(l), "=&s"(a), "=&s"(r), "=&s"(s)
      : "s"(pl), "s"(pa), "s"(pr), "s"(ps));
}

// Workgroup barrier that orders the LDS instructions (ds_*) only: global
// loads and stores and asynchronous global-to-LDS loads in flight stay in
// flight (__syncthreads, and an LDS fence, wait for all of them).  The
// memory clobber keeps the compiler from moving memory accesses across it.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// 8 floats from 16-byte aligned memory (LDS or global) as two 16-byte loads.
__device__ __forceinline__ void load_f8(const float *src, float *out) {
  const float4 a = reinterpret_cast<const float4 *>(src)[0];
  const float4 b = reinterpret_cast<const float4 *>(src)[1];
  out[0] = a.x; out[1] = a.y; out[2] = a.z; out[3] = a.w;
  out[4] = b.x; out[5] = b.y; out[6] = b.z; out[7] = b.w;
}

// CH floats that are exact KV values back into 16 bytes of KV elements.
template <typename KV>
__device__ __forceinline__ uint4 pack_chunk(const float *x) {
  if constexpr (sizeof(KV) == 2) {
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
      w[i] = (__float_as_uint(x[2 * i]) >> 16) |
             (__float_as_uint(x[2 * i + 1]) & 0xFFFF0000u);
    return make_uint4(w[0], w[1], w[2], w[3]);
  } else {
    return make_uint4(__float_as_uint(x[0]), __float_as_uint(x[1]),
                      __float_as_uint(x[2]), __float_as_uint(x[3]));
  }
}

// ---------------------------------------------------------------------------
// cross-workgroup publication ("last arriving workgroup" pattern)
// ---------------------------------------------------------------------------

// A store that is coherent device-wide by itself: the relaxed agent-scope
// atomic store (`global_store ... sc1`) is written through this XCD's L2 to
// where every XCD reads it, and its completion (vmcnt) waits for that.  Data
// handed to another workgroup only through such stores and through atomics
// needs no L2 writeback before the hand-over (arrive_last with writeback
// false).  A plain store may stay dirty in this XCD's L2: on 252 workgroups
// in rows of 7 (each row over several XCDs), 3000 hand-overs of plain stores
// without the writeback left 2.6 % of the words stale for the last
// workgroup, these stores none.
//
// Why this is the release without its writeback: in LLVM's AMDGPU memory
// model for GFX942 (gfx950 follows it), an agent-scope release fence is
// `buffer_wbl2 sc1` (write back the lines this XCD's L2 holds dirty) then
// `s_waitcnt vmcnt(0)`, and an agent-scope monotonic store is
// `global_store ... sc1`, which the L2 does not hold dirty.  For data
// written only through such stores and through atomics the writeback has
// nothing to write, and the wait is the `s_waitcnt(0)` that arrive_last
// issues itself; the last arrival still runs the agent-scope acquire
// (`buffer_inv sc1`) before it reads.  A plain store among the handed-over
// data breaks this: its writer must arrive with writeback true.
template <typename T>
__device__ __forceinline__ void store_coherent(T *p, T v) {
  static_assert(sizeof(T) == 2 || sizeof(T) == 4, "16- or 32-bit elements");
  if constexpr (sizeof(T) == 2) {
    uint16_t u;
    __builtin_memcpy(&u, &v, 2);
    __hip_atomic_store(reinterpret_cast<uint16_t *>(p), u, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
  } else {
    uint32_t u;
    __builtin_memcpy(&u, &v, 4);
    __hip_atomic_store(reinterpret_cast<uint32_t *>(p), u, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
  }
}

// Arrival counters sit one per 128-byte line (kArriveStride unsigned ints
// apart): device-scope atomics on one line from many workgroups are served
// one after another, so counters packed into a line make every row's last
// arrival wait behind the other rows' tickets (at 128K, 256 tiles over 8
// rows: the last ticket 1.7 us packed, 0.6 us one per line).
constexpr int kArriveStride = 32;

// Every wave completes its own global stores, the workgroup meets at a
// barrier, then one wave makes them visible device-wide (with `writeback`,
// one agent-scope release -- an L2 writeback, 1-2 us -- for the whole
// workgroup, not one per wave; without it the data must have been written
// with store_coherent or atomics, whose completion the wait already covers)
// and takes a ticket from the device-scope counter.  Returns true in every
// thread of the workgroup that arrives last of `n`; that workgroup has
// acquired (one agent-scope acquire, then a barrier) and resets the counter,
// so no memset is needed between launches.  `s_flag` is one int of LDS.
// Callers without the writeback, and what their last arrival reads:
//   selector tile -> row tail: the page keys, the per-tile page lists and
//     their counts, the decode token's K row and L2 side row (all
//     store_coherent), the row histograms (atomics); a statistics rebuild
//     writes plain stores and arrives with the writeback;
//   attention and latent attention splits -> merge: each split's (m, z, acc)
//     partial (store_coherent).
__device__ __forceinline__ bool arrive_last(unsigned int *counter,
                                            unsigned int n, int *s_flag,
                                            bool writeback = true) {
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x == 0) {
    if (writeback) __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
    const unsigned int before =
        __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
    const bool last = before == n - 1;
    if (last) {
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
      __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    *s_flag = last;
  }
  __syncthreads();
  return *s_flag != 0;
}

// ---------------------------------------------------------------------------
// DPP reductions of the attention kernels
// ---------------------------------------------------------------------------

// DPP lane moves (VALU, no LDS round trip).
template <int CTRL>
__device__ __forceinline__ float dppf(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xF, 0xF, false));
}

// Sum over each group of 8 consecutive lanes, in every lane of the group:
// quad_perm xor 1, quad_perm xor 2, then row_half_mirror (lane i <-> 7 - i).
__device__ __forceinline__ float sum8(float x) {
  x += dppf<0xB1>(x);
  x += dppf<0x4E>(x);
  x += dppf<0x141>(x);
  return x;
}

// Wave-wide maximum / sum: the three 8-lane steps and row_mirror (lane
// i <-> 15 - i) give every lane its row's result; the four rows combine in
// scalar registers.
__device__ __forceinline__ float wave_max_dpp(float x) {
  x = fmaxf(x, dppf<0xB1>(x));
  x = fmaxf(x, dppf<0x4E>(x));
  x = fmaxf(x, dppf<0x141>(x));
  x = fmaxf(x, dppf<0x140>(x));
  const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 0));
  const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 16));
  const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 32));
  const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 48));
  return fmaxf(fmaxf(r0, r1), fmaxf(r2, r3));
}
__device__ __forceinline__ float wave_sum_dpp(float x) {
  x += dppf<0xB1>(x);
  x += dppf<0x4E>(x);
  x += dppf<0x141>(x);
  x += dppf<0x140>(x);
  const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 0));
  const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 16));
  const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 32));
  const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 48));
  return (r0 + r1) + (r2 + r3);
}

// ---------------------------------------------------------------------------
// block-level (256 threads) scans and reductions
// ---------------------------------------------------------------------------

__device__ __forceinline__ int lane_id() { return threadIdx.x & 63; }
// wave index within the workgroup, as a scalar (uniform) value
__device__ __forceinline__ int wave_id() {
  return __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
}

// Exclusive prefix sum of an int over a block of WAVES waves; two barriers.
// Wave-wide inclusive prefix sum in lane order with DPP moves (VALU, no LDS
// round trips): shifts of 1, 2, 4, 8 within each 16-lane row, then the row
// totals broadcast upward (row_bcast:15 into rows 1 and 3, row_bcast:31 into
// rows 2 and 3).
__device__ __forceinline__ int wave_incl_sum(int x) {
  x += __builtin_amdgcn_update_dpp(0, x, 0x111, 0xF, 0xF, true);  // row_shr:1
  x += __builtin_amdgcn_update_dpp(0, x, 0x112, 0xF, 0xF, true);  // row_shr:2
  x += __builtin_amdgcn_update_dpp(0, x, 0x114, 0xF, 0xF, true);  // row_shr:4
  x += __builtin_amdgcn_update_dpp(0, x, 0x118, 0xF, 0xF, true);  // row_shr:8
  x += __builtin_amdgcn_update_dpp(0, x, 0x142, 0xA, 0xF, false);  // row_bcast:15
  x += __builtin_amdgcn_update_dpp(0, x, 0x143, 0xC, 0xF, false);  // row_bcast:31
  return x;
}

// Bitwise OR over each group of four consecutive lanes (DPP quad_perm).
__device__ __forceinline__ uint32_t quad_or(uint32_t x) {
  x |= (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0xB1, 0xF, 0xF, false);
  x |= (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x4E, 0xF, 0xF, false);
  return x;
}

template <int WAVES = NFA_WAVES>
__device__ __forceinline__ int block_scan_exclusive(int v, int *scratch,
                                                    int *total) {
  static_assert(WAVES <= 64, "one wave scans the wave totals");
  const int lane = lane_id();
  const int w = wave_id();
  const int x = wave_incl_sum(v);
  if (lane == 63) scratch[w] = x;
  __syncthreads();
  // every wave scans the wave totals itself (DPP), then picks its own
  const int t = wave_incl_sum(lane < WAVES ? scratch[lane] : 0);
  const int before = w > 0 ? __builtin_amdgcn_readlane(t, w - 1) : 0;
  *total = __builtin_amdgcn_readlane(t, WAVES - 1);
  __syncthreads();
  return before + x - v;
}

// Exclusive prefix sums of N ints at once over a block of WAVES waves (one
// pair of barriers for all N); v is replaced by its exclusive prefix, total
// receives the block totals.  `scratch` needs WAVES * N ints.  Without
// `kTrailing` the second barrier is left out: the caller guarantees that
// another barrier comes before anything writes `scratch` again.
template <int N, int WAVES = NFA_WAVES, bool kTrailing = true>
__device__ __forceinline__ void block_scan_n(int (&v)[N], int *scratch,
                                             int (&total)[N]) {
  const int lane = lane_id();
  const int w = wave_id();
  static_assert(WAVES <= 64, "one wave scans the wave totals");
  int x[N];
#pragma unroll
  for (int k = 0; k < N; ++k) x[k] = wave_incl_sum(v[k]);
  if (lane == 63) {
#pragma unroll
    for (int k = 0; k < N; ++k) scratch[w * N + k] = x[k];
  }
  __syncthreads();
#pragma unroll
  for (int k = 0; k < N; ++k) {
    const int t = wave_incl_sum(lane < WAVES ? scratch[lane * N + k] : 0);
    const int before = w > 0 ? __builtin_amdgcn_readlane(t, w - 1) : 0;
    total[k] = __builtin_amdgcn_readlane(t, WAVES - 1);
    v[k] = before + x[k] - v[k];
  }
  if constexpr (kTrailing) __syncthreads();
}

// One wave: threshold bin of the top-K over a 256-bin histogram (bin = high
// byte of a 16-bit key, higher is better).  out[0] = bin b with
// above(b) < K <= above(b) + hist[b], or -1 when every counted entry fits
// (total < K, or total == K unless `exact`, or K <= 0); out[1] = above(b);
// out[2] = total.  The second-level pass over the low bytes of one
// high-byte bin passes `exact`: there a total equal to K means the whole bin
// is taken, and the threshold is its lowest non-empty low byte.  Must be
// called by all 64 lanes of one wave.
__device__ __forceinline__ void wave_threshold_bin(const int *hist, int K,
                                                   int *out, bool exact = false) {
  const int lane = lane_id();
  const int h0 = hist[4 * lane + 0], h1 = hist[4 * lane + 1];
  const int h2 = hist[4 * lane + 2], h3 = hist[4 * lane + 3];
  const int s = h0 + h1 + h2 + h3;
  const int pre = wave_incl_sum(s);
  const int total = __builtin_amdgcn_readlane(pre, 63);
  const int x = total - pre + s;  // lanes lane..63
  if (total < K || (total == K && !exact) || K <= 0) {
    if (lane == 0) {
      out[0] = -1;
      out[1] = 0;
      out[2] = total;
    }
    return;
  }
  int above = x - s;
  const int hb[4] = {h3, h2, h1, h0};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    if (above < K && K <= above + hb[i]) {
      out[0] = 4 * lane + 3 - i;
      out[1] = above;
    }
    above += hb[i];
  }
  if (lane == 0) out[2] = total;
}

// Wave-wide exclusive prefix sum of v in lane order, and the wave total.
__device__ __forceinline__ int wave_scan_excl(int v, int *total) {
  const int x = wave_incl_sum(v);
  *total = __builtin_amdgcn_readlane(x, 63);
  return x - v;
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
