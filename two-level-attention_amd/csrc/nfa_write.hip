// Paged KV writes (decode token and prefill scatter) plus the C-ABI glue:
// error reporting and ABI queries.
//
// Reference: _paged_write_kernel / _paged_write_prefill_kernel,
// sparse_attn/ops/paged_region_kernels.py:15-103, host :610-724.
// Pool layout [P+1, 1, hkv, page, D]; physical slot = page_id * page + offset.
#include "nfa_common.h"

#include <stdarg.h>
#include <stdio.h>

namespace nfa {

// One workgroup per (row, kv head); 16-byte vector copies of the K and V rows.
template <typename KV>
__global__ void __launch_bounds__(128)
    paged_write_decode_kernel(const KV *__restrict__ keys,
                              const KV *__restrict__ values,
                              const int32_t *__restrict__ slots, int hkv, int D,
                              int DV, int page, KV *__restrict__ kpool,
                              KV *__restrict__ vpool) {
  const int b = blockIdx.x;
  const int h = blockIdx.y;
  const int slot = slots[b];
  if (slot < 0) return;
  const int64_t phys = slot / page;
  const int64_t off = slot % page;
  KV *kd = kpool + ((phys * hkv + h) * page + off) * D;
  KV *vd = vpool + ((phys * hkv + h) * page + off) * DV;
  const KV *ks = keys + ((int64_t)b * hkv + h) * D;
  const KV *vs = values + ((int64_t)b * hkv + h) * DV;
  for (int d = threadIdx.x; d < D; d += blockDim.x) kd[d] = ks[d];
  for (int d = threadIdx.x; d < DV; d += blockDim.x) vd[d] = vs[d];
}

// Grid (ceil(n / 16), hkv): 16 tokens of one kv head per workgroup.
template <typename KV>
__global__ void __launch_bounds__(256)
    paged_write_prefill_kernel(const KV *__restrict__ keys,
                               const KV *__restrict__ values, int64_t n,
                               const int32_t *__restrict__ bt, int hkv, int D,
                               int DV, int page, KV *__restrict__ kpool,
                               KV *__restrict__ vpool) {
  const int h = blockIdx.y;
  const int64_t t0 = (int64_t)blockIdx.x * 16;
  for (int i = threadIdx.x; i < 16 * D; i += blockDim.x) {
    const int64_t tok = t0 + i / D;
    const int d = i % D;
    if (tok >= n) break;
    const int64_t phys = bt[tok / page];
    kpool[((phys * hkv + h) * page + tok % page) * D + d] =
        keys[((int64_t)h * n + tok) * D + d];
  }
  for (int i = threadIdx.x; i < 16 * DV; i += blockDim.x) {
    const int64_t tok = t0 + i / DV;
    const int d = i % DV;
    if (tok >= n) break;
    const int64_t phys = bt[tok / page];
    vpool[((phys * hkv + h) * page + tok % page) * DV + d] =
        values[((int64_t)h * n + tok) * DV + d];
  }
}

}  // namespace nfa

// ---------------------------------------------------------------------------
// error reporting
// ---------------------------------------------------------------------------

static thread_local char g_err[512] = "";

extern "C" void nfa_set_error(const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}

extern "C" const char *nfa_last_error(void) { return g_err; }
extern "C" int32_t nfa_abi_version(void) { return NFA_ABI_VERSION; }
extern "C" int32_t nfa_wall_clock_khz(void) {
  int dev = 0, rate = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 0;
  if (hipDeviceGetAttribute(&rate, hipDeviceAttributeWallClockRate, dev) != hipSuccess)
    return 0;
  return rate;
}
extern "C" int32_t nfa_select_params_size(void) {
  return (int32_t)sizeof(NfaSelectParams);
}
extern "C" int32_t nfa_attn_params_size(void) {
  return (int32_t)sizeof(NfaAttnParams);
}

// DV == 0 writes keys only (values and the V pool may then be NULL): a
// latent arena whose values are part of the key rows.
static int check_write(int batch, int hkv, int D, int DV, int page, int dtype,
                       const void *k, const void *v, const void *kp,
                       const void *vp, const char *who) {
  if (hkv <= 0 || D <= 0 || DV < 0 || page <= 0 || batch < 0) {
    nfa_set_error("%s: bad geometry", who);
    return NFA_EINVAL;
  }
  if (dtype != NFA_DTYPE_BF16 && dtype != NFA_DTYPE_F32) {
    nfa_set_error("%s: unsupported dtype %d", who, dtype);
    return NFA_EINVAL;
  }
  if (!k || !kp || (DV > 0 && (!v || !vp))) {
    nfa_set_error("%s: null device pointer", who);
    return NFA_EINVAL;
  }
  return NFA_OK;
}

extern "C" int32_t nfa_paged_write_decode(const void *keys, const void *values,
                                          const int32_t *slots, int32_t batch,
                                          int32_t hkv, int32_t head_dim,
                                          int32_t head_dim_v, int32_t page,
                                          int32_t kv_dtype, void *k_pool,
                                          void *v_pool, void *stream) {
  int rc = check_write(batch, hkv, head_dim, head_dim_v, page, kv_dtype, keys,
                       values, k_pool, v_pool, "nfa_paged_write_decode");
  if (rc != NFA_OK) return rc;
  if (slots == nullptr) {
    nfa_set_error("nfa_paged_write_decode: null slots");
    return NFA_EINVAL;
  }
  if (batch == 0) return NFA_OK;
  dim3 grid(batch, hkv);
  hipStream_t s = (hipStream_t)stream;
  if (kv_dtype == NFA_DTYPE_BF16)
    hipLaunchKernelGGL(nfa::paged_write_decode_kernel<uint16_t>, grid, dim3(128),
                       0, s, (const uint16_t *)keys, (const uint16_t *)values,
                       slots, hkv, head_dim, head_dim_v, page,
                       (uint16_t *)k_pool, (uint16_t *)v_pool);
  else
    hipLaunchKernelGGL(nfa::paged_write_decode_kernel<float>, grid, dim3(128), 0,
                       s, (const float *)keys, (const float *)values, slots,
                       hkv, head_dim, head_dim_v, page, (float *)k_pool,
                       (float *)v_pool);
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess) {
    nfa_set_error("nfa_paged_write_decode: launch failed: %s",
                  hipGetErrorString(err));
    return NFA_ELAUNCH;
  }
  return NFA_OK;
}

extern "C" int32_t nfa_paged_write_prefill(const void *keys, const void *values,
                                           int64_t n,
                                           const int32_t *block_table_row,
                                           int32_t hkv, int32_t head_dim,
                                           int32_t head_dim_v, int32_t page,
                                           int32_t kv_dtype, void *k_pool,
                                           void *v_pool, void *stream) {
  int rc = check_write(0, hkv, head_dim, head_dim_v, page, kv_dtype, keys,
                       values, k_pool, v_pool, "nfa_paged_write_prefill");
  if (rc != NFA_OK) return rc;
  if (block_table_row == nullptr || n < 0) {
    nfa_set_error("nfa_paged_write_prefill: bad block table / length");
    return NFA_EINVAL;
  }
  if (n == 0) return NFA_OK;
  dim3 grid((unsigned)((n + 15) / 16), hkv);
  hipStream_t s = (hipStream_t)stream;
  if (kv_dtype == NFA_DTYPE_BF16)
    hipLaunchKernelGGL(nfa::paged_write_prefill_kernel<uint16_t>, grid, dim3(256),
                       0, s, (const uint16_t *)keys, (const uint16_t *)values, n,
                       block_table_row, hkv, head_dim, head_dim_v, page,
                       (uint16_t *)k_pool, (uint16_t *)v_pool);
  else
    hipLaunchKernelGGL(nfa::paged_write_prefill_kernel<float>, grid, dim3(256), 0,
                       s, (const float *)keys, (const float *)values, n,
                       block_table_row, hkv, head_dim, head_dim_v, page,
                       (float *)k_pool, (float *)v_pool);
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess) {
    nfa_set_error("nfa_paged_write_prefill: launch failed: %s",
                  hipGetErrorString(err));
    return NFA_ELAUNCH;
  }
  return NFA_OK;
}
