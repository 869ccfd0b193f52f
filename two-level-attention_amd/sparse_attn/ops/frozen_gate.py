"""Prefill region-mass profile on the GPU (libnfa_hip.so).

Reference: sparse_attn/ops/frozen_gate_triton.py:84-111 (``fused_region_profile``).
"""
import ctypes

import torch

from .. import _native as nat

GROUP_VECTORS = 64  # query vectors per workgroup: the GQA group divides it


def fused_region_profile(q, k, geometry, rows, scale):
    """Head-averaged near and far attention mass ``[2, rows]`` (fp32) of the
    last ``rows`` positions of a one-request prefill: ``q`` [1, hq, L, D],
    ``k`` [1, hkv, L, D], post-RoPE bf16 device tensors."""
    nat.require_hip(q, 'fused_region_profile')
    if q.dtype != torch.bfloat16 or k.dtype != torch.bfloat16:
        raise nat.NativeError('fused_region_profile takes bf16 q and k')
    length = q.shape[2]
    n = min(rows, length)
    hq, hkv, d = q.shape[1], k.shape[1], q.shape[-1]
    if q.stride(-1) != 1:
        q = q.contiguous()
    if k.stride(-1) != 1:
        k = k.contiguous()
    out = torch.empty((2, hq, n), dtype=torch.float32, device=q.device)
    p = nat.NfaGateParams()
    p.abi_version = nat.ABI_VERSION
    p.struct_size = ctypes.sizeof(nat.NfaGateParams)
    p.hq, p.hkv, p.head_dim = hq, hkv, d
    p.length, p.rows = length, n
    p.sink, p.window = geometry.sink, geometry.window
    p.near, p.page = geometry.near, geometry.page
    p.q_dtype = nat.DTYPE_BF16
    p.scale = float(scale)
    p.q, p.q_stride_h, p.q_stride_l = q.data_ptr(), q.stride(1), q.stride(2)
    p.k, p.k_stride_h, p.k_stride_l = k.data_ptr(), k.stride(1), k.stride(2)
    p.out = out.data_ptr()
    lib = nat.load_library()
    nat.check(lib.nfa_region_profile(ctypes.byref(p), nat.stream_handle()),
              'fused_region_profile')
    return out.mean(dim=1)
