"""Decode-step dense kernels around the sparse attention (libnfa_hip.so).

Reference counterparts: sparse_attn/ops/qwen3_rmsnorm_triton.py:207-300
(``is_fusable``, ``fused_rmsnorm_decode``), ops/qwen3_mlp_silu_triton.py:87-130
(``fused_silu_mul_decode``) and ops/qwen3_rope_triton.py:118-160
(``qwen3_decode_rope``).  Here the projections are fused too: one launch per
linear layer with an RMSNorm prologue and a residual or SiLU-gate epilogue.
Inputs outside the kernels' shapes (batch above 4, activations above 48 KiB,
non-bf16) take the equivalent torch ops, as the reference's ``is_fusable``
gates do.
"""
import ctypes

import torch
import torch.nn.functional as F

from .. import _native as nat

LINEAR_MAX_ROWS = 4
LINEAR_LDS_BYTES = 48 * 1024


def linear_fusable(x, *weights):
    """True when ``x`` [m, k] and the weights fit the decode linear kernel."""
    if x.dim() != 2 or x.dtype != torch.bfloat16 or not x.is_cuda:
        return False
    m, k = x.shape
    if not 1 <= m <= LINEAR_MAX_ROWS or k % 8 or m * k * 2 > LINEAR_LDS_BYTES:
        return False
    if x.stride(1) != 1 or x.stride(0) % 8 or x.data_ptr() % 16:
        return False
    return all(w.dtype == torch.bfloat16 and w.is_cuda and w.is_contiguous()
               and w.shape[1] == k and w.data_ptr() % 16 == 0 for w in weights)


def _rms_torch(x, weight, eps):
    h = x.float()
    h = h * torch.rsqrt(h.pow(2).mean(-1, keepdim=True) + eps)
    return weight * h.to(x.dtype)


def decode_linear(x, weights, *, norm_weight=None, eps=1e-6, residual=None,
                  silu_gate=False):
    """``x`` [m, k] bf16 (RMS-normalised first when ``norm_weight`` is given)
    times each weight [n_s, k]^T.  Returns one output per weight; with
    ``residual`` [m, n] the single output is ``residual + x W^T``; with
    ``silu_gate`` (weights = gate, up) the single output is
    ``silu(x Wg^T) * (x Wu^T)``.  Each bf16 rounding as HF's op chain."""
    weights = list(weights)
    if not linear_fusable(x, *weights) or (
            norm_weight is not None and (norm_weight.dtype != torch.bfloat16
                                         or not norm_weight.is_contiguous())):
        h = x if norm_weight is None else _rms_torch(x, norm_weight, eps)
        outs = [F.linear(h, w) for w in weights]
        if silu_gate:
            return [F.silu(outs[0]) * outs[1]]
        if residual is not None:
            return [residual + outs[0]]
        return outs
    if silu_gate and (len(weights) != 2 or weights[0].shape != weights[1].shape):
        raise ValueError('SiLU gate needs gate and up weights of one shape')
    if residual is not None and (len(weights) != 1 or residual.shape != (
            x.shape[0], weights[0].shape[0]) or residual.stride(1) != 1):
        raise ValueError('residual must be [m, n] with one weight')
    if not 1 <= len(weights) <= 3:
        raise ValueError('one to three weight segments')
    m, k = x.shape
    lib = nat.load_library()
    p = nat.NfaLinearParams()
    p.abi_version = nat.ABI_VERSION
    p.struct_size = ctypes.sizeof(nat.NfaLinearParams)
    p.m, p.k = m, k
    p.x, p.x_stride = x.data_ptr(), x.stride(0)
    if norm_weight is not None:
        p.norm_weight, p.norm_eps = norm_weight.data_ptr(), float(eps)
    if silu_gate:
        p.epilogue = nat.EPI_SILU_GATE
        outs = [torch.empty((m, weights[0].shape[0]), dtype=x.dtype, device=x.device)]
        segs = [(weights[0], outs[0]), (weights[1], outs[0])]
    else:
        p.epilogue = nat.EPI_RESIDUAL if residual is not None else nat.EPI_PLAIN
        outs = [torch.empty((m, w.shape[0]), dtype=x.dtype, device=x.device)
                for w in weights]
        segs = list(zip(weights, outs))
    p.nseg = len(segs)
    for i, (w, y) in enumerate(segs):
        p.w[i], p.n[i] = w.data_ptr(), w.shape[0]
        p.y[i], p.y_stride[i] = y.data_ptr(), y.stride(0)
    if residual is not None:
        p.residual, p.residual_stride = residual.data_ptr(), residual.stride(0)
    nat.check(lib.nfa_decode_linear(ctypes.byref(p), nat.stream_handle()),
              'decode_linear')
    return outs


def qk_norm_rope_decode(q, k, q_weight, k_weight, cos, sin, eps, *, hq, hkv,
                        head_dim):
    """Per-head RMSNorm (when weights are given) and rotate-half RoPE of one
    token per row.  ``q`` [B, hq*D], ``k`` [B, hkv*D] bf16 projection rows,
    ``cos``/``sin`` [B, 1, D] or [B, D].  Returns ``q`` [B, hq, D] and ``k``
    [B, hkv, D]."""
    b = q.shape[0]
    cos = cos.reshape(b, -1)
    sin = sin.reshape(b, -1)
    for t in (q, k, cos, sin):
        if t.dtype != torch.bfloat16 or not t.is_cuda or t.stride(-1) != 1:
            raise ValueError('q/k/cos/sin must be bf16 device rows')
    if cos.shape[1] != head_dim or sin.stride() != cos.stride():
        raise ValueError('cos/sin must be [B, head_dim] with equal strides')
    if q.shape[1] != hq * head_dim or k.shape[1] != hkv * head_dim:
        raise ValueError('q/k rows do not match the head geometry')
    lib = nat.load_library()
    q_out = torch.empty((b, hq, head_dim), dtype=q.dtype, device=q.device)
    k_out = torch.empty((b, hkv, head_dim), dtype=k.dtype, device=k.device)
    p = nat.NfaRopeParams()
    p.abi_version = nat.ABI_VERSION
    p.struct_size = ctypes.sizeof(nat.NfaRopeParams)
    p.batch, p.hq, p.hkv, p.head_dim = b, hq, hkv, head_dim
    p.q, p.q_stride_b = q.data_ptr(), q.stride(0)
    p.k, p.k_stride_b = k.data_ptr(), k.stride(0)
    if q_weight is not None:
        p.q_weight, p.k_weight = q_weight.data_ptr(), k_weight.data_ptr()
    p.eps = float(eps)
    p.cos, p.sin, p.cs_stride_b = cos.data_ptr(), sin.data_ptr(), cos.stride(0)
    p.q_out, p.k_out = q_out.data_ptr(), k_out.data_ptr()
    nat.check(lib.nfa_qk_norm_rope_decode(ctypes.byref(p), nat.stream_handle()),
              'qk_norm_rope_decode')
    return q_out, k_out


def rmsnorm_fusable(x, weight):
    return (x.dtype == torch.bfloat16 and x.is_cuda and x.is_contiguous()
            and weight.dtype == torch.bfloat16 and weight.is_contiguous()
            and x.shape[-1] % 8 == 0 and x.dim() >= 2 and x.shape[-2] == 1)


def rmsnorm_decode(x, weight, eps):
    """HF RMSNorm over the last dim of ``x`` (contiguous bf16 rows)."""
    dim = x.shape[-1]
    rows = x.numel() // dim
    out = torch.empty_like(x)
    lib = nat.load_library()
    nat.check(lib.nfa_rmsnorm_decode(x.data_ptr(), dim, weight.data_ptr(),
                                     out.data_ptr(), dim, rows, dim, float(eps),
                                     nat.stream_handle()), 'rmsnorm_decode')
    return out
