"""Fused decode kernels of the dense layers vs torch fp32 references.

``nfa_decode_linear`` (plain / three segments, RMSNorm prologue, residual
and SiLU-gate epilogues), ``nfa_qk_norm_rope_decode`` and
``nfa_rmsnorm_decode`` against the HF op chain in torch.  The kernels sum in
their own order, so outputs are compared within bf16 rounding: rtol 1e-2
relative to the output scale (a bf16 ulp is 2^-8 relative).
"""
import pytest
import torch
import torch.nn.functional as F

from sparse_attn.ops.decode_fused import (decode_linear, linear_fusable,
                                          qk_norm_rope_decode, rmsnorm_decode)

pytestmark = pytest.mark.gpu
DEV = 'cuda'


def _rand(shape, gen, scale=1.0):
    return (torch.randn(shape, generator=gen, device=DEV) * scale).to(torch.bfloat16)


def _hf_rms(x, w, eps):
    h = x.float()
    h = h * torch.rsqrt(h.pow(2).mean(-1, keepdim=True) + eps)
    return w * h.to(torch.bfloat16)


def _close(got, want, rel=1e-2):
    got, want = got.float(), want.float()
    scale = want.abs().max().item() + 1e-6
    err = (got - want).abs().max().item()
    assert err <= rel * scale, (err, scale)


@pytest.mark.parametrize('m,k', [(1, 4096), (2, 512), (4, 1000), (2, 12288)])
def test_linear_three_segments_with_norm(m, k):
    gen = torch.Generator(device=DEV).manual_seed(m * 100 + k)
    x = _rand((m, k), gen)
    ws = [_rand((n, k), gen, 0.02) for n in (384, 128, 130)]
    nw = _rand((k,), gen, 0.1) + 1
    print(f'# linear m={m} k={k}', flush=True)
    assert linear_fusable(x, *ws)
    outs = decode_linear(x, ws, norm_weight=nw, eps=1e-6)
    h = _hf_rms(x, nw, 1e-6).float()
    for w, y in zip(ws, outs):
        assert y.shape == (m, w.shape[0]) and y.dtype == torch.bfloat16
        _close(y, h @ w.float().T)
    plain = decode_linear(x, ws[:1])[0]
    _close(plain, x.float() @ ws[0].float().T)


@pytest.mark.parametrize('m', [1, 3])
def test_linear_residual_and_silu_gate(m):
    gen = torch.Generator(device=DEV).manual_seed(77 + m)
    k, n = 2048, 1536
    x = _rand((m, k), gen)
    wo = _rand((n, k), gen, 0.02)
    res = _rand((m, n), gen)
    y, = decode_linear(x, (wo,), residual=res)
    want = (res.float() + (x.float() @ wo.float().T).to(torch.bfloat16).float())
    _close(y, want)
    wg, wu = _rand((n, k), gen, 0.02), _rand((n, k), gen, 0.02)
    nw = _rand((k,), gen, 0.1) + 1
    a, = decode_linear(x, (wg, wu), norm_weight=nw, eps=1e-5, silu_gate=True)
    h = _hf_rms(x, nw, 1e-5).float()
    g = (h @ wg.float().T).to(torch.bfloat16)
    u = (h @ wu.float().T).to(torch.bfloat16)
    _close(a, F.silu(g) * u)


def test_linear_fallback_outside_kernel_shapes():
    gen = torch.Generator(device=DEV).manual_seed(5)
    x = _rand((6, 256), gen)
    w = _rand((64, 256), gen, 0.05)
    assert not linear_fusable(x, w)
    y, = decode_linear(x, (w,))
    _close(y, x.float() @ w.float().T)


@pytest.mark.parametrize('norm', [True, False])
def test_qk_norm_rope_matches_hf(norm):
    from transformers.models.qwen3.modeling_qwen3 import (Qwen3RMSNorm,
                                                          apply_rotary_pos_emb)
    gen = torch.Generator(device=DEV).manual_seed(3)
    b, hq, hkv, d = 3, 32, 8, 128
    q = _rand((b, hq * d), gen, 2.0)
    k = _rand((b, hkv * d), gen, 2.0)
    pos = torch.tensor([5, 70000, 131071], device=DEV, dtype=torch.float32)
    inv = 1e6 ** (-torch.arange(0, d, 2, device=DEV, dtype=torch.float32) / d)
    ang = pos[:, None] * inv[None]
    emb = torch.cat((ang, ang), dim=-1)
    cos, sin = emb.cos().to(torch.bfloat16)[:, None], emb.sin().to(torch.bfloat16)[:, None]
    qn, kn = Qwen3RMSNorm(d, eps=1e-6).to(DEV), Qwen3RMSNorm(d, eps=1e-6).to(DEV)
    with torch.no_grad():
        qn.weight.copy_(_rand((d,), gen, 0.2) + 1)
        kn.weight.copy_(_rand((d,), gen, 0.2) + 1)
    qn, kn = qn.to(torch.bfloat16), kn.to(torch.bfloat16)
    qh = q.view(b, 1, hq, d)
    kh = k.view(b, 1, hkv, d)
    with torch.no_grad():
        if norm:
            qh, kh = qn(qh), kn(kh)
        want_q, want_k = apply_rotary_pos_emb(qh.transpose(1, 2), kh.transpose(1, 2),
                                              cos, sin)
        got_q, got_k = qk_norm_rope_decode(
            q, k, qn.weight if norm else None, kn.weight if norm else None,
            cos, sin, 1e-6, hq=hq, hkv=hkv, head_dim=d)
    _close(got_q, want_q[:, :, 0])
    _close(got_k, want_k[:, :, 0])
    if not norm:  # no reduction involved: every rounding matches HF's
        assert torch.equal(got_q, want_q[:, :, 0])
        assert torch.equal(got_k, want_k[:, :, 0])


def test_rmsnorm_matches_hf_module():
    from transformers.models.qwen3.modeling_qwen3 import Qwen3RMSNorm
    gen = torch.Generator(device=DEV).manual_seed(9)
    x = _rand((2, 1, 4096), gen, 3.0)
    mod = Qwen3RMSNorm(4096, eps=1e-6).to(DEV)
    with torch.no_grad():
        mod.weight.copy_(_rand((4096,), gen, 0.2) + 1)
    mod = mod.to(torch.bfloat16)
    with torch.no_grad():
        want = mod(x)
    got = rmsnorm_decode(x, mod.weight, 1e-6)
    _close(got, want)
    exact = (got == want).float().mean().item()
    assert exact > 0.95, exact
