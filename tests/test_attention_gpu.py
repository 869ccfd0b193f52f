"""Sparse gather attention on the GPU vs a float64 textbook softmax.

Tolerance: bf16 outputs within rtol 2e-2 / atol 2e-3 of the float64
reference (the reference's own test uses 3e-2); fp32 within 1e-4.
"""
import numpy as np
import pytest
import torch

from nfa_case import bf16_randn, make_cache, to_np
from oracle import nfa_oracle as orc
from sparse_attn.ops.paged_region_kernels import sparse_paged_attention_gather
from sparse_attn.policies.region_geometry import RegionGeometry

pytestmark = pytest.mark.gpu
DEV = 'cuda'
GEO = RegionGeometry(sink=4, near=4096, window=128, page=16, max_new_tokens=64)


def _setup(dtype, hkv=8, hq=32, max_vis=1024, rows=3, pages=400, seed=7,
           head_dim=128, head_dim_v=None):
    cache = make_cache(DEV, geometry=GEO, max_blocks=64, max_physical_pages=pages,
                       max_visible_len=max_vis, hkv=hkv, hq=hq, dtype=dtype,
                       max_requests=rows, head_dim=head_dim, head_dim_v=head_dim_v)
    gen = torch.Generator(device=DEV).manual_seed(seed)
    layer = cache.layers[0]
    layer.kv_pool_k.copy_(bf16_randn(layer.kv_pool_k.shape, gen, DEV).to(dtype))
    layer.kv_pool_v.copy_(bf16_randn(layer.kv_pool_v.shape, gen, DEV).to(dtype))
    total = pages * GEO.page
    gather = torch.stack([torch.randperm(total, generator=gen, device=DEV)[:max_vis]
                          for _ in range(rows * hkv)]).view(rows, hkv, max_vis)
    gather = gather.to(torch.int32).contiguous()
    return cache, gen, gather


def _check(cache, q, gather, lens, q2r, scale, dtype, **kw):
    layer = cache.layers[0]
    out = sparse_paged_attention_gather(layer, q, gather, lens, q2r, scale=scale, **kw)
    torch.cuda.synchronize()
    ref = orc.sparse_attention(to_np(layer.kv_pool_k), to_np(layer.kv_pool_v),
                               to_np(q), gather.cpu().numpy(), lens.cpu().numpy(),
                               q2r.cpu().numpy(), scale, GEO.page)
    got = out.float().cpu().numpy()
    if dtype == torch.bfloat16:
        np.testing.assert_allclose(got, ref, rtol=2e-2, atol=2e-3)
    else:
        np.testing.assert_allclose(got, ref, rtol=1e-4, atol=1e-5)
    assert out.dtype == q.dtype
    return got


@pytest.mark.parametrize('dtype', [torch.bfloat16, torch.float32])
def test_qwen3_geometry_b1_full_width(dtype):
    cache, gen, gather = _setup(dtype, rows=1)
    lens = torch.full((1, 8), 1024, dtype=torch.int32, device=DEV)
    q = bf16_randn((1, 32, 128), gen, DEV).to(dtype)
    q2r = torch.zeros(1, dtype=torch.int32, device=DEV)
    _check(cache, q, gather, lens, q2r, 128 ** -0.5, dtype)


def test_ragged_lengths_padding_rows_and_invalid_slots():
    dtype = torch.bfloat16
    cache, gen, gather = _setup(dtype, rows=3)
    lens = torch.tensor([[1024, 1, 0, 77, 500, 1023, 64, 65],
                         [5000, 33, 2, 3, 4, 5, 6, 1000],
                         [1024] * 8], dtype=torch.int32, device=DEV)
    gather[0, 3, 10:20] = -1
    q = bf16_randn((4, 32, 128), gen, DEV)
    q2r = torch.tensor([0, -1, 1, 2], dtype=torch.int32, device=DEV)
    got = _check(cache, q, gather, lens, q2r, 0.1, dtype)
    assert np.all(got[1] == 0)
    assert np.all(got[0, 2 * 4:3 * 4] == 0)


@pytest.mark.parametrize("split", [0, 16, 64])
def test_split_sizes_agree(split):
    dtype = torch.bfloat16
    cache, gen, gather = _setup(dtype, rows=2, hkv=2, hq=8, max_vis=700)
    lens = torch.tensor([[700, 350], [699, 1]], dtype=torch.int32, device=DEV)
    q = bf16_randn((2, 8, 128), gen, DEV)
    q2r = torch.tensor([0, 1], dtype=torch.int32, device=DEV)
    _check(cache, q, gather, lens, q2r, 0.125, dtype, tokens_per_split=split)


def test_wide_rows_take_several_chunks_per_workgroup():
    """20000-slot rows: 625 chunks of 32 over at most 256 workgroups per row,
    so each workgroup carries its running softmax over several chunks."""
    dtype = torch.bfloat16
    cache, gen, gather = _setup(dtype, rows=2, hkv=2, hq=8, max_vis=20000, pages=1400)
    lens = torch.tensor([[20000, 8193], [12345, 0]], dtype=torch.int32, device=DEV)
    gather[1, 0, 100:3000] = -1
    q = bf16_randn((2, 8, 128), gen, DEV)
    q2r = torch.tensor([0, 1], dtype=torch.int32, device=DEV)
    got = _check(cache, q, gather, lens, q2r, 0.09, dtype)
    assert np.all(got[1, 4:] == 0)


@pytest.mark.parametrize('dtype', [torch.bfloat16, torch.float32])
def test_head_dim_64_group_8(dtype):
    """head_dim 64 with 8 query heads per kv head: the merge stages fewer
    splits in LDS (128 for bf16), so 5000-slot rows loop over chunks."""
    cache, gen, gather = _setup(dtype, rows=2, hkv=2, hq=16, max_vis=5000,
                                pages=400, head_dim=64)
    lens = torch.tensor([[5000, 1000], [4097, 31]], dtype=torch.int32, device=DEV)
    q = bf16_randn((2, 16, 64), gen, DEV).to(dtype)
    q2r = torch.tensor([0, 1], dtype=torch.int32, device=DEV)
    _check(cache, q, gather, lens, q2r, 64 ** -0.5, dtype)


def test_many_rows_one_workgroup_each():
    """512 (row, kv head) pairs: one workgroup per pair takes all its chunks
    and writes the output without a split merge."""
    dtype = torch.bfloat16
    cache, gen, gather = _setup(dtype, rows=64, hkv=8, hq=32, max_vis=256, pages=200)
    lens = torch.randint(0, 257, (64, 8), generator=torch.Generator().manual_seed(4),
                         dtype=torch.int32).to(DEV)
    lens[0, 0], lens[1, 1] = 256, 0
    q = bf16_randn((64, 32, 128), gen, DEV)
    q2r = torch.arange(64, dtype=torch.int32, device=DEV)
    got = _check(cache, q, gather, lens, q2r, 128 ** -0.5, dtype)
    assert np.all(got[1, 4:8] == 0)


@pytest.mark.parametrize('dtype', [torch.bfloat16, torch.float32])
@pytest.mark.parametrize('dims', [(192, 128), (64, 256), (256, 64)])
def test_key_and_value_widths_differ(dtype, dims):
    """K and V rows of different widths: DeepSeek-V2's expanded heads (192 /
    128, one kv head per query head) and the other extremes the kernel
    takes; fp32 caps rows at 128 dims (32 chunks of 16 bytes)."""
    dk, dv = dims
    if dtype == torch.float32 and max(dk, dv) > 128:
        dk, dv = dk // 2, dv // 2
    cache, gen, gather = _setup(dtype, rows=2, hkv=16, hq=16, max_vis=1024,
                                pages=400, head_dim=dk, head_dim_v=dv)
    lens = torch.full((2, 16), 1024, dtype=torch.int32, device=DEV)
    lens[1, :8] = 333
    q = bf16_randn((2, 16, dk), gen, DEV).to(dtype)
    q2r = torch.tensor([0, 1], dtype=torch.int32, device=DEV)
    got = _check(cache, q, gather, lens, q2r, dk ** -0.5, dtype)
    assert got.shape == (2, 16, dv)
