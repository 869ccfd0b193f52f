"""Shared builders for selector tests: caches, indexers and oracle inputs."""
from types import SimpleNamespace

import numpy as np
import torch

from oracle import nfa_oracle as orc
from sparse_attn.cache import GraphReadyPagedRegionCache
from sparse_attn.indexer.nfa_indexer import NFAIndexer
from sparse_attn.ops.paged_region_kernels_nfa import nfa_args
from sparse_attn.policies.region_geometry import RegionGeometry


def make_indexer(*, bs=16, k1=128, near_pages=32, k2=1024, sink=4, swa=128,
                 near_len=4096, subspace='tail', l2_subspace='same',
                 near_tokens='off', far_method='minmax', near_method='avg',
                 cmp_ratio=4, l2_quant=False):
    args = nfa_args(subspace=subspace)
    args.tia_block_size = bs
    args.tia_level1_topk = k1
    args.tia_level2_topk = k2
    args.nfa_near_pages = near_pages
    args.nfa_near_tokens = near_tokens
    args.nfa_near_len = near_len
    args.nfa_swa_size = swa
    args.nfa_sink_tokens = sink
    args.nfa_l2_subspace = l2_subspace
    args.nfa_far_method = far_method
    args.nfa_near_method = near_method
    args.tia_level2_cmp_ratio = cmp_ratio
    args.nfa_l2_quant = l2_quant
    return NFAIndexer(args)


def make_cache(device, *, geometry, n_layers=1, max_requests=4, max_blocks,
               max_physical_pages, max_visible_len=1024, hkv=2, hq=8,
               head_dim=128, head_dim_v=None, dtype=torch.bfloat16,
               max_query_tokens=8):
    return GraphReadyPagedRegionCache(
        n_layers, geometry, max_requests=max_requests,
        max_physical_pages=max_physical_pages, max_blocks=max_blocks,
        max_visible_len=max_visible_len, max_query_tokens=max_query_tokens,
        num_kv_heads=hkv, num_query_heads=hq, head_dim_k=head_dim,
        head_dim_v=head_dim if head_dim_v is None else head_dim_v,
        dtype=dtype, device=device)


def indexer_dims(indexer, head_dim=128):
    cpu = torch.device('cpu')
    full = np.arange(head_dim)
    l1 = (indexer._subspace_indices(cpu).numpy() if indexer.enable_subspace
          else full)
    if indexer.l2_subspace == 'full':
        fine = full
    elif indexer.enable_subspace:
        fine = l1
    else:
        fine = indexer._qat_indices(cpu).numpy()
    return np.asarray(l1), np.asarray(fine)


def cfg_from(cache, indexer, scaling):
    layer = cache.layers[0]
    l1, fine = indexer_dims(indexer, layer.head_dim_k)
    nb_near = max(0, int(indexer.nt_near_pages))
    return orc.NfaConfig(
        hq=cache.num_query_heads, hkv=layer.num_kv_heads,
        head_dim=layer.head_dim_k, head_dim_v=layer.head_dim_v,
        bs=int(indexer.args.tia_block_size), page=cache.geometry.page,
        max_blocks=cache.max_blocks, geo_sink=cache.geometry.sink,
        geo_near=cache.geometry.near, geo_window=cache.geometry.window,
        sink_tokens=int(indexer.sink_tokens),
        swa=int(indexer.sliding_window_size), near_len=int(indexer.nt_near_len),
        k1=int(indexer.args.tia_level1_topk), near_pages=nb_near,
        k2=int(indexer.args.tia_level2_topk), dims=l1, fine_dims=fine,
        scale=float(scaling), far_method=indexer.far_method,
        near_method=indexer.near_method,
        kv_dtype='bf16' if layer.kv_pool_k.dtype == torch.bfloat16 else 'fp32',
        near_tokens=indexer.nt_near_tokens, l2_quant=indexer.l2_quant)


def to_np(t):
    return t.detach().float().cpu().numpy() if t.is_floating_point() else \
        t.detach().cpu().numpy()


def snapshot(cache, layer_idx, batch):
    """Numpy copy of everything the selector reads for ``layer_idx``."""
    layer = cache.layers[layer_idx]
    return dict(
        k_pool=to_np(layer.kv_pool_k), v_pool=to_np(layer.kv_pool_v),
        block_table=to_np(cache.block_table_buf[layer_idx]).astype(np.int64),
        lengths=to_np(cache.planned_lengths_buf[:batch]).astype(np.int64),
        req_ids=to_np(cache.valid_req_ids_buf[:batch]).astype(np.int64),
        active=to_np(cache.active_req_ids_buf[:batch]) >= 0,
        skip_far=to_np(cache.skip_far_layer_buf[layer_idx]),
        skip_near=to_np(cache.skip_near_layer_buf[layer_idx]))


def run_oracle(cfg, snap, q, decode=None, max_vis=1024, middle_only=False):
    """Oracle selection on a snapshot; ``decode`` = (keys, values, slots)."""
    k_pool = snap['k_pool'].copy()
    v_pool = snap['v_pool'].copy()
    if decode is not None:
        keys, values, slots = decode
        active = snap['active']
        slots = np.where(active, np.asarray(slots), -1)
        orc.apply_decode_write(k_pool, v_pool, np.asarray(keys, np.float32),
                               np.asarray(values, np.float32), slots, cfg.page)
    res = orc.select_layer(cfg, k_pool, snap['block_table'], snap['lengths'],
                           snap['req_ids'], snap['active'], snap['skip_far'],
                           snap['skip_near'], np.asarray(q, np.float32),
                           max_vis, middle_only)
    return res, k_pool, v_pool


def bf16_randn(shape, gen, device, scale=1.0):
    return (torch.randn(shape, generator=gen, device=device) * scale).to(
        torch.bfloat16)


def attention_ns(indexer, scaling=1.0):
    return SimpleNamespace(indexer=indexer, scaling=scaling)


def logical_ids(cache, request_id, row, layer_idx=0, kv_head=0):
    """Selected logical token ids of one row, through the inverse block table."""
    page = cache.geometry.page
    count = int(cache.visible_lens_for_layer(layer_idx)[row, kv_head])
    width = cache.gather_indices_for_layer(layer_idx).shape[-1]
    slots = cache.gather_indices_for_layer(layer_idx)[
        row, kv_head, :min(count, width)].cpu().tolist()
    inverse = {phys: lp for lp, phys in
               cache.states[request_id].block_tables[layer_idx].items()}
    return sorted(inverse[s // page] * page + s % page for s in slots)
