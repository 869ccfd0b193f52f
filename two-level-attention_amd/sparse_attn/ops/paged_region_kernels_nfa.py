"""NFA protected-set helpers and the graph-ready gather attention entry.

Reference: sparse_attn/ops/paged_region_kernels_nfa.py:7-162.
"""
import argparse
import ctypes

import torch

from .. import _native as nat
from ..arguments import add_sparse_attn_args

INVALID_GATHER_IDX = -1


def nfa_args(subspace='tail'):
    """The production NFA flag set (reference paged_region_kernels_nfa.py:10-20)."""
    parser = argparse.ArgumentParser()
    add_sparse_attn_args(parser)
    return parser.parse_args([
        '--method', 'nfa', '--nfa_far_method', 'minmax',
        '--nfa_near_method', 'avg', '--nfa_near_pages', '32',
        '--nfa_near_tokens', 'off', '--nfa_near_len', '4096',
        '--nfa_subspace', subspace, '--tia_level2_cmp_ratio', '4',
        '--nfa_sink_tokens', '4', '--nfa_swa_size', '128',
        '--tia_level1_topk', '128', '--tia_level2_topk', '1024',
        '--nfa_enable_layer_skip', 'false', '--nfa_far_skip_backend', 'legacy',
        '--nfa_far_skip_cache', 'retain'])


def split_gather_buffers(cache, layer_idx, batch):
    """Fixed-address gather rows and visible lengths of the protected and the
    middle selection of ``layer_idx``: ``(prot_gather, prot_lens,
    mid_gather, mid_lens)``, shaped ``[batch, HKV, W]`` / ``[batch, HKV]``
    for the active visible bucket ``W``.

    Each layer owns one int32 arena sized for the cache's largest batch and
    visible length; every (batch, bucket) shape is a contiguous prefix view
    of it, so the addresses a captured graph holds stay valid and no shape
    allocates again.  The arena is created by the first (eager) call.
    """
    arenas = cache.__dict__.setdefault('_nfa_split_arenas', {})
    arena = arenas.get(layer_idx)
    layer = cache.layers[layer_idx]
    hkv = layer.num_kv_heads
    rows = cache.max_requests * hkv
    if arena is None:
        if torch.cuda.is_current_stream_capturing():
            raise RuntimeError('split gather buffers must be warmed before capture')
        arena = (torch.empty((2, rows * cache.max_visible_len), dtype=torch.int32,
                             device=layer.kv_pool_k.device),
                 torch.empty((2, rows), dtype=torch.int32,
                             device=layer.kv_pool_k.device))
        arenas[layer_idx] = arena
    width = cache.active_visible_bucket
    if batch > cache.max_requests:
        raise ValueError('split gather batch exceeds the cache request capacity')
    n = batch * hkv
    slots, lens = arena
    return (slots[0, :n * width].view(batch, hkv, width), lens[0, :n].view(batch, hkv),
            slots[1, :n * width].view(batch, hkv, width), lens[1, :n].view(batch, hkv))


def build_protected_gather(cache, layer_idx, indexer, gather_out, vis_out):
    """Write only the protected sink/SWA set as physical slots into
    ``gather_out`` [B, HKV, W] / ``vis_out`` [B, HKV] (protected-only launch
    of the selector kernel)."""
    layer0 = cache.layers[0]
    nat.require_hip(gather_out, 'build_protected_gather')
    lib = nat.load_library()
    batch, hkv, width = gather_out.shape
    p = nat.NfaSelectParams()
    p.abi_version = nat.ABI_VERSION
    p.struct_size = ctypes.sizeof(nat.NfaSelectParams)
    p.batch, p.hq, p.hkv = batch, cache.num_query_heads, hkv
    p.head_dim, p.head_dim_v = layer0.head_dim_k, layer0.head_dim_v
    p.bs = int(indexer.args.tia_block_size)
    p.page = cache.geometry.page
    p.max_blocks, p.max_req = cache.max_blocks, cache.max_requests
    p.sink_tokens = int(indexer.sink_tokens)
    p.swa = int(indexer.sliding_window_size)
    p.k2 = int(indexer.args.tia_level2_topk)
    p.dsub = 32
    p.fine_dsub = 32
    p.kv_dtype = nat.dtype_code(layer0.kv_pool_k.dtype)
    p.max_vis = width
    p.protected_only = 1
    layer = cache.layers[layer_idx]
    p.pool_pages = layer.kv_pool_k.shape[0]
    p.k_pool_l = layer.kv_pool_k.data_ptr()
    p.v_pool_l = layer.kv_pool_v.data_ptr()
    p.block_table_l = cache.block_table_buf[layer_idx].data_ptr()
    p.lengths = cache.planned_lengths_buf.data_ptr()
    p.active_req = cache.active_req_ids_buf.data_ptr()
    p.valid_req = cache.valid_req_ids_buf.data_ptr()
    p.skip_far_l = cache.skip_far_layer_buf[layer_idx].data_ptr()
    p.skip_near_l = cache.skip_near_layer_buf[layer_idx].data_ptr()
    # unused by the protected-only launch but checked for presence
    p.dims = p.fine_dims = p.q = cache.planned_lengths_buf.data_ptr()
    p.stat_min_l = p.stat_max_l = p.stat_sum_l = p.q
    p.stats_len_l = p.q
    p.gather = gather_out.data_ptr()
    p.vis_lens = vis_out.data_ptr()
    ws = getattr(cache, '_nfa_selector_workspace', None)
    if ws is None:
        ws = cache._nfa_selector_workspace = {}
    need = lib.nfa_select_workspace_bytes(ctypes.byref(p))
    key = ('nfa_protected_scratch', batch, hkv)
    scratch = ws.get(key)
    if scratch is None or scratch.numel() < need:
        if torch.cuda.is_current_stream_capturing():
            raise RuntimeError('protected scratch must be warmed before capture')
        scratch = ws[key] = torch.zeros(max(need, 1), dtype=torch.uint8,
                                        device=gather_out.device)
    p.workspace = scratch.data_ptr()
    p.workspace_bytes = scratch.numel()
    nat.check(lib.nfa_select_layer(ctypes.byref(p), nat.stream_handle()),
              'build_protected_gather')


def decode_graph_ready(module, q, cache, *, gather_indices=None,
                       visible_lens=None, query_to_req=None, scale=None):
    """Sparse gather attention for one decode step of ``module``'s layer.

    ``q`` is ``[T, HQ, D]`` or ``[B, 1, HQ, D]`` / ``[B, HQ, 1, D]``.
    """
    from .paged_region_kernels import sparse_paged_attention_gather

    layer_idx = module.layer_idx
    layer = cache.layers[layer_idx]
    scale = module.scaling if scale is None else scale
    if q.ndim == 4:
        if q.shape[2] == 1 and q.shape[1] != 1:
            q = q[:, :, 0].contiguous()
        elif q.shape[1] == 1:
            q = q[:, 0].contiguous()
        else:
            raise ValueError('graph-ready decode expects one query per row')
    if q.ndim != 3:
        raise ValueError('graph-ready decode expects [T,HQ,D] query')
    gather_indices = (cache.gather_indices_buf[layer_idx]
                      if gather_indices is None else gather_indices)
    visible_lens = (cache.visible_lens_buf[layer_idx]
                    if visible_lens is None else visible_lens)
    query_to_req = cache.query_to_req_buf if query_to_req is None else query_to_req
    return sparse_paged_attention_gather(
        layer, q, gather_indices, visible_lens, query_to_req, scale=scale,
        workspace=getattr(cache, '_nfa_selector_workspace', None))
