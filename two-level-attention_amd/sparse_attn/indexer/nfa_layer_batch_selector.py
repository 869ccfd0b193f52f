"""Request-batched, current-query NFA selector for one decode layer.

Drop-in for the reference's production entry
``select_topk_for_layer_batched`` (sparse_attn/indexer/nfa_layer_batch_selector.py:2649-2720,
implementation :2723-3091).  The host side validates the call exactly where
the reference does, resolves the geometry once per (layer, batch, bucket) and
hands one ``NfaSelectParams`` block to ``nfa_select_layer`` in libnfa_hip.so,
which runs the whole selector (decode write, page statistics, L1 scores and
top-k, candidates, L2 logits and top-k with hole fill, sink/SWA union) as one
kernel launch on the current stream.  Outputs land in the cache's fixed
``gather_indices`` / ``visible_lens`` rows; nothing is allocated after the
first call for a geometry, so the call can be captured into a hipGraph.
"""
from __future__ import annotations

import ctypes

import torch

from .. import _native as nat
from ..ops.paged_region_kernels_nfa import INVALID_GATHER_IDX  # noqa: F401
from .selection.selector import TokenSelection  # noqa: F401


class FallbackRequired(Exception):
    """The request-batched selector does not support this geometry."""


_GMAX = 8
_FAR_METHODS = {'minmax': nat.METHOD_MINMAX, 'avg': nat.METHOD_AVG,
                'avg_top2': nat.METHOD_AVG_TOP2}


def _dims_for(indexer, device, head_dim):
    """(l1_dims, fine_dims) as int32 device tensors (selector:2775-2794, 2933-2938)."""
    cache = getattr(indexer, '_nfa_hip_dims', None)
    key = (str(device), head_dim, indexer.subspace, indexer.l2_subspace,
           indexer.cmp_ratio, indexer.enable_subspace)
    if cache is not None and cache[0] == key:
        return cache[1], cache[2], cache[3], cache[4]
    cpu = torch.device('cpu')
    full = torch.arange(head_dim, dtype=torch.int64)
    if indexer.enable_subspace:
        l1 = indexer._subspace_indices(cpu).long()
    else:
        l1 = full
    if indexer.l2_subspace == 'full':
        fine = full
    elif indexer.enable_subspace:
        fine = l1
    else:
        fine = indexer._qat_indices(cpu).long()
    l1_key = tuple(l1.tolist())
    fine_key = tuple(fine.tolist())
    l1 = l1.to(device=device, dtype=torch.int32).contiguous()
    fine = fine.to(device=device, dtype=torch.int32).contiguous()
    indexer._nfa_hip_dims = (key, l1, fine, l1_key, fine_key)
    return l1, fine, l1_key, fine_key


def _latent_dims(indexer, device, layer0):
    """L1 / L2 dims of a latent arena row ``[c (head_dim_v) | k_pe]``: the
    RoPE part, where the expanded heads' ``mla_rope`` dims (128..191 of
    ``[k_nope | k_pe]``, ``nfa_indexer.py:133-134``) come from -- every
    expanded head holds the same k_pe, so selections agree bit for bit."""
    if (not indexer.enable_subspace or indexer.subspace != 'mla_rope'
            or indexer.l2_subspace != 'same'):
        raise ValueError('a latent (absorbed MLA) cache selects on the mla_rope '
                         'subspace with the same L2 dims')
    cache = getattr(indexer, '_nfa_hip_latent_dims', None)
    key = (str(device), layer0.head_dim_k, layer0.head_dim_v)
    if cache is not None and cache[0] == key:
        return cache[1], cache[1], cache[2], cache[2]
    dims = torch.arange(layer0.head_dim_v, layer0.head_dim_k, dtype=torch.int64)
    dims_key = tuple(dims.tolist())
    dims = dims.to(device=device, dtype=torch.int32).contiguous()
    indexer._nfa_hip_latent_dims = (key, dims, dims_key)
    return dims, dims, dims_key, dims_key


def _workspace(cache):
    ws = getattr(cache, '_nfa_selector_workspace', None)
    if ws is None:
        ws = cache._nfa_selector_workspace = {}
    return ws


def _no_capture_alloc(what):
    if torch.cuda.is_current_stream_capturing():
        raise RuntimeError(f'{what} must be allocated by a warm-up call before '
                           'graph capture')


def _page_stats_buffers(cache, layer_idx, dims, dims_key, dtype, fine_key,
                        head_dim, bs, quant=False):
    """Persistent per-layer page statistics [max_req, hkv, dsub, max_blocks]
    in the KV dtype, chunk-major, the fp32 running sums of each request's last
    page [max_req, hkv, dsub], and the L2 side copy [max_req, hkv,
    max_blocks * bs, fine_dsub] of every visible token's L2 dims (None for a
    full-width L2 subspace, or when ``cache.nfa_l2_side_copy`` is False) --
    with ``quant``, fine_dsub / 2 + 4 bytes per token slot instead (4-bit
    codes, then bf16 scale and zero); a new dims set for a layer forces
    rebuilds of both."""
    layer0 = cache.layers[0]
    device = layer0.kv_pool_k.device
    lengths = getattr(cache, '_nfa_page_stats_lengths', None)
    if lengths is None:
        _no_capture_alloc('page statistics')
        lengths = cache._nfa_page_stats_lengths = torch.zeros(
            (cache.n_layers, cache.max_requests), dtype=torch.int32, device=device)
        cache._nfa_stats_dirty = True
    store = getattr(cache, '_nfa_page_stats_persistent', None)
    if store is None:
        store = cache._nfa_page_stats_persistent = {}
    keys_by_layer = getattr(cache, '_nfa_stats_key_by_layer', None)
    if keys_by_layer is None:
        keys_by_layer = cache._nfa_stats_key_by_layer = {}
    want_side = (len(fine_key) < head_dim
                 and getattr(cache, 'nfa_l2_side_copy', True))
    key = (layer_idx, 1, int(dims.numel()), dtype, dims_key,
           (fine_key, bs, bool(quant)) if want_side else None)
    bufs = store.get(key)
    if bufs is None:
        _no_capture_alloc('page statistics')
        numel = (cache.max_requests * layer0.num_kv_heads * int(dims.numel())
                 * cache.max_blocks)
        stats = tuple(torch.empty(numel, dtype=dtype, device=device)
                      for _ in range(3))
        # fp32 running sums of each request's last page
        stats += (torch.zeros(cache.max_requests * layer0.num_kv_heads
                              * int(dims.numel()), dtype=torch.float32,
                              device=device),)
        side = None
        slots = cache.max_requests * layer0.num_kv_heads * cache.max_blocks * bs
        if want_side and quant:
            # fine_dsub / 2 bytes of codes, then bf16 scale and zero, per slot
            side = torch.empty(slots * (len(fine_key) // 2 + 4), dtype=torch.uint8,
                               device=device)
        elif want_side:
            side = torch.empty(slots * len(fine_key), dtype=dtype, device=device)
        bufs = store[key] = (stats, side)
    if keys_by_layer.get(layer_idx) != key:
        _no_capture_alloc('page statistics')
        lengths[layer_idx].zero_()
        keys_by_layer[layer_idx] = key
    return bufs[0], bufs[1], lengths[layer_idx]


def _check_decode_write(decode_write, b, hkv, device, latent=False):
    keys, values, slots = decode_write
    if keys.ndim != 4 or keys.shape[-2] != 1:
        raise ValueError('graph-ready decode KV must be one token per row')
    if values is None:
        # a latent arena's values are the key rows' first dims
        if not latent:
            raise ValueError('paged write decode expects [B,HK,1,DV] values')
    elif values.ndim != 4 or values.shape[-2] != 1:
        raise ValueError('paged write decode expects [B,HK,1,DV] values')
    if keys.shape[0] != b or keys.shape[0] != slots.shape[0]:
        raise ValueError('request batch must match KV batch')
    if keys.shape[1] != hkv:
        raise ValueError('KV head count does not match arena')
    if slots.device != device:
        slots = slots.to(device)
    if slots.dtype != torch.int32:
        slots = slots.to(torch.int32)
    return (keys.contiguous(), None if values is None else values.contiguous(),
            slots.contiguous())


def _alloc_debug(debug, b, hkv, max_blocks, k_f, k_n, k2, cand_cap, device):
    i32 = torch.int32
    debug['far'] = torch.full((b, hkv, max_blocks), -128, dtype=torch.int16,
                              device=device)
    debug['near'] = debug['far'].clone()
    debug['i_f'] = torch.zeros((b, hkv, max(k_f, 1)), dtype=i32, device=device)
    debug['i_n'] = torch.zeros((b, hkv, max(k_n, 1)), dtype=i32, device=device)
    debug['middle'] = torch.zeros((b, hkv, k2), dtype=i32, device=device)
    debug['counts'] = torch.zeros((b, hkv), dtype=i32, device=device)
    debug['bounds'] = torch.zeros((b, 3), dtype=torch.int64, device=device)
    debug['cand_tok'] = torch.full((b, hkv, cand_cap), -1, dtype=i32, device=device)
    debug['cand_logit'] = torch.zeros((b, hkv, cand_cap), dtype=torch.int16,
                                      device=device)
    debug['cand_count'] = torch.zeros((b, hkv), dtype=i32, device=device)


def select_layer_params(cache, layer_idx, req_ids, query_states,
                        attention=None, decode_write=None, middle_only=False,
                        selection_output=None):
    """Validate one selector call and describe it as ``NfaSelectParams``.

    Returns ``(params, keep)`` -- ``keep`` holds tensors the parameters
    point into (converted decode K/V), which must outlive the launch -- or
    None for an empty batch.  The workspace fields are left unset.
    """
    if query_states is None:
        raise ValueError('production selection requires current post-RoPE query')
    if middle_only:
        if selection_output is None or len(selection_output) != 2:
            raise ValueError('middle-only selection requires gather/lens output')
    elif selection_output is not None:
        raise ValueError('custom selection output requires middle_only=True')
    layer0 = cache.layers[0]
    if layer0.kv_pool_k.device.type != 'cuda':
        raise FallbackRequired('HIP device required')
    b = len(req_ids)
    if b == 0:
        return None
    indexer = attention.indexer
    if not hasattr(indexer, 'args') or indexer.args is None:
        raise FallbackRequired('missing indexer config')
    if b > cache.planned_lengths_buf.numel():
        raise ValueError('selector batch exceeds fixed query metadata capacity')
    hq = cache.num_query_heads
    latent = bool(getattr(cache, 'latent', False))
    arena_heads = layer0.num_kv_heads
    # selection rows per batch row: the kv heads, or every query head of a
    # latent arena (one shared row per token, selected per query head)
    hkv = cache.selection_heads if latent else arena_heads
    head_dim = layer0.head_dim_k
    if query_states.shape != (b, hq, head_dim):
        raise ValueError(f'current query must be [{b},{hq},{head_dim}] for one '
                         f'layer, got {tuple(query_states.shape)}')
    if hq % hkv or hq // hkv > _GMAX:
        raise FallbackRequired(f'unsupported GQA group {hq}/{hkv}')
    if indexer.far_method not in _FAR_METHODS:
        raise FallbackRequired(f'far method {indexer.far_method} is not supported')
    if indexer.far_method == 'avg_top2' and hq // hkv < 2:
        # the reference takes torch.topk(2) over the group's heads
        raise ValueError('nfa_far_method avg_top2 needs at least 2 query heads '
                         f'per kv head, got {hq}/{hkv}')
    if query_states.stride(-1) != 1:
        query_states = query_states.contiguous()
    device = layer0.kv_pool_k.device
    lib = nat.load_library()

    bs = int(indexer.args.tia_block_size)
    geo = cache.geometry
    if latent:
        l1_dims, fine_dims, l1_key, fine_key = _latent_dims(indexer, device, layer0)
    else:
        l1_dims, fine_dims, l1_key, fine_key = _dims_for(indexer, device, head_dim)
    if l1_dims.numel() not in (32, 64, 128):
        raise FallbackRequired(f'{l1_dims.numel()} L1 dims are not supported')
    nb_near = max(0, int(indexer.nt_near_pages))
    k1 = int(indexer.args.tia_level1_topk)
    k_f = min(max(0, k1 - nb_near), cache.max_blocks)
    k_n = min(nb_near, cache.max_blocks)
    k2 = int(indexer.args.tia_level2_topk)

    signature = cache.nfa_skip_signature(req_ids)
    live = any(item is not None for item in signature)
    region_mode = cache.nfa_region_mode(signature, layer_idx) if live else 0

    if middle_only:
        gather_out, vis_out = selection_output
    else:
        gather_out = cache.gather_indices_for_layer(layer_idx)
        vis_out = cache.visible_lens_for_layer(layer_idx)
    if (gather_out.dtype != torch.int32 or not gather_out.is_contiguous()
            or vis_out.dtype != torch.int32 or not vis_out.is_contiguous()):
        raise ValueError('selection outputs must be contiguous int32')
    if (gather_out.ndim != 3 or vis_out.ndim != 2 or gather_out.shape[0] < b
            or vis_out.shape[0] < b or gather_out.shape[1] != hkv
            or vis_out.shape[1] != hkv):
        # the kernel writes one gather row per (batch row, kv head)
        raise ValueError(f'selection outputs hold {gather_out.shape[0]} rows of '
                         f'{gather_out.shape[1]} kv heads; the call needs {b} of {hkv}')

    kv_dtype = layer0.kv_pool_k.dtype
    quant = bool(getattr(indexer, 'l2_quant', False))
    if quant and (fine_dims.numel() not in (32, 64) or kv_dtype != torch.bfloat16):
        raise ValueError('--nfa_l2_quant needs 32 or 64 L2 dims and a bf16 KV cache '
                         f'(got {fine_dims.numel()} dims, {kv_dtype})')
    (smin, smax, ssum, psum), l2_side, stats_len = _page_stats_buffers(
        cache, layer_idx, l1_dims, l1_key, kv_dtype, fine_key, head_dim, bs, quant)
    if quant and l2_side is None:
        raise ValueError('--nfa_l2_quant needs the L2 side cache (a sub-width L2 '
                         'subspace and cache.nfa_l2_side_copy)')
    layer = cache.layers[layer_idx]

    p = nat.NfaSelectParams()
    p.abi_version = nat.ABI_VERSION
    p.struct_size = ctypes.sizeof(nat.NfaSelectParams)
    p.batch = b
    p.hq, p.hkv = hq, hkv
    p.kv_heads_mem = arena_heads if not latent else 1
    p.head_dim, p.head_dim_v = head_dim, layer0.head_dim_v
    p.bs, p.page = bs, geo.page
    p.max_blocks, p.max_req = cache.max_blocks, cache.max_requests
    p.geo_sink, p.geo_near, p.geo_window = geo.sink, geo.near, geo.window
    p.sink_tokens = int(indexer.sink_tokens)
    p.swa = int(indexer.sliding_window_size)
    p.near_len = int(indexer.nt_near_len)
    p.k_f, p.k_n, p.k2 = k_f, k_n, k2
    p.near_tokens = -1 if indexer.nt_near_tokens is None else int(indexer.nt_near_tokens)
    p.far_method = _FAR_METHODS[indexer.far_method]
    p.near_method = (nat.METHOD_MINMAX if indexer.near_method == 'minmax'
                     else nat.METHOD_AVG)
    p.dsub, p.fine_dsub = l1_dims.numel(), fine_dims.numel()
    p.kv_dtype = nat.dtype_code(kv_dtype)
    p.q_dtype = nat.dtype_code(query_states.dtype)
    p.max_vis = gather_out.shape[-1]
    p.middle_only = int(bool(middle_only))
    p.l2_quant = int(quant)
    p.protected_only = int(region_mode == 3)
    p.scale = float(attention.scaling)
    p.pool_pages = layer.kv_pool_k.shape[0]
    p.k_pool_l = layer.kv_pool_k.data_ptr()
    p.v_pool_l = layer.kv_pool_v.data_ptr()
    p.block_table_l = cache.block_table_buf[layer_idx].data_ptr()
    p.lengths = cache.planned_lengths_buf.data_ptr()
    p.active_req = cache.active_req_ids_buf.data_ptr()
    p.valid_req = cache.valid_req_ids_buf.data_ptr()
    p.skip_far_l = cache.skip_far_layer_buf[layer_idx].data_ptr()
    p.skip_near_l = cache.skip_near_layer_buf[layer_idx].data_ptr()
    p.dims = l1_dims.data_ptr()
    p.fine_dims = fine_dims.data_ptr()
    p.q = query_states.data_ptr()
    p.q_stride_b = query_states.stride(0)
    p.q_stride_h = query_states.stride(1)
    keep = []
    if decode_write is not None:
        # converted copies are stream-ordered allocations: safe to drop after
        # the asynchronous launch
        keys, values, slots = _check_decode_write(decode_write, b, arena_heads, device,
                                                  latent)
        keys = keys.to(kv_dtype)
        keep += [keys, slots]
        p.k_new, p.slots = keys.data_ptr(), slots.data_ptr()
        if values is not None and not latent:
            values = values.to(kv_dtype)
            keep.append(values)
            p.v_new = values.data_ptr()
    p.stat_min_l, p.stat_max_l, p.stat_sum_l = (
        smin.data_ptr(), smax.data_ptr(), ssum.data_ptr())
    p.stats_len_l = stats_len.data_ptr()
    p.l2_keys_l = l2_side.data_ptr() if l2_side is not None else None
    p.page_sum_l = psum.data_ptr()
    p.gather = gather_out.data_ptr()
    p.vis_lens = vis_out.data_ptr()
    p._region_mode = region_mode
    keep.append(query_states)
    return p, keep


def select_topk_for_layer_batched(cache, layer_idx, req_ids, query_states,
                                  attention=None, decode_write=None,
                                  middle_only=False, selection_output=None,
                                  _debug=None):
    """Select this layer's attended tokens for every batch row.

    ``query_states`` is the current post-RoPE query ``[B, HQ, D]``;
    ``decode_write=(k [B,HKV,1,D], v [B,HKV,1,DV], slots [B])`` writes the
    current token into the arena before anything reads it.  Results go to
    ``cache.gather_indices_for_layer(layer_idx)[:B]`` (absolute physical
    slots, ascending logical order) and ``cache.visible_lens_for_layer``;
    with ``middle_only`` only the middle selection is written to
    ``selection_output=(gather, lens)``.  Returns None.
    """
    built = select_layer_params(cache, layer_idx, req_ids, query_states,
                                attention, decode_write, middle_only,
                                selection_output)
    if built is None:
        return
    p, keep = built
    lib = nat.load_library()
    b, hkv = p.batch, p.hkv
    k_f, k_n, k2, bs = p.k_f, p.k_n, p.k2, p.bs
    region_mode = p._region_mode
    device = keep[-1].device
    need = lib.nfa_select_workspace_bytes(ctypes.byref(p))
    ws = _workspace(cache)
    scratch_key = ('nfa_select_scratch', b, hkv, cache.max_blocks, k_f, k_n)
    scratch = ws.get(scratch_key)
    if scratch is None or scratch.numel() < need:
        _no_capture_alloc('selector scratch')
        scratch = ws[scratch_key] = torch.zeros(need, dtype=torch.uint8,
                                                device=device)
    p.workspace = scratch.data_ptr()
    p.workspace_bytes = scratch.numel()
    if _debug is not None and _debug.get('clock_only'):
        # phase timeline only: the production path plus wall-clock marks
        ntiles = -(-cache.max_blocks // nat.SELECT_CLOCK_PAGES)
        _debug['clock'] = torch.zeros((b * hkv, ntiles + 1, 32),
                                      dtype=torch.int64, device=device)
        p.dbg_clock = _debug['clock'].data_ptr()
    elif _debug is not None:
        want_clock = _debug.get('want_clock', False)
        _debug.clear()
        _debug['want_clock'] = want_clock
        cand_cap = (k_f + k_n + 2) * bs
        _alloc_debug(_debug, b, hkv, cache.max_blocks, k_f, k_n, k2, cand_cap,
                     device)
        p.dbg_far = _debug['far'].data_ptr()
        p.dbg_near = _debug['near'].data_ptr()
        p.dbg_i_f = _debug['i_f'].data_ptr()
        p.dbg_i_n = _debug['i_n'].data_ptr()
        p.dbg_middle = _debug['middle'].data_ptr()
        p.dbg_counts = _debug['counts'].data_ptr()
        p.dbg_bounds = _debug['bounds'].data_ptr()
        p.dbg_cand_tok = _debug['cand_tok'].data_ptr()
        p.dbg_cand_logit = _debug['cand_logit'].data_ptr()
        p.dbg_cand_count = _debug['cand_count'].data_ptr()
        p.dbg_cand_cap = cand_cap
        _debug['region_mode'] = region_mode
        if _debug.get('want_clock'):
            ntiles = -(-cache.max_blocks // nat.SELECT_CLOCK_PAGES)
            _debug['clock'] = torch.zeros((b * hkv, ntiles + 1, 32),
                                          dtype=torch.int64, device=device)
            p.dbg_clock = _debug['clock'].data_ptr()
    if _debug is not None:
        # the launch plan: kernel instance, tiles per row, passes of a row of
        # max_blocks pages (tests assert which instance a shape runs)
        plan = (ctypes.c_int32 * 8)()
        nat.check(lib.nfa_select_plan(ctypes.byref(p), plan, 8), 'nfa_select_plan')
        _debug['plan'] = dict(zip(('instance', 'round_tiles', 'grid_tiles',
                                   'row_tiles', 'passes', 'lds', 'segments',
                                   'workspace'), list(plan)))
    rc = lib.nfa_select_layer(ctypes.byref(p), nat.stream_handle())
    if rc == -1 and 'LDS' in lib.nfa_last_error().decode():
        raise FallbackRequired(lib.nfa_last_error().decode())
    nat.check(rc, 'select_topk_for_layer_batched')
