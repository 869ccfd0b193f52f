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


def indexer_dims(indexer, head_dim=128, latent_value_dim=None):
    """(L1 dims, L2 dims) the selector reads; of a latent arena row
    [c (latent_value_dim) | k_pe]: the k_pe dims (the expanded heads'
    mla_rope dims)."""
    if latent_value_dim is not None:
        dims = np.arange(latent_value_dim, head_dim)
        return dims, dims
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
    """Oracle configuration of the cache's layer 0 and the indexer; a latent
    arena is seen as its expanded heads (one selection row per query head)."""
    layer = cache.layers[0]
    latent = getattr(cache, 'latent', False)
    l1, fine = indexer_dims(indexer, layer.head_dim_k,
                            layer.head_dim_v if latent else None)
    nb_near = max(0, int(indexer.nt_near_pages))
    return orc.NfaConfig(
        hq=cache.num_query_heads,
        hkv=cache.selection_heads if latent else layer.num_kv_heads,
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


def snapshot(cache, layer_idx, batch, with_v=True):
    """Numpy copy of everything the selector reads for ``layer_idx`` (the V
    pool too unless ``with_v`` is False: selection never reads it)."""
    layer = cache.layers[layer_idx]
    latent = getattr(cache, 'latent', False)
    return dict(
        k_pool=to_np(layer.kv_pool_k),
        v_pool=to_np(layer.kv_pool_v) if with_v and not latent else None,
        latent_heads=cache.selection_heads if latent else None,
        block_table=to_np(cache.block_table_buf[layer_idx]).astype(np.int64),
        lengths=to_np(cache.planned_lengths_buf[:batch]).astype(np.int64),
        req_ids=to_np(cache.valid_req_ids_buf[:batch]).astype(np.int64),
        active=to_np(cache.active_req_ids_buf[:batch]) >= 0,
        skip_far=to_np(cache.skip_far_layer_buf[layer_idx]),
        skip_near=to_np(cache.skip_near_layer_buf[layer_idx]))


def run_oracle(cfg, snap, q, decode=None, max_vis=1024, middle_only=False,
               copy=True):
    """Oracle selection on a snapshot; ``decode`` = (keys, values, slots).
    ``copy`` False applies the decode write to the snapshot's own pools."""
    k_pool = snap['k_pool'].copy() if copy else snap['k_pool']
    v_pool = snap['v_pool']
    if copy and v_pool is not None:
        v_pool = v_pool.copy()
    if decode is not None:
        keys, values, slots = decode
        active = snap['active']
        slots = np.where(active, np.asarray(slots), -1)
        orc.apply_decode_write(k_pool, v_pool, np.asarray(keys, np.float32),
                               None if values is None else np.asarray(values, np.float32),
                               slots, cfg.page)
    if snap.get('latent_heads'):
        # a latent arena as its expanded heads: every head reads the shared
        # rows (expand_kv copies k_pe into every head)
        shape = list(k_pool.shape)
        shape[2] = snap['latent_heads']
        k_pool = np.broadcast_to(k_pool, tuple(shape))
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


# ---------------------------------------------------------------------------
# selector parity runs on the GPU (shared by the selector test modules)
# ---------------------------------------------------------------------------

GPU = 'cuda'
GEO16 = RegionGeometry(sink=4, near=4096, window=128, page=16, max_new_tokens=64)


def prefill_request(cache, req, length, gen, n_layers=1, dtype=torch.bfloat16,
                    zero_keys=False, key_fn=None):
    """Write ``length`` prompt tokens of request ``req`` into every layer.
    ``key_fn(n, hkv, d, gen)`` supplies the keys (default N(0,1))."""
    hkv = cache.num_kv_heads
    d = cache.layers[0].head_dim_k
    dv = cache.layers[0].head_dim_v
    cache.add_request(req)
    for layer in range(n_layers):
        if zero_keys:
            keys = torch.zeros(1, hkv, length, d, dtype=dtype, device=GPU)
        elif key_fn is not None:
            keys = key_fn(length, hkv, d, gen).to(dtype)
        else:
            keys = bf16_randn((1, hkv, length, d), gen, GPU).to(dtype)
        values = bf16_randn((1, hkv, length, dv), gen, GPU).to(dtype)
        cache.write_prefill(layer, req, keys, values)
        del keys, values


def decode_inputs(cache, b, gen, dtype, layer_idx=0):
    """Current-token K/V of ``b`` rows and their planned slots."""
    hkv = cache.num_kv_heads
    d = cache.layers[0].head_dim_k
    dv = cache.layers[0].head_dim_v
    keys = bf16_randn((b, hkv, 1, d), gen, GPU).to(dtype)
    values = bf16_randn((b, hkv, 1, dv), gen, GPU).to(dtype)
    slots = cache.slot_mapping_for_layer(layer_idx)[:b].clone()
    return keys, values, slots


def u16(t):
    return t.cpu().numpy().astype(np.int64) & 0xFFFF


def prod_cache(lengths, *, hkv=2, hq=8, dtype=torch.bfloat16, max_req=4,
               skips=None, req_ids=None, seed=20261201, zero_keys=False,
               geometry=GEO16, key_fn=None, max_visible_len=1024, head_dim=128,
               head_dim_v=None):
    """One-layer cache holding frozen requests of the given prompt lengths."""
    page = geometry.page
    extra = geometry.max_new_tokens
    max_blocks = (max(lengths) + extra + page - 1) // page + 8
    phys = sum((n + extra + page - 1) // page for n in lengths) + 8
    cache = make_cache(GPU, geometry=geometry, max_blocks=max_blocks,
                       max_physical_pages=phys, max_visible_len=max_visible_len,
                       hkv=hkv, hq=hq, dtype=dtype, max_requests=max_req,
                       max_query_tokens=max(8, max_req), head_dim=head_dim,
                       head_dim_v=head_dim_v)
    gen = torch.Generator(device=GPU).manual_seed(seed)
    req_ids = req_ids or list(range(len(lengths)))
    skips = skips or [(False, False)] * len(lengths)
    for rid, n, (sf, sn) in zip(req_ids, lengths, skips):
        prefill_request(cache, rid, n, gen, dtype=dtype, zero_keys=zero_keys,
                        key_fn=key_fn)
        cache.freeze(rid, [sf], [sn])
    return cache, gen, req_ids


def run_and_compare(cache, indexer, req_ids, q, decode, *, scaling=1.0,
                    middle_only=False, check_debug=True, return_pools=False,
                    with_v=True, plan=None):
    """Run the HIP selector on layer 0 and the oracle on a snapshot of the
    same cache; compare every intermediate bit for bit.  Returns the oracle's
    per-row results (and the post-decode-write pools with ``return_pools``).

    ``check_debug`` False runs the production launch (no debug buffers, the
    launch the benchmarks and the model time) and compares its gather rows,
    visible lengths and decode-written rows.  ``with_v`` False leaves the V
    pool out of the snapshot (large contexts; the returned V pool is None).
    ``plan``, a dict, receives the launch plan (kernel instance, tiles,
    passes)."""
    from sparse_attn.indexer.nfa_layer_batch_selector import \
        select_topk_for_layer_batched
    b = len(req_ids)
    cfg = cfg_from(cache, indexer, scaling)
    snap = snapshot(cache, 0, b, with_v=with_v)
    max_vis = cache.gather_indices_for_layer(0).shape[-1]
    dbg = {} if check_debug else None
    if plan is not None:
        plan.clear()
        plan.update(launch_plan(cache, indexer, req_ids, q, decode, scaling,
                                middle_only))
    sel_out = None
    if middle_only:
        sel_out = (torch.full((b, cache.num_kv_heads, max_vis), -7,
                              dtype=torch.int32, device=GPU),
                   torch.zeros((b, cache.num_kv_heads), dtype=torch.int32,
                               device=GPU))
    select_topk_for_layer_batched(cache, 0, req_ids, q,
                                  attention=attention_ns(indexer, scaling),
                                  decode_write=decode, middle_only=middle_only,
                                  selection_output=sel_out, _debug=dbg)
    torch.cuda.synchronize()
    dec_np = None
    if decode is not None:
        dec_np = tuple(None if t is None else
                       t.float().cpu().numpy() if t.is_floating_point()
                       else t.cpu().numpy() for t in decode)
    res, k_pool, v_pool = run_oracle(cfg, snap, q.float().cpu().numpy(), dec_np,
                                     max_vis=max_vis, middle_only=middle_only,
                                     copy=False)
    del snap
    if middle_only:
        gather, vis = sel_out[0].cpu().numpy(), sel_out[1].cpu().numpy()
    else:
        gather = cache.gather_indices_for_layer(0).cpu().numpy()
        vis = cache.visible_lens_for_layer(0).cpu().numpy()
    region_mode = dbg.get('region_mode', 0) if dbg is not None else 0
    for row_b in range(b):
        for kv in range(cfg.hkv):
            r = res[row_b][kv]
            tag = f'row={row_b} kv={kv}'
            assert vis[row_b, kv] == r.vis_len, tag
            n = min(r.vis_len, max_vis)
            np.testing.assert_array_equal(gather[row_b, kv, :n], r.gather[:n],
                                          err_msg=tag)
            if not check_debug or region_mode == 3 or r.far is None:
                continue
            # pages past the block-table width are never scored (the
            # oracle's scores there are outside every top-k)
            kt = min(len(r.far), cfg.max_blocks)
            np.testing.assert_array_equal(u16(dbg['far'][row_b, kv, :kt]),
                                          r.far[:kt].astype(np.int64), err_msg=tag)
            np.testing.assert_array_equal(u16(dbg['near'][row_b, kv, :kt]),
                                          r.near[:kt].astype(np.int64), err_msg=tag)
            np.testing.assert_array_equal(
                dbg['i_f'][row_b, kv, :cfg.k_f].cpu().numpy(), r.i_f, err_msg=tag)
            np.testing.assert_array_equal(
                dbg['i_n'][row_b, kv, :cfg.k_n].cpu().numpy(), r.i_n, err_msg=tag)
            assert tuple(dbg['bounds'][row_b].cpu().tolist()) == (
                r.lower, r.upper, r.quota), tag
            nc = int(dbg['cand_count'][row_b, kv])
            tok = dbg['cand_tok'][row_b, kv, :nc].cpu().numpy()
            logit = u16(dbg['cand_logit'][row_b, kv, :nc])
            # dense page-major layout: slots outside the candidate range are -1
            scored = tok >= 0
            tok, logit = tok[scored], logit[scored]
            order = np.argsort(r.cand_tokens, kind='stable')
            np.testing.assert_array_equal(tok, r.cand_tokens[order], err_msg=tag)
            np.testing.assert_array_equal(logit, r.cand_logits[order].astype(np.int64),
                                          err_msg=tag)
            cnt = int(dbg['counts'][row_b, kv])
            assert cnt == r.count, tag
            np.testing.assert_array_equal(
                dbg['middle'][row_b, kv, :cnt].cpu().numpy(), r.middle[:cnt],
                err_msg=tag)
    if decode is not None:
        layer = cache.layers[0]
        slots = decode[2].cpu().numpy()
        for row_b in range(b):
            if slots[row_b] < 0:
                continue
            phys, off = divmod(int(slots[row_b]), cfg.page)
            arena = layer.num_kv_heads
            np.testing.assert_array_equal(
                layer.kv_pool_k[phys, 0, :, off].float().cpu().numpy(),
                k_pool[phys, 0, :arena, off])
            if v_pool is not None:
                np.testing.assert_array_equal(
                    layer.kv_pool_v[phys, 0, :, off].float().cpu().numpy(),
                    v_pool[phys, 0, :, off])
    if return_pools:
        return res, k_pool, v_pool
    return res


def launch_plan(cache, indexer, req_ids, q, decode=None, scaling=1.0,
                middle_only=False):
    """The selector's launch plan for this call (kernel instance, tiles per
    row, passes of a max_blocks row), queried without launching."""
    import ctypes

    from sparse_attn import _native as nat
    from sparse_attn.indexer.nfa_layer_batch_selector import \
        select_layer_params
    b = len(req_ids)
    sel_out = None
    if middle_only:
        sel_out = (cache.gather_indices_for_layer(0)[:b],
                   cache.visible_lens_for_layer(0)[:b])
    p, _keep = select_layer_params(cache, 0, req_ids, q,
                                   attention_ns(indexer, scaling), decode,
                                   middle_only, sel_out)
    out = (ctypes.c_int32 * 8)()
    lib = nat.load_library()
    nat.check(lib.nfa_select_plan(ctypes.byref(p), out, 8), 'nfa_select_plan')
    return dict(zip(('instance', 'round_tiles', 'grid_tiles', 'row_tiles',
                     'passes', 'lds', 'segments', 'workspace'), list(out)))
