"""Paged KV writes and sparse gather attention on the graph-ready arena.

Drop-in for the reference's ``sparse_attn/ops/paged_region_kernels.py``:
``paged_write_prefill`` (:610-662), ``paged_write_decode`` (:665-724) and
``sparse_paged_attention_gather`` (:800-1006).  Device work runs in
libnfa_hip.so; CPU tensors are accepted only by the two write helpers (a plain
copy, as the reference's CPU branch), never by the attention.
"""
import ctypes

import torch

from .. import _native as nat


def _kv_contiguous(x):
    return x if x.is_contiguous() else x.contiguous()


def paged_write_prefill(cache_layer, key_states, value_states, block_table, *,
                        workspace=None):
    """Scatter an unpadded ``[1, HK, N, D]`` prefill through ``block_table``.
    A latent arena takes ``value_states`` None (its values are the key rows'
    first dims)."""
    if key_states.ndim != 4 or key_states.shape[0] != 1 or key_states.shape[2] < 1:
        raise ValueError('paged write prefill expects [1,HK,N,D] keys')
    keys_only = value_states is None
    if keys_only and not getattr(cache_layer, 'latent', False):
        raise ValueError('paged write prefill expects [1,HK,N,DV] values')
    if keys_only:
        value_states = key_states[..., :cache_layer.head_dim_v]
    if value_states.ndim != 4 or value_states.shape[:3] != key_states.shape[:3]:
        raise ValueError('paged write prefill expects [1,HK,N,DV] values')
    if key_states.shape[1] != cache_layer.num_kv_heads:
        raise ValueError('KV head count does not match arena')
    if key_states.shape[-1] != cache_layer.head_dim_k:
        raise ValueError('key head dimension does not match arena')
    if value_states.shape[-1] != cache_layer.head_dim_v:
        raise ValueError('value head dimension does not match arena')
    if block_table.ndim != 1 or block_table.device != key_states.device:
        raise ValueError('prefill block table must be a device-matched 1D row')
    n = key_states.shape[2]
    page = cache_layer.geometry.page
    if n > block_table.numel() * page:
        raise ValueError('prefill length exceeds block-table capacity')
    if key_states.dtype != cache_layer.kv_pool_k.dtype:
        raise ValueError('KV dtype does not match arena')
    if not key_states.is_cuda:
        for lp in range((n + page - 1) // page):
            pid = int(block_table[lp])
            lo, hi = lp * page, min(lp * page + page, n)
            cache_layer.kv_pool_k[pid, 0, :, :hi - lo].copy_(key_states[0, :, lo:hi])
            if not keys_only:
                cache_layer.kv_pool_v[pid, 0, :, :hi - lo].copy_(value_states[0, :, lo:hi])
        return key_states, value_states
    lib = nat.load_library()
    keys = _kv_contiguous(key_states)
    values = None if keys_only else _kv_contiguous(value_states)
    table = block_table if block_table.dtype == torch.int32 else block_table.to(torch.int32)
    table = _kv_contiguous(table)
    # keys only: value width 0, no value pointers
    rc = lib.nfa_paged_write_prefill(
        keys.data_ptr(), None if keys_only else values.data_ptr(), n, table.data_ptr(),
        cache_layer.num_kv_heads, cache_layer.head_dim_k,
        0 if keys_only else cache_layer.head_dim_v,
        page, nat.dtype_code(keys.dtype), cache_layer.kv_pool_k.data_ptr(),
        None if keys_only else cache_layer.kv_pool_v.data_ptr(), nat.stream_handle())
    nat.check(rc, 'paged_write_prefill')
    return key_states, value_states


def paged_write_decode(cache_layer, key_states, value_states, slot_mapping, *,
                       workspace=None):
    """Write ``[B, HK, 1, D]`` decode keys/values at ``slot_mapping`` [B]."""
    if key_states.ndim != 4 or key_states.shape[-2] != 1:
        raise ValueError('paged write decode expects [B,HK,1,D] keys')
    if value_states.ndim != 4 or value_states.shape[-2] != 1:
        raise ValueError('paged write decode expects [B,HK,1,DV] values')
    if key_states.shape[0] != slot_mapping.shape[0]:
        raise ValueError('slot mapping batch must match KV batch')
    if key_states.shape[1] != cache_layer.num_kv_heads:
        raise ValueError('KV head count does not match arena')
    if key_states.device != slot_mapping.device:
        slot_mapping = slot_mapping.to(key_states.device)
    batch = key_states.shape[0]
    page = cache_layer.geometry.page
    if not key_states.is_cuda:
        pad_slot = cache_layer.PAD_PAGE_ID * page
        for b in range(batch):
            slot = int(slot_mapping[b])
            pid, off = divmod(slot if slot >= 0 else pad_slot, page)
            cache_layer.kv_pool_k[pid, 0, :, off] = key_states[b, :, 0]
            cache_layer.kv_pool_v[pid, 0, :, off] = value_states[b, :, 0]
        return key_states, value_states
    lib = nat.load_library()
    keys = _kv_contiguous(key_states.to(cache_layer.kv_pool_k.dtype))
    values = _kv_contiguous(value_states.to(cache_layer.kv_pool_v.dtype))
    slots = slot_mapping if slot_mapping.dtype == torch.int32 else slot_mapping.to(torch.int32)
    slots = _kv_contiguous(slots)
    rc = lib.nfa_paged_write_decode(
        keys.data_ptr(), values.data_ptr(), slots.data_ptr(), batch,
        cache_layer.num_kv_heads, cache_layer.head_dim_k, cache_layer.head_dim_v,
        page, nat.dtype_code(keys.dtype), cache_layer.kv_pool_k.data_ptr(),
        cache_layer.kv_pool_v.data_ptr(), nat.stream_handle())
    nat.check(rc, 'paged_write_decode')
    return key_states, value_states


def _scratch(workspace, key, nbytes, device):
    """Zero-initialised byte scratch, cached in ``workspace`` when given."""
    if workspace is None:
        return torch.zeros(nbytes, dtype=torch.uint8, device=device)
    buf = workspace.get(key)
    if buf is None or buf.numel() < nbytes:
        if torch.cuda.is_current_stream_capturing():
            raise RuntimeError(f'scratch {key!r} must be allocated before capture')
        buf = torch.zeros(nbytes, dtype=torch.uint8, device=device)
        workspace[key] = buf
    return buf


def sparse_paged_attention_gather(cache_layer, q, gather_indices, visible_lens,
                                  query_to_req, *, scale, workspace=None,
                                  split_kv=False, tokens_per_split=0):
    """Attention of each query head over its kv group's selected slots.

    ``q`` is ``[T, HQ, D]``; ``gather_indices`` ``[B, HK, MAX_VISIBLE]`` holds
    absolute physical slots, ``visible_lens`` ``[B, HK]`` their counts and
    ``query_to_req`` ``[T]`` the gather row of each query row (-1 = padding,
    output zero).  Softmax in fp32; output in the dtype of ``q``.
    ``split_kv`` is accepted for compatibility; the kernel always splits the
    selected slots across workgroups and merges the partial softmax states.
    """
    if q.ndim != 3 or q.shape[-1] != cache_layer.head_dim_k:
        raise ValueError('sparse gather attention expects flat [T,HQ,D] query')
    hq = q.shape[1]
    hk = cache_layer.num_kv_heads
    if hq % hk != 0:
        raise ValueError('GQA requires HQ % HK == 0')
    page = cache_layer.geometry.page
    if page & (page - 1):
        raise ValueError('sparse gather attention requires power-of-two page size')
    _check_gather(gather_indices, visible_lens, hk)
    nat.require_hip(q, 'sparse_paged_attention_gather')
    lib = nat.load_library()
    total_q = q.shape[0]
    out = q.new_empty((total_q, hq, cache_layer.head_dim_v))
    if total_q == 0:
        return out
    p, keep = _attn_params(cache_layer, q, gather_indices, visible_lens,
                           query_to_req, scale, tokens_per_split)
    p.out = out.data_ptr()
    need = lib.nfa_attn_workspace_bytes(ctypes.byref(p))
    ws = _scratch(workspace, ('nfa_attn_scratch', total_q, hk, p.max_vis, hq,
                              p.head_dim_v, p.tokens_per_split), need, q.device)
    p.workspace = ws.data_ptr()
    p.workspace_bytes = ws.numel()
    nat.check(lib.nfa_sparse_attn_decode(ctypes.byref(p), nat.stream_handle()),
              'sparse_paged_attention_gather')
    del keep
    return out


def sparse_mla_attention_gather(cache_layer, q, gather_indices, visible_lens,
                                query_to_req, *, scale, workspace=None,
                                out_dtype=None, w_uv=None):
    """Absorbed latent attention of each query head over its own selection.

    ``cache_layer`` is a latent arena (one kv head, rows of ``head_dim_k`` =
    value dims + 64 RoPE dims, the values the rows' first ``head_dim_v``
    dims); ``q`` ``[T, H, head_dim_k]`` holds per head ``[W_uk^T q_nope |
    q_pe]``; ``gather_indices`` ``[B, H, W]`` / ``visible_lens`` ``[B, H]``
    are the per-head selections.  Returns ``[T, H, head_dim_v]`` -- each
    head's softmax-weighted latent rows -- or, with ``w_uv`` ``[H, V,
    head_dim_v]`` (bf16, each head's value up-projection), ``[T, H, V]`` =
    ``W_uv,h`` applied to them, in ``out_dtype`` (default: the dtype of
    ``q``).  No reference
    counterpart: the reference attends over expanded heads
    (``sparse_paged_attention_gather``), which this equals up to rounding.
    """
    if q.ndim != 3 or q.shape[-1] != cache_layer.head_dim_k:
        raise ValueError('latent attention expects flat [T,H,latent] query')
    if cache_layer.num_kv_heads != 1:
        raise ValueError('latent attention expects a single-head latent arena')
    heads = q.shape[1]
    _check_gather(gather_indices, visible_lens, heads)
    if (gather_indices.dtype != torch.int32 or not gather_indices.is_contiguous()
            or visible_lens.dtype != torch.int32 or not visible_lens.is_contiguous()):
        raise ValueError('gather indices and lens must be contiguous int32')
    nat.require_hip(q, 'sparse_mla_attention_gather')
    lib = nat.load_library()
    total_q = q.shape[0]
    if w_uv is not None:
        if (w_uv.dtype != torch.bfloat16 or w_uv.ndim != 3 or w_uv.shape[0] != heads
                or w_uv.shape[2] != cache_layer.head_dim_v or not w_uv.is_contiguous()):
            raise ValueError('w_uv must be a contiguous bf16 [H, V, head_dim_v] tensor')
    width = cache_layer.head_dim_v if w_uv is None else w_uv.shape[1]
    out = q.new_empty((total_q, heads, width), dtype=out_dtype or q.dtype)
    if total_q == 0:
        return out
    qc = q if q.is_contiguous() else q.contiguous()
    q2r = query_to_req
    if q2r.dtype != torch.int32:
        q2r = q2r.to(torch.int32)
    q2r = q2r.contiguous()
    p = nat.NfaMlaAttnParams()
    p.abi_version = nat.ABI_VERSION
    p.struct_size = ctypes.sizeof(nat.NfaMlaAttnParams)
    p.total_q, p.heads = total_q, heads
    p.latent_dim, p.value_dim = cache_layer.head_dim_k, cache_layer.head_dim_v
    p.page = cache_layer.geometry.page
    p.gather_rows = gather_indices.shape[0]
    p.max_vis = gather_indices.shape[-1]
    p.kv_dtype = nat.dtype_code(cache_layer.kv_pool_k.dtype)
    p.q_dtype = nat.dtype_code(qc.dtype)
    p.out_dtype = nat.dtype_code(out.dtype)
    p.pool_pages = cache_layer.kv_pool_k.shape[0]
    p.scale = float(scale)
    p.q = qc.data_ptr()
    p.kv_pool = cache_layer.kv_pool_k.data_ptr()
    p.gather = gather_indices.data_ptr()
    p.vis_lens = visible_lens.data_ptr()
    p.query_to_req = q2r.data_ptr()
    if w_uv is not None:
        p.w_uv = w_uv.data_ptr()
        p.out_dim = w_uv.shape[1]
    p.out = out.data_ptr()
    need = lib.nfa_mla_attn_workspace_bytes(ctypes.byref(p))
    ws = _scratch(workspace, ('nfa_mla_attn_scratch', total_q, heads, p.max_vis,
                              p.value_dim), need, q.device)
    p.workspace = ws.data_ptr()
    p.workspace_bytes = ws.numel()
    nat.check(lib.nfa_mla_attn_decode(ctypes.byref(p), nat.stream_handle()),
              'sparse_mla_attention_gather')
    del qc, q2r
    return out


def _check_gather(gather_indices, visible_lens, hk):
    if (gather_indices.ndim != 3 or gather_indices.shape[1] != hk
            or visible_lens.shape != gather_indices.shape[:2]):
        raise ValueError('gather attention expects indices [B,HK,K] and lens [B,HK]')


def _attn_params(cache_layer, q, gather_indices, visible_lens, query_to_req, scale,
                 tokens_per_split):
    """NfaAttnParams of a gather attention call (``out`` and the workspace
    left unset) and the converted tensors it points into."""
    hq = q.shape[1]
    hk = cache_layer.num_kv_heads
    total_q = q.shape[0]
    qc = q if q.is_contiguous() else q.contiguous()
    gather = gather_indices
    if gather.dtype != torch.int32 or not gather.is_contiguous():
        raise ValueError('gather indices must be contiguous int32')
    lens = visible_lens
    if lens.dtype != torch.int32 or not lens.is_contiguous():
        raise ValueError('visible lens must be contiguous int32')
    q2r = query_to_req
    if q2r.dtype != torch.int32:
        q2r = q2r.to(torch.int32)
    q2r = q2r.contiguous()
    p = nat.NfaAttnParams()
    p.abi_version = nat.ABI_VERSION
    p.struct_size = ctypes.sizeof(nat.NfaAttnParams)
    p.total_q = total_q
    p.hq, p.hkv = hq, hk
    p.head_dim, p.head_dim_v = cache_layer.head_dim_k, cache_layer.head_dim_v
    p.page = cache_layer.geometry.page
    p.gather_rows = gather.shape[0]
    p.max_vis = gather.shape[-1]
    p.kv_dtype = nat.dtype_code(cache_layer.kv_pool_k.dtype)
    p.q_dtype = nat.dtype_code(q.dtype)
    p.tokens_per_split = int(tokens_per_split)
    p.pool_pages = cache_layer.kv_pool_k.shape[0]
    p.scale = float(scale)
    p.q = qc.data_ptr()
    p.k_pool = cache_layer.kv_pool_k.data_ptr()
    p.v_pool = cache_layer.kv_pool_v.data_ptr()
    p.gather = gather.data_ptr()
    p.vis_lens = lens.data_ptr()
    p.query_to_req = q2r.data_ptr()
    return p, (qc, q2r)


def _partial_block_tokens(cache_layer, total_q):
    """Token block of the split partition (reference
    ops/paged_region_kernels.py:752-757)."""
    if cache_layer.head_dim_k >= 256 or cache_layer.head_dim_v >= 256:
        return 64
    return 128 if total_q <= 8 else 64


def sparse_paged_attention_gather_partial(cache_layer, q, gather_indices, visible_lens,
                                          query_to_req, *, scale, workspace, name, nsplit):
    """One region's attention as fp32 split states, without normalising
    (reference ops/paged_region_kernels.py:727-780).

    Split ``s`` of a (query row, kv head) with ``n`` visible slots covers the
    token blocks ``[s*nb//nsplit, (s+1)*nb//nsplit)`` of ``nb =
    ceil(n / block)`` (block 128 for at most 8 query rows, else 64; 64 for
    head dims of 256).  Returns ``(acc [nsplit, T, HQ, DV], m [nsplit, T,
    HQ], z [nsplit, T, HQ])`` from fixed buffers of ``workspace`` keyed by
    ``name``: ``m`` the split's maximum score (``-inf`` if it has none),
    ``z = sum exp(s_i - m)``, ``acc = sum exp(s_i - m) v_i``."""
    if not q.is_cuda:
        raise RuntimeError('split regions require a HIP device')
    if q.ndim != 3 or q.shape[-1] != cache_layer.head_dim_k:
        raise ValueError('split regions expect flat [T,HQ,D] query')
    hq = q.shape[1]
    hk = cache_layer.num_kv_heads
    if hq % hk != 0:
        raise ValueError('GQA requires HQ % HK == 0')
    page = cache_layer.geometry.page
    if page & (page - 1):
        raise ValueError('split regions require power-of-two page size')
    if cache_layer.head_dim_k < 16 or cache_layer.head_dim_v < 16:
        raise RuntimeError('split regions require grouped attention geometry')
    nsplit = int(nsplit)
    if nsplit < 1:
        raise ValueError('nsplit must be positive')
    _check_gather(gather_indices, visible_lens, hk)
    nat.require_hip(q, 'sparse_paged_attention_gather_partial')
    lib = nat.load_library()
    total_q = q.shape[0]
    dv = cache_layer.head_dim_v
    part_acc = _state(workspace, f'gather_split_{name}_acc', (nsplit, total_q, hq, dv),
                      q.device)
    part_m = _state(workspace, f'gather_split_{name}_m', (nsplit, total_q, hq), q.device)
    part_z = _state(workspace, f'gather_split_{name}_z', (nsplit, total_q, hq), q.device)
    if total_q == 0:
        return part_acc, part_m, part_z
    p, keep = _attn_params(cache_layer, q, gather_indices, visible_lens, query_to_req,
                           scale, 0)
    pt = nat.NfaAttnPartial()
    pt.abi_version = nat.ABI_VERSION
    pt.struct_size = ctypes.sizeof(nat.NfaAttnPartial)
    pt.nsplit = nsplit
    pt.block_tokens = _partial_block_tokens(cache_layer, total_q)
    pt.acc, pt.m, pt.z = part_acc.data_ptr(), part_m.data_ptr(), part_z.data_ptr()
    need = lib.nfa_attn_partial_workspace_bytes(ctypes.byref(p), ctypes.byref(pt))
    ws = _scratch(workspace, ('nfa_attn_partial_scratch', name, total_q, hk, p.max_vis,
                              hq, dv, nsplit, pt.block_tokens), need, q.device)
    p.workspace = ws.data_ptr()
    p.workspace_bytes = ws.numel()
    nat.check(lib.nfa_sparse_attn_partial(ctypes.byref(p), ctypes.byref(pt),
                                          nat.stream_handle()),
              'sparse_paged_attention_gather_partial')
    del keep
    return part_acc, part_m, part_z


def _state(workspace, key, shape, device):
    """fp32 state buffer of a fixed address, cached in ``workspace``."""
    if workspace is None:
        return torch.empty(shape, dtype=torch.float32, device=device)
    buf = workspace.get(key)
    if buf is None or tuple(buf.shape) != tuple(shape):
        if torch.cuda.is_current_stream_capturing():
            raise RuntimeError(f'state {key!r} must be allocated before capture')
        buf = torch.empty(shape, dtype=torch.float32, device=device)
        workspace[key] = buf
    return buf


def sparse_paged_attention_regions_combine(q, protected_parts, middle_parts, *, workspace):
    """Merge two disjoint regions' split states into the attention output
    ``[T, HQ, DV]`` in the dtype of ``q`` (reference
    ops/paged_region_kernels.py:783-797): protected splits first, then the
    middle's, each folded in with the online-softmax rescaling; rows whose
    denominator is 0 output 0."""
    del workspace  # the combine keeps no state
    total_q, hq = q.shape[:2]
    dv = protected_parts[0].shape[-1]
    for parts in (protected_parts, middle_parts):
        acc, m, z = parts
        if (acc.dtype != torch.float32 or acc.shape[1:] != (total_q, hq, dv)
                or m.shape != acc.shape[:3] or z.shape != acc.shape[:3]
                or not (acc.is_contiguous() and m.is_contiguous() and z.is_contiguous())):
            raise ValueError('region states must be contiguous fp32 [S,T,HQ,DV] / [S,T,HQ]')
    nat.require_hip(q, 'sparse_paged_attention_regions_combine')
    lib = nat.load_library()
    out = q.new_empty((total_q, hq, dv))
    if total_q == 0:
        return out
    c = nat.NfaAttnCombineParams()
    c.abi_version = nat.ABI_VERSION
    c.struct_size = ctypes.sizeof(nat.NfaAttnCombineParams)
    c.total_q, c.hq, c.head_dim_v = total_q, hq, dv
    c.out_dtype = nat.dtype_code(q.dtype)
    c.nsplit_a, c.nsplit_b = protected_parts[0].shape[0], middle_parts[0].shape[0]
    c.acc_a, c.m_a, c.z_a = (t.data_ptr() for t in protected_parts)
    c.acc_b, c.m_b, c.z_b = (t.data_ptr() for t in middle_parts)
    c.out = out.data_ptr()
    nat.check(lib.nfa_attn_regions_combine(ctypes.byref(c), nat.stream_handle()),
              'sparse_paged_attention_regions_combine')
    return out
