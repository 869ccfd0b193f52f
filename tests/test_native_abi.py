"""The C ABI of libnfa_hip.so: exported symbols, struct layout, host checks.

Runs without a GPU: only entry points that reject their arguments before
any HIP call are invoked.
"""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, 'include', 'nfa_hip.h')


@pytest.fixture(scope='module')
def lib():
    import torch  # noqa: F401  (bind to torch's HIP runtime first)
    from sparse_attn import _native
    if not os.path.exists(_native.LIB_PATH):
        from sparse_attn import _build
        _build.build()
    return _native.load_library()


def _declared():
    text = open(HEADER).read()
    return sorted(set(re.findall(r'\b(nfa_[a-z0-9_]+)\s*\(', text)))


def test_every_declared_symbol_is_exported(lib):
    names = _declared()
    assert len(names) >= 10
    for name in names:
        assert hasattr(lib, name), name


def test_struct_layout_matches(lib):
    from sparse_attn import _native
    assert lib.nfa_select_params_size() == ctypes.sizeof(_native.NfaSelectParams)
    assert lib.nfa_attn_params_size() == ctypes.sizeof(_native.NfaAttnParams)
    assert lib.nfa_abi_version() == _native.ABI_VERSION


def test_null_and_bad_params_are_rejected_before_launch(lib):
    from sparse_attn import _native
    assert lib.nfa_select_layer(None, None) == -1
    assert b'null params' in lib.nfa_last_error()
    p = _native.NfaSelectParams()
    p.abi_version = 99
    p.struct_size = ctypes.sizeof(p)
    assert lib.nfa_select_layer(ctypes.byref(p), None) == -1
    assert b'ABI mismatch' in lib.nfa_last_error()
    p.abi_version = _native.ABI_VERSION
    p.batch, p.hq, p.hkv = 1, 32, 8
    p.dsub = 48
    assert lib.nfa_select_layer(ctypes.byref(p), None) == -1
    assert b'L1 dim' in lib.nfa_last_error()


def test_workspace_size_is_host_computed(lib):
    from sparse_attn import _native
    p = _native.NfaSelectParams()
    p.abi_version = _native.ABI_VERSION
    p.struct_size = ctypes.sizeof(p)
    p.batch, p.hq, p.hkv, p.bs, p.max_blocks = 1, 32, 8, 16, 8216
    p.k_f, p.k_n, p.k2, p.dsub, p.fine_dsub = 96, 32, 1024, 32, 32
    need = lib.nfa_select_workspace_bytes(ctypes.byref(p))
    # per (row, kv head): a 16-bit key per page and two 256-bin histograms
    # (candidate pages and L2 keys stay in the tail workgroup's LDS)
    rows = 8
    assert need >= rows * (2 * 8216 + 4 * 512)
    a = _native.NfaAttnParams()
    a.abi_version = _native.ABI_VERSION
    a.struct_size = ctypes.sizeof(a)
    a.total_q, a.hq, a.hkv, a.head_dim_v, a.max_vis = 1, 32, 8, 128, 1024
    assert lib.nfa_attn_workspace_bytes(ctypes.byref(a)) > 0


def test_partial_combine_and_quant_checks_reject_before_launch(lib):
    from sparse_attn import _native
    assert lib.nfa_attn_partial_size() == ctypes.sizeof(_native.NfaAttnPartial)
    assert lib.nfa_attn_combine_params_size() == ctypes.sizeof(_native.NfaAttnCombineParams)
    a = _native.NfaAttnParams()
    a.abi_version, a.struct_size = _native.ABI_VERSION, ctypes.sizeof(a)
    pt = _native.NfaAttnPartial()
    pt.abi_version, pt.struct_size = 99, ctypes.sizeof(pt)
    assert lib.nfa_sparse_attn_partial(ctypes.byref(a), ctypes.byref(pt), None) == -1
    assert b'ABI mismatch' in lib.nfa_last_error()
    pt.abi_version = _native.ABI_VERSION
    a.total_q, a.hq, a.hkv, a.head_dim, a.head_dim_v = 1, 32, 8, 128, 128
    a.page, a.gather_rows, a.max_vis, a.pool_pages = 16, 1, 1024, 10
    for name in ('q', 'k_pool', 'v_pool', 'gather', 'vis_lens', 'query_to_req'):
        setattr(a, name, 16)  # never dereferenced: rejected first
    pt.nsplit, pt.block_tokens = 0, 128
    assert lib.nfa_sparse_attn_partial(ctypes.byref(a), ctypes.byref(pt), None) == -1
    assert b'nsplit' in lib.nfa_last_error()
    c = _native.NfaAttnCombineParams()
    c.abi_version, c.struct_size = _native.ABI_VERSION, ctypes.sizeof(c)
    c.total_q, c.hq, c.head_dim_v, c.out_dtype = 1, 4, 8, 7
    assert lib.nfa_attn_regions_combine(ctypes.byref(c), None) == -1
    assert b'shape or dtype' in lib.nfa_last_error()
    p = _native.NfaSelectParams()
    p.abi_version, p.struct_size = _native.ABI_VERSION, ctypes.sizeof(p)
    p.batch, p.hq, p.hkv, p.head_dim, p.dsub, p.fine_dsub = 1, 32, 8, 128, 32, 48
    p.l2_quant = 1
    assert lib.nfa_select_layer(ctypes.byref(p), None) == -1
    assert b'4-bit L2 keys' in lib.nfa_last_error()
    assert b'32 or 64' in lib.nfa_last_error()
    # arena heads shared by the selection rows: hkv, 0 (= hkv) or 1 only
    p.l2_quant, p.fine_dsub, p.kv_heads_mem = 0, 32, 4
    assert lib.nfa_select_layer(ctypes.byref(p), None) == -1
    assert b'kv_heads_mem' in lib.nfa_last_error()
    # the fused decode write puts one element of the row on each of the
    # workgroup's 1024 threads: wider rows are refused
    w = _native.NfaSelectParams()
    w.abi_version, w.struct_size = _native.ABI_VERSION, ctypes.sizeof(w)
    w.batch, w.hq, w.hkv, w.head_dim, w.head_dim_v = 1, 1, 1, 1100, 1024
    w.dsub, w.fine_dsub, w.bs, w.page, w.max_blocks = 32, 32, 16, 16, 512
    w.k_f, w.k_n, w.k2, w.pool_pages, w.max_vis, w.max_req = 96, 32, 1024, 10, 1024, 1
    for name in ('q', 'k_pool_l', 'v_pool_l', 'block_table_l', 'lengths', 'active_req',
                 'valid_req', 'slots', 'k_new', 'v_new', 'stat_min_l', 'stat_max_l',
                 'stat_sum_l', 'stats_len_l', 'skip_far_l', 'skip_near_l', 'gather',
                 'vis_lens', 'dims', 'fine_dims'):
        setattr(w, name, 16)  # never dereferenced: rejected first
    assert lib.nfa_select_layer(ctypes.byref(w), None) == -1
    assert b'fused decode write' in lib.nfa_last_error()
