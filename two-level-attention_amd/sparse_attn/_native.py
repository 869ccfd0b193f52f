"""ctypes binding of libnfa_hip.so (the gfx950 kernels behind this package).

The library exposes a plain C ABI (``include/nfa_hip.h``).  It is loaded after
``import torch`` so that it binds to the HIP runtime torch already loaded and
shares its streams.  There is no fallback: if the library is missing or the
device is not a HIP GPU the calls raise.
"""
from __future__ import annotations

import ctypes
import os
import threading

import torch

_LIB_NAME = 'libnfa_hip.so'
_PKG_ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_PATH = os.path.join(_PKG_ROOT, 'lib', _LIB_NAME)

ABI_VERSION = 1
SELECT_CLOCK_PAGES = 64  # NFA_SELECT_CLOCK_PAGES
DTYPE_BF16 = 0
DTYPE_F32 = 1
METHOD_MINMAX = 0
METHOD_AVG = 1
METHOD_AVG_TOP2 = 2

_i32 = ctypes.c_int32
_i64 = ctypes.c_int64
_f32 = ctypes.c_float
_ptr = ctypes.c_void_p


class NfaSelectParams(ctypes.Structure):
    _fields_ = [
        ('abi_version', _i32), ('struct_size', _i32),
        ('batch', _i32), ('hq', _i32), ('hkv', _i32),
        ('head_dim', _i32), ('head_dim_v', _i32),
        ('bs', _i32), ('page', _i32), ('max_blocks', _i32), ('max_req', _i32),
        ('geo_sink', _i32), ('geo_near', _i32), ('geo_window', _i32),
        ('sink_tokens', _i32), ('swa', _i32), ('near_len', _i32),
        ('k_f', _i32), ('k_n', _i32), ('k2', _i32), ('near_tokens', _i32),
        ('far_method', _i32), ('near_method', _i32),
        ('dsub', _i32), ('fine_dsub', _i32),
        ('kv_dtype', _i32), ('q_dtype', _i32),
        ('max_vis', _i32), ('middle_only', _i32), ('pool_pages', _i32),
        ('protected_only', _i32), ('scale', _f32), ('l2_quant', _i32),
        ('kv_heads_mem', _i32),
        ('k_pool_l', _ptr), ('v_pool_l', _ptr), ('block_table_l', _ptr),
        ('lengths', _ptr), ('active_req', _ptr), ('valid_req', _ptr),
        ('skip_far_l', _ptr), ('skip_near_l', _ptr),
        ('dims', _ptr), ('fine_dims', _ptr),
        ('q', _ptr), ('q_stride_b', _i64), ('q_stride_h', _i64),
        ('k_new', _ptr), ('v_new', _ptr), ('slots', _ptr),
        ('stat_min_l', _ptr), ('stat_max_l', _ptr), ('stat_sum_l', _ptr),
        ('stats_len_l', _ptr),
        ('l2_keys_l', _ptr), ('page_sum_l', _ptr),
        ('gather', _ptr), ('vis_lens', _ptr),
        ('workspace', _ptr), ('workspace_bytes', _i64),
        ('dbg_far', _ptr), ('dbg_near', _ptr),
        ('dbg_i_f', _ptr), ('dbg_i_n', _ptr),
        ('dbg_middle', _ptr), ('dbg_counts', _ptr), ('dbg_bounds', _ptr),
        ('dbg_cand_tok', _ptr), ('dbg_cand_logit', _ptr),
        ('dbg_cand_count', _ptr), ('dbg_cand_cap', _i64),
        ('dbg_clock', _ptr),
    ]


class NfaAttnParams(ctypes.Structure):
    _fields_ = [
        ('abi_version', _i32), ('struct_size', _i32),
        ('total_q', _i32), ('hq', _i32), ('hkv', _i32),
        ('head_dim', _i32), ('head_dim_v', _i32), ('page', _i32),
        ('gather_rows', _i32), ('max_vis', _i32),
        ('kv_dtype', _i32), ('q_dtype', _i32),
        ('tokens_per_split', _i32), ('pool_pages', _i32),
        ('scale', _f32), ('pad1', _f32),
        ('q', _ptr), ('k_pool', _ptr), ('v_pool', _ptr),
        ('gather', _ptr), ('vis_lens', _ptr), ('query_to_req', _ptr),
        ('out', _ptr), ('workspace', _ptr), ('workspace_bytes', _i64),
    ]


class NfaMlaAttnParams(ctypes.Structure):
    _fields_ = [
        ('abi_version', _i32), ('struct_size', _i32),
        ('total_q', _i32), ('heads', _i32), ('latent_dim', _i32),
        ('value_dim', _i32), ('page', _i32), ('gather_rows', _i32),
        ('max_vis', _i32), ('kv_dtype', _i32), ('q_dtype', _i32),
        ('out_dtype', _i32), ('pool_pages', _i32), ('scale', _f32),
        ('q', _ptr), ('kv_pool', _ptr), ('gather', _ptr), ('vis_lens', _ptr),
        ('query_to_req', _ptr), ('w_uv', _ptr), ('out_dim', _i32), ('pad0', _i32),
        ('out', _ptr), ('workspace', _ptr), ('workspace_bytes', _i64),
    ]


class NfaAttnPartial(ctypes.Structure):
    _fields_ = [
        ('abi_version', _i32), ('struct_size', _i32),
        ('nsplit', _i32), ('block_tokens', _i32),
        ('acc', _ptr), ('m', _ptr), ('z', _ptr),
    ]


class NfaAttnCombineParams(ctypes.Structure):
    _fields_ = [
        ('abi_version', _i32), ('struct_size', _i32),
        ('total_q', _i32), ('hq', _i32), ('head_dim_v', _i32), ('out_dtype', _i32),
        ('nsplit_a', _i32), ('nsplit_b', _i32),
        ('acc_a', _ptr), ('m_a', _ptr), ('z_a', _ptr),
        ('acc_b', _ptr), ('m_b', _ptr), ('z_b', _ptr),
        ('out', _ptr),
    ]


EPI_PLAIN = 0
EPI_RESIDUAL = 1
EPI_SILU_GATE = 2


class NfaLinearParams(ctypes.Structure):
    _fields_ = [
        ('abi_version', _i32), ('struct_size', _i32),
        ('m', _i32), ('k', _i32), ('nseg', _i32), ('epilogue', _i32),
        ('x', _ptr), ('x_stride', _i64),
        ('norm_weight', _ptr), ('norm_eps', _f32), ('pad0', _f32),
        ('w', _ptr * 3), ('n', _i32 * 3), ('pad1', _i32),
        ('y', _ptr * 3), ('y_stride', _i64 * 3),
        ('residual', _ptr), ('residual_stride', _i64),
    ]


class NfaRopeParams(ctypes.Structure):
    _fields_ = [
        ('abi_version', _i32), ('struct_size', _i32),
        ('batch', _i32), ('hq', _i32), ('hkv', _i32), ('head_dim', _i32),
        ('q', _ptr), ('q_stride_b', _i64), ('k', _ptr), ('k_stride_b', _i64),
        ('q_weight', _ptr), ('k_weight', _ptr), ('eps', _f32), ('pad0', _f32),
        ('cos', _ptr), ('sin', _ptr), ('cs_stride_b', _i64),
        ('q_out', _ptr), ('k_out', _ptr),
    ]


class NfaGateParams(ctypes.Structure):
    _fields_ = [
        ('abi_version', _i32), ('struct_size', _i32),
        ('hq', _i32), ('hkv', _i32), ('head_dim', _i32),
        ('length', _i32), ('rows', _i32),
        ('sink', _i32), ('window', _i32), ('near', _i32), ('page', _i32),
        ('q_dtype', _i32), ('scale', _f32), ('pad0', _i32),
        ('q', _ptr), ('q_stride_h', _i64), ('q_stride_l', _i64),
        ('k', _ptr), ('k_stride_h', _i64), ('k_stride_l', _i64),
        ('out', _ptr),
    ]


EXPORTS = (
    'nfa_abi_version', 'nfa_wall_clock_khz', 'nfa_select_params_size', 'nfa_attn_params_size',
    'nfa_last_error', 'nfa_select_workspace_bytes', 'nfa_attn_workspace_bytes',
    'nfa_select_layer', 'nfa_select_plan', 'nfa_sparse_attn_decode', 'nfa_paged_write_decode',
    'nfa_paged_write_prefill', 'nfa_linear_params_size', 'nfa_rope_params_size',
    'nfa_decode_linear', 'nfa_qk_norm_rope_decode', 'nfa_rmsnorm_decode',
    'nfa_gate_params_size', 'nfa_region_profile', 'nfa_attn_partial_size',
    'nfa_attn_combine_params_size', 'nfa_sparse_attn_partial', 'nfa_attn_regions_combine',
    'nfa_attn_partial_workspace_bytes', 'nfa_mla_attn_decode',
    'nfa_mla_attn_workspace_bytes', 'nfa_mla_attn_params_size',
)

_lib = None
_lock = threading.Lock()


class NativeError(RuntimeError):
    """A libnfa_hip call rejected its arguments or failed to launch."""


def load_library(path: str = None):
    """Load (once) and type the C ABI; raises if the library is missing."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    with _lock:
        if _lib is not None and path is None:
            return _lib
        lib_path = path or LIB_PATH
        if not os.path.exists(lib_path):
            raise NativeError(
                f'{lib_path} is not built; run __graft_entry__.build() '
                '(hipcc --offload-arch=gfx950)')
        lib = ctypes.CDLL(lib_path)
        lib.nfa_abi_version.restype = _i32
        lib.nfa_wall_clock_khz.restype = _i32
        lib.nfa_select_params_size.restype = _i32
        lib.nfa_attn_params_size.restype = _i32
        lib.nfa_last_error.restype = ctypes.c_char_p
        lib.nfa_select_workspace_bytes.restype = _i64
        lib.nfa_select_workspace_bytes.argtypes = [ctypes.POINTER(NfaSelectParams)]
        lib.nfa_attn_workspace_bytes.restype = _i64
        lib.nfa_attn_workspace_bytes.argtypes = [ctypes.POINTER(NfaAttnParams)]
        lib.nfa_select_layer.restype = _i32
        lib.nfa_select_layer.argtypes = [ctypes.POINTER(NfaSelectParams), _ptr]
        lib.nfa_select_plan.restype = _i32
        lib.nfa_select_plan.argtypes = [ctypes.POINTER(NfaSelectParams),
                                        ctypes.POINTER(_i32), _i32]
        lib.nfa_select_layer_noalloc.restype = _i32
        lib.nfa_select_layer_noalloc.argtypes = [ctypes.POINTER(NfaSelectParams), _ptr]
        lib.nfa_sparse_attn_decode.restype = _i32
        lib.nfa_sparse_attn_decode.argtypes = [ctypes.POINTER(NfaAttnParams), _ptr]
        lib.nfa_paged_write_decode.restype = _i32
        lib.nfa_paged_write_decode.argtypes = [
            _ptr, _ptr, _ptr, _i32, _i32, _i32, _i32, _i32, _i32, _ptr, _ptr, _ptr]
        lib.nfa_paged_write_prefill.restype = _i32
        lib.nfa_paged_write_prefill.argtypes = [
            _ptr, _ptr, _i64, _ptr, _i32, _i32, _i32, _i32, _i32, _ptr, _ptr, _ptr]
        lib.nfa_linear_params_size.restype = _i32
        lib.nfa_rope_params_size.restype = _i32
        lib.nfa_decode_linear.restype = _i32
        lib.nfa_decode_linear.argtypes = [ctypes.POINTER(NfaLinearParams), _ptr]
        lib.nfa_qk_norm_rope_decode.restype = _i32
        lib.nfa_qk_norm_rope_decode.argtypes = [ctypes.POINTER(NfaRopeParams), _ptr]
        lib.nfa_rmsnorm_decode.restype = _i32
        lib.nfa_rmsnorm_decode.argtypes = [
            _ptr, _i64, _ptr, _ptr, _i64, _i32, _i32, _f32, _ptr]
        lib.nfa_gate_params_size.restype = _i32
        lib.nfa_region_profile.restype = _i32
        lib.nfa_region_profile.argtypes = [ctypes.POINTER(NfaGateParams), _ptr]
        lib.nfa_attn_partial_size.restype = _i32
        lib.nfa_attn_combine_params_size.restype = _i32
        lib.nfa_sparse_attn_partial.restype = _i32
        lib.nfa_sparse_attn_partial.argtypes = [
            ctypes.POINTER(NfaAttnParams), ctypes.POINTER(NfaAttnPartial), _ptr]
        lib.nfa_attn_partial_workspace_bytes.restype = _i64
        lib.nfa_attn_partial_workspace_bytes.argtypes = [
            ctypes.POINTER(NfaAttnParams), ctypes.POINTER(NfaAttnPartial)]
        lib.nfa_attn_regions_combine.restype = _i32
        lib.nfa_attn_regions_combine.argtypes = [ctypes.POINTER(NfaAttnCombineParams), _ptr]
        lib.nfa_mla_attn_params_size.restype = _i32
        lib.nfa_mla_attn_decode.restype = _i32
        lib.nfa_mla_attn_decode.argtypes = [ctypes.POINTER(NfaMlaAttnParams), _ptr]
        lib.nfa_mla_attn_workspace_bytes.restype = _i64
        lib.nfa_mla_attn_workspace_bytes.argtypes = [ctypes.POINTER(NfaMlaAttnParams)]
        if lib.nfa_abi_version() != ABI_VERSION:
            raise NativeError('libnfa_hip ABI version mismatch')
        if lib.nfa_select_params_size() != ctypes.sizeof(NfaSelectParams):
            raise NativeError('NfaSelectParams layout mismatch')
        if lib.nfa_attn_params_size() != ctypes.sizeof(NfaAttnParams):
            raise NativeError('NfaAttnParams layout mismatch')
        if lib.nfa_linear_params_size() != ctypes.sizeof(NfaLinearParams):
            raise NativeError('NfaLinearParams layout mismatch')
        if lib.nfa_rope_params_size() != ctypes.sizeof(NfaRopeParams):
            raise NativeError('NfaRopeParams layout mismatch')
        if lib.nfa_gate_params_size() != ctypes.sizeof(NfaGateParams):
            raise NativeError('NfaGateParams layout mismatch')
        if lib.nfa_attn_partial_size() != ctypes.sizeof(NfaAttnPartial):
            raise NativeError('NfaAttnPartial layout mismatch')
        if lib.nfa_attn_combine_params_size() != ctypes.sizeof(NfaAttnCombineParams):
            raise NativeError('NfaAttnCombineParams layout mismatch')
        if lib.nfa_mla_attn_params_size() != ctypes.sizeof(NfaMlaAttnParams):
            raise NativeError('NfaMlaAttnParams layout mismatch')
        if path is None:
            _lib = lib
        return lib


def check(rc: int, what: str):
    if rc != 0:
        msg = load_library().nfa_last_error().decode(errors='replace')
        raise NativeError(f'{what} failed ({rc}): {msg}')


def dtype_code(dtype: torch.dtype) -> int:
    if dtype == torch.bfloat16:
        return DTYPE_BF16
    if dtype == torch.float32:
        return DTYPE_F32
    raise NativeError(f'unsupported dtype {dtype}; use bfloat16 or float32')


def require_hip(tensor: torch.Tensor, what: str):
    if tensor.device.type != 'cuda':
        raise NativeError(
            f'{what} runs on the HIP device only (got a {tensor.device} tensor)')


def stream_handle() -> int:
    return torch.cuda.current_stream().cuda_stream


def ptr(t) -> int:
    return 0 if t is None else t.data_ptr()
