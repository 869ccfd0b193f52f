"""Decode-step RMSNorm on one HIP launch.

Reference: sparse_attn/patches/qwen3_rmsnorm_patch.py:37-91
(``register_rmsnorm_patch`` / ``unregister_rmsnorm_patch``): instance-level
forward replacement of every RMSNorm module; one-token-per-row bf16 device
inputs take the fused kernel (``nfa_rmsnorm_decode``), anything else the
original forward.  A count different from ``expected`` raises.
"""
from types import MethodType

_ORIG = '_nfa_rmsnorm_original_forward'


def _norm_classes():
    from transformers.models.llama.modeling_llama import LlamaRMSNorm
    from transformers.models.qwen3.modeling_qwen3 import Qwen3RMSNorm
    return (Qwen3RMSNorm, LlamaRMSNorm)


def _rmsnorm_forward(self, hidden_states):
    from ..ops.decode_fused import rmsnorm_decode, rmsnorm_fusable
    if rmsnorm_fusable(hidden_states, self.weight):
        return rmsnorm_decode(hidden_states, self.weight, self.variance_epsilon)
    return getattr(self, _ORIG)(hidden_states)


def register_rmsnorm_patch(model, expected=None, verbose=False):
    n = 0
    for name, module in model.named_modules():
        if isinstance(module, _norm_classes()):
            if not hasattr(module, _ORIG):
                setattr(module, _ORIG, module.forward)
            module.forward = MethodType(_rmsnorm_forward, module)
            n += 1
    if expected is not None and n != expected:
        raise RuntimeError(f'RMSNorm patch count {n} != expected {expected}')
    return n


def unregister_rmsnorm_patch(model):
    n = 0
    for module in model.modules():
        original = getattr(module, _ORIG, None)
        if original is not None:
            module.forward = original
            delattr(module, _ORIG)
            n += 1
    return n
