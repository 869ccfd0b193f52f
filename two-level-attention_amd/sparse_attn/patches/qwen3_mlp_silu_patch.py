"""Decode-step MLP on two HIP launches.

Reference: sparse_attn/patches/qwen3_mlp_silu_patch.py:22-89
(``register_mlp_silu_patch`` / ``unregister_mlp_silu_patch``): instance-level
forward replacement of every gated-SiLU MLP.  For one token per row the gate
and up projections and SiLU*up run as one launch and the down projection as
a second (the reference fuses only the elementwise SiLU*up); other inputs
take the original forward.  A count different from ``expected`` raises.
"""
from types import MethodType

import torch

_ORIG = '_nfa_mlp_silu_original_forward'


def _mlp_classes():
    from transformers.models.llama.modeling_llama import LlamaMLP
    from transformers.models.qwen3.modeling_qwen3 import Qwen3MLP
    return (Qwen3MLP, LlamaMLP)


def _mlp_forward(self, x):
    from ..ops.decode_fused import LINEAR_MAX_ROWS, decode_linear
    from .decode_layer_patch import is_silu
    if (is_silu(self.act_fn) and x.dim() == 3 and x.shape[1] == 1
            and x.shape[0] <= LINEAR_MAX_ROWS and x.dtype == torch.bfloat16
            and x.is_cuda and x.is_contiguous() and self.gate_proj.bias is None
            and self.up_proj.bias is None and self.down_proj.bias is None):
        self._nfa_fused_calls = getattr(self, '_nfa_fused_calls', 0) + 1
        b, _, h = x.shape
        a, = decode_linear(x.view(b, h), (self.gate_proj.weight, self.up_proj.weight),
                           silu_gate=True)
        y, = decode_linear(a, (self.down_proj.weight,))
        return y.view(b, 1, -1)
    return getattr(self, _ORIG)(x)


def register_mlp_silu_patch(model, expected=None, verbose=False):
    n = 0
    for module in model.modules():
        if isinstance(module, _mlp_classes()):
            if not hasattr(module, _ORIG):
                setattr(module, _ORIG, module.forward)
            module.forward = MethodType(_mlp_forward, module)
            n += 1
    if expected is not None and n != expected:
        raise RuntimeError(f'MLP patch count {n} != expected {expected}')
    return n


def unregister_mlp_silu_patch(model):
    n = 0
    for module in model.modules():
        original = getattr(module, _ORIG, None)
        if original is not None:
            module.forward = original
            delattr(module, _ORIG)
            n += 1
    return n
