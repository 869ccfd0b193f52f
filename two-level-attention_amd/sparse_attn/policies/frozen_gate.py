"""Frozen near/far region gate decided once, during prefill.

Reference: sparse_attn/policies/frozen_gate.py:8-111.  Same configuration,
profile summary and decision rule: the last ``rows`` prompt positions'
post-RoPE queries attend causally over the prompt; the head-averaged
attention mass of the near and of the far region is summarised (mean, p95,
max over the rows), and a present region whose statistic falls below
``epsilon`` is skipped for the whole decode of the request.  The profile
runs as one HIP kernel (``nfa_region_profile``); there is no CPU path.
"""
from dataclasses import dataclass
import math

import torch

from .region_geometry import RegionGeometry


@dataclass(frozen=True)
class GateConfig:
    epsilon: float = .05
    rows: int = 256
    statistic: str = 'mean'
    mode: str = 'dual'

    def __post_init__(self):
        if not math.isfinite(self.epsilon) or not 0 <= self.epsilon <= 1:
            raise ValueError('epsilon must be in [0,1]')
        if (self.rows < 1 or self.statistic not in ('mean', 'p95')
                or self.mode not in ('full', 'far', 'near', 'dual')):
            raise ValueError('invalid gate configuration')


def _validate_profile_inputs(q, k, rows, chunk, scale):
    if (q.ndim != 4 or k.ndim != 4 or q.shape[0] != 1 or k.shape[0] != 1
            or q.shape[2] != k.shape[2] or q.shape[-1] != k.shape[-1]
            or q.shape[1] % k.shape[1]):
        raise ValueError('one-shot unpadded B=1 prefill with valid GQA required')
    if rows < 1 or chunk < 1:
        raise ValueError('profile rows and chunk must be positive')
    scale = q.shape[-1] ** -.5 if scale is None else float(scale)
    if not math.isfinite(scale) or scale <= 0:
        raise ValueError('attention scale must be finite and positive')
    return scale


def _profile_summary(values):
    """``values`` [2, rows] (near, far) -> {region: {mean, p95, max}}."""
    values = values.cpu()
    return {name: {'mean': float(values[i].mean()),
                   'p95': float(torch.quantile(values[i], .95)),
                   'max': float(values[i].max())}
            for i, name in enumerate(('near', 'far'))}


def profile_regions(q, k, geometry=RegionGeometry(), rows=256, chunk=16, scale=None):
    """Near/far mass summary of one layer's prefill (``chunk`` is accepted
    for the reference's signature; the kernel needs no row chunking)."""
    from ..ops.frozen_gate import fused_region_profile
    scale = _validate_profile_inputs(q, k, rows, chunk, scale)
    return _profile_summary(
        fused_region_profile(q.detach(), k.detach(), geometry, rows, scale))


def decide_regions(profile, config, present_near=True, present_far=True):
    n, f = (profile[name][config.statistic] for name in ('near', 'far'))
    near = present_near and config.mode in ('near', 'dual') and n < config.epsilon
    far = present_far and config.mode in ('far', 'dual') and f < config.epsilon
    return dict(skip_near=bool(near), skip_far=bool(far))


def region_present(length, geometry):
    """(near region present, far region present) for a prompt of ``length``."""
    sink_hi, far_hi, near_hi = geometry.bounds(length)
    return near_hi > far_hi, far_hi > sink_hi
