"""Frozen near/far region gate, decided once per request during prefill.

Reference interface: sparse_attn/policies/frozen_gate.py:8-111 (``GateConfig``,
``profile_regions``, ``decide_regions``).  The decision is the reference's:
the last ``rows`` prompt positions' post-RoPE queries attend causally over
the prompt; for each of the near and far regions the attention mass, averaged
over the query heads, gives one value per profiled row; a region that exists
for the prompt, is gated by ``mode`` and whose ``statistic`` (mean or 95th
percentile over the rows) stays below ``epsilon`` is skipped for the whole
decode.  The mass comes from one HIP kernel per layer; there is no CPU path.
"""
from dataclasses import dataclass
import math

import torch

from .region_geometry import RegionGeometry

_REGIONS = ('near', 'far')
_STATISTICS = ('mean', 'p95')
# which regions each gate mode may skip
_MODE_REGIONS = {'full': (), 'far': ('far',), 'near': ('near',),
                 'dual': ('near', 'far')}


@dataclass(frozen=True)
class GateConfig:
    """Gate threshold, profiled rows, summary statistic and gated regions."""
    epsilon: float = .05
    rows: int = 256
    statistic: str = 'mean'
    mode: str = 'dual'

    def __post_init__(self):
        eps = float(self.epsilon)
        if not (math.isfinite(eps) and 0.0 <= eps <= 1.0):
            raise ValueError('epsilon must be in [0,1]')
        valid = (self.rows >= 1 and self.statistic in _STATISTICS
                 and self.mode in _MODE_REGIONS)
        if not valid:
            raise ValueError('invalid gate configuration')


def _prefill_scale(q, k, rows, chunk, scale):
    """Checks a one-request prefill's ``q`` [1, HQ, L, D] / ``k`` [1, HKV, L, D]
    and returns the softmax scale (1/sqrt(D) unless given)."""
    shapes_ok = (q.ndim == 4 and k.ndim == 4 and q.shape[0] == k.shape[0] == 1
                 and q.shape[2:] == k.shape[2:] and q.shape[1] % k.shape[1] == 0)
    if not shapes_ok:
        raise ValueError('one-shot unpadded B=1 prefill with valid GQA required')
    if min(rows, chunk) < 1:
        raise ValueError('profile rows and chunk must be positive')
    value = float(scale) if scale is not None else 1.0 / math.sqrt(q.shape[-1])
    if not (math.isfinite(value) and value > 0.0):
        raise ValueError('attention scale must be finite and positive')
    return value


def _summarise(mass):
    """``mass`` [2, rows] (near, far) on the device -> per region the mean,
    the 95th percentile (linear interpolation) and the maximum over the rows,
    brought to the host in one copy."""
    table = torch.stack((mass.mean(dim=1), torch.quantile(mass, 0.95, dim=1),
                         mass.amax(dim=1)), dim=1).tolist()
    return {region: dict(zip(('mean', 'p95', 'max'), row))
            for region, row in zip(_REGIONS, table)}


def profile_regions(q, k, geometry=RegionGeometry(), rows=256, chunk=16, scale=None):
    """Near/far attention-mass summary of one layer's prefill.  ``chunk`` is
    the reference's row-chunk argument, checked and otherwise unused: the
    kernel streams every profiled row in one pass."""
    from ..ops.frozen_gate import fused_region_profile
    scale = _prefill_scale(q, k, rows, chunk, scale)
    return _summarise(fused_region_profile(q.detach(), k.detach(), geometry,
                                           rows, scale))


def decide_regions(profile, config, present_near=True, present_far=True):
    """``{'skip_near': bool, 'skip_far': bool}`` for one layer's profile."""
    present = {'near': present_near, 'far': present_far}
    gated = _MODE_REGIONS[config.mode]
    decision = {}
    for region in _REGIONS:
        low = profile[region][config.statistic] < config.epsilon
        decision['skip_' + region] = bool(present[region] and region in gated and low)
    return decision


def region_present(length, geometry):
    """(near region present, far region present) for a prompt of ``length``."""
    sink_hi, far_hi, near_hi = geometry.bounds(length)
    return near_hi > far_hi, far_hi > sink_hi
