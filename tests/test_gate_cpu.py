"""Prefill region gate: configuration checks and the decision rule (CPU).

Reference: sparse_attn/policies/frozen_gate.py:8-24 (GateConfig) and
:104-111 (decide_regions).
"""
import pytest

from sparse_attn.policies.frozen_gate import (GateConfig, _summarise,
                                              decide_regions, region_present)
from sparse_attn.policies.region_geometry import RegionGeometry


def test_gate_config_validation():
    GateConfig(epsilon=0.0)
    GateConfig(epsilon=1.0, statistic='p95', mode='far')
    for bad in (dict(epsilon=-0.1), dict(epsilon=float('nan')), dict(rows=0),
                dict(statistic='median'), dict(mode='both')):
        with pytest.raises(ValueError):
            GateConfig(**bad)


def test_decision_rule():
    prof = {'near': {'mean': 0.02, 'p95': 0.2, 'max': 0.3},
            'far': {'mean': 0.04, 'p95': 0.06, 'max': 0.5}}
    assert decide_regions(prof, GateConfig(0.05)) == dict(skip_near=True, skip_far=True)
    assert decide_regions(prof, GateConfig(0.05, statistic='p95')) == dict(
        skip_near=False, skip_far=False)
    assert decide_regions(prof, GateConfig(0.05, mode='near')) == dict(
        skip_near=True, skip_far=False)
    assert decide_regions(prof, GateConfig(0.05, mode='full')) == dict(
        skip_near=False, skip_far=False)
    # an absent region is never skipped
    assert decide_regions(prof, GateConfig(0.05), present_far=False) == dict(
        skip_near=True, skip_far=False)
    # strict comparison: a statistic equal to epsilon is kept
    assert decide_regions(prof, GateConfig(0.02, mode='near'))['skip_near'] is False


def test_profile_summary_and_presence():
    import torch
    vals = torch.tensor([[0.0, 0.1, 0.2, 0.3], [1.0, 1.0, 1.0, 1.0]])
    s = _summarise(vals)
    assert s['near']['mean'] == pytest.approx(0.15)
    assert s['near']['max'] == pytest.approx(0.3)
    assert s['far'] == {'mean': 1.0, 'p95': 1.0, 'max': 1.0}
    geo = RegionGeometry(sink=4, near=4096, window=128, page=16)
    assert region_present(200, geo) == (True, False)
    assert region_present(9000, geo) == (True, True)
    assert region_present(4, geo) == (False, False)
