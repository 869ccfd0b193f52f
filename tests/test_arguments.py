"""The flag surface and configuration checks of the NFA path (CPU).

Reference: sparse_attn/arguments.py:4-11, :249-399 (the 5 TIA and 40 NFA
flags, their defaults and choices) and indexer/nfa_indexer.py:32-106 (the
configuration checks and their messages).
"""
import argparse

import pytest

from sparse_attn import arguments
from sparse_attn.indexer.nfa_indexer import NFAIndexer

# every TIA / NFA flag of the reference, with its default (SUPPRESS = absent)
REFERENCE_DEFAULTS = {
    'tia_block_size': 64, 'tia_level1_topk': 128, 'tia_level2_topk': 1024,
    'tia_level2_cmp_ratio': 2, 'tia_enable_async_topk': False,
    'nfa_enable_subspace': True, 'nfa_enable_kmeans': True,
    'nfa_far_select': '4bit', 'nfa_near_select': '4bit', 'nfa_sim': 0.9,
    'nfa_sim_dims': 'subspace', 'nfa_enable_layer_skip': True,
    'nfa_operator_mode': 'off', 'nfa_far_clusters': 256, 'nfa_far_niter': 10,
    'nfa_far_blocks': 16, 'nfa_far_tokens': 512, 'nfa_layer_skip_path': None,
    'nfa_far_method': 'minmax', 'nfa_near_method': 'avg', 'nfa_alpha': None,
    'nfa_beta': None, 'nfa_gamma': None, 'nfa_near_pages': argparse.SUPPRESS,
    'nfa_near_tokens': argparse.SUPPRESS, 'nfa_near_len': argparse.SUPPRESS,
    'nfa_boundary_bypass': True, 'nfa_l2_quant': False, 'nfa_subspace': 'full',
    'nfa_l2_subspace': 'same', 'nfa_proj_basis': None, 'nfa_static_pair': False,
    'nfa_moba': False, 'nfa_sigma_select': 'none', 'nfa_sigma': 8.0,
    'nfa_per_q_head': False, 'nfa_sink_tokens': 128, 'nfa_swa_size': 128,
    'nfa_sinkswa_only': False, 'nfa_far_skip_backend': 'legacy',
    'nfa_far_skip_cache': 'retain', 'nfa_dyn_dgate': False,
    'nfa_dyn_dgate_eps': 0.05, 'nfa_dyn_dgate_rows': 256,
    'nfa_enable_static_gate': False,
}

# the production flag set (reference paged_region_kernels_nfa.py:10-20)
PRODUCTION = ['--method', 'nfa', '--nfa_far_method', 'minmax',
              '--nfa_near_method', 'avg', '--nfa_near_pages', '32',
              '--nfa_near_tokens', 'off', '--nfa_near_len', '4096',
              '--nfa_subspace', 'tail', '--tia_level2_cmp_ratio', '4',
              '--nfa_sink_tokens', '4', '--nfa_swa_size', '128',
              '--tia_level1_topk', '128', '--tia_level2_topk', '1024',
              '--nfa_enable_layer_skip', 'false', '--nfa_far_skip_backend', 'legacy',
              '--nfa_far_skip_cache', 'retain']

# every other flag, at a value the path accepts (its default, or an inert one)
EVERY_OTHER = ['--tia_block_size', '16', '--tia_enable_async_topk',
               '--nfa_enable_subspace', 'true', '--nfa_enable_kmeans', 'false',
               '--nfa_far_select', '4bit', '--nfa_near_select', '4bit',
               '--nfa_sim', '0.8', '--nfa_sim_dims', 'tail',
               '--nfa_operator_mode', 'serial', '--nfa_far_clusters', '128',
               '--nfa_far_niter', '5', '--nfa_far_blocks', '8',
               '--nfa_far_tokens', '256', '--nfa_boundary_bypass', 'true',
               '--nfa_l2_quant', 'true', '--nfa_l2_subspace', 'same',
               '--nfa_sigma_select', 'none', '--nfa_sigma', '4.0',
               '--nfa_per_q_head', 'false', '--nfa_dyn_dgate',
               '--nfa_dyn_dgate_eps', '0.1', '--nfa_dyn_dgate_rows', '128',
               '--nfa_enable_static_gate', 'false']


def _parser():
    ap = argparse.ArgumentParser(allow_abbrev=False)
    arguments.add_sparse_attn_args(ap)
    return ap


def _flag_defaults(ap):
    return {a.dest: a.default for a in ap._actions
            if a.dest.startswith(('tia_', 'nfa_'))}


def test_every_reference_flag_with_its_default():
    got = _flag_defaults(_parser())
    assert len(REFERENCE_DEFAULTS) == 45
    assert got == REFERENCE_DEFAULTS


def test_production_command_line_with_every_flag_parses_and_builds():
    args = _parser().parse_args(PRODUCTION + EVERY_OTHER)
    indexer = NFAIndexer(args)
    assert indexer.nt_near_pages == 32 and indexer.nt_near_tokens is None
    assert indexer.subspace == 'tail' and indexer.l2_quant
    assert args.nfa_dyn_dgate and args.nfa_sim == 0.8
    # the flags that take no part in the path (listed as unimplemented) parse
    # too, at any value the reference's parser accepts
    extra = ['--nfa_layer_skip_path', 'skip.json', '--nfa_alpha', '0.5',
             '--nfa_beta', '0.25', '--nfa_gamma', 'off', '--nfa_proj_basis', 'b.pt',
             '--nfa_static_pair', '--nfa_moba', '--nfa_sinkswa_only']
    args = _parser().parse_args(PRODUCTION + EVERY_OTHER + extra)
    assert args.nfa_gamma == 'off' and args.nfa_alpha == 0.5


@pytest.mark.parametrize('flag,value', [
    ('nfa_far_select', 'cluster'), ('nfa_near_select', 'sim_greedy'),
    ('nfa_layer_skip_path', 'skip.json'), ('nfa_alpha', 0.5), ('nfa_beta', 0.25),
    ('nfa_gamma', 'off'), ('nfa_boundary_bypass', False), ('nfa_moba', True),
    ('nfa_sigma_select', 'far'), ('nfa_per_q_head', True), ('nfa_sinkswa_only', True),
])
def test_unimplemented_values_are_rejected_before_any_launch(flag, value):
    args = _parser().parse_args(PRODUCTION)
    setattr(args, flag, value)
    with pytest.raises(ValueError, match=f'--{flag}='):
        NFAIndexer(args)


@pytest.mark.parametrize('change,message', [
    (dict(nfa_subspace='bogus'), 'nfa_subspace 非法取值: bogus'),
    (dict(nfa_l2_subspace='half'), 'nfa_l2_subspace 非法取值: half'),
    (dict(nfa_sink_tokens=-1), 'nfa_sink_tokens 必须 >= 0'),
    (dict(nfa_swa_size=0), 'nfa_swa_size 必须 >= 1'),
    (dict(nfa_swa_size=100), 'nfa_swa_size 必须是 tia_block_size 的整数倍'),
    (dict(nfa_near_pages=None), '生产 NFA 必须显式传 nfa_near_pages 与 nfa_near_len'),
    (dict(nfa_near_tokens=None), "nfa_near_tokens 须传非负整数或 'off'"),
    (dict(nfa_near_pages=True), 'nfa_near_pages 须为整数计数，收到 True'),
    (dict(nfa_near_pages=-1), 'nfa_near_pages/nfa_near_len 必须非负'),
    (dict(nfa_near_pages=200), 'nfa_near_pages 不可超过 tia_level1_topk'),
    (dict(nfa_near_len=1000), '网格约束破坏：nfa_near_pages \\* block_size <= nfa_near_len'),
    (dict(tia_level2_topk=100), 'tia_level2_topk 不可小于 sink\\+swa'),
    (dict(nfa_near_tokens=-1), 'nfa_near_tokens 必须非负'),
    (dict(nfa_near_tokens=9999), '网格约束破坏：nt <= nb \\* bs'),
    (dict(nfa_near_tokens=1000), '网格约束破坏：far = K2-sink-swa-nt >= 0'),
    (dict(nfa_proj_basis='b.pt'), 'nfa_proj_basis 旧 HF Cache 路径已删除'),
    (dict(nfa_static_pair=True), 'nfa_static_pair 旧 prefill 标定路径已删除'),
    (dict(nfa_far_skip_cache='drop'), '仅支持 GraphReadyPagedRegionCache'),
])
def test_reference_configuration_messages(change, message):
    args = _parser().parse_args(PRODUCTION)
    for k, v in change.items():
        setattr(args, k, v)
    with pytest.raises(ValueError, match=message):
        NFAIndexer(args)


def test_parse_errors_of_the_typed_flags():
    for argv in (['--nfa_near_tokens', 'many'], ['--nfa_dyn_dgate_eps', '2'],
                 ['--nfa_dyn_dgate_rows', '0'], ['--tia_level2_cmp_ratio', '3']):
        with pytest.raises(SystemExit):
            _parser().parse_args(argv)
