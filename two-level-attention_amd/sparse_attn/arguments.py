"""Command-line flags of the NFA decode path.

Every flag of the reference's TIA and NFA groups (reference
sparse_attn/arguments.py:4-11 and :249-399: 5 TIA and 40 NFA flags) is
accepted with the reference's name, type, default and choices, so launch
scripts written for the reference parse unchanged.  They fall in three sets:

* flags that drive this path (block size, budgets, subspaces, L1 methods,
  near quota geometry, sink / window, 4-bit L2 keys, operator mode);
* flags the reference records but its decode selector never reads (for
  instance ``--nfa_dyn_dgate``, ``--tia_enable_async_topk``): accepted,
  inert here as there;
* flags whose non-default values ask for selection semantics this path does
  not implement (``UNIMPLEMENTED``): ``NFAIndexer`` rejects such a value with
  ``ValueError`` before any launch.  Their defaults are the path's behaviour.

Flags of the reference's other methods (quest, twilight, vendor baselines)
are not part of this package.
"""
import argparse
import math


def _bool_flag(x):
    return str(x).lower() != 'false'


def _parse_gamma(x):
    """``--nfa_gamma``: a number, or ``off`` (kept as the string)."""
    if str(x).strip().lower() == 'off':
        return 'off'
    return float(x)


def _parse_near_tokens(x):
    """``--nfa_near_tokens``: a non-negative integer quota or ``off``."""
    if str(x).strip().lower() == 'off':
        return 'off'
    try:
        return int(x)
    except (TypeError, ValueError):
        raise argparse.ArgumentTypeError(
            f"--nfa_near_tokens 须为非负整数或 'off'（自由竞争哨兵），收到 {x!r}")


def _parse_dgate_eps(x):
    try:
        v = float(x)
    except (TypeError, ValueError):
        raise argparse.ArgumentTypeError(
            f"--nfa_dyn_dgate_eps 必须是数值（far 区概率质量阈值），收到 {x!r}")
    if not math.isfinite(v) or not 0.0 <= v <= 1.0:
        raise argparse.ArgumentTypeError(
            f"--nfa_dyn_dgate_eps 必须为有限值且 0<=eps<=1"
            f"（far 区概率质量损失上界阈值），收到 {x!r}")
    return v


def _parse_dgate_rows(x):
    try:
        v = int(x)
    except (TypeError, ValueError):
        raise argparse.ArgumentTypeError(
            f"--nfa_dyn_dgate_rows 必须是整数（标定用 prefill q 尾行数），收到 {x!r}")
    if v < 1:
        raise argparse.ArgumentTypeError(
            f"--nfa_dyn_dgate_rows 必须 >= 1（标定用 prefill q 尾行数），收到 {x!r}")
    return v


# (flag, type, default, choices, help); type None = store_true
_TIA_FLAGS = [
    ('tia_block_size', int, 64, None, 'L1 statistics block (tokens per L1 page)'),
    ('tia_level1_topk', int, 128, None, 'L1 page budget (far + near)'),
    ('tia_level2_topk', int, 1024, None, 'L2 token budget (with sink and window)'),
    ('tia_level2_cmp_ratio', int, 2, [2, 4, 8], 'tail subspace: 64 / ratio dims per RoPE half'),
    ('tia_enable_async_topk', None, False, None, 'recorded; no effect on decode selection'),
]

_NFA_FLAGS = [
    ('nfa_enable_subspace', _bool_flag, True, None, 'score L1 on the --nfa_subspace dims'),
    ('nfa_enable_kmeans', _bool_flag, True, None, 'recorded; no effect on decode selection'),
    ('nfa_far_select', str, '4bit', ['4bit', 'cluster', 'sim_greedy'],
     'far L2 choice: fine-score top-k (4bit); cluster representatives are not implemented'),
    ('nfa_near_select', str, '4bit', ['4bit', 'cluster', 'sim_greedy'],
     'near L2 choice: fine-score top-k (4bit); cluster representatives are not implemented'),
    ('nfa_sim', float, 0.9, None, 'sim_greedy merge threshold (inert unless sim_greedy)'),
    ('nfa_sim_dims', str, 'subspace', ['subspace', 'nope', 'tail', 'full'],
     'sim_greedy clustering dims (inert unless sim_greedy)'),
    ('nfa_enable_layer_skip', _bool_flag, True, None, 'recorded; no effect on decode selection'),
    ('nfa_operator_mode', str, 'off', ['off', 'serial', 'overlap'],
     'decode attention: one union pass / protected and middle apart, serial or overlapped'),
    ('nfa_far_clusters', int, 256, None, 'cluster count (inert unless cluster selection)'),
    ('nfa_far_niter', int, 10, None, 'k-means iterations (inert unless cluster selection)'),
    ('nfa_far_blocks', int, 16, None, 'cluster blocks (inert unless cluster selection)'),
    ('nfa_far_tokens', int, 512, None, 'cluster token budget (inert unless cluster selection)'),
    ('nfa_layer_skip_path', str, None, None, 'static per-layer skip JSON (not implemented)'),
    ('nfa_far_method', str, 'minmax', ['minmax', 'avg', 'avg_top2'],
     'far-pool L1 score: page upper bound / head-mean page mean / mean of the top-2 heads'),
    ('nfa_near_method', str, 'avg', ['avg', 'minmax'],
     'near-pool L1 score: page mean / page upper bound'),
    ('nfa_alpha', float, None, None, 'legacy ratio geometry (not implemented: pass near_len)'),
    ('nfa_beta', float, None, None, 'legacy ratio geometry (not implemented: pass near_pages)'),
    ('nfa_gamma', _parse_gamma, None, None, 'legacy ratio geometry (not implemented: pass near_tokens)'),
    ('nfa_near_pages', int, argparse.SUPPRESS, None, 'L1 pages reserved for the near pool'),
    ('nfa_near_tokens', _parse_near_tokens, argparse.SUPPRESS, None,
     "L2 token quota of the near region, or 'off' for one shared competition"),
    ('nfa_near_len', int, argparse.SUPPRESS, None, 'near-region width in tokens'),
    ('nfa_boundary_bypass', _bool_flag, True, None,
     'sink page and SWA boundary page go straight to L2 (false is not implemented)'),
    ('nfa_l2_quant', _bool_flag, False, None, 'L2 logits on 4-bit min-max quantised keys'),
    ('nfa_subspace', str, 'full', ['full', 'rope', 'nope', 'tail', 'random', 'highfreq', 'mla_rope'],
     'dims scored by L1 (tail = low-frequency RoPE dims, mla_rope = dims 128-191 of 192)'),
    ('nfa_l2_subspace', str, 'same', ['same', 'full'], 'dims scored by L2: as L1, or all head dims'),
    ('nfa_proj_basis', str, None, None, 'projection basis (not implemented)'),
    ('nfa_static_pair', None, False, None, 'prefill pair calibration (not implemented)'),
    ('nfa_moba', None, False, None, 'MoBA chunk-gate arm (not implemented)'),
    ('nfa_sigma_select', str, 'none', ['none', 'far', 'near', 'mid'],
     'top-sigma selection side (only none is implemented)'),
    ('nfa_sigma', float, 8.0, None, 'top-sigma width (inert unless top-sigma selection)'),
    ('nfa_per_q_head', _bool_flag, False, None,
     'per-query-head selection (not implemented: selection is per kv head)'),
    ('nfa_sink_tokens', int, 128, None, 'tokens always attended at the sequence start'),
    ('nfa_swa_size', int, 128, None, 'sliding-window tokens always attended at the end'),
    ('nfa_sinkswa_only', None, False, None, 'sink and window only (not implemented)'),
    ('nfa_far_skip_backend', str, 'legacy', ['legacy'], 'compatibility no-op'),
    ('nfa_far_skip_cache', str, 'retain', ['retain'], 'compatibility no-op'),
    ('nfa_dyn_dgate', None, False, None, 'recorded; the prefill gate is GateConfig'),
    ('nfa_dyn_dgate_eps', _parse_dgate_eps, 0.05, None, 'recorded prefill gate threshold'),
    ('nfa_dyn_dgate_rows', _parse_dgate_rows, 256, None, 'recorded prefill gate rows'),
    ('nfa_enable_static_gate', _bool_flag, False, None, 'recorded; static decisions are passed to freeze'),
]

# Non-default values that ask for selection semantics this path does not
# implement: flag -> (default, what a non-default value would ask for)
UNIMPLEMENTED = {
    'nfa_far_select': ('4bit', 'cluster / sim_greedy far selection'),
    'nfa_near_select': ('4bit', 'cluster / sim_greedy near selection'),
    'nfa_layer_skip_path': (None, 'static per-layer skip file'),
    'nfa_alpha': (None, 'legacy ratio geometry'),
    'nfa_beta': (None, 'legacy ratio geometry'),
    'nfa_gamma': (None, 'legacy ratio geometry'),
    'nfa_boundary_bypass': (True, 'L1 pools without the boundary-page bypass'),
    'nfa_moba': (False, 'MoBA chunk gate'),
    'nfa_sigma_select': ('none', 'top-sigma selection'),
    'nfa_per_q_head': (False, 'per-query-head selection'),
    'nfa_sinkswa_only': (False, 'sink-and-window-only masks'),
}


def _add(group, spec):
    name, typ, default, choices, text = spec
    if typ is None:
        group.add_argument(f'--{name}', action='store_true', default=default, help=text)
        return
    kw = dict(type=typ, default=default, help=text)
    if choices is not None:
        kw['choices'] = choices
    group.add_argument(f'--{name}', **kw)


def _add_tia_args(parser):
    group = parser.add_argument_group(title='Two-level index (TIA)')
    for spec in _TIA_FLAGS:
        _add(group, spec)
    return parser


def _add_nfa_args(parser):
    group = parser.add_argument_group(title='NFA (two-level indexer)')
    for spec in _NFA_FLAGS:
        _add(group, spec)
    return parser


METHODS = ['quest', 'quest_vendor', 'quest_vendor_kernel', 'minference_vendor',
           'fasa_vendor', 'sparq_vendor', 'ffd_vendor', 'moba_vendor',
           'clusterkv_vendor', 'asynctls_vendor', 'hisa_vendor', 'jssa_vendor',
           'jssa_official', 'tia', 'twi', 'nfa', 'none']


def add_sparse_attn_args(parser):
    """Add ``--method`` plus the TIA and NFA flag groups to ``parser``."""
    parser.add_argument('--method', type=str, choices=METHODS)
    _add_tia_args(parser)
    _add_nfa_args(parser)
    return parser


def parse_args(argv=None):
    parser = argparse.ArgumentParser(description='NFA sparse attention',
                                     allow_abbrev=False)
    add_sparse_attn_args(parser)
    return parser.parse_args(argv)
