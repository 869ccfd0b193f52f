"""Command-line flags of the NFA decode path.

Flag names, defaults and choices match the reference's TIA and NFA groups
(reference arguments.py:4-11 and :249-399) so existing launch scripts parse
unchanged.  Flags of the reference's other baselines are not part of this
package.
"""
import argparse
import math


def _bool_flag(x):
    return str(x).lower() != 'false'


def _parse_near_tokens(x):
    """``--nfa_near_tokens``: a non-negative integer quota or ``off``."""
    if str(x).strip().lower() == 'off':
        return 'off'
    try:
        return int(x)
    except (TypeError, ValueError):
        raise argparse.ArgumentTypeError(
            f"--nfa_near_tokens expects an integer or 'off', got {x!r}")


def _parse_dgate_eps(x):
    try:
        v = float(x)
    except (TypeError, ValueError):
        raise argparse.ArgumentTypeError(
            f'--nfa_dyn_dgate_eps expects a number, got {x!r}')
    if not math.isfinite(v) or not 0.0 <= v <= 1.0:
        raise argparse.ArgumentTypeError(
            f'--nfa_dyn_dgate_eps must be finite and in [0, 1], got {x!r}')
    return v


def _parse_dgate_rows(x):
    try:
        v = int(x)
    except (TypeError, ValueError):
        raise argparse.ArgumentTypeError(
            f'--nfa_dyn_dgate_rows expects an integer, got {x!r}')
    if v < 1:
        raise argparse.ArgumentTypeError(
            f'--nfa_dyn_dgate_rows must be >= 1, got {x!r}')
    return v


def _add_tia_args(parser):
    group = parser.add_argument_group(title='Two-level index (TIA)')
    group.add_argument('--tia_block_size', type=int, default=64)
    group.add_argument('--tia_level1_topk', type=int, default=128)
    group.add_argument('--tia_level2_topk', type=int, default=1024)
    group.add_argument('--tia_level2_cmp_ratio', type=int, default=2,
                       choices=[2, 4, 8])
    group.add_argument('--tia_enable_async_topk', action='store_true')
    return parser


def _add_nfa_args(parser):
    group = parser.add_argument_group(title='NFA (two-level indexer)')
    group.add_argument('--nfa_enable_subspace', type=_bool_flag, default=True)
    group.add_argument('--nfa_enable_layer_skip', type=_bool_flag, default=True)
    group.add_argument('--nfa_operator_mode', choices=['off', 'serial', 'overlap'],
                       default='off',
                       help='decode attention: union / disjoint serial / overlap')
    group.add_argument('--nfa_far_method', type=str, default='minmax',
                       choices=['minmax', 'avg', 'avg_top2'],
                       help='far-pool L1 score: page upper bound / page mean')
    group.add_argument('--nfa_near_method', type=str, default='avg',
                       choices=['avg', 'minmax'],
                       help='near-pool L1 score: page mean / page upper bound')
    group.add_argument('--nfa_near_pages', type=int, default=argparse.SUPPRESS,
                       help='L1 pages reserved for the near pool')
    group.add_argument('--nfa_near_tokens', type=_parse_near_tokens,
                       default=argparse.SUPPRESS,
                       help="L2 token quota of the near pool, or 'off' for one "
                            'shared L2 competition')
    group.add_argument('--nfa_near_len', type=int, default=argparse.SUPPRESS,
                       help='near-region width in tokens')
    group.add_argument('--nfa_boundary_bypass', type=_bool_flag, default=True,
                       help='sink page and SWA boundary page go straight to L2')
    group.add_argument('--nfa_l2_quant', type=_bool_flag, default=False,
                       help='L2 logits on 4-bit min-max quantised keys')
    group.add_argument('--nfa_subspace', type=str, default='full',
                       choices=['full', 'rope', 'nope', 'tail', 'random',
                                'highfreq', 'mla_rope'],
                       help='dims scored by L1 (tail = low-frequency RoPE dims)')
    group.add_argument('--nfa_l2_subspace', type=str, default='same',
                       choices=['same', 'full'],
                       help='dims scored by L2: same as L1, or all head dims')
    group.add_argument('--nfa_proj_basis', type=str, default=None)
    group.add_argument('--nfa_static_pair', action='store_true')
    group.add_argument('--nfa_sink_tokens', type=int, default=128,
                       help='tokens always attended at the sequence start')
    group.add_argument('--nfa_swa_size', type=int, default=128,
                       help='sliding-window tokens always attended at the end')
    group.add_argument('--nfa_far_skip_backend', choices=['legacy'],
                       default='legacy')
    group.add_argument('--nfa_far_skip_cache', choices=['retain'],
                       default='retain')
    group.add_argument('--nfa_dyn_dgate', action='store_true', default=False)
    group.add_argument('--nfa_dyn_dgate_eps', type=_parse_dgate_eps, default=0.05)
    group.add_argument('--nfa_dyn_dgate_rows', type=_parse_dgate_rows, default=256)
    group.add_argument('--nfa_enable_static_gate', type=_bool_flag, default=False)
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
