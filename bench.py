#!/usr/bin/env python
"""NFA two-level sparse-attention decode at 128K context on one MI355X.

Workload (Qwen3-8B attention geometry): 36 layers, 32 query / 8 KV heads,
head_dim 128, batch 1, 131072-token context, paged bf16 KV with page = block
= 16, production NFA flags (far minmax, near avg, 32 near pages of 128 L1
pages, near_len 4096, tail subspace at cmp_ratio 4, sink 4, SWA 128, L2
top-1024).  Each layer owns its own 128K paged cache (18 GiB of KV in total,
far beyond the 256 MiB Infinity Cache).  Synthetic keys follow the
outlier-channel recipe: N(0,1) per channel times a per-channel
LogNormal(0,1) scale, RoPE theta 1e6 at positions 0..L-1; values and queries
N(0,1).

Headline (``value``, ``ms_per_step``, ``steps``, ``warmup``): whole-model
decode of a random-init bf16 Qwen3-8B after a dense prefill of the same
context -- ``--warmup`` untimed and ``--steps`` timed greedy steps replayed
from a hipGraph, HIP events around each runner step, median TPOT; value =
1000 / TPOT tok/s.

Per layer (``config.layer_us`` and the roofline): the hot path alone -- the
selector (fused decode K/V write, page statistics, L1, L2, union) and the
sparse gather attention of all 36 layers -- captured into one graph, warmed
by untimed replays, then ``--hot-steps`` replays timed with HIP events on the
replaying stream (median), the host planning of each step (plan_common /
commit_step) overlapping the previous replay.  The selector and the attention
are also captured alone and timed the same way (``select_us``,
``attention_us``, the roofline's achieved bandwidth).

CPU baseline (reported, not the target): the numpy oracle on the 32K fp32
layer, the kv heads spread over worker processes, 3 warm-up and 10 timed
steps, split into L1 / L2 / attention.

Prints one JSON line; ``--gpus`` above 1 is refused: this path runs on one
GPU.
"""
import argparse
import ctypes
import json
import math
import os
import re
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, 'two-level-attention_amd')):
    if _p not in sys.path:
        sys.path.insert(0, _p)

HBM_PEAK_GBS = 8000.0


def parse():
    ap = argparse.ArgumentParser(description=__doc__.split('\n')[0])
    ap.add_argument('--gpus', type=int, default=1)
    ap.add_argument('--steps', type=int, default=256,
                    help='timed whole-model decode steps (the headline e2e tok/s '
                         'is 1000 / their median TPOT)')
    ap.add_argument('--warmup', type=int, default=3,
                    help='untimed whole-model decode steps before them')
    ap.add_argument('--hot-steps', type=int, default=200,
                    help='timed replays of the 36-layer hot-path graph')
    ap.add_argument('--hot-warmup', type=int, default=30,
                    help='eager steps, then as many untimed graph replays, before them')
    ap.add_argument('--ctx', type=int, default=131072)
    ap.add_argument('--batch', type=int, default=1,
                    help='decode rows (requests) sharing one cache per layer')
    ap.add_argument('--ragged', type=int, nargs=2, metavar=('LO', 'HI'),
                    help='request lengths drawn uniformly from [LO, HI] (seeded) '
                         'instead of --ctx for every request')
    ap.add_argument('--layers', type=int, default=36)
    ap.add_argument('--l2-quant', action='store_true',
                    help='L2 logits over the 4-bit packed tail keys (--nfa_l2_quant)')
    ap.add_argument('--operator-mode', choices=['off', 'serial', 'overlap'], default='off',
                    help='decode attention of the timed step: one union pass (off) or '
                         'protected and middle apart, then merged (serial / overlap)')
    ap.add_argument('--kernel-rounds', type=int, default=40,
                    help='replays of the selector-only and attention-only graphs')
    ap.add_argument('--no-cpu-baseline', action='store_true')
    ap.add_argument('--seed', type=int, default=20261201)
    ap.add_argument('--timeline', type=int, default=0,
                    help='print selector phase timings of N extra decode steps')
    ap.add_argument('--no-e2e', action='store_true',
                    help='skip the whole-model decode (the headline value is then '
                         'the hot path\'s tok/s)')
    ap.add_argument('--e2e-unfused', action='store_true',
                    help='end-to-end decode with HF\'s own dense layers (only the '
                         'attention patched)')
    ap.add_argument('--e2e-only', action='store_true',
                    help='run only the end-to-end model decode')
    ap.add_argument('--mla', choices=['expanded', 'absorbed'],
                    help='only the DeepSeek-V2-Lite MLA decode layer (16 heads, '
                         'latent 512 + 64, batch 4 x 64K, 4-bit L2 keys on the 64 '
                         'RoPE dims, --layers layers): expanded heads or the '
                         'absorbed latent arena')
    ap.add_argument('--copy-calibration', type=int, default=0, metavar='MIB',
                    help='only copy a MIB-MiB device buffer three times (the '
                         'known-size kernel that scales rocprofv3 FETCH_SIZE '
                         'and WRITE_SIZE readings) and exit')
    ap.add_argument('--gather-calibration', type=int, default=0, metavar='MIB',
                    help='only gather a quarter of a MIB-MiB device buffer in '
                         'random order, three times as 1 KiB rows and three '
                         'times as 64-byte rows (the access sizes of the '
                         'selector\'s staged statistics and of one L2 side '
                         'row), and exit: FETCH_SIZE per known byte on '
                         'scattered reads')
    return ap.parse_args()


def synthetic_keys(torch, n, hkv, d, gen, device, theta=1e6, start=0,
                   dtype=None, scale=None):
    """N(0,1) x per-channel LogNormal(0,1) scale, RoPE (half-split) applied
    at positions start .. start+n-1.  Returns [1, hkv, n, d] in ``dtype``
    (bf16 by default).  ``scale`` ([hkv, 1, d]) reuses a request's channel
    scales, e.g. for its decode tokens."""
    if scale is None:
        scale = torch.exp(torch.randn(hkv, 1, d, generator=gen, device=device))
    k = torch.randn(hkv, n, d, generator=gen, device=device) * scale
    half = d // 2
    inv = theta ** (-torch.arange(0, half, device=device, dtype=torch.float32) / half)
    pos = torch.arange(start, start + n, device=device, dtype=torch.float32)
    ang = pos[:, None] * inv[None, :]
    cos, sin = torch.cos(ang), torch.sin(ang)
    x1, x2 = k[..., :half], k[..., half:]
    out = torch.cat((x1 * cos - x2 * sin, x2 * cos + x1 * sin), dim=-1)
    return out.to(dtype or torch.bfloat16).unsqueeze(0)


def build_workload(torch, args, device):
    from types import SimpleNamespace
    from sparse_attn.cache import GraphReadyPagedRegionCache
    from sparse_attn.indexer.nfa_indexer import NFAIndexer
    from sparse_attn.ops.paged_region_kernels_nfa import nfa_args
    from sparse_attn.policies.region_geometry import RegionGeometry

    hkv, hq, d, page = 8, 32, 128, 16
    new_tokens = (2 * args.hot_warmup + args.hot_steps + 2 * args.kernel_rounds
                  + args.timeline + 8)
    geo = RegionGeometry(sink=4, near=4096, window=128, page=page,
                         max_new_tokens=new_tokens)
    b = args.batch
    if args.ragged:
        lo, hi = args.ragged
        g = torch.Generator().manual_seed(args.seed)
        lengths = torch.randint(lo, hi + 1, (b,), generator=g).tolist()
    else:
        lengths = [args.ctx] * b
    pages = [(n + new_tokens + page - 1) // page for n in lengths]
    cache = GraphReadyPagedRegionCache(
        args.layers, geo, max_requests=b, max_physical_pages=sum(pages) + 1,
        max_blocks=max(pages) + 8, max_visible_len=1024, max_query_tokens=b,
        num_kv_heads=hkv, num_query_heads=hq, head_dim_k=d, head_dim_v=d,
        dtype=torch.bfloat16, device=device)
    fargs = nfa_args('tail')
    fargs.tia_block_size = page
    fargs.nfa_l2_quant = args.l2_quant
    indexer = NFAIndexer(fargs)
    gen = torch.Generator(device=device).manual_seed(args.seed)
    req_ids = list(range(b))
    for rid, n in zip(req_ids, lengths):
        cache.add_request(rid)
        for layer in range(args.layers):
            keys = synthetic_keys(torch, n, hkv, d, gen, device)
            values = torch.randn(1, hkv, n, d, generator=gen,
                                 device=device).to(torch.bfloat16)
            cache.write_prefill(layer, rid, keys, values)
            del keys, values
        cache.freeze(rid, [False] * args.layers, [False] * args.layers)
    attn = [SimpleNamespace(indexer=indexer, scaling=d ** -0.5, layer_idx=l)
            for l in range(args.layers)]
    q = [torch.randn(b, hq, d, generator=gen, device=device).to(torch.bfloat16)
         for _ in range(args.layers)]
    kn = [torch.randn(b, hkv, 1, d, generator=gen, device=device).to(torch.bfloat16)
          for _ in range(args.layers)]
    vn = [torch.randn(b, hkv, 1, d, generator=gen, device=device).to(torch.bfloat16)
          for _ in range(args.layers)]
    torch.cuda.synchronize()
    return SimpleNamespace(cache=cache, indexer=indexer, attn=attn, q=q, kn=kn,
                           vn=vn, hkv=hkv, hq=hq, d=d, page=page, req_ids=req_ids,
                           lengths=lengths, mode=args.operator_mode,
                           l2_quant=args.l2_quant)


def run_layer(w, layer, outs):
    from sparse_attn.indexer.nfa_layer_batch_selector import \
        select_topk_for_layer_batched
    from sparse_attn.ops.paged_region_kernels_nfa import decode_graph_ready
    cache = w.cache
    if w.mode != 'off':
        from sparse_attn.patches.qwen3_attn_patch import disjoint_regions_attention
        outs[layer] = disjoint_regions_attention(
            w.attn[layer], w.q[layer], w.kn[layer], w.vn[layer], cache,
            cache.slot_mapping_for_layer(layer)[:len(w.req_ids)], w.mode == 'overlap')
        return
    select_topk_for_layer_batched(
        cache, layer, w.req_ids, w.q[layer], attention=w.attn[layer],
        decode_write=(w.kn[layer], w.vn[layer],
                      cache.slot_mapping_for_layer(layer)[:len(w.req_ids)]))
    outs[layer] = decode_graph_ready(w.attn[layer], w.q[layer], cache)


def algorithmic_bytes(w, length, bs=16, window=128, near_len=4096, sink=4,
                      k_far=96, k_near=32, k2=1024, dsub=32):
    """Bytes one selector launch and one attention launch must move.

    Selector: L1 reads min+max (far pool, minmax score) or sum (near pool,
    avg score) of the 32 tail dims per page and KV head; L2 reads the 32 tail
    dims (64 B) of every candidate token, or its 4-bit codes with bf16
    scale and zero (20 B) with the 4-bit keys; plus the decode K/V write, the
    latest page's statistics update, the query and the gather row.
    Attention: K and V rows of every selected slot plus query, output and
    gather row.  Pool sizes follow the selector's region formulas.
    """
    hkv, hq, d = w.hkv, w.hq, w.d
    kt_eff = (length + bs - 1) // bs
    spl = sink // bs
    near_start = max((length - window - near_len) // bs, spl)
    swa_lo_blk = max(near_start, kt_eff - max(1, window // bs))
    p_far = max(0, near_start - spl) - (1 if sink % bs and near_start > spl else 0)
    p_near = max(0, swa_lo_blk - near_start)
    byp = max(length - window, 0)
    if byp % bs and byp // bs >= near_start and byp // bs < swa_lo_blk:
        p_near -= 1
    # candidate tokens: full far/near pages, the sink page past the sink
    # tokens and the part of the SWA boundary page before the window
    t_c = (k_far + k_near) * bs + (bs - sink % bs if sink % bs else 0) + byp % bs
    l1 = hkv * (2 * p_far * dsub * 2 + p_near * dsub * 2)
    l2 = hkv * t_c * (dsub // 2 + 4 if getattr(w, 'l2_quant', False) else dsub * 2)
    misc = (2 * hkv * d * 2 * 2        # decode K/V write (read + write)
            + 3 * hkv * dsub * 2       # latest page statistics
            + bs * hkv * dsub * 2      # latest page keys
            + hq * d * 2               # query
            + hkv * k2 * 4)            # gather row
    sel = l1 + l2 + misc
    att = hkv * k2 * (d + d) * 2 + hkv * k2 * 4 + 2 * hq * d * 2
    return dict(select=sel, attention=att, l1=l1, l2=l2, p_far=p_far,
                p_near=p_near, t_c=t_c)


# profiled workloads: (ctx, batch, ragged) -> rocprofv3 FETCH_SIZE / WRITE_SIZE summary
_TRAFFIC_PROFILES = {
    (131072, 1, None): 'nfa_select_layer_128k_hbm_traffic.md',
    (1048576, 1, None): 'nfa_select_layer_1m_kernel_trace_hbm_traffic.md',
    (131072, 16, (32768, 131072)): 'nfa_select_layer_16x_ragged_kernel_trace_hbm_traffic.md',
}


def measured_traffic(args):
    """HBM bytes per selector launch at this workload, from the committed
    rocprofv3 FETCH_SIZE / WRITE_SIZE summary (None when absent or when the
    workload differs from the profiled ones)."""
    ragged = tuple(args.ragged) if args.ragged else None
    name = _TRAFFIC_PROFILES.get((args.ctx, args.batch, ragged))
    if name is None or args.l2_quant or args.operator_mode != 'off':
        return None
    path = os.path.join(ROOT, 'profiles', name)
    try:
        with open(path) as f:
            text = f.read()
    except OSError:
        return None
    m = re.search(r'traffic_bytes_per_launch: (\d+)', text)
    return int(m.group(1)) if m else None


def time_kernels(torch, w, rounds, plan):
    """Per-launch durations of the selector entry point (kernel A + kernel B)
    and of the attention kernel.  Each is captured alone into a graph of one
    launch per layer; HIP events recorded on the launching stream bracket
    every replay, and the lengths advance between replays exactly as in
    decode (so the statistics stay on the incremental path)."""
    from sparse_attn.indexer.nfa_layer_batch_selector import \
        select_topk_for_layer_batched
    from sparse_attn.ops.paged_region_kernels_nfa import decode_graph_ready
    cache = w.cache
    layers = len(w.q)
    outs = [None] * layers

    def sel_all():
        for layer in range(layers):
            select_topk_for_layer_batched(
                cache, layer, w.req_ids, w.q[layer], attention=w.attn[layer],
                decode_write=(w.kn[layer], w.vn[layer],
                              cache.slot_mapping_for_layer(layer)[:len(w.req_ids)]))

    def att_all():
        for layer in range(layers):
            outs[layer] = decode_graph_ready(w.attn[layer], w.q[layer], cache)

    plan()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        sel_all()
        att_all()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g_sel, g_att = torch.cuda.CUDAGraph(), torch.cuda.CUDAGraph()
    with torch.cuda.graph(g_sel):
        sel_all()
    with torch.cuda.graph(g_att):
        att_all()
    cache.commit_step()
    for _ in range(rounds):  # untimed replays: graph upload, caches
        plan()
        g_sel.replay()
        g_att.replay()
        cache.commit_step()
    torch.cuda.synchronize()
    sel, att = [], []
    lengths = []
    marks = [(a, b, torch.cuda.Event(enable_timing=True))
             for a, b in warm_events(torch, rounds)]
    for m in marks:
        m[2].record()
    torch.cuda.synchronize()
    for a, b, c in marks:
        plan()
        lengths = [int(cache.pending_lengths[r]) for r in w.req_ids]
        a.record()
        g_sel.replay()
        b.record()
        g_att.replay()
        c.record()
        cache.commit_step()
        c.synchronize()
        sel.append(a.elapsed_time(b) * 1000.0 / layers)
        att.append(b.elapsed_time(c) * 1000.0 / layers)
    sel.sort()
    att.sort()
    mean = lambda v: sum(v) / len(v)
    return dict(select_us=mean(sel), attention_us=mean(att),
                select_us_median=sel[len(sel) // 2],
                attention_us_median=att[len(att) // 2], lengths=lengths)


def selector_timeline(torch, w, steps, plan):
    """Phase durations (µs) of the selector kernel from its in-kernel wall
    clock marks, over ``steps`` eager decode steps of every layer."""
    from sparse_attn import _native
    from sparse_attn.indexer.nfa_layer_batch_selector import \
        select_topk_for_layer_batched
    rate_khz = _native.load_library().nfa_wall_clock_khz() or 100000
    cache = w.cache
    tiles, tails = [], []
    for _ in range(steps):
        plan()
        for layer in range(len(w.q)):
            dbg = {'clock_only': True}
            select_topk_for_layer_batched(
                cache, layer, w.req_ids, w.q[layer], attention=w.attn[layer],
                decode_write=(w.kn[layer], w.vn[layer],
                              cache.slot_mapping_for_layer(layer)[:len(w.req_ids)]),
                _debug=dbg)
            tiles.append(dbg['clock'])
        cache.commit_step()
    torch.cuda.synchronize()
    us = 1000.0 / rate_khz
    import numpy as np
    acc = {}
    for clk in tiles:
        c = clk.cpu().numpy().astype(np.int64)
        tile, tail = c[:, :-1, :], c[:, -1, :]
        start = tile[:, :, 0][tile[:, :, 0] > 0].min()
        acc.setdefault('kernel span', []).append((tail[:, 13].max() - start) * us)
        acc.setdefault('last tile arrives', []).append(
            (tile[:, :, 4].max() - start) * us)
        # per row: its tail's first mark after its last tile's arrival mark
        # (the counters, the release and acquire, the tail's own set-up)
        gap = (tail[:, 0] - tile[:, :, 4].max(axis=1)) * us
        acc.setdefault('arrival to tail start (max row)', []).append(float(gap.max()))
        acc.setdefault('tail start (max)', []).append(float((tail[:, 0].max() - start) * us))
        if (tail[:, 27] > 0).all():
            g1 = (tail[:, 27] - tile[:, :, 4].max(axis=1)) * us
            g2 = (tail[:, 0] - tail[:, 27]) * us
            acc.setdefault('  arrival: marks flush + request counter (max row)', []).append(
                float(g1.max()))
            acc.setdefault('  arrival: row counter + tail set-up (max row)', []).append(
                float(g2.max()))
        # arrival steps of the last workgroup when the kernel records them
        # (marks 28-31: completion wait, group ticket, row ticket, acquire)
        if (tail[:, 31] > 0).all():
            for a, bb, name in ((27, 28, 'completion wait + barrier'),
                                (28, 29, 'group ticket'), (29, 30, 'row ticket'),
                                (30, 31, 'acquire + barrier'), (31, 0, 'tail set-up')):
                d = (tail[:, bb] - tail[:, a]) * us
                acc.setdefault(f'    {name} (max row)', []).append(float(d.max()))
        names = ['row scalars', 'q prep', 'page stats', 'L1 scores+publish']
        for k, name in enumerate(names):
            d = (tile[:, :, k + 1] - tile[:, :, k]) * us
            acc.setdefault(f'A tile {name} (max)', []).append(d.max())
        # summed over a tile's passes: staging wait, scores, keys + histogram;
        # then the histogram flush after the last pass
        for k, name in ((8, 'passes: staging wait'), (9, 'passes: scores'),
                        (10, 'passes: keys+hist')):
            acc.setdefault(f'A tile {name} (max)', []).append(tile[:, :, k].max() * us)
        acc.setdefault('A tile hist flush (max)', []).append(
            ((tile[:, :, 4] - tile[:, :, 6]) * us).max())
        # survivor lists of long rows (marks 11-15 when present)
        if (tile[:, :, 15] > 0).any():
            ok = tile[:, :, 15] > 0
            for a, bb, name in ((6, 11, 'coarse bins'), (11, 12, 'refine'),
                                (12, 13, 'fine bins+count'), (13, 14, 'scan'),
                                (14, 15, 'write'), (15, 4, 'hist flush')):
                acc.setdefault(f'A tile survivors: {name} (max)', []).append(
                    float(((tile[:, :, bb] - tile[:, :, a]) * us)[ok].max()))
        acc.setdefault('A tile slowest scoring tile', []).append(
            float(np.unravel_index(tile[:, :, 9].argmax(), tile.shape[:2])[1]))
        # the tile that arrives last in each row, and the median tile: their
        # start (from the kernel's first mark) and phase durations
        live = tile[:, :, 4] > 0
        arr = np.where(live, tile[:, :, 4], 0)
        last_t = arr.argmax(axis=1)
        rows_i = np.arange(tile.shape[0])
        acc.setdefault('A last-arriving tile index (median row)', []).append(
            float(np.median(last_t)))
        # the tile of median duration in each row
        dur_rt = np.where(live, tile[:, :, 4] - tile[:, :, 0], -1)
        med_t = np.array([np.argsort(r)[len(r) - 1 - int(np.sum(r >= 0)) // 2]
                          for r in dur_rt])
        for nm, sel in (('last tile', tile[rows_i, last_t]),
                        ('median tile', tile[rows_i, med_t])):
            acc.setdefault(f'A {nm}: start', []).append(
                float(np.median((sel[:, 0] - start) * us)))
            for k, name in enumerate(names):
                acc.setdefault(f'A {nm}: {name}', []).append(
                    float(np.median((sel[:, k + 1] - sel[:, k]) * us)))
            for k, name in ((8, 'staging wait'), (9, 'scores'), (10, 'keys+hist')):
                acc.setdefault(f'A {nm}: passes {name}', []).append(
                    float(np.median(sel[:, k] * us)))
        dur = np.where(live, (tile[:, :, 4] - tile[:, :, 0]) * us, np.nan)
        acc.setdefault('A tile duration (median tile)', []).append(
            float(np.nanmedian(dur)))
        st0 = np.where(live, (tile[:, :, 0] - start) * us, np.nan)
        acc.setdefault('A tile start (median tile)', []).append(float(np.nanmedian(st0)))
        acc.setdefault('A tile start (max)', []).append(float(np.nanmax(st0)))
        spans = [('tail L1 threshold', 0, 1),
                 ('  L1 thr: hist+keys load', 0, 24), ('  L1 thr: coarse bins', 24, 25),
                 ('  L1 thr: refine pass', 25, 26), ('  L1 thr: fine bins', 26, 1),
                 ('tail selection pass', 1, 2),
                 
                 ('tail bitmap compaction', 2, 3), ('tail candidate pages', 3, 4),
                 ('tail L1 end', 4, 6), ('tail L2 logits', 6, 9),
                 ('tail L2 top-k', 9, 12), ('tail union', 12, 13),
                 ('  L2 top-k: coarse hist', 16, 17), ('  L2 top-k: coarse bin', 17, 18),
                 ('  L2 top-k: fine pass+bin', 18, 19), ('  L2 top-k: count+scan', 19, 20),
                 ('  L2 top-k: emit', 20, 21), ('  L2 top-k: hole fill', 21, 22),
                 ('  L2 top-k: merge', 22, 23)]
        for name, a, b in spans:
            ok = (tail[:, a] > 0) & (tail[:, b] > 0)
            if ok.any():
                d = (tail[ok, b] - tail[ok, a]) * us
                acc.setdefault(f'{name} (max)', []).append(d.max())
    for name, vals in acc.items():
        print(f'# timeline {name:28s} median {np.median(vals):8.2f} us',
              file=sys.stderr, flush=True)


def qwen3_8b_config(ctx, new_tokens):
    """Qwen3-8B architecture (36 layers, hidden 4096, MLP 12288, 32/8 heads,
    head_dim 128, vocab 151936, RoPE theta 1e6)."""
    from transformers import Qwen3Config
    cfg = Qwen3Config(vocab_size=151936, hidden_size=4096, intermediate_size=12288,
                      num_hidden_layers=36, num_attention_heads=32,
                      num_key_value_heads=8, head_dim=128, rms_norm_eps=1e-6,
                      rope_theta=1e6, tie_word_embeddings=False,
                      max_position_embeddings=ctx + new_tokens + 64)
    cfg._attn_implementation = 'sdpa'
    return cfg


def llama31_8b_config(ctx, new_tokens):
    """Llama-3.1-8B architecture (32 layers, hidden 4096, MLP 14336, 32/8
    heads, head_dim 128, vocab 128256, RoPE theta 5e5 with llama3 scaling)."""
    from transformers import LlamaConfig
    cfg = LlamaConfig(vocab_size=128256, hidden_size=4096, intermediate_size=14336,
                      num_hidden_layers=32, num_attention_heads=32,
                      num_key_value_heads=8, head_dim=128, rms_norm_eps=1e-5,
                      rope_theta=500000.0, tie_word_embeddings=False,
                      rope_scaling={'rope_type': 'llama3', 'factor': 8.0,
                                    'low_freq_factor': 1.0, 'high_freq_factor': 4.0,
                                    'original_max_position_embeddings': 8192},
                      max_position_embeddings=max(131072, ctx + new_tokens + 64))
    cfg._attn_implementation = 'sdpa'
    return cfg


def end_to_end_batch(torch, args, device, lengths):
    """Whole-model decode of a ragged batch: random-init bf16 Llama-3.1-8B,
    one dense prefill per prompt (seeded uniform token ids of the given
    lengths) into one paged cache sized for their pages, then the batch
    decoded together: 3 warm-up steps and ``args.steps`` greedy steps
    replayed from one captured hipGraph; HIP events around every
    ``GraphRunner.step``, median step time; tok/s = batch / step."""
    from transformers import LlamaForCausalLM
    from sparse_attn.engine.frozen_runner import (build_frozen_cache,
                                                  prefill_frozen_request)
    from sparse_attn.engine.graph_runner import GraphRunner
    from sparse_attn.ops.decode_fused import LINEAR_MAX_ROWS
    from sparse_attn.ops.paged_region_kernels_nfa import nfa_args
    from sparse_attn.patches.patch import register_patch
    from sparse_attn.policies.region_geometry import RegionGeometry
    from sparse_attn.scheduler.scheduler import ContinuousBatchScheduler

    warm = args.warmup
    b = len(lengths)
    new_tokens = warm + args.steps + 8
    cfg = llama31_8b_config(max(lengths), new_tokens)
    t0 = time.perf_counter()
    torch.manual_seed(args.seed)
    prev = torch.get_default_dtype()
    torch.set_default_dtype(torch.bfloat16)
    try:
        with torch.device(device):
            model = LlamaForCausalLM(cfg).eval()
    finally:
        torch.set_default_dtype(prev)
    fargs = nfa_args('tail')
    fargs.tia_block_size = 16
    n_patched = register_patch(model, fargs, rmsnorm_decode=True, decode_layers=True)
    params = sum(p.numel() for p in model.parameters())
    torch.cuda.synchronize()
    print(f'# e2e batch model ready ({params / 1e9:.2f} B params) in '
          f'{time.perf_counter() - t0:.1f}s', file=sys.stderr, flush=True)

    page = 16
    geo = RegionGeometry(sink=4, near=4096, window=128, page=page,
                         max_new_tokens=new_tokens)
    pages = sum((n + new_tokens + page - 1) // page for n in lengths)
    cache = build_frozen_cache(model, geo, max(lengths), max_requests=b,
                               max_visible_len=1024, physical_pages=pages + 8)
    gen = torch.Generator(device=device).manual_seed(args.seed)
    from torch.nn.attention import SDPBackend, sdpa_kernel
    rids, firsts = [], []
    t0 = time.perf_counter()
    with torch.no_grad(), sdpa_kernel([SDPBackend.FLASH_ATTENTION,
                                       SDPBackend.EFFICIENT_ATTENTION]):
        for i, n in enumerate(lengths):
            ids = torch.randint(0, cfg.vocab_size, (1, n), generator=gen, device=device)
            out, audit = prefill_frozen_request(model, ids, None, geo, cache=cache)
            rids.append(audit['request_id'])
            firsts.append(int(out.logits[0, -1].argmax()))
            del out, ids
            print(f'# e2e batch prefill {i + 1}/{b}: {n} tokens', file=sys.stderr,
                  flush=True)
    torch.cuda.synchronize()
    prefill_s = time.perf_counter() - t0
    sched = ContinuousBatchScheduler(cache=cache, max_batch=b, eos_ids=(), pad_token_id=0)
    for rid, tok in zip(rids, firsts):
        sched.add_request(rid)
        sched.next_tokens[rid] = tok
    runner = GraphRunner(scheduler=sched, buckets=(b,), visible_buckets=(), device=device)
    with torch.no_grad():
        runner.capture_all(model, cache)
        for i in range(warm):
            runner.step(model, cache, generated_counts=i + 1)
        torch.cuda.synchronize()
        events = warm_events(torch, args.steps)
        t0 = time.perf_counter()
        for i, (a, e) in enumerate(events):
            a.record()
            runner.step(model, cache, generated_counts=warm + i + 1)
            e.record()
        torch.cuda.synchronize()
        wall_ms = (time.perf_counter() - t0) * 1e3 / args.steps
    step = sorted(a.elapsed_time(e) for a, e in events)
    med = step[len(step) // 2]
    tokens = len(sched.flush_ready_receipts())
    print(f'# e2e batch decode: median step {med:.3f} ms for {b} requests, '
          f'wall {wall_ms:.3f} ms/step', file=sys.stderr, flush=True)
    return {
        'model': 'Llama-3.1-8B architecture, random-init bf16 weights',
        'dense_layers': ('fused HIP decode layers' if b <= LINEAR_MAX_ROWS else
                         f'HF modules (the fused HIP decode layers take up to '
                         f'{LINEAR_MAX_ROWS} rows)'),
        'params': params, 'patched_attention_layers': n_patched,
        'prompt_tokens': list(lengths), 'prefill_s': round(prefill_s, 2),
        'decode_steps': args.steps, 'warmup_steps': warm,
        'step_ms_median': round(med, 4),
        'step_ms_p10_p90': [round(step[len(step) // 10], 4),
                            round(step[(len(step) * 9) // 10], 4)],
        'wall_ms_per_step': round(wall_ms, 4),
        'tok_s': round(b * 1e3 / med, 2),
        'graph_replays': runner.replay_count,
        'graph_eager_fallbacks': runner.eager_fallback_count,
        'receipts': tokens,
    }


def end_to_end(torch, args, device):
    """Whole-model decode: random-init bf16 Qwen3-8B, dense prefill of
    ``args.ctx`` seeded uniform token ids into the paged cache, 3 warm-up
    steps, then ``args.steps`` greedy steps replayed from one captured
    hipGraph each; HIP events around every ``GraphRunner.step``, median
    TPOT (the steady-state time per output token)."""
    from transformers import Qwen3ForCausalLM
    from sparse_attn.engine.frozen_runner import (build_frozen_cache,
                                                  prefill_frozen_request)
    from sparse_attn.engine.graph_runner import GraphRunner
    from sparse_attn.ops.paged_region_kernels_nfa import nfa_args
    from sparse_attn.patches.patch import register_patch
    from sparse_attn.policies.region_geometry import RegionGeometry
    from sparse_attn.scheduler.scheduler import ContinuousBatchScheduler

    warm = args.warmup
    new_tokens = warm + args.steps + 8
    cfg = qwen3_8b_config(args.ctx, new_tokens)
    t0 = time.perf_counter()
    torch.manual_seed(args.seed)
    prev = torch.get_default_dtype()
    torch.set_default_dtype(torch.bfloat16)
    try:
        with torch.device(device):
            model = Qwen3ForCausalLM(cfg).eval()
    finally:
        torch.set_default_dtype(prev)
    fargs = nfa_args('tail')
    fargs.tia_block_size = 16
    fused = not args.e2e_unfused
    n_patched = register_patch(model, fargs, rmsnorm_decode=fused,
                               decode_layers=fused)
    params = sum(p.numel() for p in model.parameters())
    torch.cuda.synchronize()
    print(f'# e2e model ready ({params / 1e9:.2f} B params) in '
          f'{time.perf_counter() - t0:.1f}s', file=sys.stderr, flush=True)

    geo = RegionGeometry(sink=4, near=4096, window=128, page=16,
                         max_new_tokens=new_tokens)
    cache = build_frozen_cache(model, geo, args.ctx, max_visible_len=1024)
    gen = torch.Generator(device=device).manual_seed(args.seed)
    ids = torch.randint(0, cfg.vocab_size, (1, args.ctx), generator=gen,
                        device=device)
    from torch.nn.attention import SDPBackend, sdpa_kernel
    t0 = time.perf_counter()
    with torch.no_grad(), sdpa_kernel([SDPBackend.FLASH_ATTENTION,
                                       SDPBackend.EFFICIENT_ATTENTION]):
        out, audit = prefill_frozen_request(model, ids, None, geo, cache=cache)
    torch.cuda.synchronize()
    prefill_s = time.perf_counter() - t0
    print(f'# e2e prefill of {args.ctx} tokens: {prefill_s:.1f}s', file=sys.stderr,
          flush=True)
    rid = audit['request_id']
    del ids
    sched = ContinuousBatchScheduler(cache=cache, max_batch=1, eos_ids=(),
                                     pad_token_id=0)
    sched.add_request(rid)
    sched.next_tokens[rid] = int(out.logits[0, -1].argmax())
    del out
    runner = GraphRunner(scheduler=sched, buckets=(1,), visible_buckets=(),
                         device=device)
    with torch.no_grad():
        runner.capture_all(model, cache)
        for i in range(warm):
            runner.step(model, cache, generated_counts=i + 1)
        torch.cuda.synchronize()
        events = warm_events(torch, args.steps)
        t0 = time.perf_counter()
        for i, (a, b) in enumerate(events):
            a.record()
            runner.step(model, cache, generated_counts=warm + i + 1)
            b.record()
        torch.cuda.synchronize()
        wall_ms = (time.perf_counter() - t0) * 1e3 / args.steps
    tpot = sorted(a.elapsed_time(b) for a, b in events)
    med = tpot[len(tpot) // 2]
    tokens = len(sched.flush_ready_receipts())
    print(f'# e2e decode: median TPOT {med:.3f} ms, wall {wall_ms:.3f} ms/token',
          file=sys.stderr, flush=True)
    res = {
        'model': 'Qwen3-8B architecture, random-init bf16 weights',
        'dense_layers': 'fused HIP decode layers' if fused else 'HF modules',
        'params': params, 'patched_attention_layers': n_patched,
        'prompt_tokens': args.ctx, 'prefill_s': round(prefill_s, 2),
        'decode_steps': args.steps, 'warmup_steps': warm,
        'tpot_ms_median': round(med, 4),
        'tpot_ms_p10_p90': [round(tpot[len(tpot) // 10], 4),
                            round(tpot[(len(tpot) * 9) // 10], 4)],
        'wall_ms_per_token': round(wall_ms, 4),
        'tok_s': round(1e3 / med, 2),
        'graph_replays': runner.replay_count,
        'graph_eager_fallbacks': runner.eager_fallback_count,
        'receipts': tokens,
    }
    del runner, sched, model, cache
    torch.cuda.empty_cache()
    return res


# ---------------------------------------------------------------------------
# CPU baseline: the numpy oracle on the single-layer 32K fp32 workload
# ---------------------------------------------------------------------------

_CPU = {}   # inherited by the forked workers: pools, query, geometry


def _cpu_config0(seed, extra_tokens):
    """Config-0 layer as numpy arrays: Qwen3-8B layer geometry (32 query /
    8 KV heads, head_dim 128), 32768-token context plus ``extra_tokens``
    decode tokens, page 16, fp32 paged K/V; outlier-channel keys (N(0,1) x
    per-channel LogNormal(0,1) scale, RoPE theta 1e6), N(0,1) values and
    queries."""
    import numpy as np
    from oracle import nfa_oracle as orc
    hq, hkv, d, page, ctx = 32, 8, 128, 16, 32768
    total = ctx + extra_tokens
    pages = (total + page - 1) // page
    rng = np.random.default_rng(seed)
    scale = np.exp(rng.standard_normal((hkv, 1, d), dtype=np.float32))
    keys = rng.standard_normal((hkv, total, d), dtype=np.float32) * scale
    half = d // 2
    inv = 1e6 ** (-np.arange(half, dtype=np.float64) / half)
    ang = np.arange(total, dtype=np.float64)[:, None] * inv[None, :]
    cos, sin = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
    x1, x2 = keys[..., :half], keys[..., half:]
    keys = np.concatenate((x1 * cos - x2 * sin, x2 * cos + x1 * sin), axis=-1)
    values = rng.standard_normal((hkv, total, d), dtype=np.float32)
    k_pool = np.zeros((pages + 1, 1, hkv, page, d), dtype=np.float32)
    v_pool = np.zeros_like(k_pool)
    pad = pages * page - total
    k_pool[:pages, 0] = np.pad(keys, ((0, 0), (0, pad), (0, 0))).reshape(
        hkv, pages, page, d).transpose(1, 0, 2, 3)
    v_pool[:pages, 0] = np.pad(values, ((0, 0), (0, pad), (0, 0))).reshape(
        hkv, pages, page, d).transpose(1, 0, 2, 3)
    dims = cpu_tail_dims(d, 4)
    cfg = orc.NfaConfig(
        hq=hq, hkv=hkv, head_dim=d, head_dim_v=d, bs=16, page=page,
        max_blocks=pages + 8, geo_sink=4, geo_near=4096, geo_window=128,
        sink_tokens=4, swa=128, near_len=4096, k1=128, near_pages=32, k2=1024,
        dims=dims, fine_dims=dims, scale=d ** -0.5, kv_dtype='fp32')
    bt = np.full(cfg.max_blocks, pages, dtype=np.int64)
    bt[:pages] = np.arange(pages)
    qs = rng.standard_normal((3 + extra_tokens, 1, hq, d), dtype=np.float32)
    return dict(cfg=cfg, k_pool=k_pool, v_pool=v_pool, bt=bt, ctx=ctx, q=qs,
                new_k=keys[:, ctx:], new_v=values[:, ctx:])


def cpu_tail_dims(head_dim, cmp_ratio):
    """The production L1/L2 dims (``--nfa_subspace tail``, L2 subspace
    ``same``): the last head_dim / 2 / cmp_ratio dims of each rotary half
    (reference sparse_attn/indexer/nfa_indexer.py:112-121), [48..63] and
    [112..127] for head_dim 128 at cmp_ratio 4.  Computed here without torch:
    the baseline runs before torch starts."""
    import numpy as np
    half = head_dim // 2
    delta = half // cmp_ratio
    return np.concatenate((np.arange(half - delta, half),
                           np.arange(head_dim - delta, head_dim)))


def _cpu_apply_writes(kv, upto):
    """Decode tokens 0..upto-1 of kv head ``kv`` into this process's pools
    (a worker's pools are its own copies, so every phase-1 call replays the
    writes it may have missed)."""
    c = _CPU
    page = c['cfg'].page
    for i in range(upto):
        pos = c['ctx'] + i
        c['k_pool'][pos // page, 0, kv, pos % page] = c['new_k'][kv, i]
        c['v_pool'][pos // page, 0, kv, pos % page] = c['new_v'][kv, i]


def cpu_l1_part(cfg, k_pool, bt, length, kv, q_full, p0, p1):
    """far / near bf16 score bits of pages [p0, p1) of one (row, kv head),
    no region skipped: the oracle's l1_scores restricted to a page range
    (page statistics and scores are per page; the pool masks are the
    row's).  Needs page == bs, so page p0 starts block-table entry p0."""
    import numpy as np
    from oracle import nfa_oracle as orc
    far_pool, near_pool, _ = orc.l1_pools(cfg, length, False, False)
    kmin, kmax, ksum = orc.page_stats(cfg, k_pool, bt[p0:], length - p0 * cfg.bs,
                                      kv, n_pages=p1 - p0)
    g = cfg.group
    mm, avg = orc.l1_page_scores(cfg, kmin, kmax, ksum, q_full[kv * g:(kv + 1) * g])
    far_val = mm if cfg.far_method == 'minmax' else avg
    near_val = avg if cfg.near_method == 'avg' else mm
    far = np.where(far_pool[p0:p1], far_val, orc.NEG_INF_BITS).astype(np.uint16)
    near = np.where(near_pool[p0:p1], near_val, orc.NEG_INF_BITS).astype(np.uint16)
    return far, near


def _cpu_l1(args):
    from oracle import nfa_oracle as orc
    kv, step, length, p0, p1 = args
    c = _CPU
    cfg = c['cfg']
    _cpu_apply_writes(kv, step + 1)
    q_full = orc.prepare_q(cfg, c['q'][step, 0], cfg.dims)
    return cpu_l1_part(cfg, c['k_pool'], c['bt'], length, kv, q_full, p0, p1)


def _cpu_l2(args):
    import numpy as np
    from oracle import nfa_oracle as orc
    kv, step, length, parts = args
    c = _CPU
    cfg = c['cfg']
    _cpu_apply_writes(kv, step + 1)
    far = np.concatenate([f for f, _ in parts])
    near = np.concatenate([n for _, n in parts])
    geo = orc.l1_geometry(cfg, length)
    i_f = orc.l1_topk(far, 0, geo.far_end, cfg.k_f, cfg.kt_cap)
    i_n = orc.l1_topk(near, geo.near_start, geo.near_end, cfg.k_n, cfg.kt_cap)
    q_fine = orc.prepare_q_grouped(cfg, c['q'][step, 0])
    lower, upper, quota = orc.l2_bounds(cfg, length, False, False)
    token, active, pack_r = orc.candidate_slots(cfg, i_f, i_n, far, near, length)
    load = orc.owned_slots(cfg, token, active, pack_r, lower, upper)
    logits = orc.l2_logits(cfg, c['k_pool'], c['bt'], token, load, q_fine[kv], kv,
                           quota)
    middle, count = orc.l2_middle(cfg, logits, token, length, False, False,
                                  lower, upper, quota)
    return orc.final_union(cfg, middle, count, length, c['bt'], 1024)


def _cpu_attention(args):
    import numpy as np
    from oracle import nfa_oracle as orc
    kv, step, (gather, vis) = args
    c = _CPU
    cfg = c['cfg']
    _cpu_apply_writes(kv, step + 1)   # the window holds the decode tokens
    g = cfg.group
    q = c['q'][step][:, kv * g:(kv + 1) * g]
    out = orc.sparse_attention(c['k_pool'][:, :, kv:kv + 1], c['v_pool'][:, :, kv:kv + 1],
                               q, np.asarray(gather)[None, None], np.array([[vis]]),
                               np.array([0]), cfg.scale, cfg.page)
    return out


def cpu_baseline(warmup=3, steps=10, seed=20261201):
    """Single-layer decode steps of the 32K fp32 layer on the numpy oracle:
    3 warm-up and 10 timed steps (the context grows by the decode token each
    step), each split into L1 (decode write, page
    statistics and scores), L2 (L1 top-k, candidates, logits, top-quota,
    union) and attention, one task per kv head and phase, timed with
    perf_counter around each phase; medians reported.  Runs before anything
    touches the GPU."""
    import multiprocessing as mp
    import statistics
    _CPU.clear()
    _CPU.update(_cpu_config0(seed, warmup + steps))
    hkv = _CPU['cfg'].hkv
    cores = os.cpu_count() or 1
    # one worker per kv head: the phases are bound by the host's memory
    # bandwidth (numpy gathers of the K pool), so more concurrent workers
    # slow each other down -- on the 16-CPU GPU host, 16 workers over 2
    # page ranges per kv head took the L1 phase from 23.7 ms to 92.5 ms
    workers = max(1, min(hkv, cores))
    nparts = 1
    phases = {'l1': [], 'l2': [], 'attention': []}
    with mp.get_context('fork').Pool(workers) as pool:
        for step in range(warmup + steps):
            length = _CPU['ctx'] + step + 1
            kt = -(-length // _CPU['cfg'].bs)
            cuts = [kt * i // nparts for i in range(nparts + 1)]
            t0 = time.perf_counter()
            l1 = pool.map(_cpu_l1, [(kv, step, length, cuts[i], cuts[i + 1])
                                    for kv in range(hkv) for i in range(nparts)],
                          chunksize=1)
            t1 = time.perf_counter()
            l2 = pool.map(_cpu_l2, [(kv, step, length,
                                     l1[kv * nparts:(kv + 1) * nparts])
                                    for kv in range(hkv)], chunksize=1)
            t2 = time.perf_counter()
            pool.map(_cpu_attention, [(kv, step, l2[kv]) for kv in range(hkv)],
                     chunksize=1)
            t3 = time.perf_counter()
            if step >= warmup:
                phases['l1'].append(t1 - t0)
                phases['l2'].append(t2 - t1)
                phases['attention'].append(t3 - t2)
    totals = [a + b + c for a, b, c in zip(*phases.values())]
    med = {k: statistics.median(v) * 1e6 for k, v in phases.items()}
    layer_us = statistics.median(totals) * 1e6
    _CPU.clear()
    return dict(value=round(layer_us, 1), unit='µs per decode layer (selector + attention)',
                cores=workers, kind='port',
                l1_us=round(med['l1'], 1), l2_us=round(med['l2'], 1),
                attention_us=round(med['attention'], 1),
                tok_s_36_layers=round(1e6 / (layer_us * 36), 4),
                host_cpus=cores,
                sample=f'{steps} timed single-layer decode steps after {warmup} '
                       'warm-up steps of the 32768-token fp32 layer (Qwen3-8B '
                       'layer geometry, page 16, production flags: minmax far / '
                       'avg near pools, L1 and L2 dims [48..63] + [112..127] '
                       '(tail subspace at cmp_ratio 4), 96 + 32 pages, 1024 '
                       'tokens, sink 4, window 128) on the numpy oracle in '
                       f'{workers} worker processes, one per kv head (memory-'
                       'bandwidth bound: 16 workers were 4x slower on a 16-CPU '
                       'host); median per phase')


# ---------------------------------------------------------------------------
# DeepSeek-V2-Lite MLA decode layer (expanded heads or absorbed latent arena)
# ---------------------------------------------------------------------------

MLA_HEADS, MLA_RANK, MLA_ROPE, MLA_NOPE, MLA_V = 16, 512, 64, 128, 128


def mla_algorithmic_bytes(mode, lengths, k2=1024, bs=16, window=128, near_len=4096,
                          sink=4, k_far=96, k_near=32):
    """Bytes one selector launch and one attention launch must move for the
    DeepSeek-V2-Lite layer.  Selector: page statistics of the 64 RoPE dims
    (min + max of far pages, the mean of near pages) -- once per request in
    the latent arena, where every head shares them, once per head expanded
    -- plus each head's candidate tokens' 4-bit L2 rows (32 B of codes, bf16
    scale and zero), the decode row and each head's gather row.  Attention:
    each head's selected rows (latent: the 576-dim row, 1152 B; expanded:
    192 + 128 dims, 640 B), query, output and gather row."""
    dsub, h = MLA_ROPE, MLA_HEADS
    sel = att = 0
    for n in lengths:
        kt = (n + bs - 1) // bs
        spl = sink // bs
        near_start = max((n - window - near_len) // bs, spl)
        swa_lo = max(near_start, kt - max(1, window // bs))
        p_far = max(0, near_start - spl) - (1 if sink % bs and near_start > spl else 0)
        p_near = max(0, swa_lo - near_start)
        byp = max(n - window, 0)
        t_c = (k_far + k_near) * bs + (bs - sink % bs if sink % bs else 0) + byp % bs
        stat_heads = 1 if mode == 'absorbed' else h
        l1 = stat_heads * (2 * p_far + p_near) * dsub * 2
        l2 = h * t_c * (dsub // 2 + 4)
        if mode == 'absorbed':
            row = (MLA_RANK + MLA_ROPE) * 2
            misc = row + h * (MLA_RANK + MLA_ROPE) * 2 + h * k2 * 4
            att += h * k2 * row + h * (MLA_RANK + MLA_ROPE) * 2 + h * MLA_RANK * 4 + h * k2 * 4
        else:
            row = (MLA_NOPE + MLA_ROPE + MLA_V) * 2
            misc = h * row + h * (MLA_NOPE + MLA_ROPE) * 2 + h * k2 * 4
            att += h * k2 * row + h * (MLA_NOPE + MLA_ROPE) * 2 + h * MLA_V * 2 + h * k2 * 4
        sel += l1 + l2 + misc
    return dict(select=sel, attention=att)


def mla_layer_bench(torch, args, device):
    """Selector and attention of the DeepSeek-V2-Lite decode layer, batch 4 x
    65536 tokens, ``--layers`` layers each with its own arena: selector-only
    and attention-only graphs of one launch per layer, timed like the
    Qwen3-8B layer (HIP events around each replay, lengths advancing)."""
    from types import SimpleNamespace
    from sparse_attn.cache import GraphReadyPagedRegionCache
    from sparse_attn.indexer.nfa_indexer import NFAIndexer
    from sparse_attn.indexer.nfa_layer_batch_selector import \
        select_topk_for_layer_batched
    from sparse_attn.ops.paged_region_kernels import (sparse_mla_attention_gather,
                                                      sparse_paged_attention_gather)
    from sparse_attn.ops.paged_region_kernels_nfa import nfa_args
    from sparse_attn.policies.region_geometry import RegionGeometry

    mode, layers, b, ctx = args.mla, args.layers, 4, 65536
    h, rank, rope, nope, dv = MLA_HEADS, MLA_RANK, MLA_ROPE, MLA_NOPE, MLA_V
    page = 16
    new_tokens = 2 * args.kernel_rounds + args.timeline + 8
    geo = RegionGeometry(sink=4, near=4096, window=128, page=page,
                         max_new_tokens=new_tokens)
    pages = (ctx + new_tokens + page - 1) // page
    latent = mode == 'absorbed'
    cache = GraphReadyPagedRegionCache(
        layers, geo, max_requests=b, max_physical_pages=b * pages + 1,
        max_blocks=pages + 8, max_visible_len=1024, max_query_tokens=b,
        num_kv_heads=1 if latent else h, num_query_heads=h,
        head_dim_k=rank + rope if latent else nope + rope,
        head_dim_v=rank if latent else dv, dtype=torch.bfloat16, device=device,
        latent=latent)
    fargs = nfa_args('mla_rope')
    fargs.tia_block_size = page
    fargs.nfa_l2_quant = True
    indexer = NFAIndexer(fargs)
    gen = torch.Generator(device=device).manual_seed(args.seed)
    scale = (nope + rope) ** -0.5
    w_uk, w_uv, w_exp = [], [], []
    for layer in range(layers):
        w = (torch.randn(h * (nope + dv), rank, generator=gen, device=device)
             * rank ** -0.5).to(torch.bfloat16).view(h, nope + dv, rank)
        w_uk.append(w[:, :nope].contiguous())
        w_uv.append(w[:, nope:].contiguous())
        # kv_b_proj^T as a contiguous [rank, H * (nope + v)] operand (the
        # expanded arena is c @ kv_b_proj^T, a plain 2-D product)
        w_exp.append(w.reshape(h * (nope + dv), rank).t().contiguous())
    for rid in range(b):
        cache.add_request(rid)
        for layer in range(layers):
            c = torch.randn(ctx, rank, generator=gen, device=device).to(torch.bfloat16)
            k_pe = synthetic_keys(torch, ctx, 1, rope, gen, device)[0, 0]
            if latent:
                cache.write_prefill(layer, rid, torch.cat([c, k_pe], -1)[None, None], None)
            else:
                kv = torch.matmul(c, w_exp[layer]).view(ctx, h, nope + dv).transpose(0, 1)
                k = torch.cat([kv[..., :nope], k_pe[None].expand(h, -1, -1)], dim=-1)
                v = kv[..., nope:]
                cache.write_prefill(layer, rid, k[None].contiguous(), v[None].contiguous())
                del kv, k, v
            del c, k_pe
        cache.freeze(rid, [False] * layers, [False] * layers)
    attn = [SimpleNamespace(indexer=indexer, scaling=scale, layer_idx=l)
            for l in range(layers)]
    q_nope = [torch.randn(b, h, nope, generator=gen, device=device).to(torch.bfloat16)
              for _ in range(layers)]
    q_pe = [torch.randn(b, h, rope, generator=gen, device=device).to(torch.bfloat16)
            for _ in range(layers)]
    row = [torch.randn(b, 1, 1, rank + rope if latent else nope + rope, generator=gen,
                       device=device).to(torch.bfloat16) for _ in range(layers)]
    if latent:
        q = [torch.cat([torch.bmm(qn.transpose(0, 1).contiguous(), wk).transpose(0, 1), qp],
                       -1).contiguous() for qn, qp, wk in zip(q_nope, q_pe, w_uk)]
        keys = row
        vals = [None] * layers
    else:
        q = [torch.cat([qn, qp], -1).contiguous() for qn, qp in zip(q_nope, q_pe)]
        keys = [torch.randn(b, h, 1, nope + rope, generator=gen, device=device).to(
            torch.bfloat16) for _ in range(layers)]
        vals = [torch.randn(b, h, 1, dv, generator=gen, device=device).to(torch.bfloat16)
                for _ in range(layers)]
    ws = cache.__dict__.setdefault('_nfa_selector_workspace', {})
    req_ids = list(range(b))
    outs = [None] * layers

    def sel_all():
        for layer in range(layers):
            select_topk_for_layer_batched(
                cache, layer, req_ids, q[layer], attention=attn[layer],
                decode_write=(keys[layer], vals[layer],
                              cache.slot_mapping_for_layer(layer)[:b]))

    def att_all():
        for layer in range(layers):
            if latent:
                # each head's value up-projection fused into the kernel
                outs[layer] = sparse_mla_attention_gather(
                    cache.layers[layer], q[layer], cache.gather_indices_for_layer(layer),
                    cache.visible_lens_for_layer(layer), cache.query_to_req_buf,
                    scale=scale, workspace=ws, w_uv=w_uv[layer])
            else:
                outs[layer] = sparse_paged_attention_gather(
                    cache.layers[layer], q[layer], cache.gather_indices_for_layer(layer),
                    cache.visible_lens_for_layer(layer), cache.query_to_req_buf,
                    scale=scale, workspace=ws)

    def plan():
        cache.new_step(req_ids)
        cache.plan_common(req_ids)

    w = SimpleNamespace(q=q)
    print(f'# MLA ({mode}) workload ready: {layers} layers, {b} x {ctx} tokens',
          file=sys.stderr, flush=True)
    kt = _time_graphs(torch, sel_all, att_all, layers, args.kernel_rounds, plan, cache,
                      req_ids)
    if args.timeline:
        selector_timeline(torch, SimpleNamespace(cache=cache, q=q, req_ids=req_ids,
                                                 attn=attn, kn=keys, vn=vals),
                          args.timeline, plan)
    nbytes = mla_algorithmic_bytes(mode, kt['lengths'])
    arena = cache.layers[0].kv_pool_k.numel() * 2 + (
        0 if latent else cache.layers[0].kv_pool_v.numel() * 2)
    stats, side = stats_side_bytes(cache)
    sel_gbs = nbytes['select'] / (kt['select_us_median'] * 1e-6) / 1e9
    att_gbs = nbytes['attention'] / (kt['attention_us_median'] * 1e-6) / 1e9
    layer_us = kt['select_us_median'] + kt['attention_us_median']
    tokens = cache.layers[0].max_physical_pages * page
    result = {
        'metric': 'MLA sparse-attn decode layer µs (DeepSeek-V2-Lite, batch 4 x 64K)',
        'value': round(layer_us, 3), 'unit': 'µs per layer (selector + attention)',
        'n_gpus': 1, 'steps': args.kernel_rounds, 'warmup': args.kernel_rounds,
        'ms_per_step': round(layer_us * layers / 1000.0, 4),
        'higher_is_better': False, 'scaling': 'weak', 'vs_baseline': None,
        'dtype': 'bf16', 'data': 'synthetic',
        'config': {
            'workload': f'DeepSeek-V2-Lite MLA decode layer ({mode}): 16 heads, '
                        f'latent {rank} + {rope}, nope {nope}, v {dv}, batch {b} x '
                        f'{ctx} tokens, page 16, 4-bit L2 keys on the {rope} RoPE dims, '
                        f'{layers} layers with their own arenas, hipGraph',
            'mla': mode, 'layers': layers, 'batch': b, 'context': ctx,
            'select_us': round(kt['select_us_median'], 3),
            'attention_us': round(kt['attention_us_median'], 3),
            'select_bytes': nbytes['select'], 'attention_bytes': nbytes['attention'],
            'attention_gbs': round(att_gbs, 1),
            'layer_hbm_frac': round((nbytes['select'] + nbytes['attention'])
                                    / (layer_us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
            'arena_bytes_per_token': arena // tokens,
            'arena_bytes_per_layer': arena,
            'page_stats_bytes_per_layer': stats,
            'l2_side_bytes_per_layer': side,
            'attention_includes': ('the latent kernel with the W_uv up-projection fused'
                                   if latent else 'the gather attention kernel'),
        },
        'roofline': {
            'bound': 'hbm', 'kernel': 'nfa_select_layer (nfa_select_kernel)',
            'achieved': round(sel_gbs, 1), 'peak': HBM_PEAK_GBS, 'unit': 'GB/s',
            'frac': round(sel_gbs / HBM_PEAK_GBS, 4), 'traffic': None,
        },
        'cpu_baseline': None,
    }
    print(json.dumps(result), flush=True)
    del w


def stats_side_bytes(cache, layer=0):
    """Bytes of one layer's persistent page statistics (min, max, mean and
    the fp32 running sums) and of its L2 side cache (raw L2 dims, or 4-bit
    codes with scale and zero)."""
    stats = side = 0
    for key, (st, sd) in getattr(cache, '_nfa_page_stats_persistent', {}).items():
        if key[0] != layer:
            continue
        stats += sum(t.numel() * t.element_size() for t in st)
        if sd is not None:
            side += sd.numel() * sd.element_size()
    return stats, side


def _time_graphs(torch, sel_all, att_all, layers, rounds, plan, cache, req_ids):
    """Median per-launch µs of a selector-only and an attention-only graph of
    one launch per layer (HIP events on the replaying stream, lengths
    advancing between replays as in decode)."""
    plan()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        sel_all()
        att_all()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g_sel, g_att = torch.cuda.CUDAGraph(), torch.cuda.CUDAGraph()
    with torch.cuda.graph(g_sel):
        sel_all()
    with torch.cuda.graph(g_att):
        att_all()
    cache.commit_step()
    for _ in range(rounds):
        plan()
        g_sel.replay()
        g_att.replay()
        cache.commit_step()
    torch.cuda.synchronize()
    sel, att, lengths = [], [], []
    marks = [(a, b, torch.cuda.Event(enable_timing=True))
             for a, b in warm_events(torch, rounds)]
    for m in marks:
        m[2].record()
    torch.cuda.synchronize()
    for a, b, c in marks:
        plan()
        lengths = [int(cache.pending_lengths[r]) for r in req_ids]
        a.record()
        g_sel.replay()
        b.record()
        g_att.replay()
        c.record()
        cache.commit_step()
        c.synchronize()
        sel.append(a.elapsed_time(b) * 1000.0 / layers)
        att.append(b.elapsed_time(c) * 1000.0 / layers)
    sel.sort()
    att.sort()
    return dict(select_us_median=sel[len(sel) // 2],
                attention_us_median=att[len(att) // 2], lengths=lengths)


def warm_events(torch, n):
    """``n`` pairs of timing events, each recorded once already: HIP creates
    an event at its first record, slowly for the first few hundred of a
    process, which must not happen inside a timed loop."""
    events = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
              for _ in range(n)]
    for a, b in events:
        a.record()
        b.record()
    torch.cuda.synchronize()
    return events


def hot_path_loop(torch, w, args, plan, outs):
    """The 36-layer hot path as one captured graph: ``hot_warmup`` eager
    steps (the first rebuilds the page statistics), capture, ``hot_warmup``
    untimed replays, then ``hot_steps`` timed replays with HIP events on
    the replaying stream around each.  The host planning of a step
    (plan_common, commit_step) runs while the previous replay executes."""
    for _ in range(args.hot_warmup):
        plan()
        for layer in range(args.layers):
            run_layer(w, layer, outs)
        w.cache.commit_step()
    torch.cuda.synchronize()
    plan()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        for layer in range(args.layers):  # warm the capture stream
            run_layer(w, layer, outs)
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for layer in range(args.layers):
            run_layer(w, layer, outs)
    w.cache.commit_step()
    for _ in range(args.hot_warmup):
        plan()
        graph.replay()
        w.cache.commit_step()
    torch.cuda.synchronize()
    print('# hot-path graph captured and warm', file=sys.stderr, flush=True)
    events = warm_events(torch, args.hot_steps)
    t0 = time.perf_counter()
    for a, b in events:
        plan()
        a.record()
        graph.replay()
        b.record()
        w.cache.commit_step()
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3 / args.hot_steps
    dev = sorted(a.elapsed_time(b) for a, b in events)
    med = dev[len(dev) // 2]
    print(f'# hot path: {med:.3f} ms per step (device median), {wall_ms:.3f} ms '
          'wall', file=sys.stderr, flush=True)
    return graph, dict(ms_per_step_median=med, wall_ms_per_step=wall_ms,
                       ms_p10_p90=[dev[len(dev) // 10], dev[(len(dev) * 9) // 10]])


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({'error': 'this hot path runs on one GPU; '
                                   f'--gpus {args.gpus} is not supported'}))
        sys.exit(2)
    single = args.batch == 1 and not args.ragged
    cpu = None
    if not args.no_cpu_baseline and single and not args.e2e_only \
            and args.copy_calibration == 0 and args.gather_calibration == 0 \
            and not args.mla:
        # before torch or HIP start: the baseline forks worker processes
        print('# cpu baseline ...', file=sys.stderr, flush=True)
        cpu = cpu_baseline(seed=args.seed)
        print(f'# cpu baseline: {cpu["value"]} us per layer', file=sys.stderr, flush=True)
    import torch
    from sparse_attn import _native
    if not os.path.exists(_native.LIB_PATH):
        import __graft_entry__
        __graft_entry__.build()
    device = torch.device('cuda:0')
    torch.cuda.set_device(device)
    if args.copy_calibration > 0:
        n = args.copy_calibration << 20
        src = torch.ones(n // 4, dtype=torch.float32, device=device)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({'copy_bytes_read': n, 'copy_bytes_written': n,
                          'launches': 3}), flush=True)
        return
    if args.gather_calibration > 0:
        n = args.gather_calibration << 20
        src = torch.ones(n // 4, dtype=torch.float32, device=device)
        gen = torch.Generator(device=device).manual_seed(args.seed)
        out = {}
        for name, row_bytes in (('gather_1k', 1024), ('gather_64b', 64)):
            rows = src.view(-1, row_bytes // 4)
            idx = torch.randperm(rows.shape[0], generator=gen, device=device)[
                :rows.shape[0] // 4].contiguous()
            torch.cuda.synchronize()
            for _ in range(3):
                got = rows.index_select(0, idx)
            torch.cuda.synchronize()
            out[name] = {'rows': int(idx.numel()), 'row_bytes': row_bytes,
                         'bytes_read': int(idx.numel()) * row_bytes,
                         'bytes_written': int(got.numel()) * 4,
                         'index_bytes': int(idx.numel()) * 8, 'launches': 3}
            del got, idx
        print(json.dumps(out), flush=True)
        return
    if args.mla:
        mla_layer_bench(torch, args, device)
        return
    if args.e2e_only:
        e2e = end_to_end(torch, args, device)
        print(json.dumps({
            'metric': 'e2e decode tok/s at 128K ctx', 'value': e2e['tok_s'],
            'unit': 'tok/s', 'n_gpus': 1, 'steps': args.steps, 'warmup': args.warmup,
            'ms_per_step': e2e['tpot_ms_median'], 'higher_is_better': True,
            'scaling': 'weak', 'vs_baseline': None, 'dtype': 'bf16',
            'data': 'synthetic', 'config': {'workload': 'whole-model decode', **e2e},
        }), flush=True)
        return
    t_setup = time.perf_counter()
    w = build_workload(torch, args, device)
    cache = w.cache
    outs = [None] * args.layers
    print(f'# workload ready in {time.perf_counter() - t_setup:.1f}s', file=sys.stderr,
          flush=True)

    def plan():
        cache.new_step(w.req_ids)
        cache.plan_common(w.req_ids)

    graph, hot = hot_path_loop(torch, w, args, plan, outs)
    if args.timeline:
        selector_timeline(torch, w, args.timeline, plan)
    # per-kernel durations (events around each launch), same stream
    kt = time_kernels(torch, w, args.kernel_rounds, plan)
    per_req = [algorithmic_bytes(w, n) for n in kt['lengths']]
    nbytes = {k: sum(b[k] for b in per_req) for k in ('select', 'attention')}
    sel_gbs = nbytes['select'] / (kt['select_us_median'] * 1e-6) / 1e9
    att_gbs = nbytes['attention'] / (kt['attention_us_median'] * 1e-6) / 1e9
    layer_us = hot['ms_per_step_median'] * 1e3 / args.layers
    layer_gbs = (nbytes['select'] + nbytes['attention']) / (layer_us * 1e-6) / 1e9
    hot_tok_s = args.batch * 1e3 / hot['ms_per_step_median']
    geometry = {'heads': [w.hq, w.hkv], 'head_dim': w.d, 'page': w.page}
    lengths = list(w.lengths)
    stats_bytes, side_bytes = stats_side_bytes(cache)
    e2e = None
    if not args.no_e2e:
        del graph, w, cache, outs
        torch.cuda.synchronize()
        torch.cuda.empty_cache()
        e2e = (end_to_end(torch, args, device) if single
               else end_to_end_batch(torch, args, device, lengths))

    if e2e is not None and single:
        value, ms_per_step = e2e['tok_s'], e2e['tpot_ms_median']
        steps, warmup = args.steps, args.warmup
        headline = ('whole-model decode: random-init bf16 Qwen3-8B, dense prefill '
                    f'of {args.ctx} tokens, median TPOT over {steps} greedy steps '
                    'replayed from a hipGraph; hot path = selector + attention of '
                    f'{args.layers} layers')
    elif e2e is not None:
        value, ms_per_step = e2e['tok_s'], e2e['step_ms_median']
        steps, warmup = args.steps, args.warmup
        headline = (f'whole-model decode of {args.batch} ragged requests: random-init '
                    'bf16 Llama-3.1-8B, one dense prefill per prompt, median step '
                    f'time over {steps} greedy steps of the whole batch replayed from '
                    f'a hipGraph, tok/s = {args.batch} / step; hot path = selector + '
                    f'attention of {args.layers} layers')
    else:
        value, ms_per_step = hot_tok_s, hot['ms_per_step_median']
        steps, warmup = args.hot_steps, args.hot_warmup
        headline = (f'hot path only: selector + attention of {args.layers} layers '
                    'per decode token, median device time per graph replay')
    result = {
        'metric': 'sparse-attn decode layer µs + e2e decode tok/s at 128K '
                  'ctx; % of HBM peak',
        'value': round(value, 2),
        'unit': 'tok/s',
        'n_gpus': 1,
        'steps': steps,
        'warmup': warmup,
        'ms_per_step': round(ms_per_step, 4),
        'higher_is_better': True,
        'scaling': 'weak',
        'vs_baseline': None,
        'dtype': 'bf16',
        'data': 'synthetic',
        'config': {
            'workload': f'NFA sparse-attention decode, 32/8 heads, head_dim 128 '
                        f'(Qwen3-8B and Llama-3.1-8B attention geometry), '
                        f'batch {args.batch}, '
                        + (f'contexts U({args.ragged[0]}, {args.ragged[1]})'
                           if args.ragged else f'{args.ctx // 1024}K context')
                        + ', page 16, hipGraph',
            'value_is': headline,
            'layers': args.layers, 'batch': args.batch,
            'operator_mode': args.operator_mode, 'l2_keys': '4-bit' if args.l2_quant
                                                          else 'bf16',
            'context': (lengths if args.ragged else args.ctx),
            **geometry,
            'nfa': 'far minmax / near avg, K1 128 (32 near), near_len 4096, '
                   'tail dims cmp 4, sink 4, SWA 128, K2 1024',
            'layer_us': round(layer_us, 3),
            'layer_hbm_frac': round(layer_gbs / HBM_PEAK_GBS, 4),
            'hot_path_ms_per_step': round(hot['ms_per_step_median'], 4),
            'hot_path_wall_ms_per_step': round(hot['wall_ms_per_step'], 4),
            'hot_path_ms_p10_p90': [round(x, 4) for x in hot['ms_p10_p90']],
            'hot_path_tok_s': round(hot_tok_s, 2),
            'hot_path_steps': args.hot_steps,
            'select_us': round(kt['select_us_median'], 3),
            'attention_us': round(kt['attention_us_median'], 3),
            'select_bytes': nbytes['select'],
            'attention_bytes': nbytes['attention'],
            'attention_gbs': round(att_gbs, 1),
            # persistent per-layer memory besides the KV arena (all request
            # slots): page statistics and the L2 side cache (--l2-quant: 4-bit)
            'page_stats_bytes_per_layer': stats_bytes,
            'l2_side_bytes_per_layer': side_bytes,
            'parallelism': 'single GPU',
        },
        'roofline': {
            'bound': 'hbm',
            'kernel': 'nfa_select_layer (nfa_select_kernel)',
            'achieved': round(sel_gbs, 1),
            'peak': HBM_PEAK_GBS,
            'unit': 'GB/s',
            'frac': round(sel_gbs / HBM_PEAK_GBS, 4),
            'traffic': measured_traffic(args),
        },
        'cpu_baseline': cpu,
        'e2e': e2e,
    }
    print(json.dumps(result), flush=True)


if __name__ == '__main__':
    main()
