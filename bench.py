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

One step = one decode token through the hot path of all 36 layers: the
selector (fused decode K/V write, page statistics, L1, L2, union) and the
sparse gather attention, captured once into a hipGraph and replayed, with
the host-side step planning (plan_common / commit_step) in the timed loop.
Dense projections and the MLP are outside this hot path.

Prints one JSON line (see ``_result``); ``--gpus`` above 1 is refused: this
path runs on one GPU.
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
    ap.add_argument('--steps', type=int, default=200)
    ap.add_argument('--warmup', type=int, default=30)
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
    ap.add_argument('--kernel-rounds', type=int, default=20)
    ap.add_argument('--cpu-seconds', type=float, default=15.0,
                    help='budget of the CPU oracle baseline sample')
    ap.add_argument('--no-cpu-baseline', action='store_true')
    ap.add_argument('--seed', type=int, default=20261201)
    ap.add_argument('--timeline', type=int, default=0,
                    help='print selector phase timings of N extra decode steps')
    ap.add_argument('--e2e-steps', type=int, default=256,
                    help='also run the whole Qwen3-8B-geometry model (random-init '
                         'bf16): dense prefill of --ctx tokens, then this many '
                         'greedy decode steps replayed from a hipGraph; 0 = off')
    ap.add_argument('--e2e-unfused', action='store_true',
                    help='end-to-end decode with HF\'s own dense layers (only the '
                         'attention patched)')
    ap.add_argument('--e2e-only', action='store_true',
                    help='run only the end-to-end model decode')
    ap.add_argument('--copy-calibration', type=int, default=0, metavar='MIB',
                    help='only copy a MIB-MiB device buffer three times (the '
                         'known-size kernel that scales rocprofv3 FETCH_SIZE '
                         'and WRITE_SIZE readings) and exit')
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
    new_tokens = args.warmup + args.steps + args.kernel_rounds + args.timeline + 8
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


def measured_traffic(args):
    """HBM bytes per selector launch at this workload, from the committed
    rocprofv3 FETCH_SIZE / WRITE_SIZE summary (None when absent or when the
    workload differs from the profiled one)."""
    if args.ctx != 131072 or args.batch != 1 or args.ragged:
        return None
    path = os.path.join(ROOT, 'profiles', 'nfa_select_layer_128k_hbm_traffic.md')
    try:
        with open(path) as f:
            text = f.read()
    except OSError:
        return None
    m = re.search(r'traffic_bytes_per_launch: (\d+)', text)
    return int(m.group(1)) if m else None


def _oracle_cfg(w):
    """Oracle configuration of the workload (CPU baseline leg only)."""
    from oracle import nfa_oracle as orc
    import numpy as np
    import torch
    cache = w.cache
    dims = w.indexer._subspace_indices(torch.device('cpu')).numpy()
    return orc.NfaConfig(
        hq=w.hq, hkv=w.hkv, head_dim=w.d, head_dim_v=w.d, bs=16, page=w.page,
        max_blocks=cache.max_blocks, geo_sink=4, geo_near=4096, geo_window=128,
        sink_tokens=4, swa=128, near_len=4096, k1=128, near_pages=32, k2=1024,
        dims=np.asarray(dims), fine_dims=np.asarray(dims), scale=w.d ** -0.5)


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
    torch.cuda.synchronize()
    sel, att = [], []
    lengths = []
    for _ in range(rounds):
        plan()
        lengths = [int(cache.pending_lengths[r]) for r in w.req_ids]
        a, b, c = (torch.cuda.Event(enable_timing=True) for _ in range(3))
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
        names = ['row scalars', 'q prep', 'page stats', 'L1 scores+publish']
        for k, name in enumerate(names):
            d = (tile[:, :, k + 1] - tile[:, :, k]) * us
            acc.setdefault(f'A tile {name} (max)', []).append(d.max())
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


def end_to_end(torch, args, device):
    """Whole-model decode: random-init bf16 Qwen3-8B, dense prefill of
    ``args.ctx`` seeded uniform token ids into the paged cache, 3 warm-up
    steps, then ``args.e2e_steps`` greedy steps replayed from one captured
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

    warm = 3
    new_tokens = warm + args.e2e_steps + 8
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
        events = [(torch.cuda.Event(enable_timing=True),
                   torch.cuda.Event(enable_timing=True))
                  for _ in range(args.e2e_steps)]
        t0 = time.perf_counter()
        for i, (a, b) in enumerate(events):
            a.record()
            runner.step(model, cache, generated_counts=warm + i + 1)
            b.record()
        torch.cuda.synchronize()
        wall_ms = (time.perf_counter() - t0) * 1e3 / args.e2e_steps
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
        'decode_steps': args.e2e_steps, 'warmup_steps': warm,
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


def cpu_baseline(torch, w, seconds):
    """The CPU oracle on a bounded sample: layer-0 decode steps at the same
    128K context, single-threaded numpy."""
    import numpy as np
    from oracle import nfa_oracle as orc
    try:
        from threadpoolctl import threadpool_limits
    except Exception:  # pragma: no cover
        threadpool_limits = None
    cache = w.cache
    cfg = _oracle_cfg(w)
    layer = cache.layers[0]
    k_pool = layer.kv_pool_k.float().cpu().numpy()
    v_pool = layer.kv_pool_v.float().cpu().numpy()
    bt = cache.block_table_buf[0].cpu().numpy().astype(np.int64)
    length = int(cache.states[0].logical_length) + 1
    q = w.q[0].float().cpu().numpy()
    q2r = np.zeros(1, dtype=np.int64)
    ctx = threadpool_limits(1) if threadpool_limits else None
    if ctx is not None:
        ctx.__enter__()
    try:
        n = 0
        t0 = time.perf_counter()
        while True:
            res = orc.select_layer(cfg, k_pool, bt, np.array([length]),
                                   np.array([0]), np.array([True]), np.zeros(1),
                                   np.zeros(1), q, 1024)
            gather = np.zeros((1, w.hkv, 1024), dtype=np.int64)
            vis = np.zeros((1, w.hkv), dtype=np.int64)
            for kv in range(w.hkv):
                r = res[0][kv]
                gather[0, kv, :len(r.gather)] = r.gather
                vis[0, kv] = r.vis_len
            orc.sparse_attention(k_pool, v_pool, q, gather, vis, q2r,
                                 cfg.scale, w.page)
            n += 1
            elapsed = time.perf_counter() - t0
            if elapsed >= seconds or n >= 100:
                break
    finally:
        if ctx is not None:
            ctx.__exit__(None, None, None)
    layer_s = elapsed / n
    return dict(value=1.0 / (layer_s * len(w.q)), unit='tok/s', cores=1,
                kind='port',
                sample=f'{n} single-layer decode steps (selector + attention) '
                       f'of the same 128K workload on the numpy oracle, '
                       f'{layer_s * 1e3:.1f} ms per layer, scaled to '
                       f'{len(w.q)} layers per token')


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({'error': 'this hot path runs on one GPU; '
                                   f'--gpus {args.gpus} is not supported'}))
        sys.exit(2)
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
    if args.e2e_only:
        steps = args.e2e_steps or 256
        args.e2e_steps = steps
        e2e = end_to_end(torch, args, device)
        print(json.dumps({
            'metric': 'e2e decode tok/s at 128K ctx', 'value': e2e['tok_s'],
            'unit': 'tok/s', 'n_gpus': 1, 'steps': steps, 'warmup': 3,
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

    # warm-up: first step rebuilds page statistics, later ones are incremental
    for _ in range(args.warmup):
        plan()
        for layer in range(args.layers):
            run_layer(w, layer, outs)
        cache.commit_step()
    torch.cuda.synchronize()

    # capture one decode step of all layers
    plan()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        for layer in range(args.layers):  # warm the capture stream
            run_layer(w, layer, outs)
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    with torch.cuda.graph(graph):
        for layer in range(args.layers):
            run_layer(w, layer, outs)
    cache.commit_step()
    torch.cuda.synchronize()
    print('# graph captured', file=sys.stderr, flush=True)

    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        plan()
        graph.replay()
        cache.commit_step()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    ms_per_step = elapsed * 1e3 / args.steps
    print(f'# timed {args.steps} steps: {ms_per_step:.3f} ms/step', file=sys.stderr,
          flush=True)

    if args.timeline:
        selector_timeline(torch, w, args.timeline, plan)
    # per-kernel durations (events around each launch), same stream
    kt = time_kernels(torch, w, args.kernel_rounds, plan)
    per_req = [algorithmic_bytes(w, n) for n in kt['lengths']]
    nbytes = {k: sum(b[k] for b in per_req) for k in ('select', 'attention')}
    sel_gbs = nbytes['select'] / (kt['select_us'] * 1e-6) / 1e9
    att_gbs = nbytes['attention'] / (kt['attention_us'] * 1e-6) / 1e9
    layer_us = ms_per_step * 1e3 / args.layers
    layer_gbs = (nbytes['select'] + nbytes['attention']) / (layer_us * 1e-6) / 1e9

    single = args.batch == 1 and not args.ragged
    cpu = None
    if not args.no_cpu_baseline and single:
        print('# cpu baseline ...', file=sys.stderr, flush=True)
        cpu = cpu_baseline(torch, w, args.cpu_seconds)
    geometry = {'heads': [w.hq, w.hkv], 'head_dim': w.d, 'page': w.page}
    lengths = list(w.lengths)
    e2e = None
    if args.e2e_steps > 0 and single:
        del graph, w, cache, outs
        torch.cuda.synchronize()
        torch.cuda.empty_cache()
        e2e = end_to_end(torch, args, device)

    result = {
        'metric': 'sparse-attn decode layer µs + e2e decode tok/s at 128K '
                  'ctx; % of HBM peak',
        'value': round(args.batch * 1e3 / ms_per_step, 2),
        'unit': 'tok/s',
        'n_gpus': 1,
        'steps': args.steps,
        'warmup': args.warmup,
        'ms_per_step': round(ms_per_step, 4),
        'higher_is_better': True,
        'scaling': 'weak',
        'vs_baseline': None,
        'dtype': 'bf16',
        'data': 'synthetic',
        'config': {
            'workload': f'NFA sparse-attention decode hot path (selector + '
                        f'attention) of {args.layers} layers, Qwen3-8B attention '
                        f'geometry, batch {args.batch}, '
                        + (f'contexts U({args.ragged[0]}, {args.ragged[1]})'
                           if args.ragged else f'{args.ctx // 1024}K context')
                        + ', page 16, hipGraph',
            'layers': args.layers, 'batch': args.batch,
            'operator_mode': args.operator_mode, 'l2_keys': '4-bit' if args.l2_quant
                                                          else 'bf16',
            'context': (lengths if args.ragged else args.ctx),
            **geometry,
            'nfa': 'far minmax / near avg, K1 128 (32 near), near_len 4096, '
                   'tail dims cmp 4, sink 4, SWA 128, K2 1024',
            'layer_us': round(layer_us, 3),
            'layer_hbm_frac': round(layer_gbs / HBM_PEAK_GBS, 4),
            'select_us': round(kt['select_us'], 3),
            'attention_us': round(kt['attention_us'], 3),
            'select_bytes': nbytes['select'],
            'attention_bytes': nbytes['attention'],
            'attention_gbs': round(att_gbs, 1),
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
