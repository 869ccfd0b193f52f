"""Absorbed multi-head latent attention (DeepSeek-V2 MLA) on the GPU.

The latent arena holds one row per token, [kv_a_layernorm(c) | k_pe], shared
by every head; each query head selects on the RoPE dims and attends in the
latent space.  Pinned two ways:

* selections: the kernel's per-head selections over the shared rows against
  the oracle's expanded heads (every head holding the same k_pe, as
  transformers' expand_kv builds them) -- bit-exact: far/near score bits,
  I_F / I_N, candidates and logits, middle, gather rows and visible lengths;
  and against the selections of the expanded arena of the same data;
* attention: ``nfa_mla_attn_decode`` against the float64 latent oracle
  (itself pinned against the expanded attention in test_oracle_pinning.py),
  and the up-projected result against the float64 attention over the
  expanded heads (rtol 2e-2 / atol 2e-3 in bf16).

Cases: the kernel alone (value dims 64 and 512, padding rows, empty and
ragged rows, negative slots, bf16 and fp32 outputs); a 20000 + 9000-token
batch at DeepSeek-V2-Lite's 16 heads and 512 + 64 latent rows, with raw and
4-bit L2 keys and an incremental production step; the DeepSeek-V2-Lite layer
of the benchmark (4 requests x 65536 tokens, 4-bit L2 keys on the 64 RoPE
dims) through both arenas; and a tiny random-init DeepSeek-V2 patched with
``mla='absorbed'`` against the same model patched with the expanded heads.
"""
import copy
from contextlib import contextmanager

import numpy as np
import pytest
import torch

from nfa_case import (GPU, attention_ns, bf16_randn, cfg_from, make_indexer,
                      run_and_compare, run_oracle, snapshot)
from oracle import nfa_oracle as orc
from sparse_attn.cache import GraphReadyPagedRegionCache
from sparse_attn.indexer.nfa_layer_batch_selector import \
    select_topk_for_layer_batched
from sparse_attn.ops.paged_region_kernels import (sparse_mla_attention_gather,
                                                  sparse_paged_attention_gather)
from sparse_attn.policies.region_geometry import RegionGeometry

pytestmark = pytest.mark.gpu

GEO = RegionGeometry(sink=4, near=4096, window=128, page=16, max_new_tokens=64)
HEADS, RANK, ROPE, NOPE, VDIM = 16, 512, 64, 128, 128
SCALE = (NOPE + ROPE) ** -0.5


def _latent_cache(lengths, *, heads=HEADS, rank=RANK, rope=ROPE, seed=20261201,
                  rows_fn=None):
    page = GEO.page
    extra = GEO.max_new_tokens
    max_blocks = (max(lengths) + extra + page - 1) // page + 8
    phys = sum((n + extra + page - 1) // page for n in lengths) + 8
    cache = GraphReadyPagedRegionCache(
        1, GEO, max_requests=len(lengths), max_physical_pages=phys,
        max_blocks=max_blocks, max_visible_len=1024,
        max_query_tokens=max(8, len(lengths)), num_kv_heads=1,
        num_query_heads=heads, head_dim_k=rank + rope, head_dim_v=rank,
        dtype=torch.bfloat16, device=GPU, latent=True)
    gen = torch.Generator(device=GPU).manual_seed(seed)
    for rid, n in enumerate(lengths):
        cache.add_request(rid)
        rows = (rows_fn(rid, n) if rows_fn is not None
                else bf16_randn((1, 1, n, rank + rope), gen, GPU))
        cache.write_prefill(0, rid, rows.to(torch.bfloat16), None)
        cache.freeze(rid, [False], [False])
    return cache, gen, list(range(len(lengths)))


def _decode_rows(cache, b, gen):
    d = cache.layers[0].head_dim_k
    keys = bf16_randn((b, 1, 1, d), gen, GPU)
    slots = cache.slot_mapping_for_layer(0)[:b].clone()
    return keys, None, slots


# ---------------------------------------------------------------------------
# the attention kernel
# ---------------------------------------------------------------------------

@pytest.mark.parametrize('rank,out_dtype,project', [
    (512, torch.bfloat16, False), (512, torch.float32, False), (64, torch.float32, False),
    (512, torch.float32, True), (512, torch.bfloat16, True), (64, torch.float32, True)])
def test_mla_attention_kernel_matches_oracle(rank, out_dtype, project):
    """The latent kernel against the float64 latent oracle; with ``project``
    the head-wise value up-projection (128 rows of ``rank`` dims per head)
    fused into its last step, against the oracle's result projected in
    float64."""
    gen = torch.Generator(device=GPU).manual_seed(rank)
    page, pages, heads, rows, width = 16, 300, HEADS, 3, 1024
    cache = GraphReadyPagedRegionCache(
        1, GEO, max_requests=rows, max_physical_pages=pages, max_blocks=64,
        max_visible_len=width, max_query_tokens=8, num_kv_heads=1,
        num_query_heads=heads, head_dim_k=rank + 64, head_dim_v=rank,
        dtype=torch.bfloat16, device=GPU, latent=True)
    layer = cache.layers[0]
    layer.kv_pool_k.copy_(bf16_randn(layer.kv_pool_k.shape, gen, GPU))
    total = pages * page
    gather = torch.stack([torch.randperm(total, generator=gen, device=GPU)[:width]
                          for _ in range(rows * heads)]).view(rows, heads, width)
    gather = gather.to(torch.int32)
    gather[1, 3, 5] = -1                      # a negative slot is skipped
    vis = torch.randint(1, width + 1, (rows, heads), generator=gen, device=GPU)
    vis[0, 0] = 0                             # an empty row
    vis[2, 7] = width
    vis = vis.to(torch.int32).contiguous()
    q2r = torch.tensor([2, -1, 0, 1], dtype=torch.int32, device=GPU)  # a padding row
    q = (torch.randn(4, heads, rank + 64, generator=gen, device=GPU) * 0.05).to(torch.bfloat16)
    w_uv = None
    if project:
        w_uv = (torch.randn(heads, VDIM, rank, generator=gen, device=GPU)
                * rank ** -0.5).to(torch.bfloat16)
    print(f'# mla attention rank={rank} out={out_dtype} project={project}', flush=True)
    out = sparse_mla_attention_gather(layer, q, gather.contiguous(), vis, q2r,
                                      scale=SCALE, out_dtype=out_dtype, w_uv=w_uv)
    torch.cuda.synchronize()
    want = orc.mla_sparse_attention(layer.kv_pool_k.float().cpu().numpy(),
                                    q.float().cpu().numpy(), gather.cpu().numpy(),
                                    vis.cpu().numpy(), q2r.cpu().numpy(), SCALE, page,
                                    rank)
    if project:
        want = np.einsum('thr,hvr->thv', want, w_uv.double().cpu().numpy())
    got = out.float().cpu().numpy()
    assert (got[1] == 0).all()
    if out_dtype == torch.bfloat16:
        np.testing.assert_allclose(got, want, rtol=2e-2, atol=2e-3)
    else:
        np.testing.assert_allclose(got, want, rtol=1e-4, atol=1e-5)


# ---------------------------------------------------------------------------
# latent selections vs the oracle's expanded heads
# ---------------------------------------------------------------------------

@pytest.mark.parametrize('l2_quant', [False, True])
def test_latent_selection_matches_expanded_oracle(l2_quant):
    """20000 + 9000 tokens, 16 heads, 512 + 64 latent rows: the rebuild step
    with every debug output, then an incremental step through the
    production launch."""
    cache, gen, req_ids = _latent_cache([20000, 9000])
    indexer = make_indexer(subspace='mla_rope', l2_quant=l2_quant)
    for step in range(2):
        cache.new_step(req_ids)
        cache.plan_common(req_ids)
        q = bf16_randn((2, HEADS, RANK + ROPE), gen, GPU, scale=0.1)
        decode = _decode_rows(cache, 2, gen)
        plan = {}
        res = run_and_compare(cache, indexer, req_ids, q, decode, scaling=SCALE,
                              check_debug=step == 0, plan=plan)
        assert all(res[r][h].vis_len == 1024 for r in range(2) for h in range(HEADS))
        # the decode row was written once (selection row 0), keys only
        print(f'# latent selection step {step + 1} (4-bit {l2_quant}): bit-exact',
              flush=True)
        cache.commit_step()


def _dsv2_lite_data(lengths, seed):
    """DeepSeek-V2-Lite-shaped latent data: c (512, RMS-normalised scale),
    k_pe (64, N(0,1) x per-channel LogNormal(0,1) with RoPE), the
    kv_b_proj halves W_uk [16, 128, 512] and W_uv [16, 128, 512]."""
    from bench import synthetic_keys
    gen = torch.Generator(device=GPU).manual_seed(seed)
    data = []
    for n in lengths:
        c = torch.randn(n, RANK, generator=gen, device=GPU).to(torch.bfloat16)
        k_pe = synthetic_keys(torch, n, 1, ROPE, gen, GPU, dtype=torch.float32)
        data.append((c, k_pe[0, 0].to(torch.bfloat16)))
    w = (torch.randn(HEADS * (NOPE + VDIM), RANK, generator=gen, device=GPU)
         * RANK ** -0.5).to(torch.bfloat16)
    wv = w.view(HEADS, NOPE + VDIM, RANK)
    return data, wv[:, :NOPE].contiguous(), wv[:, NOPE:].contiguous(), gen


def test_dsv2_lite_layer_4_requests_64k_latent_and_expanded():
    """The benchmark's DeepSeek-V2-Lite layer: 4 requests of 65536 tokens, 16
    heads, 512 + 64 latent rows, 4-bit L2 keys on the 64 RoPE dims.  The
    latent arena's selections are the oracle's (bit-exact, every debug
    output) and the expanded arena's (same logical ids per head); both
    attentions match the float64 attention over the expanded heads."""
    lengths = [65536] * 4
    data, w_uk, w_uv, gen = _dsv2_lite_data(lengths, 4)
    lat, _, req_ids = _latent_cache(
        lengths, rows_fn=lambda rid, n: torch.cat(data[rid], dim=-1)[None, None])
    # the expanded arena of the same tokens (transformers' expand_kv in bf16),
    # same page budget: both arenas hand out the same physical pages
    page = GEO.page
    exp = GraphReadyPagedRegionCache(
        1, GEO, max_requests=4, max_physical_pages=lat.layers[0].max_physical_pages,
        max_blocks=lat.max_blocks, max_visible_len=1024, max_query_tokens=8,
        num_kv_heads=HEADS, num_query_heads=HEADS, head_dim_k=NOPE + ROPE,
        head_dim_v=VDIM, dtype=torch.bfloat16, device=GPU)
    for rid, (c, k_pe) in enumerate(data):
        exp.add_request(rid)
        k_nope = torch.einsum('nr,hdr->hnd', c.float(), w_uk.float()).to(torch.bfloat16)
        v = torch.einsum('nr,hdr->hnd', c.float(), w_uv.float()).to(torch.bfloat16)
        k = torch.cat([k_nope, k_pe[None].expand(HEADS, -1, -1)], dim=-1)
        exp.write_prefill(0, rid, k[None].contiguous(), v[None].contiguous())
        exp.freeze(rid, [False], [False])
        del k_nope, v, k
    print('# DSV2-Lite layer, 4 x 65536 tokens: latent and expanded arenas ready',
          flush=True)
    indexer = make_indexer(subspace='mla_rope', l2_quant=True)
    b = 4
    for cache in (lat, exp):
        cache.new_step(req_ids)
        cache.plan_common(req_ids)
    q_nope = torch.randn(b, HEADS, NOPE, generator=gen, device=GPU).to(torch.bfloat16)
    q_pe = torch.randn(b, HEADS, ROPE, generator=gen, device=GPU).to(torch.bfloat16)
    c_new = torch.randn(b, RANK, generator=gen, device=GPU).to(torch.bfloat16)
    k_pe_new = torch.randn(b, ROPE, generator=gen, device=GPU).to(torch.bfloat16)
    q_abs = torch.bmm(q_nope.transpose(0, 1).contiguous(), w_uk).transpose(0, 1)
    q_lat = torch.cat([q_abs, q_pe], dim=-1).contiguous()
    row = torch.cat([c_new, k_pe_new], dim=-1)[:, None, None].contiguous()
    slots = lat.slot_mapping_for_layer(0)[:b].clone()
    res, k_pool, _ = run_and_compare(lat, indexer, req_ids, q_lat, (row, None, slots),
                                     scaling=SCALE, return_pools=True, with_v=False)
    print('# DSV2-Lite latent selections: bit-exact vs the oracle', flush=True)
    # the expanded arena: the same decode token expanded per head
    k_new = torch.cat([torch.einsum('br,hdr->bhd', c_new.float(), w_uk.float()),
                       k_pe_new.float()[:, None].expand(-1, HEADS, -1)], dim=-1)
    v_new = torch.einsum('br,hdr->bhd', c_new.float(), w_uv.float())
    q_exp = torch.cat([q_nope, q_pe], dim=-1).contiguous()
    select_topk_for_layer_batched(
        exp, 0, req_ids, q_exp, attention=attention_ns(indexer, SCALE),
        decode_write=(k_new.to(torch.bfloat16)[:, :, None].contiguous(),
                      v_new.to(torch.bfloat16)[:, :, None].contiguous(),
                      exp.slot_mapping_for_layer(0)[:b].clone()))
    torch.cuda.synchronize()
    lat_g = lat.gather_indices_for_layer(0)[:b].cpu().numpy()
    exp_g = exp.gather_indices_for_layer(0)[:b].cpu().numpy()
    lat_n = lat.visible_lens_for_layer(0)[:b].cpu().numpy()
    exp_n = exp.visible_lens_for_layer(0)[:b].cpu().numpy()
    np.testing.assert_array_equal(lat_n, exp_n)
    for r in range(b):
        assert (lat.states[r].block_tables[0].physical()
                == exp.states[r].block_tables[0].physical())
        for h in range(HEADS):
            n = lat_n[r, h]
            np.testing.assert_array_equal(lat_g[r, h, :n], exp_g[r, h, :n])
    print('# DSV2-Lite expanded selections equal the latent ones', flush=True)
    # attention: both against float64 attention over the expanded heads
    # (the head-wise W_uv up-projection fused into the latent kernel)
    out_lat = sparse_mla_attention_gather(
        lat.layers[0], q_lat, lat.gather_indices_for_layer(0),
        lat.visible_lens_for_layer(0), lat.query_to_req_buf, scale=SCALE,
        out_dtype=torch.float32, w_uv=w_uv)
    out_exp = sparse_paged_attention_gather(
        exp.layers[0], q_exp, exp.gather_indices_for_layer(0),
        exp.visible_lens_for_layer(0), exp.query_to_req_buf, scale=SCALE)
    torch.cuda.synchronize()
    # the latent form against the float64 latent algebra (exact W_uv)
    want_lat = orc.mla_sparse_attention(k_pool, q_lat.float().cpu().numpy(), lat_g, lat_n,
                                        np.arange(b), SCALE, page, RANK)
    want = np.einsum('thr,hvr->thv', want_lat, w_uv.double().cpu().numpy())
    np.testing.assert_allclose(out_lat.cpu().numpy(), want, rtol=2e-2, atol=2e-3)
    del k_pool
    # the expanded heads against float64 attention over the bf16 keys and
    # values their arena holds (W_uk c and W_uv c rounded to bf16)
    want_exp = orc.sparse_attention(exp.layers[0].kv_pool_k.float().cpu().numpy(),
                                    exp.layers[0].kv_pool_v.float().cpu().numpy(),
                                    q_exp.float().cpu().numpy(), exp_g, exp_n,
                                    np.arange(b), SCALE, page)
    np.testing.assert_allclose(out_exp.float().cpu().numpy(), want_exp, rtol=2e-2, atol=2e-3)
    gap = float(np.abs(out_lat.cpu().numpy() - out_exp.float().cpu().numpy()).max())
    print(f'# DSV2-Lite attention: latent and expanded each vs float64 '
          f'(max |latent - expanded| {gap:.2e})', flush=True)


# ---------------------------------------------------------------------------
# a tiny DeepSeek-V2 patched with mla='absorbed'
# ---------------------------------------------------------------------------

@contextmanager
def _recording_selector():
    """Record, per layer, the selector's inputs: a snapshot, the query and
    the decode row (keys only on a latent arena)."""
    from sparse_attn.indexer import nfa_layer_batch_selector as selmod
    calls = {}
    real = selmod.select_topk_for_layer_batched

    def select(cache, layer_idx, req_ids, q, attention=None, decode_write=None, **kw):
        calls[layer_idx] = dict(
            snap=snapshot(cache, layer_idx, len(req_ids)), q=q.float().cpu().numpy(),
            decode=tuple(None if t is None else t.float().cpu().numpy()
                         if t.is_floating_point() else t.cpu().numpy()
                         for t in decode_write),
            scaling=attention.scaling, indexer=attention.indexer)
        return real(cache, layer_idx, req_ids, q, attention=attention,
                    decode_write=decode_write, **kw)

    selmod.select_topk_for_layer_batched = select
    try:
        yield calls
    finally:
        selmod.select_topk_for_layer_batched = real


def _prefill(model, ids, mla):
    from sparse_attn.engine.frozen_runner import prefill_frozen_request
    from sparse_attn.patches.patch import register_patch
    from test_deepseek_v2_gpu import GEO as MGEO, _args
    register_patch(model, _args(), mla=mla)
    with torch.no_grad():
        out, audit = prefill_frozen_request(model, ids, None, MGEO)
    return out, out.past_key_values, audit['request_id']


def test_tiny_dsv2_absorbed_matches_expanded():
    """Prefill writes the module's own latent rows; a decode step selects the
    expanded path's tokens in every layer and head and gives its logits up
    to rounding; graph replays equal eager steps."""
    from test_deepseek_v2_gpu import PROMPT, _tiny_dsv2
    from test_model_patch_gpu import _arena_rows
    model = _tiny_dsv2()
    ref = copy.deepcopy(model)
    ids = torch.randint(0, 1024, (1, PROMPT),
                        generator=torch.Generator().manual_seed(13)).to(GPU)
    with torch.no_grad():
        want = ref(ids, use_cache=True)
    model_e = copy.deepcopy(model)
    out_e, cache_e, rid_e = _prefill(model_e, ids, 'expanded')
    model_a = copy.deepcopy(model)
    out_a, cache_a, rid_a = _prefill(model_a, ids, 'absorbed')
    assert cache_a.latent and cache_a.num_kv_heads == 1
    assert cache_a.layers[0].head_dim_k == 64 + 64 and cache_a.selection_heads == 16
    # the same dense prefill attention over the module's expanded heads
    torch.testing.assert_close(out_a.logits[:, -1], out_e.logits[:, -1], rtol=1e-2,
                               atol=1e-5)
    for li in range(model.config.num_hidden_layers):
        k, _ = _arena_rows(cache_a, li, rid_a, PROMPT)
        layer = want.past_key_values.layers[li]
        rows = torch.cat([layer.keys[0, 0], layer.values[0, 0]], dim=-1)
        assert torch.equal(k[0], rows)
    print('# tiny DSV2 absorbed prefill: latent rows as the module computes them',
          flush=True)
    token = out_e.logits[:, -1].argmax(-1, keepdim=True)
    pos = torch.full((1, 1), PROMPT, dtype=torch.long, device=GPU)
    outs = {}
    with torch.no_grad():
        for name, mx, cache, rid in (('expanded', model_e, cache_e, rid_e),
                                     ('absorbed', model_a, cache_a, rid_a)):
            cache.new_step([rid])
            cache.plan_common([rid])
            with _recording_selector() as calls:
                outs[name] = mx(input_ids=token, position_ids=pos, past_key_values=cache,
                                use_cache=True).logits[:, -1].float()
            if name == 'absorbed':
                calls_a = calls
    torch.cuda.synchronize()
    # layer 0 sees the same inputs on both paths: the same tokens per head
    for h in range(16):
        ne = int(cache_e.visible_lens_for_layer(0)[0, h])
        assert ne == int(cache_a.visible_lens_for_layer(0)[0, h]), h
        assert torch.equal(cache_e.gather_indices_for_layer(0)[0, h, :ne],
                           cache_a.gather_indices_for_layer(0)[0, h, :ne]), h
    # every layer (whose inputs differ by rounding from layer 1 on): the
    # oracle's selections on the absorbed path's own inputs
    for li, rec in calls_a.items():
        cfg = cfg_from(cache_a, rec['indexer'], rec['scaling'])
        res, _, _ = run_oracle(cfg, rec['snap'], rec['q'], rec['decode'],
                               max_vis=cache_a.gather_indices_for_layer(li).shape[-1])
        for h in range(16):
            r = res[0][h]
            assert int(cache_a.visible_lens_for_layer(li)[0, h]) == r.vis_len, (li, h)
            np.testing.assert_array_equal(
                cache_a.gather_indices_for_layer(li)[0, h, :r.vis_len].cpu().numpy(),
                r.gather, err_msg=f'layer {li} head {h}')
    diff = (outs['absorbed'] - outs['expanded']).abs().max().item()
    scale = outs['expanded'].abs().max().item()
    assert diff <= 2e-2 * scale, (diff, scale)
    print(f'# tiny DSV2 decode: selections equal, logits within {diff:.3g} of {scale:.3g}',
          flush=True)


def test_tiny_dsv2_absorbed_graph_replay_matches_eager():
    from sparse_attn.engine.graph_runner import GraphRunner
    from sparse_attn.scheduler.scheduler import ContinuousBatchScheduler
    from test_deepseek_v2_gpu import PROMPT, _tiny_dsv2
    steps = 4
    runs = {}
    for how in ('eager', 'graph'):
        model = _tiny_dsv2()
        ids = torch.randint(0, 1024, (1, PROMPT),
                            generator=torch.Generator().manual_seed(17)).to(GPU)
        out, cache, rid = _prefill(model, ids, 'absorbed')
        sched = ContinuousBatchScheduler(cache=cache, max_batch=1, eos_ids=(),
                                         pad_token_id=0, track_receipts=True)
        sched.add_request(rid)
        sched.next_tokens[rid] = int(out.logits[0, -1].argmax())
        runner = GraphRunner(scheduler=sched, buckets=(1,), device=GPU)
        if how == 'graph':
            runner.capture_all(model, cache)
        logits = []
        with torch.no_grad():
            for i in range(steps):
                logits.append(runner.step(model, cache, generated_counts=i + 1)
                              .logits[:1].float().clone())
        if how == 'graph':
            assert runner.replay_count == steps and runner.eager_fallback_count == 0
        runs[how] = (sorted(sched.flush_ready_receipts()), torch.stack(logits))
        print(f'# tiny DSV2 absorbed {how}: {steps} steps', flush=True)
        del runner, sched, cache, model
    assert runs['graph'][0] == runs['eager'][0]
    assert torch.equal(runs['graph'][1], runs['eager'][1])
