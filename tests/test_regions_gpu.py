"""Disjoint protected / middle attention on the GPU.

* ``sparse_paged_attention_gather_partial``: every split's (m, z, acc)
  against the oracle's float64 split states on the same partition (block
  128 for up to 8 query rows, 64 above), with padding rows, negative slots,
  empty rows and rows shorter than the split count.  Tolerances: m within
  1e-5 relative (fp32 dot products of bf16 / fp32 inputs), z and acc within
  1e-4 relative (fp32 exp and sums over up to 1024 slots).
* ``sparse_paged_attention_regions_combine``: on the kernel's own split
  states, against the oracle's float64 merge of the same states (1e-5
  relative for fp32 output), and end to end against softmax attention over
  the union of the two slot sets (bf16: rtol 2e-2 / atol 2e-3).
* ``--nfa_operator_mode serial`` / ``overlap`` in a patched tiny Qwen3 /
  Llama: per layer and kv head the protected and middle sets partition the
  union that mode ``off`` selects, the logits agree with mode ``off``, and
  graph replays (the overlap arm on a second stream inside the graph) are
  bit-identical to eager steps.
"""
import numpy as np
import pytest
import torch

from nfa_case import bf16_randn, make_cache, to_np
from oracle import nfa_oracle as orc
from sparse_attn.ops.paged_region_kernels import (sparse_paged_attention_gather,
                                                  sparse_paged_attention_gather_partial,
                                                  sparse_paged_attention_regions_combine)
from sparse_attn.policies.region_geometry import RegionGeometry

pytestmark = pytest.mark.gpu
DEV = 'cuda'
GEO = RegionGeometry(sink=4, near=4096, window=128, page=16, max_new_tokens=64)


def _pools(dtype, hkv, hq, head_dim, pages, seed, rows):
    cache = make_cache(DEV, geometry=GEO, max_blocks=64, max_physical_pages=pages,
                       max_visible_len=1024, hkv=hkv, hq=hq, dtype=dtype,
                       max_requests=rows, head_dim=head_dim)
    gen = torch.Generator(device=DEV).manual_seed(seed)
    layer = cache.layers[0]
    layer.kv_pool_k.copy_(bf16_randn(layer.kv_pool_k.shape, gen, DEV).to(dtype))
    layer.kv_pool_v.copy_(bf16_randn(layer.kv_pool_v.shape, gen, DEV).to(dtype))
    return cache, gen


def _disjoint_gathers(gen, rows, hkv, pages, widths):
    """Per (row, kv head) disjoint random slot sets of the given widths."""
    total = pages * GEO.page
    perm = torch.stack([torch.randperm(total, generator=gen, device=DEV)[:sum(widths)]
                        for _ in range(rows * hkv)]).view(rows, hkv, -1)
    out, at = [], 0
    for w in widths:
        out.append(perm[..., at:at + w].to(torch.int32).contiguous())
        at += w
    return out


def _assert_states(got, want, tag):
    acc, m, z = (t.cpu().numpy().astype(np.float64) for t in got)
    w_acc, w_m, w_z = want
    empty = w_m == -np.inf
    assert (m[empty] == -np.inf).all(), tag
    assert (z[empty] == 0).all() and not acc[empty].any(), tag
    np.testing.assert_allclose(m[~empty], w_m[~empty], rtol=1e-5, atol=1e-5, err_msg=tag)
    np.testing.assert_allclose(z, w_z, rtol=1e-4, atol=1e-6, err_msg=tag)
    np.testing.assert_allclose(acc, w_acc, rtol=1e-4, atol=1e-4, err_msg=tag)


@pytest.mark.parametrize('dtype', [torch.bfloat16, torch.float32])
@pytest.mark.parametrize('total_q,nsplit,head_dim', [
    (3, 1, 128), (3, 4, 128), (12, 4, 128), (5, 7, 64), (12, 1, 64)])
def test_partial_states_match_oracle(dtype, total_q, nsplit, head_dim):
    hkv, hq, pages, rows = 4, 16, 300, 4
    cache, gen = _pools(dtype, hkv, hq, head_dim, pages, 31 + total_q, rows)
    layer = cache.layers[0]
    gather, = _disjoint_gathers(gen, rows, hkv, pages, (1024,))
    gather[1, 2, 7] = -1  # negative slots are skipped
    lens = torch.randint(0, 1025, (rows, hkv), generator=gen, device=DEV,
                         dtype=torch.int32)
    lens[0, 0], lens[0, 1], lens[2, 3], lens[3, 0] = 1024, 0, 3, 129
    q = bf16_randn((total_q, hq, head_dim), gen, DEV).to(dtype)
    q2r = torch.randint(0, rows, (total_q,), generator=gen, device=DEV,
                        dtype=torch.int32)
    q2r[1] = -1  # padding row
    q2r[0] = 0
    scale = head_dim ** -0.5
    print(f'# partial dtype={dtype} T={total_q} nsplit={nsplit} D={head_dim}', flush=True)
    ws = {}
    got = sparse_paged_attention_gather_partial(
        layer, q, gather, lens, q2r, scale=scale, workspace=ws, name='t', nsplit=nsplit)
    torch.cuda.synchronize()
    bt = 128 if total_q <= 8 else 64
    want = orc.sparse_attention_partial(
        to_np(layer.kv_pool_k), to_np(layer.kv_pool_v), to_np(q), gather.cpu().numpy(),
        lens.cpu().numpy(), q2r.cpu().numpy(), scale, GEO.page, nsplit, bt)
    _assert_states(got, want, f'T={total_q} nsplit={nsplit}')
    # fixed addresses: the same workspace name returns the same buffers
    again = sparse_paged_attention_gather_partial(
        layer, q, gather, lens, q2r, scale=scale, workspace=ws, name='t', nsplit=nsplit)
    assert all(a.data_ptr() == b.data_ptr() for a, b in zip(got, again))


@pytest.mark.parametrize('dtype', [torch.bfloat16, torch.float32])
def test_regions_combine_matches_union_attention(dtype):
    hkv, hq, head_dim, pages, rows, total_q = 8, 32, 128, 600, 2, 3
    cache, gen = _pools(dtype, hkv, hq, head_dim, pages, 77, rows)
    layer = cache.layers[0]
    prot, mid = _disjoint_gathers(gen, rows, hkv, pages, (132, 1024))
    prot_lens = torch.full((rows, hkv), 132, dtype=torch.int32, device=DEV)
    prot_lens[1, 3] = 0
    mid_lens = torch.randint(0, 1025, (rows, hkv), generator=gen, device=DEV,
                             dtype=torch.int32)
    mid_lens[0, 0], mid_lens[1, 3] = 1024, 0  # [1, 3]: both regions empty
    q = bf16_randn((total_q, hq, head_dim), gen, DEV).to(dtype)
    q2r = torch.tensor([1, 0, -1], dtype=torch.int32, device=DEV)
    scale = head_dim ** -0.5
    ws = {}
    pa = sparse_paged_attention_gather_partial(
        layer, q, prot, prot_lens, q2r, scale=scale, workspace=ws, name='protected',
        nsplit=1)
    pb = sparse_paged_attention_gather_partial(
        layer, q, mid, mid_lens, q2r, scale=scale, workspace=ws, name='middle', nsplit=4)
    out = sparse_paged_attention_regions_combine(q, pa, pb, workspace=ws)
    torch.cuda.synchronize()
    assert out.dtype == dtype and out.shape == (total_q, hq, head_dim)
    got = out.float().cpu().numpy()
    # the combine kernel alone: the oracle's merge of the kernel's own states
    merged = orc.regions_combine(tuple(t.cpu().numpy().astype(np.float64) for t in pa),
                                 tuple(t.cpu().numpy().astype(np.float64) for t in pb))
    if dtype == torch.float32:
        np.testing.assert_allclose(got, merged, rtol=1e-5, atol=1e-6)
    else:
        np.testing.assert_allclose(got, merged, rtol=8e-3, atol=1e-5)
    # end to end: attention over the union of the two sets
    union = torch.full((rows, hkv, 132 + 1024), -1, dtype=torch.int32, device=DEV)
    ulens = prot_lens + mid_lens
    for r in range(rows):
        for kv in range(hkv):
            a, b = int(prot_lens[r, kv]), int(mid_lens[r, kv])
            union[r, kv, :a] = prot[r, kv, :a]
            union[r, kv, a:a + b] = mid[r, kv, :b]
    want = orc.sparse_attention(to_np(layer.kv_pool_k), to_np(layer.kv_pool_v), to_np(q),
                                union.cpu().numpy(), ulens.cpu().numpy(),
                                q2r.cpu().numpy(), scale, GEO.page)
    tol = dict(rtol=2e-2, atol=2e-3) if dtype == torch.bfloat16 else dict(rtol=1e-4,
                                                                            atol=1e-5)
    np.testing.assert_allclose(got, want, **tol)
    assert not got[2].any() and not got[0, 3 * 4:4 * 4].any()  # padding; empty kv 3
    fused = sparse_paged_attention_gather(layer, q, union, ulens, q2r, scale=scale)
    np.testing.assert_allclose(got, fused.float().cpu().numpy(), **tol)


# --- operator modes in the model ---------------------------------------------

def _mode_args(mode):
    from test_model_patch_gpu import _args
    args = _args()
    args.nfa_operator_mode = mode
    return args


def _prefill_mode(model, ids, mode, fused=False):
    from test_model_patch_gpu import GEO as MGEO
    from sparse_attn.engine.frozen_runner import prefill_frozen_request
    from sparse_attn.patches.patch import register_patch
    register_patch(model, _mode_args(mode), rmsnorm_decode=fused,
                   mlp_silu_decode=fused, decode_layers=fused)
    with torch.no_grad():
        out, audit = prefill_frozen_request(model, ids, None, MGEO)
    return out, out.past_key_values, audit['request_id']


@pytest.mark.parametrize('mode', ['serial', 'overlap'])
@pytest.mark.parametrize('kind', ['qwen3', 'llama'])
def test_operator_modes_partition_the_union_and_match_off(kind, mode):
    import copy
    from test_model_patch_gpu import PROMPT, _mask_arg, _tiny_model
    from sparse_attn.ops.paged_region_kernels_nfa import split_gather_buffers
    base = _tiny_model(kind)
    models = {'off': base, mode: copy.deepcopy(base)}
    gen = torch.Generator(device='cpu').manual_seed(29)
    ids = torch.randint(0, 1024, (1, PROMPT), generator=gen).to(DEV)
    state = {}
    for m, model in models.items():
        print(f'# {kind} operator mode {m}: prefill + 2 decode steps', flush=True)
        out, cache, rid = _prefill_mode(model, ids, m)
        token = out.logits[:, -1].argmax(-1, keepdim=True)
        logits = []
        for step in range(2):
            pos = torch.full((1, 1), PROMPT + step, dtype=torch.long, device=DEV)
            cache.new_step([rid])
            cache.plan_common([rid])
            with torch.no_grad():
                lg = model(input_ids=token, position_ids=pos, past_key_values=cache,
                           use_cache=True, attention_mask=_mask_arg(model)).logits
            torch.cuda.synchronize()
            cache.commit_step()
            logits.append(lg.float())
            token = lg[:, -1].argmax(-1, keepdim=True)
        state[m] = (cache, rid, logits)
    off_cache, _, off_logits = state['off']
    cache, rid, logits = state[mode]
    for layer_idx in range(base.config.num_hidden_layers):
        pg, pl, mg, ml = split_gather_buffers(cache, layer_idx, 1)
        union = off_cache.gather_indices_for_layer(layer_idx).cpu().numpy()
        ulen = off_cache.visible_lens_for_layer(layer_idx).cpu().numpy()
        for kv in range(cache.num_kv_heads):
            tag = f'{kind} {mode} layer={layer_idx} kv={kv}'
            prot = pg[0, kv, :int(pl[0, kv])].cpu().numpy()
            mid = mg[0, kv, :int(ml[0, kv])].cpu().numpy()
            assert len(np.intersect1d(prot, mid)) == 0, tag
            assert len(prot) + len(mid) == ulen[0, kv], tag
            np.testing.assert_array_equal(np.sort(np.concatenate([prot, mid])),
                                          np.sort(union[0, kv, :ulen[0, kv]]), err_msg=tag)
            assert len(prot) == 4 + 128 and len(mid) > 0, tag
    for a, b in zip(logits, off_logits):
        diff = (a - b).abs().max().item()
        scale = b.abs().max().item()
        assert diff <= 2e-2 * scale, (diff, scale)


@pytest.mark.parametrize('fused', [False, True])
@pytest.mark.parametrize('mode', ['serial', 'overlap'])
def test_operator_mode_graph_replay_matches_eager(mode, fused):
    from test_model_patch_gpu import PROMPT, _tiny_model
    from sparse_attn.engine.graph_runner import GraphRunner
    from sparse_attn.scheduler.scheduler import ContinuousBatchScheduler
    steps = 4
    model = _tiny_model('qwen3')
    gen = torch.Generator(device='cpu').manual_seed(37)
    ids = torch.randint(0, 1024, (1, PROMPT), generator=gen).to(DEV)
    runs = {}
    for run in ('eager', 'graph'):
        print(f'# qwen3 {mode} fused={fused} {run} decode {steps} steps', flush=True)
        out, cache, rid = _prefill_mode(model, ids, mode, fused=fused)
        sched = ContinuousBatchScheduler(cache=cache, max_batch=1, eos_ids=(),
                                         pad_token_id=0, track_receipts=True)
        sched.add_request(rid)
        sched.next_tokens[rid] = int(out.logits[0, -1].argmax())
        runner = GraphRunner(scheduler=sched, buckets=(1,), device=DEV)
        if run == 'graph':
            runner.capture_all(model, cache)
        logits = []
        with torch.no_grad():
            for i in range(steps):
                lg = runner.step(model, cache, generated_counts=i + 1)
                logits.append(lg.logits.float().clone())
        tokens = [t for _, t in sched.flush_ready_receipts()]
        if run == 'graph':
            assert runner.replay_count == steps and runner.eager_fallback_count == 0
        calls = [getattr(l, '_nfa_fused_calls', 0) for l in model.model.layers]
        assert all(c > 0 for c in calls) == fused, calls
        runs[run] = (tokens, torch.stack(logits))
    assert runs['graph'][0] == runs['eager'][0]
    assert torch.equal(runs['graph'][1], runs['eager'][1])
