"""Prefill region gate on the GPU vs the oracle.

``nfa_region_profile`` (through ``fused_region_profile``) against the
oracle's float64 causal softmax masses: per head and row, near and far mass
within 2e-5 absolute (fp32 online softmax over up to 5000 keys).  The q/k
inputs are transposed views, as the model's attention hands them over.
Then a tiny Qwen3 model prefilled with a request-time gate: the frozen skip
flags follow the decision rule on the returned profiles, and the next decode
step's selection in the resulting region mode matches the oracle.
"""
import numpy as np
import pytest
import torch

from oracle import nfa_oracle as orc
from sparse_attn.ops.frozen_gate import fused_region_profile
from sparse_attn.policies.frozen_gate import GateConfig, decide_regions, region_present
from sparse_attn.policies.region_geometry import RegionGeometry

pytestmark = pytest.mark.gpu
DEV = 'cuda'


@pytest.mark.parametrize('hq,hkv,d,length,rows', [
    (8, 2, 128, 3000, 256), (16, 2, 64, 700, 700), (4, 4, 128, 5000, 100)])
def test_profile_matches_oracle(hq, hkv, d, length, rows):
    geo = RegionGeometry(sink=4, near=512, window=64, page=16)
    gen = torch.Generator(device=DEV).manual_seed(length)
    # [1, L, H, D] projections viewed as [1, H, L, D], like the model's
    q = (torch.randn(1, length, hq, d, generator=gen, device=DEV) * 1.5).to(
        torch.bfloat16).transpose(1, 2)
    k = torch.randn(1, length, hkv, d, generator=gen, device=DEV).to(
        torch.bfloat16).transpose(1, 2)
    scale = d ** -0.5
    print(f'# gate profile hq={hq} hkv={hkv} d={d} L={length} rows={rows}', flush=True)
    from sparse_attn import _native as nat
    import ctypes
    # per-head values straight from the kernel, before the head mean
    out = torch.empty((2, hq, rows), dtype=torch.float32, device=DEV)
    p = nat.NfaGateParams()
    p.abi_version, p.struct_size = nat.ABI_VERSION, ctypes.sizeof(nat.NfaGateParams)
    p.hq, p.hkv, p.head_dim, p.length, p.rows = hq, hkv, d, length, rows
    p.sink, p.window, p.near, p.page = geo.sink, geo.window, geo.near, geo.page
    p.q_dtype, p.scale = nat.DTYPE_BF16, scale
    p.q, p.q_stride_h, p.q_stride_l = q.data_ptr(), q.stride(1), q.stride(2)
    p.k, p.k_stride_h, p.k_stride_l = k.data_ptr(), k.stride(1), k.stride(2)
    p.out = out.data_ptr()
    nat.check(nat.load_library().nfa_region_profile(ctypes.byref(p), nat.stream_handle()),
              'region_profile')
    mean = fused_region_profile(q, k, geo, rows, scale)
    torch.cuda.synchronize()
    want = orc.region_profile(q[0].float().cpu().numpy(), k[0].float().cpu().numpy(),
                              rows, scale, geo.sink, geo.window, geo.near, geo.page)
    np.testing.assert_allclose(out.cpu().numpy(), want, atol=2e-5, rtol=0)
    np.testing.assert_allclose(mean.cpu().numpy(), want.mean(axis=1), atol=2e-5, rtol=0)


def test_gated_prefill_freezes_decisions_and_decodes():
    from test_model_patch_gpu import (GEO, PROMPT, _args, _mask_arg, _recording,
                                      _tiny_model)
    from nfa_case import cfg_from, run_oracle
    from sparse_attn.engine.frozen_runner import prefill_frozen_request
    from sparse_attn.patches.patch import register_patch

    model = _tiny_model('qwen3')
    register_patch(model, _args())
    gen = torch.Generator(device='cpu').manual_seed(23)
    ids = torch.randint(0, 1024, (1, PROMPT), generator=gen).to(DEV)
    # random weights attend almost uniformly: near ~ 4096 / 9000, far ~ 0.5
    config = GateConfig(epsilon=0.5, rows=64)
    with torch.no_grad():
        out, audit = prefill_frozen_request(model, ids, config, GEO)
    cache, rid = out.past_key_values, audit['request_id']
    present = region_present(PROMPT, GEO)
    assert present == (True, True)
    state = cache.states[rid]
    for layer, prof in audit['profiles'].items():
        want = decide_regions(prof, config, *present)
        assert audit['decisions'][layer] == want
        assert state.skip_far_by_layer[layer] == want['skip_far']
        assert state.skip_near_by_layer[layer] == want['skip_near']
        assert 0.3 < prof['near']['mean'] < 0.6 and 0.3 < prof['far']['mean'] < 0.7
    assert any(state.skip_near_by_layer)
    # one decode step in the gated region mode: selections as the oracle's
    token = out.logits[:, -1].argmax(-1, keepdim=True)
    pos = torch.full((1, 1), PROMPT, dtype=torch.long, device=DEV)
    cache.new_step([rid])
    cache.plan_common([rid])
    with torch.no_grad(), _recording() as calls:
        model(input_ids=token, position_ids=pos, past_key_values=cache,
              use_cache=True, attention_mask=_mask_arg(model))
    torch.cuda.synchronize()
    for layer, rec in calls.items():
        cfg = cfg_from(cache, rec['indexer'], rec['scaling'])
        width = cache.gather_indices_for_layer(layer).shape[-1]
        res, _, _ = run_oracle(cfg, rec['snap'], rec['q'], rec['decode'], max_vis=width)
        gather = cache.gather_indices_for_layer(layer).cpu().numpy()
        vis = cache.visible_lens_for_layer(layer).cpu().numpy()
        for kv in range(cache.num_kv_heads):
            r = res[0][kv]
            assert vis[0, kv] == r.vis_len
            np.testing.assert_array_equal(gather[0, kv, :r.vis_len], r.gather[:r.vis_len])
