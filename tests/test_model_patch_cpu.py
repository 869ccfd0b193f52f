"""Host-side checks of the model patches, prefill lifecycle and graph runner.

CPU only (fp32 tiny models): which modules get patched and the errors of
``register_patch``; dense prefill into the paged arena (the arena holds the
model's own K/V and the logits equal the unpatched model's); skip decisions
frozen from a static gate; bucket choice of the graph runner; EOS masking of
the greedy step.
"""
import copy
from types import SimpleNamespace

import pytest
import torch

from sparse_attn.engine.frozen_runner import prefill_frozen_request
from sparse_attn.engine.graph_runner import GraphRunner
from sparse_attn.ops.paged_region_kernels_nfa import nfa_args
from sparse_attn.patches.patch import register_patch, unregister_patch
from sparse_attn.policies.region_geometry import RegionGeometry
from sparse_attn.scheduler.scheduler import greedy_next_tokens

GEO = RegionGeometry(sink=4, near=64, window=16, page=16, max_new_tokens=8)


def _tiny(kind, layers=2):
    torch.manual_seed(3)
    common = dict(vocab_size=256, hidden_size=128, intermediate_size=256,
                  num_hidden_layers=layers, num_attention_heads=4,
                  num_key_value_heads=2, head_dim=64,
                  max_position_embeddings=4096, rope_theta=1e6)
    if kind == 'qwen3':
        from transformers import Qwen3Config, Qwen3ForCausalLM
        cfg, cls = Qwen3Config(**common), Qwen3ForCausalLM
    else:
        from transformers import LlamaConfig, LlamaForCausalLM
        cfg, cls = LlamaConfig(**common), LlamaForCausalLM
    cfg._attn_implementation = 'sdpa'
    return cls(cfg).eval()


def _args(**kw):
    args = nfa_args('tail')
    args.tia_block_size = 16
    for k, v in kw.items():
        setattr(args, k, v)
    return args


@pytest.mark.parametrize('kind', ['qwen3', 'llama'])
def test_register_patch_counts_and_restores(kind):
    model = _tiny(kind, layers=3)
    originals = [m.forward for m in model.modules() if hasattr(m, 'q_proj')]
    assert register_patch(model, _args()) == 3
    attn = [m for m in model.modules() if hasattr(m, 'q_proj')]
    assert all(m.indexer.layer_idx == m.layer_idx for m in attn)
    assert all(m.indexer.head_dim == 64 for m in attn)
    assert all(m.forward.__func__.__name__.endswith('_attn_forward') for m in attn)
    # registering again keeps the first original forward
    assert register_patch(model, _args()) == 3
    assert unregister_patch(model) == 3
    assert [m.forward for m in attn] == originals


def test_register_patch_errors():
    model = _tiny('qwen3')
    with pytest.raises(ValueError, match='removed'):
        register_patch(model, _args(nfa_far_skip_cache='drop'))
    with pytest.raises(ValueError, match='not support'):
        register_patch(model, _args(method='quest'))
    with pytest.raises(RuntimeError, match='patched=0'):
        register_patch(torch.nn.Sequential(torch.nn.Linear(2, 2)), _args())
    assert register_patch(model, _args(method='none')) == 0


@pytest.mark.parametrize('kind', ['qwen3', 'llama'])
def test_prefill_into_arena_matches_model(kind):
    model = _tiny(kind)
    ref_model = copy.deepcopy(model)
    ids = torch.randint(0, 256, (1, 200), generator=torch.Generator().manual_seed(5))
    with torch.no_grad():
        ref = ref_model(ids, use_cache=True)
    register_patch(model, _args())
    with torch.no_grad():
        out, audit = prefill_frozen_request(model, ids, None, GEO)
    cache = out.past_key_values
    rid = audit['request_id']
    torch.testing.assert_close(out.logits[:, -1], ref.logits[:, -1],
                               rtol=1e-5, atol=1e-5)
    page = GEO.page
    for layer_idx in range(2):
        layer = cache.layers[layer_idx]
        table = cache.states[rid].block_tables[layer_idx]
        pids = torch.tensor([table[lp] for lp in range((200 + page - 1) // page)])
        k = layer.kv_pool_k[pids, 0].permute(1, 0, 2, 3).reshape(2, -1, 64)[:, :200]
        v = layer.kv_pool_v[pids, 0].permute(1, 0, 2, 3).reshape(2, -1, 64)[:, :200]
        assert torch.equal(k, ref.past_key_values.layers[layer_idx].keys[0])
        assert torch.equal(v, ref.past_key_values.layers[layer_idx].values[0])
    assert cache.states[rid].logical_length == 200
    assert cache.states[rid].frozen
    assert all(d == {'skip_near': False, 'skip_far': False}
               for d in audit['decisions'].values())


def test_prefill_static_gate_and_guards():
    model = _tiny('qwen3')
    register_patch(model, _args())
    ids = torch.randint(0, 256, (1, 100), generator=torch.Generator().manual_seed(1))
    gate = SimpleNamespace(num_layers=2, skip_far=(True, False), skip_near=(False, True))
    with torch.no_grad():
        out, audit = prefill_frozen_request(model, ids, None, GEO, static_gate=gate)
    state = out.past_key_values.states[audit['request_id']]
    assert state.skip_far_by_layer == [True, False]
    assert state.skip_near_by_layer == [False, True]
    with pytest.raises(ValueError, match='num_layers'):
        prefill_frozen_request(model, ids, None, GEO,
                               static_gate=SimpleNamespace(num_layers=5))


def test_decode_rejects_unknown_operator_modes():
    model = _tiny('qwen3')
    register_patch(model, _args(nfa_operator_mode='parallel'))
    ids = torch.randint(0, 256, (1, 100), generator=torch.Generator().manual_seed(2))
    with torch.no_grad():
        out, audit = prefill_frozen_request(model, ids, None, GEO)
    cache = out.past_key_values
    rid = audit['request_id']
    cache.new_step([rid])
    cache.plan_common([rid])
    with pytest.raises(ValueError, match='unknown NFA operator mode'), torch.no_grad():
        model(input_ids=ids[:, :1], position_ids=torch.tensor([[100]]),
              past_key_values=cache, use_cache=True,
              attention_mask={'full_attention': None})


def test_graph_runner_buckets():
    runner = GraphRunner(scheduler=None, buckets=(1, 2, 4, 8), device='cpu')
    assert [runner.bucket_for(n) for n in (1, 2, 3, 5, 8)] == [1, 2, 4, 8, 8]
    assert runner.bucket_for(3, max_requests=3) == 3
    assert runner.bucket_for(2, max_requests=4) == 2
    with pytest.raises(ValueError, match='capacity'):
        runner.bucket_for(9, max_requests=8)
    assert runner._key(2, 1024, ((False, True),)) == (2, 1024, ((False, True),))


def test_greedy_next_tokens_masks_eos_until_min_tokens():
    logits = torch.zeros(2, 1, 5)
    logits[:, 0, 3] = 2.0  # EOS
    logits[:, 0, 1] = 1.0
    out = greedy_next_tokens(logits, (3,), generated_counts=[0, 4], min_new_tokens=2)
    assert out.tolist() == [1, 3]
    assert logits[0, 0, 3] == 2.0  # the caller's logits are untouched
    assert greedy_next_tokens(logits, (3,)).tolist() == [3, 3]
    with pytest.raises(ValueError):
        greedy_next_tokens(logits[:, 0], (3,))
