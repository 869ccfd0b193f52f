"""hipGraph capture and replay of whole-model decode steps.

Reference: sparse_attn/engine/graph_runner.py:7-200 (``GraphRunner``) and
:203-302 (``GraphSessionPool``, ``session_graph_runner``).  Same API and keys:
one graph per (batch bucket, visible-length bucket, frozen skip signature);
a step pads the scheduler's active requests to a bucket, refreshes the
cache's fixed-address metadata, replays the graph (or runs the model eagerly
when no graph matches) and hands the logits to the scheduler.

Every layer's selection runs inside the graph on that layer's current
post-RoPE query; nothing is selected ahead of the forward.  All graphs of a
runner share one memory pool.
"""
import time
import weakref

import torch


class GraphRunner:
    def __init__(self, *, scheduler, buckets=(1, 2, 4, 8, 16, 32, 64),
                 visible_buckets=(512, 1024, 2048, 4096), device='cuda'):
        self.scheduler = scheduler
        self.buckets = tuple(int(b) for b in buckets)
        self.visible_buckets = tuple(int(v) for v in visible_buckets)
        self.device = torch.device(device)
        self.graphs = {}
        self.static_logits = {}
        self.capture_count = 0
        self.replay_count = 0
        self.eager_fallback_count = 0
        self.input_ids_buf = {b: torch.zeros((b, 1), dtype=torch.long, device=self.device)
                              for b in self.buckets}
        self.position_ids_buf = {b: torch.zeros((b, 1), dtype=torch.long,
                                                device=self.device)
                                 for b in self.buckets}
        self._pool = None

    @staticmethod
    def _key(bucket, visible_bucket, skip_signature=()):
        return (int(bucket), int(visible_bucket), skip_signature)

    def bucket_for(self, batch, max_requests=None):
        """Smallest bucket holding ``batch`` rows (within ``max_requests``)."""
        for bucket in self.buckets:
            if max_requests is not None and bucket > max_requests:
                continue
            if bucket >= batch:
                return bucket
        if max_requests is not None:
            if batch > max_requests:
                raise ValueError('active batch exceeds fixed cache capacity')
            return max_requests
        return max(self.buckets)

    @staticmethod
    def _attention_mask_arg(model):
        # Qwen3 takes a per-layer-type mask mapping: no mask is built at all
        if getattr(getattr(model, 'config', None), 'model_type', None) == 'qwen3':
            return {'full_attention': None}
        return None

    def visible_bucket_for(self, cache, padded_ids):
        width = cache.choose_visible_bucket(padded_ids, self.visible_buckets)
        return min(width, cache.max_visible_len)

    def _capture_request_ids(self, cache, bucket):
        active = list(getattr(self.scheduler, 'active_req_ids', ()) or ())
        if not active:
            active = [r for r in getattr(cache, 'active_req_ids', ())
                      if r is not None and r >= 0 and r in cache.states]
        if len(active) > bucket:
            raise ValueError('capture bucket is smaller than the frozen batch')
        return active + [-1] * (bucket - len(active))

    def _prepare_metadata(self, cache, padded_ids, visible_bucket):
        cache.plan_common(padded_ids)
        cache.set_active_visible_bucket(visible_bucket)

    def _forward(self, model, cache, bucket):
        return model(input_ids=self.input_ids_buf[bucket],
                     position_ids=self.position_ids_buf[bucket],
                     past_key_values=cache, use_cache=True,
                     attention_mask=self._attention_mask_arg(model))

    def capture(self, model, cache, bucket, visible_bucket=None):
        """Capture one decode step for ``bucket`` rows.  The capture runs on
        padding rows only (no request's length or KV changes); the frozen
        skip signature of the live requests picks the region mode."""
        if visible_bucket is None:
            visible_bucket = cache.max_visible_len
        if bucket not in self.input_ids_buf:
            raise ValueError(f'unsupported batch bucket {bucket}')
        if visible_bucket > cache.max_visible_len:
            raise ValueError(
                f'visible bucket {visible_bucket} exceeds cache {cache.max_visible_len}')
        signature = cache.nfa_skip_signature(self._capture_request_ids(cache, bucket))
        key = self._key(bucket, visible_bucket, signature)
        if key in self.graphs:
            return self.graphs[key]
        padded = [-1] * bucket
        cache.ensure_visible_buckets((visible_bucket,))
        cache.new_step(padded)
        self._prepare_metadata(cache, padded, visible_bucket)
        self.input_ids_buf[bucket].zero_()
        self.position_ids_buf[bucket].zero_()
        missing = object()
        previous = getattr(cache, '_nfa_capture_skip_signature', missing)
        cache._nfa_capture_skip_signature = signature
        try:
            # eager pass first: library handles, scratch and workspaces are
            # created outside the capture
            self._forward(model, cache, bucket)
            torch.cuda.synchronize(self.device)
            if self._pool is None:
                self._pool = torch.cuda.graph_pool_handle()
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph, pool=self._pool):
                logits = self._forward(model, cache, bucket)
        finally:
            if previous is missing:
                del cache._nfa_capture_skip_signature
            else:
                cache._nfa_capture_skip_signature = previous
        self.graphs[key] = graph
        self.static_logits[key] = logits
        self.capture_count += 1
        return graph

    def capture_all(self, model, cache):
        if not all(state.frozen for state in cache.states.values()):
            raise RuntimeError('all active requests must be frozen before graph capture')
        widths = tuple(w for w in self.visible_buckets if w <= cache.max_visible_len)
        cache.ensure_visible_buckets(widths)
        active = len(getattr(self.scheduler, 'active_req_ids', ()) or ())
        for bucket in self.buckets:
            if bucket > cache.max_requests or bucket < active:
                continue
            for width in widths:
                self.capture(model, cache, bucket, width)
            if cache.max_visible_len not in widths:
                self.capture(model, cache, bucket, cache.max_visible_len)
        return self.graphs

    def step(self, model, cache, *, generated_counts=0, min_new_tokens=0,
             return_next_tokens=False, forced_tokens=None, stop_on_eos=True):
        """One decode step of every active request."""
        req_ids, input_ids, position_ids = self.scheduler.prepare_step()
        bucket = self.bucket_for(len(req_ids), cache.max_requests)
        padded = (req_ids if len(req_ids) == bucket
                  else list(req_ids) + [-1] * (bucket - len(req_ids)))
        width = self.visible_bucket_for(cache, padded)
        self._prepare_metadata(cache, padded, width)
        rows = input_ids.shape[0]
        self.input_ids_buf[bucket][:rows].copy_(input_ids, non_blocking=True)
        self.position_ids_buf[bucket][:rows].copy_(position_ids, non_blocking=True)
        if rows < bucket:
            self.input_ids_buf[bucket][rows:].zero_()
            self.position_ids_buf[bucket][rows:].zero_()
        key = self._key(bucket, width, cache.nfa_skip_signature(padded))
        graph = self.graphs.get(key)
        if graph is not None:
            graph.replay()
            self.replay_count += 1
            logits = self.static_logits[key]
        else:
            self.eager_fallback_count += 1
            logits = self._forward(model, cache, bucket)
        self.scheduler._drain_pending_next_tokens()
        cache.nfa_decode_steps += 1
        cache.commit_step()
        next_tokens = self.scheduler.record_next_tokens(
            padded, logits, generated_counts=generated_counts,
            min_new_tokens=min_new_tokens, forced_tokens=forced_tokens,
            stop_on_eos=stop_on_eos)
        if return_next_tokens:
            return logits, next_tokens
        return logits


class GraphSessionPool:
    """Runners keyed by everything a captured graph depends on (model,
    cache object and its buffer addresses, buckets, device)."""

    def __init__(self):
        self._entries = {}
        self.hit_count = 0
        self.miss_count = 0
        self.warmup_seconds = 0.0

    @staticmethod
    def _descriptor(model, cache, buckets, visible_buckets, device):
        ptrs = [cache.layer_kv_ptrs_buf.data_ptr(), cache.block_table_buf.data_ptr(),
                cache.slot_mapping_buf.data_ptr(), cache.query_to_req_buf.data_ptr(),
                cache.active_req_ids_buf.data_ptr(), cache.valid_req_ids_buf.data_ptr(),
                cache.planned_lengths_buf.data_ptr(), cache.skip_far_layer_buf.data_ptr(),
                cache.skip_near_layer_buf.data_ptr(), cache.gather_indices_buf.data_ptr(),
                cache.visible_lens_buf.data_ptr()]
        ptrs += [layer.kv_pool_k.data_ptr() for layer in cache.layers]
        ptrs += [layer.kv_pool_v.data_ptr() for layer in cache.layers]
        ptrs += [t.data_ptr() for _, t in sorted(cache._gather_indices_by_vis.items())]
        ptrs += [t.data_ptr() for _, t in sorted(cache._visible_lens_by_vis.items())]
        return (id(model), id(cache), str(torch.device(device)), tuple(buckets),
                tuple(visible_buckets), cache.max_requests, cache.max_visible_len,
                cache.max_blocks, cache.n_layers, cache.num_kv_heads,
                cache.num_query_heads, tuple(ptrs))

    def get_runner(self, model, cache, scheduler, *, buckets=(1,),
                   visible_buckets=(512, 1024, 2048, 4096), device='cuda',
                   capture=False):
        cache.ensure_visible_buckets(
            w for w in visible_buckets if w <= cache.max_visible_len)
        desc = self._descriptor(model, cache, buckets, visible_buckets, device)
        runner = None
        entry = self._entries.get(desc)
        if entry is not None:
            cache_ref, candidate = entry
            if cache_ref() is cache:
                runner = candidate
            else:
                self._entries.pop(desc, None)
        if runner is None:
            self.miss_count += 1
            runner = GraphRunner(scheduler=scheduler, buckets=buckets,
                                 visible_buckets=visible_buckets, device=device)
            self._entries[desc] = (weakref.ref(cache), runner)
        else:
            self.hit_count += 1
            runner.scheduler = scheduler
        if capture:
            started = time.perf_counter()
            try:
                runner.capture_all(model, cache)
            except Exception:
                self._entries.pop(desc, None)
                runner.scheduler = None
                raise
            finally:
                self.warmup_seconds += time.perf_counter() - started
        return runner

    @staticmethod
    def release(runner):
        runner.scheduler = None


def session_graph_runner(model, cache, scheduler, *, buckets=(1,),
                         visible_buckets=(512, 1024, 2048, 4096), device='cuda',
                         capture=False):
    pool = getattr(model, '_nfa_graph_session_pool', None)
    if pool is None:
        pool = model._nfa_graph_session_pool = GraphSessionPool()
    return pool.get_runner(model, cache, scheduler, buckets=buckets,
                           visible_buckets=visible_buckets, device=device,
                           capture=capture)
