"""hipGraph capture and replay of whole-model decode steps.

Reference interface: sparse_attn/engine/graph_runner.py:7-200 (``GraphRunner``:
constructor, ``bucket_for``, ``visible_bucket_for``, ``capture``,
``capture_all``, ``step``, the capture/replay/eager counters) and :203-302
(``GraphSessionPool``, ``session_graph_runner``).  The behaviour a caller sees
is the reference's: a step pads the scheduler's active requests to a batch
bucket, picks the graph of (batch bucket, visible-length bucket, frozen skip
signature), replays it -- or runs the model eagerly when no graph was
captured for that key -- and hands the logits to the scheduler.

Design.  Every captured step is a ``_StepGraph`` record: the graph, its
static logits and the key it serves.  The model inputs of all buckets live in
one device buffer of the largest bucket; a bucket reads a prefix view of it,
so the addresses a graph holds never move.  Capture runs on padding rows
only (no request's length or KV changes), with the cache told which skip
signature the live rows carry so that each layer captures the selector's
region mode for them.  The session pool keys runners by the model, the cache
and a fingerprint of every device buffer the cache owns: a runner (and its
graphs) is reused only while all of those addresses are unchanged.
"""
from contextlib import contextmanager
from dataclasses import dataclass
import time
import weakref

import torch


@dataclass
class _StepGraph:
    """One captured decode step."""
    key: tuple
    graph: object
    logits: object
    replays: int = 0


@contextmanager
def _frozen_signature(cache, signature):
    """While capturing on padding rows, report the live rows' frozen skip
    signature to the selector."""
    saved = cache.__dict__.get('_nfa_signature_override')
    cache._nfa_signature_override = signature
    try:
        yield
    finally:
        cache._nfa_signature_override = saved


class GraphRunner:
    """Decode-step graphs of one (model, cache) pair."""

    def __init__(self, *, scheduler, buckets=(1, 2, 4, 8, 16, 32, 64),
                 visible_buckets=(512, 1024, 2048, 4096), device='cuda'):
        self.scheduler = scheduler
        self.buckets = tuple(sorted(int(b) for b in buckets))
        self.visible_buckets = tuple(int(v) for v in visible_buckets)
        self.device = torch.device(device)
        self._table = {}
        self.capture_count = 0
        self.replay_count = 0
        self.eager_fallback_count = 0
        width = max(self.buckets)
        # [0]: input token ids, [1]: positions; bucket b reads rows [:b]
        self._inputs = torch.zeros((2, width, 1), dtype=torch.long, device=self.device)
        self._pool = None

    # -- the graph table ------------------------------------------------
    @staticmethod
    def _key(bucket, visible_bucket, skip_signature=()):
        return (int(bucket), int(visible_bucket), skip_signature)

    @property
    def graphs(self):
        return {k: entry.graph for k, entry in self._table.items()}

    @property
    def static_logits(self):
        return {k: entry.logits for k, entry in self._table.items()}

    def _bucket_inputs(self, bucket):
        return self._inputs[0, :bucket], self._inputs[1, :bucket]

    # -- shapes ---------------------------------------------------------
    def bucket_for(self, batch, max_requests=None):
        """Smallest batch bucket holding ``batch`` rows within
        ``max_requests``; the capacity itself when no bucket fits in it."""
        fitting = [b for b in self.buckets
                   if b >= batch and (max_requests is None or b <= max_requests)]
        if fitting:
            return fitting[0]
        if max_requests is None:
            return self.buckets[-1]
        if batch > max_requests:
            raise ValueError('active batch exceeds fixed cache capacity')
        return max_requests

    def visible_bucket_for(self, cache, padded_ids):
        return min(cache.choose_visible_bucket(padded_ids, self.visible_buckets),
                   cache.max_visible_len)

    @staticmethod
    def _mask_arg(model):
        # Qwen3 takes a mapping of attention kinds to masks: build none
        kind = getattr(getattr(model, 'config', None), 'model_type', None)
        return {'full_attention': None} if kind == 'qwen3' else None

    def _run_model(self, model, cache, bucket):
        ids, pos = self._bucket_inputs(bucket)
        return model(input_ids=ids, position_ids=pos, past_key_values=cache,
                     use_cache=True, attention_mask=self._mask_arg(model))

    # -- capture ----------------------------------------------------------
    def _live_rows(self, cache, bucket):
        """The frozen requests a graph of ``bucket`` rows will serve, padded."""
        live = list(getattr(self.scheduler, 'active_req_ids', None) or [])
        if not live:
            live = [r for r in getattr(cache, 'active_req_ids', ())
                    if r is not None and r >= 0 and r in cache.states]
        if len(live) > bucket:
            raise ValueError('capture bucket is smaller than the frozen batch')
        return live + [-1] * (bucket - len(live))

    def capture(self, model, cache, bucket, visible_bucket=None):
        """Capture one decode step of ``bucket`` rows at ``visible_bucket``
        gather width (the cache's full width by default)."""
        width = cache.max_visible_len if visible_bucket is None else int(visible_bucket)
        if bucket not in self.buckets:
            raise ValueError(f'unsupported batch bucket {bucket}')
        if width > cache.max_visible_len:
            raise ValueError(
                f'visible bucket {width} exceeds cache {cache.max_visible_len}')
        signature = cache.nfa_skip_signature(self._live_rows(cache, bucket))
        key = self._key(bucket, width, signature)
        entry = self._table.get(key)
        if entry is not None:
            return entry.graph
        padding = [-1] * bucket
        cache.ensure_visible_buckets((width,))
        cache.new_step(padding)
        cache.plan_common(padding)
        cache.set_active_visible_bucket(width)
        self._inputs[:, :bucket].zero_()
        with _frozen_signature(cache, signature):
            # one eager pass creates every library handle, scratch buffer and
            # workspace outside the capture
            self._run_model(model, cache, bucket)
            torch.cuda.synchronize(self.device)
            if self._pool is None:
                self._pool = torch.cuda.graph_pool_handle()
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph, pool=self._pool):
                logits = self._run_model(model, cache, bucket)
        self._table[key] = _StepGraph(key, graph, logits)
        self.capture_count += 1
        return graph

    def capture_all(self, model, cache):
        """Capture every (batch bucket, visible bucket) the cache can serve
        for the frozen requests; the full-width graph always."""
        if any(not state.frozen for state in cache.states.values()):
            raise RuntimeError('all active requests must be frozen before graph capture')
        widths = [w for w in self.visible_buckets if w <= cache.max_visible_len]
        if cache.max_visible_len not in widths:
            widths.append(cache.max_visible_len)
        cache.ensure_visible_buckets(w for w in widths if w != cache.max_visible_len)
        floor = len(getattr(self.scheduler, 'active_req_ids', None) or ())
        for bucket in self.buckets:
            if floor <= bucket <= cache.max_requests:
                for width in widths:
                    self.capture(model, cache, bucket, width)
        return self.graphs

    # -- one step ---------------------------------------------------------
    def step(self, model, cache, *, generated_counts=0, min_new_tokens=0,
             return_next_tokens=False, forced_tokens=None, stop_on_eos=True):
        """One decode token for every active request."""
        req_ids, input_ids, position_ids = self.scheduler.prepare_step()
        rows = len(req_ids)
        bucket = self.bucket_for(rows, cache.max_requests)
        padded = list(req_ids) + [-1] * (bucket - rows)
        width = self.visible_bucket_for(cache, padded)
        cache.plan_common(padded)
        # a runner that never captured (eager only) has not prepared the
        # narrower visible buckets: the step prepares the one it uses (never
        # under capture; capture_all prepares them all up front)
        cache.ensure_visible_buckets((width,))
        cache.set_active_visible_bucket(width)
        ids, pos = self._bucket_inputs(bucket)
        n = input_ids.shape[0]
        ids[:n].copy_(input_ids, non_blocking=True)
        pos[:n].copy_(position_ids, non_blocking=True)
        if n < bucket:
            self._inputs[:, n:bucket].zero_()
        entry = self._table.get(self._key(bucket, width, cache.nfa_skip_signature(padded)))
        if entry is None:
            self.eager_fallback_count += 1
            logits = self._run_model(model, cache, bucket)
        else:
            entry.graph.replay()
            entry.replays += 1
            self.replay_count += 1
            logits = entry.logits
        # the previous step's host receipts, now that this step is queued
        self.scheduler._drain_pending_next_tokens()
        cache.nfa_decode_steps += 1
        cache.commit_step()
        next_tokens = self.scheduler.record_next_tokens(
            padded, logits, generated_counts=generated_counts,
            min_new_tokens=min_new_tokens, forced_tokens=forced_tokens,
            stop_on_eos=stop_on_eos)
        return (logits, next_tokens) if return_next_tokens else logits


def _cache_fingerprint(cache):
    """Addresses and shapes of every device buffer the cache holds (its
    metadata buffers, bucketed gather rows and KV arenas) plus its
    capacities: graphs captured against one fingerprint stay valid while it
    is unchanged."""
    found = []

    def visit(name, value):
        if isinstance(value, torch.Tensor) and value.device.type != 'cpu':
            found.append((name, value.data_ptr(), tuple(value.shape)))
        elif isinstance(value, dict):
            for k in sorted(value, key=repr):
                visit(f'{name}[{k!r}]', value[k])

    for name in sorted(vars(cache)):
        visit(name, vars(cache)[name])
    for i, layer in enumerate(cache.layers):
        visit(f'k{i}', layer.kv_pool_k)
        visit(f'v{i}', layer.kv_pool_v)
    caps = (cache.max_requests, cache.max_visible_len, cache.max_blocks,
            cache.n_layers, cache.num_kv_heads, cache.num_query_heads)
    return caps, tuple(found)


class GraphSessionPool:
    """Graph runners shared across requests of one model: a request reuses
    the runner (and its captured graphs) of an earlier one only when model,
    cache object, device, buckets and every cache buffer address match."""

    def __init__(self):
        self._runners = {}
        self.hit_count = 0
        self.miss_count = 0
        self.warmup_seconds = 0.0

    def get_runner(self, model, cache, scheduler, *, buckets=(1,),
                   visible_buckets=(512, 1024, 2048, 4096), device='cuda',
                   capture=False):
        # create the bucketed gather rows first: they are part of the
        # fingerprint, and capture would otherwise add them afterwards
        cache.ensure_visible_buckets(
            w for w in visible_buckets if w < cache.max_visible_len)
        key = (id(model), id(cache), str(torch.device(device)),
               tuple(buckets), tuple(visible_buckets))
        print_ = _cache_fingerprint(cache)
        held = self._runners.get(key)
        runner = None
        if held is not None:
            cache_ref, held_print, candidate = held
            if cache_ref() is cache and held_print == print_:
                runner = candidate
        if runner is None:
            self.miss_count += 1
            runner = GraphRunner(scheduler=scheduler, buckets=buckets,
                                 visible_buckets=visible_buckets, device=device)
            self._runners[key] = (weakref.ref(cache), print_, runner)
        else:
            self.hit_count += 1
            runner.scheduler = scheduler
        if capture:
            t0 = time.perf_counter()
            try:
                runner.capture_all(model, cache)
                # a capture may create cache buffers (workspaces, statistics):
                # the runner now serves the cache as it is after capture
                self._runners[key] = (weakref.ref(cache), _cache_fingerprint(cache),
                                      runner)
            except Exception:
                self._runners.pop(key, None)
                runner.scheduler = None
                raise
            finally:
                self.warmup_seconds += time.perf_counter() - t0
        return runner

    @staticmethod
    def release(runner):
        """Drop the runner's scheduler (and through it the cache arena)."""
        runner.scheduler = None


def session_graph_runner(model, cache, scheduler, *, buckets=(1,),
                         visible_buckets=(512, 1024, 2048, 4096), device='cuda',
                         capture=False):
    """The model's session pool (created on first use) hands out the runner."""
    pool = model.__dict__.get('_nfa_graph_session_pool')
    if pool is None:
        pool = model._nfa_graph_session_pool = GraphSessionPool()
    return pool.get_runner(model, cache, scheduler, buckets=buckets,
                           visible_buckets=visible_buckets, device=device,
                           capture=capture)
