"""Graph-ready paged KV cache with a continuous-batching request lifecycle.

Reference interface: sparse_attn/cache/paged_region_cache.py
(``GraphReadyPagedRegionLayer`` :60-112, ``GraphReadyPagedRegionCache``
:115-1113): the constructor, the device buffers (names, shapes, dtypes), the
public methods and their errors are the reference's, so callers and kernels
index the same memory.  The implementation is this project's own:

* **Pages.**  A request's pages per layer form an append-only ``_PageRun``
  (logical page i -> physical id); each layer's arena hands out pages from a
  bump pointer and re-uses returned pages lowest id first.  The last arena
  page is a zeroed PAD page that invalid block-table entries point at; the
  physical slot of a token is ``page_id * page + offset``.
* **Step metadata.**  Planned lengths, slot mapping, query->row map and
  query start offsets share one device int32 arena, request ids one int64
  arena; the buffers are views into them.  The host fills a pinned bank of
  the same layout and uploads it with one copy per arena.  Two banks
  alternate, so planning the next step never waits for the copy of the
  current one.  A steady decode step computes every slot on the host from
  each row's current physical page per layer (a small vector, refreshed when
  the row's token opens a page) and uploads only lengths and slots, plus the
  block-table entries of pages opened this step.
* **Visible buckets.**  The gather width a step needs is the largest union
  of a row's kept regions at its planned length, a closed form of
  ``RegionGeometry.bounds``; no per-step cache of earlier answers is kept.
"""
import bisect
from dataclasses import dataclass, field
from enum import Enum

import numpy as np
import torch

INVALID_PAGE_IDX = -1
INVALID_GATHER_IDX = -1
PAD_SLOT = -1

SINK = 0b0001
FAR = 0b0010
NEAR = 0b0100
SWA = 0b1000
REGION_BITS = (SINK, FAR, NEAR, SWA)


class RequestPhase(str, Enum):
    PREFILL = 'PREFILL'
    FREEZE = 'FREEZE'
    SUFFIX = 'SUFFIX'
    GENERATE = 'GENERATE'
    FINISHED = 'FINISHED'
    FAILED = 'FAILED'


def _phase_graph():
    """Allowed phase changes: a request may fail from any live phase and
    finishes after it is frozen."""
    P = RequestPhase
    live_order = [P.PREFILL, P.FREEZE, P.SUFFIX, P.GENERATE]
    edges = {p: {P.FAILED} for p in live_order}
    edges[P.PREFILL].add(P.FREEZE)
    edges[P.FREEZE] |= {P.SUFFIX, P.GENERATE, P.FINISHED}
    edges[P.SUFFIX] |= {P.GENERATE, P.FINISHED}
    edges[P.GENERATE].add(P.FINISHED)
    edges[P.FINISHED] = set()
    edges[P.FAILED] = set()
    return edges


_NEXT_PHASES = _phase_graph()


class _PageRun:
    """Append-only map of one request's logical pages to physical pages in
    one layer, read like the reference's ``{logical: physical}`` dict."""

    __slots__ = ('_ids',)

    def __init__(self, ids=()):
        self._ids = list(ids)

    def append(self, pid):
        self._ids.append(int(pid))

    def __len__(self):
        return len(self._ids)

    def __bool__(self):
        return bool(self._ids)

    def __getitem__(self, lp):
        if not 0 <= lp < len(self._ids):
            raise KeyError(lp)
        return self._ids[lp]

    def get(self, lp, default=None):
        return self._ids[lp] if 0 <= lp < len(self._ids) else default

    def __contains__(self, lp):
        return 0 <= lp < len(self._ids)

    def __iter__(self):
        return iter(range(len(self._ids)))

    def keys(self):
        return range(len(self._ids))

    def values(self):
        return list(self._ids)

    def items(self):
        return list(enumerate(self._ids))

    def physical(self):
        return self._ids


@dataclass
class RequestState:
    """One request slot: lengths, lifecycle phase, per-layer page runs and
    frozen per-layer region skips."""
    logical_length: int = 0
    prompt_length: int = 0
    phase: RequestPhase = RequestPhase.PREFILL
    block_tables: list = field(default_factory=list)
    skip_far_by_layer: list = field(default_factory=list)
    skip_near_by_layer: list = field(default_factory=list)
    frozen: bool = False
    active: bool = True
    skip_policy_groups: tuple = ()


class GraphReadyPagedRegionLayer:
    """One layer's physical KV arena ``[P + 1, 1, HKV, page, D]`` and its page
    allocator (the PAD page ``P`` is never handed out).  A ``latent`` arena
    (absorbed multi-head latent attention) holds one row per token and kv
    head, ``[c | k_pe]``, whose first ``head_dim_v`` dims are the values:
    ``kv_pool_v`` is then a view of ``kv_pool_k``, not a second pool."""

    def __init__(self, *, geometry, max_physical_pages, num_kv_heads,
                 num_query_heads=None, head_dim_k, head_dim_v, dtype, device,
                 latent=False):
        self.geometry = geometry
        self.max_physical_pages = max_physical_pages
        self.PAD_PAGE_ID = max_physical_pages
        self.num_kv_heads = num_kv_heads
        self.head_dim_k = head_dim_k
        self.head_dim_v = head_dim_v
        self.latent = bool(latent)
        self.dtype = dtype
        self.device = device
        shape = (max_physical_pages + 1, 1, num_kv_heads, geometry.page)
        self.kv_pool_k = torch.empty(shape + (head_dim_k,), dtype=dtype, device=device)
        if self.latent:
            if head_dim_v > head_dim_k:
                raise ValueError('latent values are the first dims of the key rows')
            self.kv_pool_v = self.kv_pool_k[..., :head_dim_v]
        else:
            self.kv_pool_v = torch.empty(shape + (head_dim_v,), dtype=dtype, device=device)
        self.kv_pool_k[-1].zero_()
        self.kv_pool_v[-1].zero_()
        self._fresh = 0          # pages [_fresh, P) were never handed out
        self._returned = []      # sorted ids handed back by finished requests

    @property
    def free_ids(self):
        return self._returned + list(range(self._fresh, self.max_physical_pages))

    def free_count(self):
        return len(self._returned) + self.max_physical_pages - self._fresh

    def alloc_pages(self, count):
        if count > self.free_count():
            raise RuntimeError('graph-ready physical page pool exhausted')
        reuse = min(count, len(self._returned))
        out = self._returned[:reuse]
        del self._returned[:reuse]
        out += range(self._fresh, self._fresh + count - reuse)
        self._fresh += count - reuse
        return out

    def release_pages(self, ids):
        for pid in ids:
            if pid == self.PAD_PAGE_ID:
                raise RuntimeError('PAD page leaked into free_ids')
            bisect.insort(self._returned, pid)


class _Bank:
    """Pinned host mirror of the step-metadata arenas plus the block-table
    entries of pages opened in a step, and the event after its uploads."""

    def __init__(self, n32, n64, cross, pinned):
        def buf(n, dtype):
            t = torch.zeros(n, dtype=dtype)
            return t.pin_memory() if pinned else t
        self.i32 = buf(n32, torch.int32)
        self.i64 = buf(n64, torch.int64)
        self.cross_at = buf(cross, torch.int64)
        self.cross_pid = buf(cross, torch.int32)
        self.a32, self.a64 = self.i32.numpy(), self.i64.numpy()
        self.at, self.pid = self.cross_at.numpy(), self.cross_pid.numpy()
        self.done = None

    def wait(self):
        if self.done is not None:
            self.done.synchronize()
            self.done = None


class GraphReadyPagedRegionCache:
    """Continuous-batching coordinator over per-layer arenas.

    Block tables and slot mapping are per layer; ``gather_indices_buf`` and
    ``visible_lens_buf`` are per layer because layers may skip different
    regions.  The selector writes them in place.
    """

    INVALID_REQ_ID = -1
    paged_regions = True
    nfa_regions = True
    is_compileable = False

    def __init__(self, n_layers, geometry, *, max_requests, max_physical_pages,
                 max_blocks, max_visible_len, max_query_tokens, num_kv_heads,
                 num_query_heads=None, head_dim_k, head_dim_v, dtype, device,
                 visible_buckets=None, latent=False):
        device = torch.device(device)
        self.geometry = geometry
        self.n_layers = n_layers
        self.max_requests = max_requests
        self.max_blocks = max_blocks
        self.max_visible_len = max_visible_len
        self.max_query_tokens = max_query_tokens
        self.num_kv_heads = num_kv_heads
        self.num_query_heads = num_query_heads or num_kv_heads
        # a latent arena (absorbed MLA: one shared row per token) selects per
        # query head, so its gather rows are per query head
        self.latent = bool(latent)
        if self.latent and num_kv_heads != 1:
            raise ValueError('a latent arena holds one kv head')
        self.selection_heads = self.num_query_heads if self.latent else num_kv_heads
        self.layers = [
            GraphReadyPagedRegionLayer(
                geometry=geometry, max_physical_pages=max_physical_pages,
                num_kv_heads=num_kv_heads, head_dim_k=head_dim_k,
                head_dim_v=head_dim_v, dtype=dtype, device=device,
                latent=self.latent)
            for _ in range(n_layers)]
        self.layer_kv_ptrs_buf = torch.tensor(
            [layer.kv_pool_k.data_ptr() for layer in self.layers],
            dtype=torch.int64, device=device)

        self.states = {}
        self.request_phases = {}
        self.pending_lengths = {}
        self.active_request_id = None
        self.active_req_ids = []
        self.nfa_decode_steps = 0
        self.step_opens_page = False      # this step's token opens a page
        self._layout = None               # (row ids, state refs) of new_step
        self._planned_layout = None       # the layout the device metadata has
        self._row_pages = {}              # row -> current physical page per layer

        pad = max_physical_pages
        q, r, nl = max_query_tokens, max_requests, n_layers
        i32, i64 = torch.int32, torch.int64
        # step-metadata arenas: [planned lengths | slots per layer | query ->
        # row | query start offsets] and [active ids | valid ids]
        self._o_slots, self._o_q2r = q, q + nl * q
        self._o_qsl = self._o_q2r + q
        n32 = self._o_qsl + r + 1
        self._meta32 = torch.zeros(n32, dtype=i32, device=device)
        self._meta64 = torch.zeros(2 * q, dtype=i64, device=device)
        self.planned_lengths_buf = self._meta32[:q]
        self.slot_mapping_buf = self._meta32[q:self._o_q2r].view(nl, q)
        self.query_to_req_buf = self._meta32[self._o_q2r:self._o_qsl]
        self.query_start_loc_buf = self._meta32[self._o_qsl:]
        self.active_req_ids_buf = self._meta64[:q]
        self.valid_req_ids_buf = self._meta64[q:]
        self.slot_mapping_buf.fill_(PAD_SLOT)
        self.query_to_req_buf.fill_(-1)
        self.active_req_ids_buf.fill_(self.INVALID_REQ_ID)
        self.query_req_ids_buf = torch.arange(q, dtype=i64, device=device)
        self.block_table_buf = torch.full((nl, r, max_blocks), pad, dtype=i32,
                                          device=device)
        sh = self.selection_heads
        self.gather_indices_buf = torch.full((nl, r, sh, max_visible_len),
                                             INVALID_GATHER_IDX, dtype=i32, device=device)
        self.visible_lens_buf = torch.zeros((nl, r, sh), dtype=i32, device=device)
        self.skip_far_layer_buf = torch.zeros((nl, r), dtype=i32, device=device)
        self.skip_near_layer_buf = torch.zeros((nl, r), dtype=i32, device=device)

        self._pinned = device.type == 'cuda'
        self._banks = [_Bank(n32, 2 * q, q * nl, self._pinned) for _ in range(2)]
        for bank in self._banks:   # the device arenas' initial contents
            bank.a32[self._o_slots:self._o_qsl] = -1
            bank.a64[:q] = self.INVALID_REQ_ID
        self._bank_turn = 0
        self._cross_at_dev = torch.zeros(q * nl, dtype=i64, device=device)
        self._cross_pid_dev = torch.zeros(q * nl, dtype=i32, device=device)

        self._gather_indices_by_vis = {}
        self._visible_lens_by_vis = {}
        self.active_visible_bucket = max_visible_len
        if visible_buckets:
            self.ensure_visible_buckets(visible_buckets)

    # ------------------------------------------------------------------
    # visible-length buckets
    # ------------------------------------------------------------------
    def ensure_visible_buckets(self, buckets):
        for width in (int(w) for w in buckets):
            if not 0 < width <= self.max_visible_len:
                raise ValueError(
                    f'visible bucket {width} outside (0, {self.max_visible_len}]')
            if width < self.max_visible_len and width not in self._gather_indices_by_vis:
                shape = (self.n_layers, self.max_requests, self.selection_heads)
                dev = self.gather_indices_buf.device
                self._gather_indices_by_vis[width] = torch.full(
                    shape + (width,), INVALID_GATHER_IDX, dtype=torch.int32, device=dev)
                self._visible_lens_by_vis[width] = torch.zeros(
                    shape, dtype=torch.int32, device=dev)

    def set_active_visible_bucket(self, width):
        width = int(width)
        if width != self.max_visible_len and width not in self._gather_indices_by_vis:
            raise ValueError(f'visible bucket {width} has not been prepared')
        self.active_visible_bucket = width

    def _bucket_buffers(self):
        width = self.active_visible_bucket
        if width == self.max_visible_len:
            return self.gather_indices_buf, self.visible_lens_buf
        return self._gather_indices_by_vis[width], self._visible_lens_by_vis[width]

    def gather_indices_for_layer(self, layer_idx):
        return self._bucket_buffers()[0][layer_idx]

    def visible_lens_for_layer(self, layer_idx):
        return self._bucket_buffers()[1][layer_idx]

    def slot_mapping_for_layer(self, layer_idx):
        return self.slot_mapping_buf[layer_idx]

    def _visible_spans(self, state, layer_idx, length):
        """Token intervals a layer keeps visible for a row of ``length``:
        sink and window always, far and near unless frozen as skipped."""
        sink_hi, far_hi, near_hi = self.geometry.bounds(length)
        spans = [(0, sink_hi)]
        if not state.skip_far_by_layer[layer_idx]:
            spans.append((sink_hi, far_hi))
        if not state.skip_near_by_layer[layer_idx]:
            spans.append((far_hi, near_hi))
        spans.append((near_hi, length))
        return [(a, b) for a, b in spans if a < b]

    def choose_visible_bucket(self, req_ids, visible_buckets):
        """Smallest bucket holding every live row's kept regions at the
        length its next step plans (the full width when none does)."""
        need = 0
        for rid in req_ids:
            state = self.states.get(rid) if rid is not None and rid >= 0 else None
            if state is None:
                continue
            length = self.pending_lengths.get(rid, state.logical_length + 1)
            groups = state.skip_policy_groups or self._policy_groups(state)
            for _, layer_idx in groups:
                need = max(need, sum(b - a for a, b in
                                     self._visible_spans(state, layer_idx, length)))
        fits = [w for w in sorted(visible_buckets) if w >= need]
        return fits[0] if fits else self.max_visible_len

    # ------------------------------------------------------------------
    # request lifecycle
    # ------------------------------------------------------------------
    def add_request(self, request_id=None):
        if request_id is None:
            free = [r for r in range(self.max_requests) if r not in self.states]
            if not free:
                raise RuntimeError('no free request slot')
            request_id = free[0]
        if not 0 <= request_id < self.max_requests:
            raise ValueError('request_id outside fixed batch capacity')
        if request_id in self.states:
            raise ValueError(f'request {request_id} already active')
        self.states[request_id] = RequestState(
            block_tables=[_PageRun() for _ in range(self.n_layers)])
        self.request_phases[request_id] = RequestPhase.PREFILL
        return request_id

    def transition_request(self, request_id, phase):
        phase = RequestPhase(phase)
        now = self.request_phases.get(request_id)
        if now is None:
            raise ValueError(f'unknown request phase slot {request_id}')
        if phase == now:
            return
        if phase not in _NEXT_PHASES[now]:
            raise ValueError(
                f'invalid request phase transition {now.value} -> {phase.value}')
        self.request_phases[request_id] = phase
        if request_id in self.states:
            self.states[request_id].phase = phase

    def remove_request(self, request_id):
        state = self.states.pop(request_id, None)
        if state is None:
            return
        if self.layers[0].kv_pool_k.is_cuda:
            # queued kernels may still read the pages
            torch.cuda.synchronize(self.layers[0].kv_pool_k.device)
        for layer, run in zip(self.layers, state.block_tables):
            layer.release_pages(run.physical())
        self._planned_layout = None
        if self.active_request_id == request_id:
            self.active_request_id = None

    def set_active_request(self, request_id):
        if request_id not in self.states:
            raise ValueError(f'unknown request {request_id}')
        self.active_request_id = request_id

    # ------------------------------------------------------------------
    # prefill and freeze
    # ------------------------------------------------------------------
    def _table_row(self, run):
        row = np.full(self.max_blocks, self.layers[0].PAD_PAGE_ID, dtype=np.int32)
        ids = run.physical()[:self.max_blocks]
        row[:len(ids)] = ids
        return row

    def _upload_rows(self, request_id, layer_ids):
        """Write the block-table rows of ``request_id`` for ``layer_ids``."""
        state = self.states[request_id]
        rows = np.stack([self._table_row(state.block_tables[l]) for l in layer_ids])
        src = torch.from_numpy(rows)
        if len(layer_ids) == self.n_layers:
            self.block_table_buf[:, request_id].copy_(src)
        else:
            for i, l in enumerate(layer_ids):
                self.block_table_buf[l, request_id].copy_(src[i])

    def write_prefill(self, layer_idx, request_id, keys, values):
        state = self.states[request_id]
        layer = self.layers[layer_idx]
        page = self.geometry.page
        if keys.ndim != 4 or keys.shape[0] != 1 or keys.shape[-2] < 1:
            raise ValueError('graph-ready prefill expects unpadded B1 KV')
        if keys.shape[1] != layer.num_kv_heads:
            raise ValueError('KV head count does not match arena')
        if values is None:
            if not layer.latent:
                raise ValueError('prefill values are required (not a latent arena)')
        elif keys.device != values.device or keys.dtype != values.dtype:
            raise ValueError('KV dtype/device mismatch')
        n = keys.shape[-2]
        pages = -(-n // page)
        if pages > self.max_blocks:
            raise ValueError('prefill length exceeds fixed block-table capacity')
        run = state.block_tables[layer_idx]
        if run:
            if n != state.prompt_length:
                raise ValueError('prefill length diverged across layers')
        else:
            for pid in layer.alloc_pages(pages):
                run.append(pid)
            state.prompt_length = state.logical_length = n
        self._upload_rows(request_id, [layer_idx])
        from ..ops.paged_region_kernels import paged_write_prefill
        return paged_write_prefill(
            layer, keys, values, self.block_table_buf[layer_idx, request_id],
            workspace=getattr(self, '_nfa_selector_workspace', None))

    def freeze(self, request_id, skip_far_list, skip_near_list):
        state = self.states[request_id]
        if len(skip_far_list) != self.n_layers or len(skip_near_list) != self.n_layers:
            raise ValueError('freeze expects per-layer skip decisions')
        if state.logical_length == 0:
            raise ValueError('prefill before freeze')
        page = self.geometry.page
        if -(-(state.prompt_length + self.geometry.max_new_tokens) // page) > self.max_blocks:
            raise ValueError('prompt + max_new_tokens exceeds fixed block-table capacity')
        state.skip_far_by_layer = [bool(x) for x in skip_far_list]
        state.skip_near_by_layer = [bool(x) for x in skip_near_list]
        state.skip_policy_groups = self._policy_groups(state)
        flags = torch.tensor([state.skip_far_by_layer, state.skip_near_by_layer],
                             dtype=torch.int32)
        self.skip_far_layer_buf[:, request_id].copy_(flags[0])
        self.skip_near_layer_buf[:, request_id].copy_(flags[1])
        # a re-used request slot rebuilds its persistent page statistics
        lengths = getattr(self, '_nfa_page_stats_lengths', None)
        if lengths is not None:
            lengths[:, request_id].zero_()
        self._nfa_stats_dirty = True
        self._upload_rows(request_id, list(range(self.n_layers)))
        self._planned_layout = None
        state.frozen = True
        self.transition_request(request_id, RequestPhase.FREEZE)

    # ------------------------------------------------------------------
    # region helpers
    # ------------------------------------------------------------------
    def nfa_skip_signature(self, req_ids):
        """Per batch row, the frozen per-layer (skip_far, skip_near) pairs
        (None for padding rows); a graph capture on padding rows reports the
        live rows' signature instead."""
        override = self.__dict__.get('_nfa_signature_override')
        if override is not None:
            return override
        out = []
        for rid in req_ids:
            state = self.states.get(rid) if rid is not None and rid >= 0 else None
            out.append(None if state is None else
                       tuple(zip(state.skip_far_by_layer, state.skip_near_by_layer)))
        return tuple(out)

    @staticmethod
    def nfa_region_mode(signature, layer_idx):
        """Selector region mode of a layer: 0 none skipped (or rows differ),
        1 far skipped, 2 near skipped, 3 both."""
        pairs = {row[layer_idx] for row in signature if row is not None}
        if len(pairs) != 1:
            return 0
        skip_far, skip_near = pairs.pop()
        return (1 if skip_far else 0) + (2 if skip_near else 0)

    def _intervals_for_layer(self, state, layer_idx, length):
        return self._visible_spans(state, layer_idx, length)

    def _policy_groups(self, state):
        """((skip_far, skip_near), first layer) per distinct frozen policy."""
        first = {}
        for l, key in enumerate(zip(state.skip_far_by_layer, state.skip_near_by_layer)):
            first.setdefault((bool(key[0]), bool(key[1])), l)
        return tuple(first.items())

    # ------------------------------------------------------------------
    # step planning
    # ------------------------------------------------------------------
    def _next_bank(self):
        bank = self._banks[self._bank_turn]
        self._bank_turn ^= 1
        bank.wait()
        return bank

    def _mark(self, bank):
        if self._pinned and not torch.cuda.is_current_stream_capturing():
            bank.done = torch.cuda.Event()
            bank.done.record()

    def _grow(self, rid, state, length, opened):
        """Give every layer of ``state`` the pages ``length`` tokens need;
        new (flat block-table index, page) pairs are appended to ``opened``."""
        if length < state.logical_length:
            raise ValueError('paged block tables cannot move backwards')
        capacity = state.prompt_length + self.geometry.max_new_tokens
        if length > capacity:
            raise RuntimeError(
                f'planned length {length} exceeds request capacity {capacity}')
        need = -(-length // self.geometry.page)
        if need > self.max_blocks:
            raise RuntimeError('planned length exceeds fixed block-table capacity')
        for l, (layer, run) in enumerate(zip(self.layers, state.block_tables)):
            if len(run) >= need:
                continue
            start = len(run)
            for lp, pid in enumerate(layer.alloc_pages(need - start), start):
                run.append(pid)
                opened.append(((l * self.max_requests + rid) * self.max_blocks + lp, pid))

    def _upload_opened(self, bank, opened):
        """Scatter the block-table entries of newly opened pages."""
        if not opened:
            return
        n = len(opened)
        bank.at[:n] = [a for a, _ in opened]
        bank.pid[:n] = [p for _, p in opened]
        nb = self._pinned
        at = self._cross_at_dev[:n]
        pid = self._cross_pid_dev[:n]
        at.copy_(bank.cross_at[:n], non_blocking=nb)
        pid.copy_(bank.cross_pid[:n], non_blocking=nb)
        # scatter_ queues without a host synchronisation (index_copy_ waits)
        self.block_table_buf.view(-1).scatter_(0, at, pid)

    def new_step(self, active_req_ids):
        rows = tuple(active_req_ids)
        refs = tuple(self.states.get(r) if r is not None and r >= 0 else None
                     for r in rows)
        self._layout = (rows, refs)
        self.active_req_ids = list(rows)
        page = self.geometry.page
        self.step_opens_page = any(s is not None and s.logical_length % page == 0
                                   for s in refs)

    def plan_common(self, active_req_ids, query_lengths=None):
        """Plan this step's device metadata (lengths, slots, block-table
        growth).  A decode step of an unchanged layout only moves each live
        row forward by one token."""
        rows = tuple(active_req_ids)
        self.new_step(rows)
        if query_lengths is None:
            query_lengths = [1 if (r >= 0 and r in self.states) else 0 for r in rows]
        if not self._plan_decode(query_lengths):
            self._plan_full(query_lengths)

    def _plan_decode(self, query_lengths):
        rows, refs = self._layout
        if self._planned_layout is None or self._planned_layout != (
                rows, tuple(map(id, refs))):
            return False
        page = self.geometry.page
        for i, state in enumerate(refs):
            want = 0 if state is None else 1
            if (query_lengths[i] if i < len(query_lengths) else 0) != want:
                return False
            if state is not None and (
                    state.logical_length + 1 > state.prompt_length + self.geometry.max_new_tokens
                    or state.logical_length // page >= self.max_blocks):
                return False
        bank = self._next_bank()
        batch = len(rows)
        slots = bank.a32[self._o_slots:self._o_q2r].reshape(self.n_layers, -1)
        opened = []
        self.pending_lengths.clear()
        tok = 0
        for b, (rid, state) in enumerate(zip(rows, refs)):
            if state is None:
                bank.a32[b] = 0
                continue
            pos = state.logical_length
            if pos % page == 0:
                self._grow(rid, state, pos + 1, opened)
                self._row_pages[b] = np.array(
                    [run[pos // page] for run in state.block_tables], dtype=np.int64)
            slots[:, tok] = self._row_pages[b] * page + pos % page
            bank.a32[b] = pos + 1
            self.pending_lengths[rid] = pos + 1
            tok += 1
        slots[:, tok:batch] = PAD_SLOT
        nb = self._pinned
        # lengths and the slots of the first `batch` query tokens of every
        # layer: the arena prefix up to the last layer's row
        end = self._o_slots + (self.n_layers - 1) * self.max_query_tokens + batch
        self._meta32[:end].copy_(bank.i32[:end], non_blocking=nb)
        self._upload_opened(bank, opened)
        self._mark(bank)
        return True

    def _plan_full(self, query_lengths):
        rows, refs = self._layout
        batch = len(rows)
        page = self.geometry.page
        bank = self._next_bank()
        a32, a64 = bank.a32, bank.a64
        q = self.max_query_tokens
        a32[:] = 0
        a32[self._o_slots:self._o_qsl] = -1          # slots and query -> row
        a64[:q] = self.INVALID_REQ_ID
        a64[q:] = 0
        slots = a32[self._o_slots:self._o_q2r].reshape(self.n_layers, q)
        self.pending_lengths.clear()
        self._row_pages = {}
        opened = []
        tok = 0
        for b, (rid, state) in enumerate(zip(rows, refs)):
            a32[self._o_qsl + b] = tok
            qlen = int(query_lengths[b]) if b < len(query_lengths) else 0
            if state is None:
                tok += qlen
                continue
            planned = state.logical_length + qlen
            self._grow(rid, state, planned, opened)
            a32[b] = planned
            a64[b] = a64[q + b] = rid
            self.pending_lengths[rid] = planned
            for pos in range(state.logical_length, planned):
                lp = pos // page
                pids = np.array([run.get(lp, -1) for run in state.block_tables],
                                dtype=np.int64)
                if (pids < 0).any():
                    raise RuntimeError(f'missing logical page {lp} for request {rid}')
                slots[:, tok] = pids * page + pos % page
                a32[self._o_q2r + tok] = b
                tok += 1
            last = max(planned - 1, 0) // page
            self._row_pages[b] = np.array(
                [run.get(last, self.layers[0].PAD_PAGE_ID) for run in state.block_tables],
                dtype=np.int64)
        a32[self._o_qsl + batch:] = tok
        nb = self._pinned
        for rid, state in zip(rows, refs):
            if state is not None:
                self._upload_rows(rid, list(range(self.n_layers)))
        self._meta32.copy_(bank.i32, non_blocking=nb)
        self._meta64.copy_(bank.i64, non_blocking=nb)
        self._mark(bank)
        self._planned_layout = (rows, tuple(map(id, refs)))
        self.step_opens_page = False

    # ------------------------------------------------------------------
    # dense (region-interval) and given selections -> gather rows
    # ------------------------------------------------------------------
    def _physical(self, state, layer_idx, ids):
        """Physical slots of logical token ids (negative ids stay invalid)."""
        ids = np.asarray(ids, dtype=np.int64)
        page = self.geometry.page
        run = np.asarray(state.block_tables[layer_idx].physical(), dtype=np.int64)
        ok = (ids >= 0) & (ids // page < len(run))
        pages = run[np.where(ok, ids // page, 0)] if len(run) else np.zeros_like(ids)
        return np.where(ok, pages * page + ids % page, INVALID_GATHER_IDX).astype(np.int32)

    def _layer_gather(self, layer_idx, req_ids, selected_ids_by_req=None):
        dev = self.gather_indices_buf.device
        width = self.max_visible_len
        lens = np.zeros((self.max_requests, self.num_kv_heads), dtype=np.int32)
        for b, rid in enumerate(req_ids):
            state = self.states.get(rid) if rid >= 0 else None
            if state is None:
                continue
            length = self.pending_lengths.get(rid, state.logical_length)
            chosen = None if selected_ids_by_req is None else selected_ids_by_req.get(rid)
            count = None
            if chosen is None:
                ids = np.concatenate([np.arange(a, e) for a, e in
                                      self._visible_spans(state, layer_idx, length)]
                                     or [np.zeros(0, np.int64)])
                if len(ids) > width:
                    raise RuntimeError(
                        f'request {rid} layer {layer_idx} visible_len {len(ids)} '
                        f'exceeds fixed capacity {width}')
            else:
                if isinstance(chosen, tuple):
                    chosen, count = chosen
                ids = (chosen.detach().reshape(-1).cpu().numpy()
                       if isinstance(chosen, torch.Tensor) else np.asarray(chosen).reshape(-1))
                if count is None and len(ids) > width:
                    raise RuntimeError(
                        f'request {rid} layer {layer_idx} visible_len {len(ids)} '
                        f'exceeds fixed capacity {width}')
                ids = ids[:width]
            n = len(ids)
            if count is not None:
                count = int(torch.as_tensor(count).reshape(()))
                if count > width:
                    raise RuntimeError(f'request {rid} layer {layer_idx} visible_len '
                                       f'{count} exceeds fixed capacity {width}')
            lens[b] = n if count is None else count
            if n:
                slots = torch.from_numpy(self._physical(state, layer_idx, ids))
                self.gather_indices_buf[layer_idx, b, :, :n].copy_(
                    slots.to(dev).expand(self.num_kv_heads, n))
        self.visible_lens_buf[layer_idx].copy_(torch.from_numpy(lens))

    def _plan_if_stale(self, active_req_ids, query_lengths):
        rows = tuple(active_req_ids)
        if self._layout is None or self._layout[0] != rows:
            self.new_step(rows)
        stale = (self._planned_layout is None or self.step_opens_page
                 or self._planned_layout[0] != rows)
        if stale:
            if query_lengths is None:
                query_lengths = [1 if (r >= 0 and r in self.states) else 0 for r in rows]
            self._plan_full(query_lengths)

    def prepare_metadata(self, active_req_ids, current_layer_id,
                         query_lengths=None, selected_ids_by_req=None):
        """Gather rows of one layer: the kept region intervals of every row,
        or the given logical ids (a tensor/list, or ``(ids, count)``)."""
        if not 0 <= current_layer_id < self.n_layers:
            raise ValueError('invalid layer id')
        self._plan_if_stale(active_req_ids, query_lengths)
        self._layer_gather(current_layer_id, active_req_ids, selected_ids_by_req)
        return (self.gather_indices_buf[current_layer_id],
                self.visible_lens_buf[current_layer_id])

    def prepare_all_layers(self, active_req_ids, query_lengths=None,
                           selected_ids_by_layer=None, visible_bucket=None):
        """``prepare_metadata`` for every layer (a layer given as the string
        ``'__prepared__'`` is left as it is), then a copy into the visible
        bucket's rows, which becomes the active bucket."""
        self.active_req_ids = list(active_req_ids)
        self._plan_if_stale(active_req_ids, query_lengths)
        for layer_idx in range(self.n_layers):
            chosen = (None if selected_ids_by_layer is None
                      else selected_ids_by_layer.get(layer_idx))
            if isinstance(chosen, str) and chosen == '__prepared__':
                continue
            self._layer_gather(layer_idx, active_req_ids, chosen)
        if visible_bucket is not None:
            width = int(visible_bucket)
            if width != self.max_visible_len:
                self.ensure_visible_buckets((width,))
                self._gather_indices_by_vis[width].copy_(
                    self.gather_indices_buf[..., :width])
                self._visible_lens_by_vis[width].copy_(self.visible_lens_buf)
            self.active_visible_bucket = width

    def commit_step(self):
        """Advance request lengths once every layer of the step has run."""
        for rid, length in self.pending_lengths.items():
            self.states[rid].logical_length = length
        self.pending_lengths.clear()

    # ------------------------------------------------------------------
    # decode write and HF-cache compatibility
    # ------------------------------------------------------------------
    def write_decode(self, layer_idx, key_states, value_states, slot_mapping):
        if key_states.ndim != 4 or key_states.shape[-2] != 1:
            raise ValueError('graph-ready decode KV must be one token per row')
        if key_states.shape[0] != slot_mapping.shape[0]:
            raise ValueError('request batch must match KV batch')
        from ..ops.paged_region_kernels import paged_write_decode
        return paged_write_decode(
            self.layers[layer_idx], key_states, value_states, slot_mapping,
            workspace=getattr(self, '_nfa_selector_workspace', None))

    def block_table(self):
        return self.block_table_buf

    def slot_mapping(self):
        return self.slot_mapping_buf

    def query_start_loc(self):
        return self.query_start_loc_buf

    def get_max_cache_shape(self):
        return -1

    def get_seq_length(self, layer_idx=0):
        if self.active_request_id is not None:
            return self.states[self.active_request_id].logical_length
        return max((s.logical_length for s in self.states.values()), default=0)

    def get_query_offset(self, layer_idx=0):
        """Position of the first query token: the tokens already cached."""
        return self.get_seq_length(layer_idx)

    def get_mask_sizes(self, cache_position, layer_idx=0):
        query_len = (cache_position if isinstance(cache_position, int)
                     else cache_position.shape[0])
        return self.get_seq_length(layer_idx) + query_len, 0

    def report(self):
        return {
            'requests': len(self.states),
            'active_requests': list(self.states),
            'n_layers': self.n_layers,
            'layers': [{'num_kv_heads': l.num_kv_heads, 'head_dim_k': l.head_dim_k,
                        'head_dim_v': l.head_dim_v} for l in self.layers],
        }
