"""Graph-ready paged KV cache with a continuous-batching request lifecycle.

Drop-in for the reference's ``sparse_attn/cache/paged_region_cache.py``
(``GraphReadyPagedRegionLayer`` :60-112, ``GraphReadyPagedRegionCache``
:115-1113): same constructor, buffer names, shapes and dtypes, same public
methods and error behaviour.  Every device buffer has a fixed address for the
cache's lifetime, metadata reaches the device through pinned staging copies,
and steady-state decode only advances planned lengths and slots, so a decode
step can be captured into a hipGraph.

Layout of the KV arena per layer: ``[P + 1, 1, hkv, page, D]``; the extra
last page is a zeroed PAD page that invalid block-table entries point at.
Physical slot of a token = ``page_id * page + offset``.
"""
import heapq
from dataclasses import dataclass, field
from enum import Enum

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


_PHASE_NEXT = {
    RequestPhase.PREFILL: {RequestPhase.FREEZE, RequestPhase.FAILED},
    RequestPhase.FREEZE: {RequestPhase.SUFFIX, RequestPhase.GENERATE,
                          RequestPhase.FINISHED, RequestPhase.FAILED},
    RequestPhase.SUFFIX: {RequestPhase.GENERATE, RequestPhase.FINISHED,
                          RequestPhase.FAILED},
    RequestPhase.GENERATE: {RequestPhase.FINISHED, RequestPhase.FAILED},
    RequestPhase.FINISHED: set(),
    RequestPhase.FAILED: set(),
}


@dataclass
class RequestState:
    """One request slot.  ``block_tables[layer]`` maps logical page ->
    physical page and only ever grows while the request lives."""
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
    """Physical KV arena of one layer plus its page free-list."""

    def __init__(self, *, geometry, max_physical_pages, num_kv_heads,
                 num_query_heads=None, head_dim_k, head_dim_v, dtype, device):
        self.geometry = geometry
        self.max_physical_pages = max_physical_pages
        self.PAD_PAGE_ID = max_physical_pages
        self.num_kv_heads = num_kv_heads
        self.head_dim_k = head_dim_k
        self.head_dim_v = head_dim_v
        self.dtype = dtype
        self.device = device
        pages = max_physical_pages + 1
        self.kv_pool_k = torch.empty(
            (pages, 1, num_kv_heads, geometry.page, head_dim_k),
            dtype=dtype, device=device)
        self.kv_pool_v = torch.empty(
            (pages, 1, num_kv_heads, geometry.page, head_dim_v),
            dtype=dtype, device=device)
        self.kv_pool_k[self.PAD_PAGE_ID].zero_()
        self.kv_pool_v[self.PAD_PAGE_ID].zero_()
        self.free_ids = list(range(max_physical_pages))
        heapq.heapify(self.free_ids)

    def alloc_pages(self, count):
        if len(self.free_ids) < count:
            raise RuntimeError('graph-ready physical page pool exhausted')
        return [heapq.heappop(self.free_ids) for _ in range(count)]


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
                 visible_buckets=None):
        device = torch.device(device)
        self.geometry = geometry
        self.n_layers = n_layers
        self.max_requests = max_requests
        self.max_blocks = max_blocks
        self.max_visible_len = max_visible_len
        self.max_query_tokens = max_query_tokens
        self.num_kv_heads = num_kv_heads
        self.num_query_heads = (num_kv_heads if num_query_heads is None
                                else num_query_heads)
        self.layers = [
            GraphReadyPagedRegionLayer(
                geometry=geometry, max_physical_pages=max_physical_pages,
                num_kv_heads=num_kv_heads, head_dim_k=head_dim_k,
                head_dim_v=head_dim_v, dtype=dtype, device=device)
            for _ in range(n_layers)]
        self.layer_kv_ptrs_buf = torch.tensor(
            [layer.kv_pool_k.data_ptr() for layer in self.layers],
            dtype=torch.int64, device=device)

        self.states = {}
        self.request_phases = {}
        self.pending_lengths = {}
        self.active_request_id = None
        self.active_req_ids = []
        self.common_dirty = True
        self._page_cross = False  # a row's next token opens a new logical page
        self._common_active_req_ids = ()
        self._common_state_refs = ()
        self._common_layout_revision = -1
        self.request_layout_revision = 0
        self._layout_req_ids = ()
        self._layout_state_refs = ()
        self._layout_source = None
        self._visible_bucket_cache = {}
        self.nfa_decode_steps = 0

        pad = self.layers[0].PAD_PAGE_ID
        i32, i64 = torch.int32, torch.int64
        self.block_table_buf = torch.full(
            (n_layers, max_requests, max_blocks), pad, dtype=i32, device=device)
        self.slot_mapping_buf = torch.full(
            (n_layers, max_query_tokens), PAD_SLOT, dtype=i32, device=device)
        self.query_start_loc_buf = torch.zeros(
            (max_requests + 1,), dtype=i32, device=device)
        self.query_to_req_buf = torch.full(
            (max_query_tokens,), -1, dtype=i32, device=device)
        self.active_req_ids_buf = torch.full(
            (max_query_tokens,), self.INVALID_REQ_ID, dtype=i64, device=device)
        self.valid_req_ids_buf = torch.zeros(
            (max_query_tokens,), dtype=i64, device=device)
        self.query_req_ids_buf = torch.arange(
            max_query_tokens, dtype=i64, device=device)
        self.planned_lengths_buf = torch.zeros(
            (max_query_tokens,), dtype=i32, device=device)
        self.gather_indices_buf = torch.full(
            (n_layers, max_requests, num_kv_heads, max_visible_len),
            INVALID_GATHER_IDX, dtype=i32, device=device)
        self.visible_lens_buf = torch.zeros(
            (n_layers, max_requests, num_kv_heads), dtype=i32, device=device)
        self.skip_far_layer_buf = torch.zeros(
            (n_layers, max_requests), dtype=i32, device=device)
        self.skip_near_layer_buf = torch.zeros(
            (n_layers, max_requests), dtype=i32, device=device)

        pin = device.type == 'cuda'
        # pinned staging buffers feed asynchronous copies; a buffer is only
        # rewritten once the device has executed the last copy out of it
        self._pinned_staging = pin
        self._staging_event = None

        def staging(shape, fill, dtype):
            t = torch.full(shape, fill, dtype=dtype, device='cpu')
            return t.pin_memory() if pin else t

        self._cpu_gather_staging = torch.full(
            (max_requests, num_kv_heads, max_visible_len), INVALID_GATHER_IDX,
            dtype=i32, device='cpu')
        self._gather_logical_tmp = torch.empty(
            (max_visible_len,), dtype=i32, device=device)
        self._cpu_block_table_staging = staging(
            (n_layers, max_requests, max_blocks), pad, i32)
        self._cpu_slot_mapping_staging = staging(
            (n_layers, max_query_tokens), PAD_SLOT, i32)
        self._cpu_query_start_loc_staging = staging((max_requests + 1,), 0, i32)
        self._cpu_query_to_req_staging = staging((max_query_tokens,), -1, i32)
        self._cpu_active_req_ids_staging = staging(
            (max_query_tokens,), self.INVALID_REQ_ID, i64)
        self._cpu_valid_req_ids_staging = torch.zeros(
            (max_query_tokens,), dtype=i64, device='cpu')
        self._cpu_planned_lengths_staging = staging((max_query_tokens,), 0, i32)
        # rows opening a new page in a steady step: (query token index,
        # request, logical page, physical page of every layer)
        self._cpu_cross_staging = staging((max_query_tokens, 3 + n_layers), 0, i64)
        self._cpu_skip_far_layer_staging = staging((n_layers, max_requests), 0, i32)
        self._cpu_skip_near_layer_staging = staging((n_layers, max_requests), 0, i32)

        self._gather_indices_by_vis = {}
        self._visible_lens_by_vis = {}
        self.active_visible_bucket = max_visible_len
        if visible_buckets:
            self.ensure_visible_buckets(visible_buckets)

    # ------------------------------------------------------------------
    # visible-length buckets
    # ------------------------------------------------------------------
    def ensure_visible_buckets(self, buckets):
        for width in buckets:
            width = int(width)
            if width <= 0 or width > self.max_visible_len:
                raise ValueError(
                    f'visible bucket {width} outside (0, {self.max_visible_len}]')
            if width == self.max_visible_len or width in self._gather_indices_by_vis:
                continue
            dev = self.gather_indices_buf.device
            self._gather_indices_by_vis[width] = torch.full(
                (self.n_layers, self.max_requests, self.num_kv_heads, width),
                INVALID_GATHER_IDX, dtype=torch.int32, device=dev)
            self._visible_lens_by_vis[width] = torch.zeros(
                (self.n_layers, self.max_requests, self.num_kv_heads),
                dtype=torch.int32, device=dev)

    def set_active_visible_bucket(self, width):
        width = int(width)
        if width != self.max_visible_len and width not in self._gather_indices_by_vis:
            raise ValueError(f'visible bucket {width} has not been prepared')
        self.active_visible_bucket = width

    def gather_indices_for_layer(self, layer_idx):
        width = self.active_visible_bucket
        if width != self.max_visible_len:
            return self._gather_indices_by_vis[width][layer_idx]
        return self.gather_indices_buf[layer_idx]

    def visible_lens_for_layer(self, layer_idx):
        width = self.active_visible_bucket
        if width != self.max_visible_len:
            return self._visible_lens_by_vis[width][layer_idx]
        return self.visible_lens_buf[layer_idx]

    def slot_mapping_for_layer(self, layer_idx):
        return self.slot_mapping_buf[layer_idx]

    def choose_visible_bucket(self, req_ids, visible_buckets):
        """Smallest bucket covering every request's dense region intervals;
        a cached answer is reused while the length growth fits in it."""
        states, lengths, policies = [], [], []
        for rid in req_ids:
            if rid is None or rid < 0 or rid not in self.states:
                states.append(None)
                lengths.append(-1)
                policies.append(None)
                continue
            state = self.states[rid]
            states.append(state)
            lengths.append(self.pending_lengths.get(rid, state.logical_length))
            groups = state.skip_policy_groups or self._build_skip_policy_groups(state)
            policies.append(tuple(key for key, _ in groups))
        key = (tuple(policies), len(req_ids), tuple(sorted(visible_buckets)))
        cached = self._visible_bucket_cache.get(key)
        refs = tuple(states)
        cur = tuple(lengths)
        if cached is not None:
            old_refs, old_lengths, old_max, old_width = cached
            if old_refs == refs and all(n >= o for n, o in zip(cur, old_lengths)):
                grow = max((n - o for n, o in zip(cur, old_lengths)), default=0)
                if old_max + grow <= old_width:
                    return old_width
        max_total = 0
        for state, length in zip(states, lengths):
            if state is None:
                continue
            groups = state.skip_policy_groups or self._build_skip_policy_groups(state)
            for _, layer_idx in groups:
                spans = self._intervals_for_layer(state, layer_idx, length)
                max_total = max(max_total, sum(b - a for a, b in spans))
        width = self.max_visible_len
        for cand in sorted(visible_buckets):
            if cand >= max_total:
                width = cand
                break
        self._visible_bucket_cache[key] = (refs, cur, max_total, width)
        return width

    # ------------------------------------------------------------------
    # request lifecycle
    # ------------------------------------------------------------------
    def _alloc_pages(self, layer_idx, count):
        return self.layers[layer_idx].alloc_pages(count)

    def _staging_wait(self):
        """Block until the device has executed the last asynchronous copy
        out of the pinned staging buffers, so that they can be rewritten."""
        ev = self._staging_event
        if ev is not None:
            self._staging_event = None
            ev.synchronize()

    def _staging_mark(self):
        """Mark the copies just enqueued out of the staging buffers."""
        if self._pinned_staging and not torch.cuda.is_current_stream_capturing():
            ev = torch.cuda.Event()
            ev.record()
            self._staging_event = ev

    def add_request(self, request_id=None):
        if request_id is None:
            request_id = self._next_free_slot()
        if request_id < 0 or request_id >= self.max_requests:
            raise ValueError('request_id outside fixed batch capacity')
        if request_id in self.states:
            raise ValueError(f'request {request_id} already active')
        self.states[request_id] = RequestState(
            block_tables=[{} for _ in range(self.n_layers)])
        self.request_phases[request_id] = RequestPhase.PREFILL
        self._staging_wait()
        self._cpu_block_table_staging[:, request_id].fill_(self.layers[0].PAD_PAGE_ID)
        return request_id

    def transition_request(self, request_id, phase):
        phase = RequestPhase(phase)
        current = self.request_phases.get(request_id)
        if current is None:
            raise ValueError(f'unknown request phase slot {request_id}')
        if current == phase:
            return
        if phase not in _PHASE_NEXT[current]:
            raise ValueError(
                f'invalid request phase transition {current.value} -> {phase.value}')
        self.request_phases[request_id] = phase
        state = self.states.get(request_id)
        if state is not None:
            state.phase = phase

    def _next_free_slot(self):
        for rid in range(self.max_requests):
            if rid not in self.states:
                return rid
        raise RuntimeError('no free request slot')

    def remove_request(self, request_id):
        state = self.states.pop(request_id, None)
        if state is None:
            return
        freed = [set(state.block_tables[l].values()) for l in range(self.n_layers)]
        self._staging_wait()
        self._cpu_block_table_staging[:, request_id].fill_(self.layers[0].PAD_PAGE_ID)
        if self.layers[0].kv_pool_k.is_cuda:
            # pages may still be read by queued kernels; return them only
            # after the device is idle
            torch.cuda.synchronize(self.layers[0].kv_pool_k.device)
        for layer_idx, ids in enumerate(freed):
            layer = self.layers[layer_idx]
            for pid in sorted(ids):
                if pid == layer.PAD_PAGE_ID:
                    raise RuntimeError('PAD page leaked into free_ids')
                heapq.heappush(layer.free_ids, pid)
        if self.active_request_id == request_id:
            self.active_request_id = None

    def set_active_request(self, request_id):
        if request_id not in self.states:
            raise ValueError(f'unknown request {request_id}')
        self.active_request_id = request_id

    # ------------------------------------------------------------------
    # prefill and freeze
    # ------------------------------------------------------------------
    def write_prefill(self, layer_idx, request_id, keys, values):
        state = self.states[request_id]
        layer = self.layers[layer_idx]
        page = self.geometry.page
        if keys.ndim != 4 or keys.shape[0] != 1 or keys.shape[-2] < 1:
            raise ValueError('graph-ready prefill expects unpadded B1 KV')
        if keys.shape[1] != layer.num_kv_heads:
            raise ValueError('KV head count does not match arena')
        if keys.device != values.device or keys.dtype != values.dtype:
            raise ValueError('KV dtype/device mismatch')
        n = keys.shape[-2]
        if (n + page - 1) // page > self.max_blocks:
            raise ValueError('prefill length exceeds fixed block-table capacity')
        table = state.block_tables[layer_idx]
        if not table:
            logical = list(range((n + page - 1) // page))
            state.block_tables[layer_idx] = dict(
                zip(logical, self._alloc_pages(layer_idx, len(logical))))
            table = state.block_tables[layer_idx]
            state.prompt_length = n
            state.logical_length = n
        elif n != state.prompt_length:
            raise ValueError('prefill length diverged across layers')
        self._staging_wait()
        row = self._cpu_block_table_staging[layer_idx, request_id]
        row.fill_(self.layers[0].PAD_PAGE_ID)
        for lp, pid in table.items():
            if 0 <= lp < self.max_blocks:
                row[lp] = pid
        self.block_table_buf[layer_idx, request_id].copy_(row, non_blocking=keys.is_cuda)
        self._staging_mark()
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
        state.skip_far_by_layer = [bool(x) for x in skip_far_list]
        state.skip_near_by_layer = [bool(x) for x in skip_near_list]
        state.skip_policy_groups = self._build_skip_policy_groups(state)
        self._staging_wait()
        self._cpu_skip_far_layer_staging[:, request_id] = torch.as_tensor(
            state.skip_far_by_layer, dtype=torch.int32)
        self._cpu_skip_near_layer_staging[:, request_id] = torch.as_tensor(
            state.skip_near_by_layer, dtype=torch.int32)
        nb = self.layers[0].kv_pool_k.is_cuda
        self.skip_far_layer_buf[:, request_id].copy_(
            self._cpu_skip_far_layer_staging[:, request_id], non_blocking=nb)
        self.skip_near_layer_buf[:, request_id].copy_(
            self._cpu_skip_near_layer_staging[:, request_id], non_blocking=nb)
        # a reused request slot must rebuild its persistent page statistics
        if hasattr(self, '_nfa_page_stats_lengths'):
            self._nfa_page_stats_lengths[:, request_id].zero_()
        self._nfa_stats_dirty = True
        page = self.geometry.page
        cap_pages = (state.prompt_length + self.geometry.max_new_tokens
                     + page - 1) // page
        if cap_pages > self.max_blocks:
            raise ValueError('prompt + max_new_tokens exceeds fixed block-table capacity')
        self._write_block_table_row(request_id, state)
        self.block_table_buf[:, request_id].copy_(
            self._cpu_block_table_staging[:, request_id], non_blocking=nb)
        self._staging_mark()
        self.common_dirty = True
        self.request_layout_revision += 1
        self._layout_source = None
        state.frozen = True
        self.transition_request(request_id, RequestPhase.FREEZE)

    # ------------------------------------------------------------------
    # region helpers
    # ------------------------------------------------------------------
    def nfa_skip_signature(self, req_ids):
        """Per batch row, the frozen per-layer (skip_far, skip_near) tuple."""
        override = getattr(self, '_nfa_capture_skip_signature', None)
        if override is not None:
            return override
        sig = []
        for rid in req_ids:
            state = self.states.get(rid) if rid is not None and rid >= 0 else None
            sig.append(None if state is None else tuple(
                zip(state.skip_far_by_layer, state.skip_near_by_layer)))
        return tuple(sig)

    @staticmethod
    def nfa_region_mode(signature, layer_idx):
        """0 full, 1 skip-far, 2 skip-near, 3 both skipped; 0 if rows differ."""
        modes = [item[layer_idx] for item in signature if item is not None]
        if not modes or any(m != modes[0] for m in modes[1:]):
            return 0
        skip_far, skip_near = modes[0]
        if skip_far and skip_near:
            return 3
        if skip_far:
            return 1
        if skip_near:
            return 2
        return 0

    def _intervals_for_layer(self, state, layer_idx, length):
        sink_hi, far_hi, near_hi = self.geometry.bounds(length)
        spans = [(0, sink_hi), (near_hi, length)]
        if not state.skip_far_by_layer[layer_idx]:
            spans.append((sink_hi, far_hi))
        if not state.skip_near_by_layer[layer_idx]:
            spans.append((far_hi, near_hi))
        return sorted((a, b) for a, b in spans if a < b)

    def _build_skip_policy_groups(self, state):
        groups, seen = [], set()
        for layer_idx in range(self.n_layers):
            key = (bool(state.skip_far_by_layer[layer_idx]),
                   bool(state.skip_near_by_layer[layer_idx]))
            if key not in seen:
                seen.add(key)
                groups.append((key, layer_idx))
        return tuple(groups)

    def _write_block_table_row(self, request_id, state):
        pad = self.layers[0].PAD_PAGE_ID
        for layer_idx in range(self.n_layers):
            row = self._cpu_block_table_staging[layer_idx, request_id]
            row.fill_(pad)
            for lp, pid in state.block_tables[layer_idx].items():
                if 0 <= lp < self.max_blocks:
                    row[lp] = pid

    def _sync_block_table(self, state, length, request_id=None):
        """Append physical pages for newly reached logical pages only."""
        if length < state.logical_length:
            raise ValueError('paged block tables cannot move backwards')
        capacity = state.prompt_length + self.geometry.max_new_tokens
        if length > capacity:
            raise RuntimeError(
                f'planned length {length} exceeds request capacity {capacity}')
        page = self.geometry.page
        needed = (length + page - 1) // page
        if needed > self.max_blocks:
            raise RuntimeError('planned length exceeds fixed block-table capacity')
        for layer_idx in range(self.n_layers):
            table = state.block_tables[layer_idx]
            first_missing = len(table)
            if first_missing >= needed:
                continue
            # logical pages are only ever appended, so the table holds exactly
            # 0 .. first_missing - 1 when its last key is first_missing - 1
            if first_missing and next(reversed(table)) != first_missing - 1:
                raise RuntimeError('physical block table is not append-only')
            missing = range(first_missing, needed)
            ids = self._alloc_pages(layer_idx, len(missing))
            for lp, pid in zip(missing, ids):
                table[lp] = pid
                if request_id is not None:
                    self._cpu_block_table_staging[layer_idx, request_id, lp] = pid

    # ------------------------------------------------------------------
    # metadata
    # ------------------------------------------------------------------
    def _logical_to_slots(self, layer_idx, batch_idx, ids):
        page = self.geometry.page
        if page & (page - 1) == 0:
            pages = ids >> (page.bit_length() - 1)
            offsets = ids & (page - 1)
        else:
            pages = torch.div(ids, page, rounding_mode='floor')
            offsets = torch.remainder(ids, page)
        safe = torch.clamp(pages, min=0, max=self.max_blocks - 1)
        table = self.block_table_buf[layer_idx, batch_idx]
        phys = table.gather(-1, safe.to(torch.int64))
        slots = phys.to(torch.int32) * page + offsets.to(torch.int32)
        return torch.where(ids >= 0, slots, torch.full_like(slots, INVALID_GATHER_IDX))

    def _store_gather_slots(self, layer_idx, batch_idx, logical_ids, width):
        """Write ``logical_ids[:width]`` as absolute physical slots."""
        if width <= 0:
            return
        ids = logical_ids[:width].to(self.gather_indices_buf.device,
                                     torch.int32).contiguous()
        slots = self._logical_to_slots(layer_idx, batch_idx, ids)
        self.gather_indices_buf[layer_idx, batch_idx, :, :width].copy_(
            slots.unsqueeze(0), non_blocking=True)

    def _store_gather_slots_batch(self, layer_idx, logical_ids, counts):
        """Batch form of ``_store_gather_slots`` for ``[B,W]``/``[B,Hkv,W]``."""
        if logical_ids.numel() == 0 or counts.numel() == 0:
            return
        if logical_ids.ndim == 2:
            logical_ids = logical_ids.unsqueeze(1)
        if logical_ids.ndim != 3 or logical_ids.shape[1] != self.num_kv_heads:
            raise ValueError('logical gather ids must be [B,W] or [B,Hkv,W]')
        batch, _, width = logical_ids.shape
        ids = logical_ids.to(self.gather_indices_buf.device, torch.int32).contiguous()
        page = self.geometry.page
        pages = torch.div(ids, page, rounding_mode='floor')
        offsets = torch.remainder(ids, page)
        safe = torch.clamp(pages, min=0, max=self.max_blocks - 1)
        table = self.block_table_buf[layer_idx, :batch, None, :].expand(
            -1, ids.shape[1], -1)
        phys = table.gather(2, safe.to(torch.int64))
        slots = phys.to(torch.int32) * page + offsets.to(torch.int32)
        slots = torch.where(ids >= 0, slots, torch.full_like(slots, INVALID_GATHER_IDX))
        self.gather_indices_buf[layer_idx, :batch, :, :width].copy_(slots, non_blocking=True)
        if counts.ndim == 1:
            counts = counts.unsqueeze(1)
        self.visible_lens_buf[layer_idx, :batch].copy_(
            counts.to(torch.int32), non_blocking=True)

    def new_step(self, active_req_ids):
        req_ids = tuple(active_req_ids)
        refs = tuple(self.states.get(r) if r is not None and r >= 0 else None
                     for r in req_ids)
        changed = (req_ids != self._layout_req_ids
                   or len(refs) != len(self._layout_state_refs)
                   or any(n is not o for n, o in zip(refs, self._layout_state_refs)))
        if changed:
            self.request_layout_revision += 1
            self._layout_req_ids = req_ids
            self._layout_state_refs = refs
        self._layout_source = active_req_ids
        page = self.geometry.page
        # the next token of a row opens a new logical page: the steady plan
        # appends that page; the dense-metadata planners re-plan fully
        self._page_cross = any(state is not None and state.logical_length % page == 0
                               for state in refs)
        self.active_req_ids = list(req_ids)
        self.common_dirty = self.common_dirty or changed

    def plan_common(self, active_req_ids, query_lengths=None):
        """Plan this step's metadata; steady decode only advances lengths."""
        if active_req_ids is not self._layout_source:
            self.new_step(active_req_ids)
        if query_lengths is None:
            query_lengths = [1 if (r >= 0 and r in self.states) else 0
                             for r in active_req_ids]
        self.active_req_ids = list(active_req_ids)
        if self.common_dirty:
            self._prepare_common(active_req_ids, query_lengths)
        elif not self._prepare_decode_common_fast(active_req_ids, query_lengths):
            self._prepare_common(active_req_ids, query_lengths)

    def _prepare_decode_common_fast(self, req_ids, query_lengths):
        """Steady decode: one token per live row.  Every slot moves by one;
        a row whose token opens a new logical page gets that page appended
        in every layer and its slots pointed at the page's first slot."""
        if self.request_layout_revision != self._common_layout_revision:
            return False
        req_ids = self._layout_req_ids
        refs = self._layout_state_refs
        batch = len(req_ids)
        planned = []
        crossing = []  # (batch row, query token index) of rows opening a page
        flat = 0
        page = self.geometry.page
        for row, (rid, state) in enumerate(zip(req_ids, refs)):
            qlen = int(query_lengths[row]) if row < len(query_lengths) else 0
            if qlen != (1 if state is not None else 0):
                return False
            if state is None:
                planned.append(0)
                continue
            length = state.logical_length + qlen
            if length > state.prompt_length + self.geometry.max_new_tokens:
                return False
            if qlen and state.logical_length % page == 0:  # the token opens a page
                if (length - 1) // page >= self.max_blocks:
                    return False
                crossing.append((row, flat))
            planned.append(length)
            flat += qlen
        slots = self.slot_mapping_buf[:, :batch]
        slots.add_(slots >= 0)
        self._staging_wait()
        self.pending_lengths.clear()
        for row, (rid, state) in enumerate(zip(req_ids, refs)):
            self._cpu_planned_lengths_staging[row] = planned[row]
            if state is not None:
                self.pending_lengths[rid] = planned[row]
        self.planned_lengths_buf[:batch].copy_(
            self._cpu_planned_lengths_staging[:batch], non_blocking=True)
        if crossing:
            st = self._cpu_cross_staging
            for i, (row, tok) in enumerate(crossing):
                rid, state = req_ids[row], refs[row]
                self._sync_block_table(state, planned[row], request_id=rid)
                lp = (planned[row] - 1) // page
                st[i, 0], st[i, 1], st[i, 2] = tok, rid, lp
                for layer_idx in range(self.n_layers):
                    st[i, 3 + layer_idx] = state.block_tables[layer_idx][lp]
            dev = st[:len(crossing)].to(slots.device, non_blocking=True)
            pids = dev[:, 3:].t().to(torch.int32)  # [layers, rows]
            self.block_table_buf[:, dev[:, 1], dev[:, 2]] = pids
            self.slot_mapping_buf[:, dev[:, 0]] = pids * page
        self._staging_mark()
        return True

    def _prepare_common(self, req_ids, query_lengths):
        page = self.geometry.page
        batch = len(req_ids)
        self._staging_wait()
        self._cpu_slot_mapping_staging[:, :batch].fill_(PAD_SLOT)
        self._cpu_query_to_req_staging.fill_(-1)  # tokens of padding rows
        self._cpu_active_req_ids_staging[:batch].fill_(self.INVALID_REQ_ID)
        self._cpu_valid_req_ids_staging[:batch].zero_()
        self._cpu_planned_lengths_staging[:batch].zero_()
        self.pending_lengths.clear()
        cumsum = 0
        flat = 0
        for b, rid in enumerate(req_ids):
            self._cpu_query_start_loc_staging[b] = cumsum
            qlen = int(query_lengths[b]) if b < len(query_lengths) else 0
            if rid < 0 or rid not in self.states:
                cumsum += qlen
                continue
            state = self.states[rid]
            planned = state.logical_length + qlen
            self._cpu_active_req_ids_staging[b] = rid
            self._cpu_valid_req_ids_staging[b] = rid
            self._cpu_planned_lengths_staging[b] = planned
            self._sync_block_table(state, planned, request_id=rid)
            self.pending_lengths[rid] = planned
            self.block_table_buf[:, rid].copy_(
                self._cpu_block_table_staging[:, rid], non_blocking=True)
            for t in range(qlen):
                pos = state.logical_length + t
                lp, off = divmod(pos, page)
                for layer_idx in range(self.n_layers):
                    pid = state.block_tables[layer_idx].get(lp)
                    if pid is None:
                        raise RuntimeError(
                            f'missing logical page {lp} for request {rid} '
                            f'layer {layer_idx}')
                    self._cpu_slot_mapping_staging[layer_idx, flat] = pid * page + off
                self._cpu_query_to_req_staging[flat] = b
                flat += 1
            cumsum += qlen
        self._cpu_query_start_loc_staging[batch] = cumsum
        self.slot_mapping_buf[:, :flat].copy_(
            self._cpu_slot_mapping_staging[:, :flat], non_blocking=True)
        self.query_start_loc_buf.copy_(self._cpu_query_start_loc_staging, non_blocking=True)
        self.query_to_req_buf.copy_(self._cpu_query_to_req_staging, non_blocking=True)
        self.active_req_ids_buf.copy_(self._cpu_active_req_ids_staging, non_blocking=True)
        self.valid_req_ids_buf.copy_(self._cpu_valid_req_ids_staging, non_blocking=True)
        self.planned_lengths_buf.copy_(
            self._cpu_planned_lengths_staging, non_blocking=True)
        self._staging_mark()
        self._common_active_req_ids = tuple(req_ids)
        self._common_state_refs = tuple(
            self.states.get(r) if r is not None and r >= 0 else None for r in req_ids)
        self._common_layout_revision = self.request_layout_revision
        self.common_dirty = False
        self._page_cross = False

    def _prepare_layer_gather(self, layer_idx, req_ids, selected_ids_by_req=None):
        """Dense (region-interval) or given selections as physical slots."""
        self.visible_lens_buf[layer_idx].zero_()
        for b, rid in enumerate(req_ids):
            if rid < 0 or rid not in self.states:
                continue
            state = self.states[rid]
            length = self.pending_lengths.get(rid, state.logical_length)
            selected = None
            if selected_ids_by_req is not None:
                selected = selected_ids_by_req.get(rid)
            if selected is None:
                spans = self._intervals_for_layer(state, layer_idx, length)
                total = sum(e - a for a, e in spans)
                if total > self.max_visible_len:
                    raise RuntimeError(
                        f'request {rid} layer {layer_idx} visible_len {total} '
                        f'exceeds fixed capacity {self.max_visible_len}')
                off = 0
                for a, e in spans:
                    if e > a:
                        torch.arange(a, e, dtype=torch.int32,
                                     out=self._gather_logical_tmp[off:off + e - a])
                        off += e - a
                self._store_gather_slots(layer_idx, b, self._gather_logical_tmp, total)
                self.visible_lens_buf[layer_idx, b] = total
                continue
            count = None
            if isinstance(selected, tuple):
                selected, count = selected
                count = count.reshape(())
            elif not isinstance(selected, torch.Tensor):
                selected = torch.as_tensor(selected, dtype=torch.int32,
                                           device=self.gather_indices_buf.device)
            selected = selected.to(self.gather_indices_buf.device).reshape(-1)
            width = min(selected.numel(), self.max_visible_len)
            if count is not None:
                torch._assert_async(count <= self.max_visible_len)
                self.visible_lens_buf[layer_idx, b].copy_(count, non_blocking=True)
            else:
                if selected.numel() > self.max_visible_len:
                    raise RuntimeError(
                        f'request {rid} layer {layer_idx} visible_len '
                        f'{selected.numel()} exceeds fixed capacity '
                        f'{self.max_visible_len}')
                self.visible_lens_buf[layer_idx, b] = width
            if width:
                self._store_gather_slots(layer_idx, b, selected, width)

    def prepare_metadata(self, active_req_ids, current_layer_id,
                         query_lengths=None, selected_ids_by_req=None):
        if current_layer_id < 0 or current_layer_id >= self.n_layers:
            raise ValueError('invalid layer id')
        if self.common_dirty or self._page_cross:
            if query_lengths is None:
                query_lengths = [1 if (r >= 0 and r in self.states) else 0
                                 for r in active_req_ids]
            self._prepare_common(active_req_ids, query_lengths)
        self._prepare_layer_gather(current_layer_id, active_req_ids,
                                   selected_ids_by_req)
        return (self.gather_indices_buf[current_layer_id],
                self.visible_lens_buf[current_layer_id])

    def prepare_all_layers(self, active_req_ids, query_lengths=None,
                           selected_ids_by_layer=None, visible_bucket=None):
        if query_lengths is None:
            query_lengths = [1 if (r >= 0 and r in self.states) else 0
                             for r in active_req_ids]
        self.active_req_ids = list(active_req_ids)
        if self.common_dirty or self._page_cross:
            self._prepare_common(active_req_ids, query_lengths)
        for layer_idx in range(self.n_layers):
            selected = None
            if selected_ids_by_layer is not None:
                selected = selected_ids_by_layer.get(layer_idx)
            if isinstance(selected, str) and selected == '__prepared__':
                continue
            self._prepare_layer_gather(layer_idx, active_req_ids, selected)
        if visible_bucket is not None:
            visible_bucket = int(visible_bucket)
            if visible_bucket != self.max_visible_len:
                self.ensure_visible_buckets((visible_bucket,))
                dst_g = self._gather_indices_by_vis[visible_bucket]
                dst_l = self._visible_lens_by_vis[visible_bucket]
                for layer_idx in range(self.n_layers):
                    dst_g[layer_idx].copy_(
                        self.gather_indices_buf[layer_idx, :, :, :visible_bucket],
                        non_blocking=True)
                    dst_l[layer_idx].copy_(self.visible_lens_buf[layer_idx],
                                           non_blocking=True)
            self.active_visible_bucket = visible_bucket

    def commit_step(self):
        """Advance request lengths once after every layer of the step ran."""
        for rid, length in self.pending_lengths.items():
            self.states[rid].logical_length = length
        self.pending_lengths.clear()

    # ------------------------------------------------------------------
    # decode write and HF-cache compatibility
    # ------------------------------------------------------------------
    def write_decode(self, layer_idx, key_states, value_states, slot_mapping):
        layer = self.layers[layer_idx]
        if key_states.ndim != 4 or key_states.shape[-2] != 1:
            raise ValueError('graph-ready decode KV must be one token per row')
        if key_states.shape[0] != slot_mapping.shape[0]:
            raise ValueError('request batch must match KV batch')
        from ..ops.paged_region_kernels import paged_write_decode
        return paged_write_decode(
            layer, key_states, value_states, slot_mapping,
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
        if self.states:
            return max(s.logical_length for s in self.states.values())
        return 0

    def get_query_offset(self, layer_idx=0):
        """Position of the first query token: the tokens already cached."""
        return self.get_seq_length(layer_idx)

    def get_mask_sizes(self, cache_position, layer_idx=0):
        query_len = (cache_position if isinstance(cache_position, int)
                     else cache_position.shape[0])
        if self.active_request_id is not None:
            kv_len = self.states[self.active_request_id].logical_length
        else:
            kv_len = max((s.logical_length for s in self.states.values()), default=0)
        return kv_len + query_len, 0

    def report(self):
        return {
            'requests': len(self.states),
            'active_requests': list(self.states),
            'n_layers': self.n_layers,
            'layers': [{'num_kv_heads': l.num_kv_heads, 'head_dim_k': l.head_dim_k,
                        'head_dim_v': l.head_dim_v} for l in self.layers],
        }
