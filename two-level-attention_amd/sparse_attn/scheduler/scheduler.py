"""Device-resident continuous-batching scheduler for graph decode.

Reference: sparse_attn/scheduler/scheduler.py:38-328 (``greedy_next_tokens``,
``ContinuousBatchScheduler``).  Same public API and the same contract: the
next input token and position of every request live on the device, greedy
argmax never leaves it on the decode path, and each step's tokens reach the
host through a pinned double buffer copied on a side stream and drained at
the start of a later step.

Every device update here has a fixed shape (padded batch rows scatter into
one spare table row), so no step needs a host synchronisation or a
data-dependent allocation.
"""
import torch


def greedy_next_tokens(logits, eos_ids, *, generated_counts=0, min_new_tokens=0):
    """Argmax of the last position, EOS masked for rows that have generated
    fewer than ``min_new_tokens`` tokens (``generated_counts``: int, list or
    ``[B]`` tensor).  Returns ``[B]`` int64."""
    logits = getattr(logits, 'logits', logits)
    if logits.ndim != 3:
        raise ValueError('greedy decoding expects [B,T,V] logits')
    if min_new_tokens < 0:
        raise ValueError('min_new_tokens must be non-negative')
    last = logits[:, -1]
    batch = last.shape[0]
    counts = torch.as_tensor(generated_counts, dtype=torch.long, device=last.device)
    if counts.ndim == 0:
        counts = counts.expand(batch)
    if counts.ndim != 1 or counts.numel() != batch:
        raise ValueError('generated_counts must be scalar or [B]')
    eos_ids = tuple(int(t) for t in eos_ids)
    if eos_ids and min_new_tokens > 0:
        last = last.clone()  # never modify a graph's static output
        eos = torch.tensor(eos_ids, dtype=torch.long, device=last.device)
        blocked = (counts < min_new_tokens)[:, None]
        last[:, eos] = torch.where(blocked, last.new_full((), -torch.inf),
                                   last[:, eos])
    return last.argmax(dim=-1).to(torch.int64)


class ContinuousBatchScheduler:
    """Active request list plus device tables of next token / position."""

    def __init__(self, *, cache, max_batch, eos_ids, pad_token_id,
                 track_receipts=False, auto_finish_requests=True):
        self.cache = cache
        self.max_batch = int(max_batch)
        self.eos_ids = set(int(t) for t in eos_ids)
        self.pad_token_id = int(pad_token_id)
        self.track_receipts = track_receipts
        self.auto_finish_requests = auto_finish_requests
        self.active_req_ids = []
        self.next_tokens = {}
        self.device = cache.layers[0].kv_pool_k.device
        if self.device.type != 'cuda' or not torch.cuda.is_available():
            raise RuntimeError('ContinuousBatchScheduler requires a GPU')
        dev, i64 = self.device, torch.long
        self._spare = cache.max_requests  # padded rows scatter here
        rows = cache.max_requests + 1
        self._req_input = torch.full((rows,), self.pad_token_id, dtype=i64, device=dev)
        self._req_pos = torch.zeros((rows,), dtype=i64, device=dev)
        self._req_alive = torch.zeros((rows,), dtype=torch.bool, device=dev)
        self._req_ids_dev = torch.full((self.max_batch,), -1, dtype=i64, device=dev)
        self._input_ids = torch.full((self.max_batch, 1), self.pad_token_id,
                                     dtype=i64, device=dev)
        self._positions = torch.zeros((self.max_batch, 1), dtype=i64, device=dev)
        self._counts_dev = torch.zeros((self.max_batch,), dtype=i64, device=dev)
        self._eos_dev = torch.tensor(sorted(self.eos_ids) or [-1], dtype=i64, device=dev)
        self._req_staging = torch.full((self.max_batch,), -1, dtype=i64).pin_memory()
        self._counts_staging = torch.zeros((self.max_batch,), dtype=i64).pin_memory()
        self._seen = set()
        self._staged = None
        self._staged_copy = None
        # two receipt slots: device tokens, pinned host copy, their request ids
        self._tok_dev = [torch.zeros((self.max_batch,), dtype=i64, device=dev)
                         for _ in range(2)]
        self._tok_host = [torch.zeros((self.max_batch,), dtype=i64).pin_memory()
                          for _ in range(2)]
        self._tok_req = [torch.zeros((self.max_batch,), dtype=i64) for _ in range(2)]
        self._copy_stream = torch.cuda.Stream(device=dev)
        self._copy_done = [torch.cuda.Event() for _ in range(2)]
        self._pending = [None, None]  # (sequence, batch, stop_on_eos) per slot
        self._step_counter = 0
        self._ready_receipts = []

    # -- request set ---------------------------------------------------
    def add_request(self, request_id):
        if request_id not in self.active_req_ids:
            self.active_req_ids.append(request_id)
            self._seen.discard(request_id)

    def finish_request(self, request_id):
        self.cache.transition_request(request_id, 'FINISHED')
        self.cache.remove_request(request_id)
        if request_id in self.active_req_ids:
            self.active_req_ids.remove(request_id)
        self.next_tokens.pop(request_id, None)
        self._seen.discard(request_id)

    def _pad_to_bucket(self, req_ids):
        bucket = 1
        while bucket < len(req_ids):
            bucket <<= 1
        bucket = min(bucket, self.max_batch)
        if len(req_ids) > bucket:
            raise ValueError('active requests exceed the scheduler batch')
        return list(req_ids) + [-1] * (bucket - len(req_ids))

    # -- receipts ------------------------------------------------------
    def _drain_pending_next_tokens(self):
        """Consume the receipt slots whose copy has finished, oldest first;
        never waits."""
        ready = [(p[0], i) for i, p in enumerate(self._pending)
                 if p is not None and self._copy_done[i].query()]
        for _, idx in sorted(ready):
            _, batch, stop_on_eos = self._pending[idx]
            self._pending[idx] = None
            toks = self._tok_host[idx][:batch].tolist()
            rids = self._tok_req[idx][:batch].tolist()
            finished = []
            for rid, tok in zip(rids, toks):
                if rid < 0:
                    continue
                self.next_tokens[rid] = tok
                if self.track_receipts:
                    self._ready_receipts.append((rid, tok))
                if stop_on_eos and tok in self.eos_ids:
                    finished.append(rid)
            if self.auto_finish_requests:
                for rid in finished:
                    if rid in self.active_req_ids:
                        self.finish_request(rid)

    def pop_ready_receipts(self):
        """``(request_id, token)`` pairs whose copy has finished, in order."""
        self._drain_pending_next_tokens()
        out, self._ready_receipts = self._ready_receipts, []
        return out

    def flush_ready_receipts(self):
        """Wait for every pending copy and return all unread receipts."""
        for idx, pending in enumerate(self._pending):
            if pending is not None:
                self._copy_done[idx].synchronize()
        return self.pop_ready_receipts()

    # -- one step ------------------------------------------------------
    def _seed_new_requests(self, padded):
        fresh = [r for r in padded if r >= 0 and r not in self._seen]
        if not fresh:
            return
        for rid in fresh:
            self._seen.add(rid)
        idx = torch.tensor(fresh, dtype=torch.long)
        tok = torch.tensor([self.next_tokens.get(r, self.pad_token_id) for r in fresh],
                           dtype=torch.long)
        pos = torch.tensor([self.cache.states[r].logical_length for r in fresh],
                           dtype=torch.long)
        idx = idx.to(self.device)
        self._req_input[idx] = tok.to(self.device)
        self._req_pos[idx] = pos.to(self.device)
        self._req_alive[idx] = True

    def prepare_step(self):
        """Pad the active set to a batch bucket and gather each row's input
        token and position on the device.  Returns ``(padded_ids,
        input_ids [B,1], position_ids [B,1])``."""
        self._drain_pending_next_tokens()
        padded = self._pad_to_bucket(self.active_req_ids)
        batch = len(padded)
        if padded != self._staged:
            # the pinned row may still feed the last asynchronous copy
            if self._staged_copy is not None:
                self._staged_copy.synchronize()
            self._req_staging[:batch] = torch.tensor(padded, dtype=torch.long)
            self._staged = padded
        rids = self._req_ids_dev[:batch]
        rids.copy_(self._req_staging[:batch], non_blocking=True)
        self._staged_copy = torch.cuda.Event()
        self._staged_copy.record()
        self._req_ids_dev[batch:].fill_(-1)
        self._seed_new_requests(padded)
        valid = rids >= 0
        row = torch.where(valid, rids, torch.full_like(rids, self._spare))
        self._input_ids[:batch, 0] = torch.where(
            valid, self._req_input[row], torch.full_like(rids, self.pad_token_id))
        self._positions[:batch, 0] = torch.where(
            valid, self._req_pos[row], torch.zeros_like(rids))
        self.cache.new_step(padded)
        return padded, self._input_ids[:batch], self._positions[:batch]

    def record_next_tokens(self, req_ids, logits, *, generated_counts=0,
                           min_new_tokens=0, forced_tokens=None, stop_on_eos=True):
        """Greedy (or forced) next token per row; advances each live
        request's device input token and position and queues the host copy."""
        logits = getattr(logits, 'logits', logits)
        if logits.device.type != 'cuda':
            raise RuntimeError('ContinuousBatchScheduler requires device logits')
        batch = len(req_ids)
        if forced_tokens is None:
            counts = generated_counts
            if not isinstance(counts, torch.Tensor):
                staging = self._counts_staging[:batch]
                if isinstance(counts, int):
                    staging.fill_(counts)
                else:
                    staging.copy_(torch.as_tensor(counts, dtype=torch.long))
                counts = self._counts_dev[:batch]
                counts.copy_(staging, non_blocking=True)
            nxt = greedy_next_tokens(logits, self.eos_ids, generated_counts=counts,
                                     min_new_tokens=min_new_tokens)
        else:
            if len(forced_tokens) != batch:
                raise ValueError('forced token count must match the padded batch')
            nxt = torch.as_tensor(forced_tokens, dtype=torch.long, device=logits.device)
        slot = self._step_counter & 1
        if self._pending[slot] is not None:
            # reuse of a receipt slot: consume its tokens first
            self._copy_done[slot].synchronize()
            self._drain_pending_next_tokens()
        rids = self._req_ids_dev[:batch]
        valid = rids >= 0
        if stop_on_eos:
            alive = valid & ~torch.isin(nxt, self._eos_dev)
        else:
            alive = valid
        row = torch.where(valid, rids, torch.full_like(rids, self._spare))
        self._req_alive[row] = alive
        self._req_input[row] = torch.where(
            alive, nxt, torch.full_like(nxt, self.pad_token_id))
        self._req_pos.index_add_(0, row, alive.to(torch.long))

        self._tok_req[slot][:batch] = torch.tensor(req_ids, dtype=torch.long)
        self._tok_dev[slot][:batch].copy_(nxt)
        self._copy_stream.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(self._copy_stream):
            self._tok_host[slot][:batch].copy_(self._tok_dev[slot][:batch],
                                               non_blocking=True)
            self._copy_done[slot].record(self._copy_stream)
        self._pending[slot] = (self._step_counter, batch, stop_on_eos)
        self._step_counter += 1
        return nxt
