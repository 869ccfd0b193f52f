"""Deferred device error flags read at request boundaries.

Reference: sparse_attn/ops/eager_decoding.py:10-69.  One int32 flag per
device; 0 means no error, codes 1-4 name the failed contract.  Flags are
shared per device, so request boundaries using the guard must be serialised.
"""
from contextlib import contextmanager

import torch

_ERR_FLAG = {}

_MESSAGES = {
    1: 'eager_decoding_attn: a selection row is empty; softmax would be NaN '
       '(check the sink/SWA forced-selection contract)',
    2: 'eager_decoding_attn: a row selects more tokens than its upper bound; '
       'the request was rejected',
    3: 'eager_decoding_attn: cu_seqlens_k contract broken; the request was '
       'rejected (check the caller length metadata)',
    4: 'ordered attention: invalid selected token IDs, counts or live '
       'lengths; request rejected',
}


def _err_flag(device: torch.device) -> torch.Tensor:
    buf = _ERR_FLAG.get(device)
    if buf is None:
        with torch.inference_mode(False):
            buf = torch.zeros(1, dtype=torch.int32, device=device)
        _ERR_FLAG[device] = buf
    return buf


def _raise_for_code(code: int):
    if code in _MESSAGES:
        raise RuntimeError(_MESSAGES[code])


def eager_decoding_check_errors(device=None, clear: bool = True):
    """Read (and by default clear) the deferred flags; raise on a set code."""
    if device is None:
        bufs = list(_ERR_FLAG.values())
    else:
        buf = _ERR_FLAG.get(torch.device(device))
        bufs = [] if buf is None else [buf]
    for buf in bufs:
        code = int(buf.item())
        if clear:
            buf.zero_()
        _raise_for_code(code)


@contextmanager
def eager_decoding_request_guard(device=None):
    """Clear stale flags, run the request, then consume its flags."""
    for buf in list(_ERR_FLAG.values()):
        buf.zero_()
    try:
        yield
    finally:
        eager_decoding_check_errors(device)
