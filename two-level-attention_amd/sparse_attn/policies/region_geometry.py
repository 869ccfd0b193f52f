"""Token-region boundaries of a sequence (reference policies/region_geometry.py:6-23)."""
from dataclasses import dataclass


@dataclass(frozen=True)
class RegionGeometry:
    """Sink / far / near / sliding-window layout of one request.

    ``bounds(length)`` returns ``(sink_hi, far_hi, near_hi)``: sink tokens are
    ``[0, sink_hi)``, far ``[sink_hi, far_hi)``, near ``[far_hi, near_hi)`` and
    the window ``[near_hi, length)``; ``far_hi`` is page aligned.
    """
    sink: int = 4
    near: int = 4096
    window: int = 128
    page: int = 64
    max_new_tokens: int = 512

    def __post_init__(self):
        for name in ('sink', 'near', 'window', 'page', 'max_new_tokens'):
            value = getattr(self, name)
            floor = 0 if name == 'sink' else 1
            if isinstance(value, bool) or not isinstance(value, int) or value < floor:
                raise ValueError(f'invalid {name}: {value}')

    def bounds(self, length):
        sink_hi = min(self.sink, length)
        near_hi = max(sink_hi, length - self.window)
        aligned = ((length - self.window - self.near) // self.page) * self.page
        far_hi = min(near_hi, max(sink_hi, aligned))
        return sink_hi, far_hi, near_hi
