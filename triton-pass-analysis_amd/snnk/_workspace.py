"""Device workspace for the split-K conv / linear entry points.

One zero-filled buffer per device, shared by every call on it (the kernels
leave their ticket counters at zero, so it never needs clearing).  It grows
when a call needs more; a replaced buffer is kept alive because a captured
HIP graph may still point at it.  Growing inside a graph capture would record
an allocation and a fill into the graph, so it raises instead: run the layer
once before capturing it.
"""
from __future__ import annotations

import torch

_MIN_BYTES = 32 << 20
_current: dict[int, torch.Tensor] = {}
_retired: list[torch.Tensor] = []


def get(device: torch.device, nbytes: int) -> torch.Tensor | None:
    if nbytes <= 0:
        return None
    idx = device.index if device.index is not None else torch.cuda.current_device()
    t = _current.get(idx)
    if t is None or t.numel() < nbytes:
        if torch.cuda.is_current_stream_capturing():
            raise RuntimeError(
                f"snnk needs a {nbytes}-byte split-K workspace on cuda:{idx} during graph "
                "capture; run the same layer once before capturing")
        if t is not None:
            _retired.append(t)
        size = max(_MIN_BYTES, (nbytes + (1 << 20) - 1) >> 20 << 20)
        t = torch.zeros(size, dtype=torch.uint8, device=f"cuda:{idx}")
        _current[idx] = t
    return t
