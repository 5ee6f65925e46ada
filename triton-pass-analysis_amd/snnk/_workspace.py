"""Device workspaces for the split-K conv / Linear entry points.

A workspace holds a region of ticket counters followed by the partial sums
of one call; calls that run at the same time must not share one.  Work on
one stream runs in order, so the pool keeps one zero-filled buffer per
(device, stream): split-K calls on two streams get distinct buffers and
cannot race.  The kernels leave their ticket counters at zero, so a buffer
never needs clearing.  A buffer grows when a call needs more; a replaced
buffer is kept alive because a captured HIP graph may still point at it.

Growing inside a graph capture would record an allocation and a fill into
the graph, so it raises instead: run the layer once on the capture stream
before capturing it (the capture then reuses that stream's buffer, and the
graph owns its address for the rest of the process).
"""
from __future__ import annotations

from typing import Callable, Optional

import torch

MIN_BYTES = 32 << 20


def _zeros(device_index: int, nbytes: int) -> torch.Tensor:
    return torch.zeros(nbytes, dtype=torch.uint8, device=f"cuda:{device_index}")


class WorkspacePool:
    """Zero-filled byte buffers keyed by (device index, stream handle)."""

    def __init__(self, alloc: Callable[[int, int], torch.Tensor] = _zeros,
                 min_bytes: int = MIN_BYTES):
        self._alloc = alloc
        self._min = min_bytes
        self._current: dict[tuple[int, int], torch.Tensor] = {}
        self._retired: list[torch.Tensor] = []

    def get(self, device_index: int, stream: int, nbytes: int,
            capturing: bool = False) -> Optional[torch.Tensor]:
        if nbytes <= 0:
            return None
        key = (device_index, stream)
        buf = self._current.get(key)
        if buf is not None and buf.numel() >= nbytes:
            return buf
        if capturing:
            raise RuntimeError(
                f"snnk needs a {nbytes}-byte split-K workspace on cuda:{device_index} "
                f"for stream {stream:#x} during graph capture; run the same layer once on "
                "the capture stream before capturing")
        if buf is not None:
            self._retired.append(buf)
        size = max(self._min, (nbytes + (1 << 20) - 1) >> 20 << 20)
        buf = self._alloc(device_index, size)
        self._current[key] = buf
        return buf

    def buffers(self) -> dict[tuple[int, int], torch.Tensor]:
        return dict(self._current)


_pool = WorkspacePool()


def get(device: torch.device, nbytes: int) -> torch.Tensor | None:
    """The workspace of the current stream on ``device`` (at least ``nbytes``)."""
    if nbytes <= 0:
        return None
    idx = device.index if device.index is not None else torch.cuda.current_device()
    stream = torch.cuda.current_stream(idx).cuda_stream
    return _pool.get(idx, stream, nbytes, torch.cuda.is_current_stream_capturing())
