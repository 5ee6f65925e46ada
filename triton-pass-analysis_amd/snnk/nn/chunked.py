"""T-chunked execution driver (snn_compiler/nn/chunked.py:31-79).

A network whose neurons carry their membrane across calls (``StatefulLIFNode``
with ``v_init`` / ``return_v``) can run a long sequence chunk by chunk: each
chunk of ``chunk_t`` steps flows through every layer, the per-layer membranes
go into a state dict, and the next chunk resumes from it.  Peak activation
memory then scales with ``chunk_t`` instead of T.  Spikes are identical to one
pass over the whole sequence, since the LIF recurrence is serial in t and the
carried fp32 membrane is exactly the state the single pass holds at the chunk
boundary.
"""
from __future__ import annotations

from typing import Callable

import torch
import torch.nn as nn


def run_chunked(
    forward_fn: Callable[[torch.Tensor, dict | None], tuple[torch.Tensor, dict]],
    x_seq: torch.Tensor,
    *,
    chunk_t: int = 16,
) -> torch.Tensor:
    """Drive ``forward_fn(x_chunk, state) -> (y_chunk, state)`` over ``[T, B, ...]``.

    ``state`` is ``None`` on the first call and whatever the previous call
    returned afterwards.  With ``chunk_t >= T`` the whole sequence is one call
    (snn_compiler/nn/chunked.py:49-51); otherwise the outputs of the chunks
    (the last one may be shorter) are concatenated along T.
    """
    if chunk_t < 1:
        raise ValueError(f"chunk_t must be >= 1, got {chunk_t}")
    T = x_seq.shape[0]
    if chunk_t >= T:
        out, _ = forward_fn(x_seq, None)
        return out
    outs = []
    state = None
    for t0 in range(0, T, chunk_t):
        y, state = forward_fn(x_seq[t0:t0 + chunk_t].contiguous(), state)
        outs.append(y)
    return torch.cat(outs, dim=0)


class ChunkedForward(nn.Module):
    """Wrap a network so that ``forward(x_seq)`` runs chunked
    (snn_compiler/nn/chunked.py:64-79).

    The network provides ``forward_chunked(x_chunk, state) -> (y, state)``;
    without it the wrapper calls the plain forward (no chunking).
    """

    def __init__(self, model: nn.Module, *, chunk_t: int = 16):
        super().__init__()
        self.model = model
        self.chunk_t = chunk_t

    def forward(self, x_seq):
        if not hasattr(self.model, "forward_chunked"):
            return self.model(x_seq)
        return run_chunked(self.model.forward_chunked, x_seq, chunk_t=self.chunk_t)
