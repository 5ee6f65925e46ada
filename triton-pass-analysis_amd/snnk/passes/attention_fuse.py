"""Replace spiking attention blocks by FusedSpikeAttention
(mirror of snn_compiler/passes/attention_fuse.py:14-35)."""
from __future__ import annotations

import torch.nn as nn

from ..nn.attention import FusedSpikeAttention, is_spiking_attention
from .fuse import _set_submodule


def fuse_spiking_attention(model: nn.Module, *, fold_bn: bool = False,
                           ktv_mode: str = "bmm") -> int:
    """Swap every detected spiking attention block (ssa / ms) for
    ``FusedSpikeAttention.from_reference`` in place; returns the count.
    ``fold_bn=False`` keeps the result bit-identical to the blocks."""
    targets = [(n, m) for n, m in model.named_modules() if n and is_spiking_attention(m)]
    for name, m in targets:
        _set_submodule(model, name,
                       FusedSpikeAttention.from_reference(m, fold_bn=fold_bn, ktv_mode=ktv_mode))
    return len(targets)
