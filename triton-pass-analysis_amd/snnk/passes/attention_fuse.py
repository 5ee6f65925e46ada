"""Swap spiking attention blocks for FusedSpikeAttention.

Public API of ``snn_compiler/passes/attention_fuse.py:14-30``.
"""
from __future__ import annotations

import torch.nn as nn

from ..nn.attention import FusedSpikeAttention, attention_variant
from .fuse import replace_module


def fuse_spiking_attention(model: nn.Module, *, fold_bn: bool = False,
                           ktv_mode: str = "bmm") -> int:
    """Replace, in place, every block that :func:`attention_variant` recognises
    by ``FusedSpikeAttention.from_reference``; returns how many were replaced.
    ``fold_bn=False`` keeps the result bit-identical to the original blocks.
    Blocks are collected before any replacement, outermost first; a block
    nested inside one already replaced is left alone, and the model itself is
    never replaced (wrap it in a container to fuse a bare block)."""
    found = [name for name, m in model.named_modules()
             if name and attention_variant(m) is not None]
    done: list[str] = []
    for name in found:
        if any(name == d or name.startswith(d + ".") for d in done):
            continue
        fused = FusedSpikeAttention.from_reference(model.get_submodule(name), fold_bn=fold_bn,
                                                   ktv_mode=ktv_mode)
        replace_module(model, name, fused)
        done.append(name)
    return len(done)
