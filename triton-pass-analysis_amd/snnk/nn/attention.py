"""Fused spike attention module (mirror of snn_compiler/nn/attention.py, ssa variant).

``FusedSpikeAttention.from_reference`` takes a Spikingformer-style
SpikingSelfAttention block (Conv1d-1x1 q/k/v/proj + BatchNorm1d + LIF nodes,
``num_heads`` and ``scale``; detected like snn_compiler/nn/attention.py:40-59)
and runs it as: input LIF, one fused QKV projection (BN folded, bf16 MFMA,
LIF epilogue), the int8-MFMA attention core with its LIF, and the output
projection (BN folded).  forward takes and returns [T, B, C, H, W].
"""
from __future__ import annotations

import torch
import torch.nn as nn

from ..kernels.attention import spike_self_attention


def fold_conv1d_bn(conv: nn.Conv1d, bn: nn.BatchNorm1d):
    """Fold eval BatchNorm1d into a 1x1 Conv1d: W' = W*g/sqrt(var+eps),
    b' = (b - mean)*g/sqrt(var+eps) + beta (snn_compiler/nn/attention.py:28-33)."""
    inv = bn.weight.detach() / torch.sqrt(bn.running_var.detach() + bn.eps)
    w = conv.weight.detach() * inv.view(-1, 1, 1)
    cb = conv.bias.detach() if conv.bias is not None else torch.zeros_like(bn.bias)
    b = (cb - bn.running_mean.detach()) * inv + bn.bias.detach()
    return w, b.float().contiguous()


def _lif_pv(node):
    return float(getattr(node, "tau", 2.0)), float(getattr(node, "v_threshold", 1.0))


def _has_lifs_and_core(m):
    return all(hasattr(m, n) for n in ("q_lif", "k_lif", "v_lif", "attn_lif", "q_conv",
                                       "k_conv", "v_conv", "proj_conv", "num_heads", "scale"))


def is_spiking_self_attention(m: nn.Module) -> bool:
    """Spikingformer SSA: Conv1d projections + BatchNorm1d + proj_lif."""
    return (_has_lifs_and_core(m) and isinstance(getattr(m, "q_conv"), nn.Conv1d)
            and hasattr(m, "q_bn") and hasattr(m, "proj_lif"))


class FusedSpikeAttention(nn.Module):
    """forward(x [T, B, C, H, W]) -> [T, B, C, H, W] fp32 (ssa variant)."""

    def __init__(self, num_heads: int, scale: float):
        super().__init__()
        self.num_heads = num_heads
        self.scale = float(scale)
        self.variant = "ssa"

    @classmethod
    def from_reference(cls, ref: nn.Module, *, fold_bn: bool = True, ktv_mode: str = "mfma"):
        """Build from a reference block (snn_compiler/nn/attention.py:76-108).
        BN is always folded here (the projections run in bf16); the attention
        counts are exact integers whatever ``ktv_mode`` says."""
        if not is_spiking_self_attention(ref):
            raise TypeError(f"not a recognized spiking self-attention block: {type(ref).__name__}")
        self = cls(ref.num_heads, ref.scale)
        self.in_tau, self.in_vth = _lif_pv(ref.proj_lif)
        q_tau, self.q_vth = _lif_pv(ref.q_lif)
        k_tau, k_vth = _lif_pv(ref.k_lif)
        v_tau, v_vth = _lif_pv(ref.v_lif)
        self.a_tau, self.a_vth = _lif_pv(ref.attn_lif)
        if not (q_tau == k_tau == v_tau == self.in_tau == self.a_tau and self.q_vth == k_vth == v_vth):
            raise ValueError("the fused QKV projection needs one tau and one q/k/v threshold")
        ws, bs = [], []
        for nm in ("q", "k", "v"):
            w, b = fold_conv1d_bn(getattr(ref, f"{nm}_conv"), getattr(ref, f"{nm}_bn"))
            ws.append(w.squeeze(-1))
            bs.append(b)
        pw, pb = fold_conv1d_bn(ref.proj_conv, ref.proj_bn)
        self.register_buffer("w_qkv", torch.cat(ws, 0).to(torch.bfloat16).contiguous())
        self.register_buffer("b_qkv", torch.cat(bs, 0).float().contiguous())
        self.register_buffer("w_proj", pw.squeeze(-1).to(torch.bfloat16).contiguous())
        self.register_buffer("b_proj", pb.float().contiguous())
        return self

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        T, B, C, H, W = x.shape
        N = H * W
        tokens = x.reshape(T, B, C, N).transpose(2, 3)           # [T, B, N, C]
        out = spike_self_attention(tokens, self.w_qkv, self.b_qkv, self.w_proj, self.b_proj,
                                   heads=self.num_heads, scale=self.scale, tau=self.a_tau,
                                   vth_qkv=self.q_vth, vth_attn=self.a_vth,
                                   input_vth=self.in_vth)
        return out.transpose(2, 3).reshape(T, B, C, H, W)
