"""Fused spike attention module (mirror of snn_compiler/nn/attention.py).

``FusedSpikeAttention.from_reference`` takes a spiking attention block --
Spikingformer ``SpikingSelfAttention`` (variant ``ssa``: Conv1d-1x1 q/k/v/proj
+ BatchNorm1d + LIF nodes) or SDT-V2 ``MS_Attention`` (variant ``ms``:
Sequential(conv, BN) projections + ``head_lif``) -- detected like
snn_compiler/nn/attention.py:40-59, and runs it on libsnnk:

* ``ktv_mode='bmm'`` / ``'popcount'`` (the reference's modes,
  attention.py:76-164): reference linear order ``(q @ (k^T v)) * scale``.
  Every LIF runs in the HIP neuron kernel (bit-exact with the reference
  neuron), ``k^T v`` is an fp32 bmm of 0/1 values or the bit-packed popcount
  GEMM (exact integer counts either way), and ``spike_av_lif`` fuses the
  product with the attention LIF.  With ``fold_bn=False`` the projections
  are the block's own conv + BN, so the block output is bit-identical to the
  reference block's.
* ``ktv_mode='mfma'`` (ssa only, N <= 64, d <= 64, d % 8 == 0): the fast
  path -- one fused QKV projection (BN folded, bf16 MFMA, LIF epilogue), the
  int8-MFMA attention core (exact counts in the quadratic order
  ``(q k^T) v``, equal to the linear order over the integers) and the folded
  output projection.

forward takes and returns ``[T, B, C, H, W]`` (fp32 for the reference
modes, the projection's fp32 output for ``mfma``).
"""
from __future__ import annotations

import copy

import torch
import torch.nn as nn
import torch.nn.functional as F

from ..kernels.attention import spike_self_attention, spike_av_lif, spike_ktv_popcount
from ..kernels.fused import fused_bias_if_lif


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


def is_ms_attention(m: nn.Module) -> bool:
    """SDT-V2 MS_Attention: Sequential(conv, BN) projections + head_lif."""
    return (_has_lifs_and_core(m) and isinstance(getattr(m, "q_conv"), nn.Sequential)
            and hasattr(m, "head_lif"))


def is_spiking_attention(m: nn.Module) -> bool:
    return is_spiking_self_attention(m) or is_ms_attention(m)


def _to_heads(s, T, B, N, heads, d):
    """[T, B, C, N] -> [T, B, heads, N, d]."""
    return s.transpose(-1, -2).reshape(T, B, N, heads, d).permute(0, 1, 3, 2, 4).contiguous()


class FusedSpikeAttention(nn.Module):
    """Spiking attention block on libsnnk (variant ``ssa`` or ``ms``)."""

    def __init__(self, num_heads: int, scale: float, variant: str = "ssa",
                 fold_bn: bool = False, ktv_mode: str = "bmm"):
        super().__init__()
        if ktv_mode not in ("bmm", "popcount", "mfma"):
            raise ValueError(f"unknown ktv_mode {ktv_mode!r} ('bmm', 'popcount' or 'mfma')")
        if ktv_mode == "mfma" and variant != "ssa":
            raise ValueError("ktv_mode='mfma' is the fused ssa path")
        self.num_heads = num_heads
        self.scale = float(scale)
        self.variant = variant
        # the ms projection chains stay eager, as in the reference
        self.fold_bn = (fold_bn and variant == "ssa") or ktv_mode == "mfma"
        self.ktv_mode = ktv_mode

    @classmethod
    def from_reference(cls, ref: nn.Module, *, fold_bn: bool = False, ktv_mode: str = "bmm"):
        """Build from a reference block (snn_compiler/nn/attention.py:76-108).

        ``fold_bn=False`` keeps the projections' conv + BN (bit-exact);
        ``ktv_mode='mfma'`` always folds BN (bf16 projections)."""
        if is_spiking_self_attention(ref):
            variant = "ssa"
        elif is_ms_attention(ref):
            variant = "ms"
        else:
            raise TypeError(f"not a recognized spiking attention block: {type(ref).__name__}")
        self = cls(ref.num_heads, ref.scale, variant, fold_bn=fold_bn, ktv_mode=ktv_mode)
        in_lif = ref.proj_lif if variant == "ssa" else ref.head_lif
        self.in_tau, self.in_vth = _lif_pv(in_lif)
        self.q_tau, self.q_vth = _lif_pv(ref.q_lif)
        self.k_tau, self.k_vth = _lif_pv(ref.k_lif)
        self.v_tau, self.v_vth = _lif_pv(ref.v_lif)
        self.a_tau, self.a_vth = _lif_pv(ref.attn_lif)
        if ktv_mode == "mfma":
            if not (self.q_tau == self.k_tau == self.v_tau == self.in_tau == self.a_tau
                    and self.q_vth == self.k_vth == self.v_vth):
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
        elif variant == "ssa" and self.fold_bn:
            for nm in ("q", "k", "v", "proj"):
                w, b = fold_conv1d_bn(getattr(ref, f"{nm}_conv"), getattr(ref, f"{nm}_bn"))
                self.register_buffer(f"{nm}_w", w)
                self.register_buffer(f"{nm}_b", b)
        elif variant == "ssa":
            for nm in ("q", "k", "v", "proj"):
                setattr(self, f"{nm}_conv", copy.deepcopy(getattr(ref, f"{nm}_conv")).eval())
                setattr(self, f"{nm}_bn", copy.deepcopy(getattr(ref, f"{nm}_bn")).eval())
        else:
            for nm in ("q", "k", "v", "proj"):
                setattr(self, f"{nm}_conv", copy.deepcopy(getattr(ref, f"{nm}_conv")).eval())
        return self

    # -- reference linear order ------------------------------------------------
    @staticmethod
    def _lif(x, bias, tau, vth):
        return fused_bias_if_lif(x.contiguous(), bias, neuron="lif", tau=tau, decay_input=True,
                                 soft_reset=False, v_threshold=vth, v_reset=0.0, layout="NCHW")

    def _proj(self, xf, nm, tau, vth, T, B, C, N, H, W):
        """Projection + LIF -> spikes [T, B, C, N]."""
        if self.variant == "ssa":
            if self.fold_bn:
                y = F.conv1d(xf, getattr(self, f"{nm}_w"), bias=None)
                bias = getattr(self, f"{nm}_b")
            else:
                y = getattr(self, f"{nm}_bn")(getattr(self, f"{nm}_conv")(xf))
                bias = None
            return self._lif(y.reshape(T, B, C, N).unsqueeze(-1), bias, tau, vth).squeeze(-1)
        y = getattr(self, f"{nm}_conv")(xf).reshape(T, B, C, H, W)
        return self._lif(y, None, tau, vth).flatten(3)

    def _forward_linear(self, x):
        T, B, C, H, W = x.shape
        N, heads = H * W, self.num_heads
        d = C // heads
        x = self._lif(x, None, self.in_tau, self.in_vth).reshape(T, B, C, H, W)
        xf = x.flatten(3).flatten(0, 1) if self.variant == "ssa" else x.flatten(0, 1)
        q = _to_heads(self._proj(xf, "q", self.q_tau, self.q_vth, T, B, C, N, H, W), T, B, N, heads, d)
        k = _to_heads(self._proj(xf, "k", self.k_tau, self.k_vth, T, B, C, N, H, W), T, B, N, heads, d)
        v = _to_heads(self._proj(xf, "v", self.v_tau, self.v_vth, T, B, C, N, H, W), T, B, N, heads, d)
        if self.ktv_mode == "popcount":
            kv = spike_ktv_popcount(k, v)
        else:
            kv = torch.matmul(k.transpose(-2, -1).contiguous(), v)
        s = spike_av_lif(q, kv, scale=self.scale, tau=self.a_tau, v_threshold=self.a_vth,
                         v_reset=0.0)
        s = s.transpose(3, 4).reshape(T, B, C, N)
        if self.variant == "ssa":
            sf = s.flatten(0, 1)
            if self.fold_bn:
                out = F.conv1d(sf, self.proj_w, bias=self.proj_b)
            else:
                out = self.proj_bn(self.proj_conv(sf))
            return out.reshape(T, B, C, H, W)
        return self.proj_conv(s.reshape(T, B, C, H, W).flatten(0, 1)).reshape(T, B, C, H, W)

    # -- fused int8-MFMA path ---------------------------------------------------
    def _forward_mfma(self, x):
        T, B, C, H, W = x.shape
        N = H * W
        tokens = x.reshape(T, B, C, N).transpose(2, 3)           # [T, B, N, C]
        out = spike_self_attention(tokens, self.w_qkv, self.b_qkv, self.w_proj, self.b_proj,
                                   heads=self.num_heads, scale=self.scale, tau=self.a_tau,
                                   vth_qkv=self.q_vth, vth_attn=self.a_vth,
                                   input_vth=self.in_vth)
        return out.transpose(2, 3).reshape(T, B, C, H, W)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if self.ktv_mode == "mfma":
            return self._forward_mfma(x)
        return self._forward_linear(x)
