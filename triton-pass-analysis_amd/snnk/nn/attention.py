"""Spiking attention block on libsnnk.

Public API of ``snn_compiler/nn/attention.py``: :class:`FusedSpikeAttention`
with ``from_reference(block, fold_bn=False, ktv_mode='bmm')``,
:func:`fold_conv1d_bn` and the detectors :func:`is_spiking_self_attention`,
:func:`is_ms_attention`, :func:`is_spiking_attention`.

Two block families are recognised by the attributes they carry (the
interface the reference detects, snn_compiler/nn/attention.py:40-59):

  ``ssa``  Spikingformer SpikingSelfAttention: Conv1d-1x1 q/k/v/proj convs,
           a BatchNorm1d after each (``q_bn`` ...), input neuron ``proj_lif``;
  ``ms``   SDT-V2 MS_Attention: q/k/v/proj are Sequential (conv ..., BN2d)
           chains over the 2-D map, input neuron ``head_lif``.

Both compute, per step, ``attn_lif(scale * q (k^T v))`` with no softmax.

Design.  ``from_reference`` reads a block into four projection modules and
five (tau, threshold) neuron settings; ``forward`` is one pipeline: input
neuron -> each projection and its neuron -> split heads -> attention core ->
merge heads -> output projection.  A projection maps the flattened
``[T*B, C, ...]`` spikes to a pre-activation and an optional per-channel bias
that the neuron kernel adds.  ``ktv_mode`` picks the core:

  ``'bmm'``       K^T V as an exact binary GEMM of the spikes (MFMA where the
                  shape allows), then the fused ``spike_av_lif`` kernel;
  ``'popcount'``  K^T V by bit packing along the tokens and the VALU popcount
                  GEMM (the reference's popcount mode), then ``spike_av_lif``;
  ``'mfma'``      (ssa) the fused SSA block: BN folded into one bf16 QKV
                  projection with the LIF in its epilogue, the MFMA attention
                  core and the folded output projection.

With ``fold_bn=False`` the first two keep the block's own layers as the
projections, so the output is bit-identical to the block's.
"""
from __future__ import annotations

import copy
from typing import NamedTuple, Optional

import torch
import torch.nn as nn
import torch.nn.functional as F

from ..kernels.attention import (
    spike_self_attention, spike_av_lif, spike_ktv_popcount, spike_ktv,
)
from ..kernels.fused import fused_bias_if_lif, fold_conv_bn

# every block has these; the variants differ in the type of q_conv and in
# the attributes only they carry
_SHARED = ("q_lif", "k_lif", "v_lif", "attn_lif", "q_conv", "k_conv", "v_conv", "proj_conv",
           "num_heads", "scale")
_VARIANTS = (("ssa", nn.Conv1d, ("q_bn", "proj_lif")),
             ("ms", nn.Sequential, ("head_lif",)))
_INPUT_NEURON = {"ssa": "proj_lif", "ms": "head_lif"}


def attention_variant(m: nn.Module) -> Optional[str]:
    """'ssa' / 'ms' for a recognised spiking attention block, else None."""
    if not all(hasattr(m, a) for a in _SHARED):
        return None
    for name, conv_type, own in _VARIANTS:
        if isinstance(m.q_conv, conv_type) and all(hasattr(m, a) for a in own):
            return name
    return None


def is_spiking_self_attention(m: nn.Module) -> bool:
    return attention_variant(m) == "ssa"


def is_ms_attention(m: nn.Module) -> bool:
    return attention_variant(m) == "ms"


def is_spiking_attention(m: nn.Module) -> bool:
    return attention_variant(m) is not None


def fold_conv1d_bn(conv: nn.Conv1d, bn: nn.BatchNorm1d):
    """(W', b') of an eval BatchNorm1d folded into the conv before it (the
    same eval-BN algebra as :func:`snnk.kernels.fused.fold_conv_bn`)."""
    return fold_conv_bn(conv.weight.detach(),
                        conv.bias.detach() if conv.bias is not None else None,
                        bn.weight.detach(), bn.bias.detach(), bn.running_mean.detach(),
                        bn.running_var.detach(), bn.eps)


class _Neuron(NamedTuple):
    tau: float
    vth: float

    @classmethod
    def of(cls, node) -> "_Neuron":
        # SpikingJelly-style node attributes, with their defaults
        return cls(float(getattr(node, "tau", 2.0)), float(getattr(node, "v_threshold", 1.0)))


# ---- projections: flattened spikes -> (pre-activation, per-channel bias) -----
class _Layers(nn.Module):
    """The block's own layers, run as they are (bit-identical)."""

    def __init__(self, *layers: nn.Module):
        super().__init__()
        self.body = nn.Sequential(*[copy.deepcopy(m).eval() for m in layers])

    def forward(self, xf):
        return self.body(xf), None


class _Folded1x1(nn.Module):
    """Conv1d-1x1 with its BatchNorm1d folded in; the neuron adds the bias."""

    def __init__(self, conv: nn.Conv1d, bn: nn.BatchNorm1d):
        super().__init__()
        w, b = fold_conv1d_bn(conv, bn)
        self.register_buffer("weight", w.contiguous())
        self.register_buffer("bias", b.float().contiguous())

    def forward(self, xf):
        return F.conv1d(xf, self.weight), self.bias


def _projections(ref: nn.Module, variant: str, fold: bool) -> nn.ModuleDict:
    if variant == "ms":   # the conv chains stay as they are
        return nn.ModuleDict({n: _Layers(getattr(ref, f"{n}_conv")) for n in ("q", "k", "v", "proj")})
    if fold:
        return nn.ModuleDict({n: _Folded1x1(getattr(ref, f"{n}_conv"), getattr(ref, f"{n}_bn"))
                              for n in ("q", "k", "v", "proj")})
    return nn.ModuleDict({n: _Layers(getattr(ref, f"{n}_conv"), getattr(ref, f"{n}_bn"))
                          for n in ("q", "k", "v", "proj")})


class FusedSpikeAttention(nn.Module):
    """Spiking attention block on libsnnk (variant ``ssa`` or ``ms``);
    forward takes and returns ``[T, B, C, H, W]``."""

    CORES = ("bmm", "popcount", "mfma")

    def __init__(self, num_heads: int, scale: float, variant: str = "ssa",
                 fold_bn: bool = False, ktv_mode: str = "bmm"):
        super().__init__()
        if ktv_mode not in self.CORES:
            raise ValueError(f"unknown ktv_mode {ktv_mode!r}; one of {self.CORES}")
        if variant not in _INPUT_NEURON:
            raise ValueError(f"unknown variant {variant!r}")
        if ktv_mode == "mfma" and variant != "ssa":
            raise ValueError("ktv_mode='mfma' is the fused ssa block")
        self.num_heads, self.scale = int(num_heads), float(scale)
        self.variant, self.ktv_mode = variant, ktv_mode
        # the ms conv chains are never folded; the mfma core always is
        self.fold_bn = ktv_mode == "mfma" or (fold_bn and variant == "ssa")
        self.neurons: dict[str, _Neuron] = {}
        self.proj: nn.ModuleDict | None = None

    # kept as attributes for callers that read them
    @property
    def in_tau(self):
        return self.neurons["in"].tau

    @property
    def in_vth(self):
        return self.neurons["in"].vth

    @classmethod
    def from_reference(cls, ref: nn.Module, *, fold_bn: bool = False, ktv_mode: str = "bmm"):
        """Build from a reference block.  ``fold_bn=False`` keeps the block's
        projection layers (bit-identical output); ``ktv_mode='mfma'`` always
        folds BN into bf16 projections."""
        variant = attention_variant(ref)
        if variant is None:
            raise TypeError(f"{type(ref).__name__} is not a spiking attention block this "
                            "package recognises (ssa or ms)")
        mod = cls(ref.num_heads, ref.scale, variant, fold_bn=fold_bn, ktv_mode=ktv_mode)
        mod.neurons = {"in": _Neuron.of(getattr(ref, _INPUT_NEURON[variant])),
                       **{n: _Neuron.of(getattr(ref, f"{n}_lif")) for n in ("q", "k", "v")},
                       "attn": _Neuron.of(ref.attn_lif)}
        if ktv_mode == "mfma":
            mod._prepare_fused_block(ref)
        else:
            mod.proj = _projections(ref, variant, mod.fold_bn)
        return mod

    # ---- the fused SSA block (ktv_mode='mfma') ---------------------------------
    def _prepare_fused_block(self, ref):
        taus = {p.tau for p in self.neurons.values()}
        vths = {self.neurons[n].vth for n in ("q", "k", "v")}
        if len(taus) != 1 or len(vths) != 1:
            raise ValueError("the fused QKV projection needs one tau for every neuron and one "
                             "threshold for q, k and v")
        folded = {n: fold_conv1d_bn(getattr(ref, f"{n}_conv"), getattr(ref, f"{n}_bn"))
                  for n in ("q", "k", "v", "proj")}
        self.register_buffer("w_qkv", torch.cat([folded[n][0].squeeze(-1) for n in "qkv"])
                             .to(torch.bfloat16).contiguous())
        self.register_buffer("b_qkv", torch.cat([folded[n][1] for n in "qkv"]).float().contiguous())
        self.register_buffer("w_proj", folded["proj"][0].squeeze(-1).to(torch.bfloat16).contiguous())
        self.register_buffer("b_proj", folded["proj"][1].float().contiguous())

    def _fused_block(self, x):
        T, B, C, H, W = x.shape
        tokens = x.reshape(T, B, C, H * W).transpose(2, 3)           # [T, B, N, C]
        nq, na = self.neurons["q"], self.neurons["attn"]
        out = spike_self_attention(tokens, self.w_qkv, self.b_qkv, self.w_proj, self.b_proj,
                                   heads=self.num_heads, scale=self.scale, tau=na.tau,
                                   vth_qkv=nq.vth, vth_attn=na.vth,
                                   input_vth=self.neurons["in"].vth)
        return out.transpose(2, 3).reshape(T, B, C, H, W)

    # ---- the reference-order pipeline ('bmm', 'popcount') ------------------------
    @staticmethod
    def _fire(y, bias, neuron: _Neuron):
        """LIF (decay_input, hard reset to 0) over [T, B, C, ...] pre-activations."""
        return fused_bias_if_lif(y.contiguous(), bias, neuron="lif", tau=neuron.tau,
                                 decay_input=True, soft_reset=False, v_threshold=neuron.vth,
                                 v_reset=0.0, layout="NCHW")

    def _project(self, name, flat, T, B):
        y, bias = self.proj[name](flat)
        return y.reshape(T, B, *y.shape[1:]), bias

    def _split_heads(self, s):
        """[T, B, C, N] -> [T, B, heads, N, d], channel c = head * d + dim."""
        T, B, C, N = s.shape
        return s.view(T, B, self.num_heads, C // self.num_heads, N).transpose(3, 4).contiguous()

    def _core(self, q, k, v):
        kv = spike_ktv_popcount(k, v) if self.ktv_mode == "popcount" else spike_ktv(k, v)
        na = self.neurons["attn"]
        return spike_av_lif(q, kv, scale=self.scale, tau=na.tau, v_threshold=na.vth, v_reset=0.0)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if self.ktv_mode == "mfma":
            return self._fused_block(x)
        T, B, C, H, W = x.shape
        s = self._fire(x, None, self.neurons["in"]).flatten(0, 1)       # [T*B, C, H, W]
        flat = s.flatten(2) if self.variant == "ssa" else s
        heads = []
        for name in ("q", "k", "v"):
            y, bias = self._project(name, flat, T, B)
            heads.append(self._split_heads(self._fire(y, bias, self.neurons[name]).flatten(3)))
        a = self._core(*heads)                                            # [T, B, h, N, d]
        merged = a.transpose(3, 4).reshape(T * B, C, H * W)
        if self.variant == "ms":
            merged = merged.view(T * B, C, H, W)
        y, bias = self.proj["proj"](merged)
        if bias is not None:
            y = y + bias.view(1, -1, 1)
        return y.reshape(T, B, C, H, W)
