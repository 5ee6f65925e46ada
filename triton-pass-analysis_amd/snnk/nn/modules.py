"""nn.Module layer (mirror of snn_compiler/nn/modules.py).

Every module takes ``[T, B, ...]`` and returns spikes ``[T, B, ...]``; the
neuron arithmetic runs in libsnnk (HIP).  Constructor arguments follow the
reference classes one to one; ``FusedConvBNLIFPool`` is new: the whole
conv3x3 + BN + LIF + 2x2 max-pool block in one MFMA kernel.
"""
from __future__ import annotations

import torch
import torch.nn as nn
import torch.nn.functional as F

from ..kernels.neurons import if_lif, neuron_params
from ..kernels.fused import (
    fused_bias_if_lif, fused_bias_if_lif_rate, fused_bias_if_lif_stateful, fold_conv_bn,
)
from ..kernels.conv import (
    prepare_conv3x3_weight, to_nhwc_bf16, conv3x3_bn_lif_nhwc, conv3x3_bn_lif_act,
    conv3x3_dense_weight,
)
from ..kernels.linear import (
    linear_bias_lif, linear_bias_lif_act, linear_bias_lif_pool4, linear_fusable,
)


def _thr(module, v_threshold):
    if isinstance(v_threshold, torch.Tensor):
        module.register_buffer("v_threshold", v_threshold.float().contiguous())
    else:
        module.v_threshold = float(v_threshold)


class IFNode(nn.Module):
    """Integrate-and-fire (snn_compiler/nn/modules.py:26-49)."""

    def __init__(self, *, decay: float = 1.0, soft_reset: bool = False,
                 v_threshold=1.0, v_reset: float = 0.0, layout: str = "NCHW"):
        super().__init__()
        self.decay, self.soft_reset, self.v_reset, self.layout = decay, soft_reset, v_reset, layout
        _thr(self, v_threshold)

    def forward(self, x_seq):
        return if_lif(x_seq if self.layout == "NHWC" else x_seq.contiguous(), neuron="if",
                      decay=self.decay, soft_reset=self.soft_reset,
                      v_threshold=self.v_threshold, v_reset=self.v_reset, layout=self.layout)


class LIFNode(nn.Module):
    """Leaky integrate-and-fire (snn_compiler/nn/modules.py:52-85)."""

    def __init__(self, *, tau: float = 2.0, decay: float | None = None,
                 decay_input: bool = True, soft_reset: bool = False, v_threshold=1.0,
                 v_reset: float = 0.0, layout: str = "NCHW"):
        super().__init__()
        self.tau, self.decay, self.decay_input = tau, decay, decay_input
        self.soft_reset, self.v_reset, self.layout = soft_reset, v_reset, layout
        _thr(self, v_threshold)

    def forward(self, x_seq):
        return if_lif(x_seq if self.layout == "NHWC" else x_seq.contiguous(), neuron="lif",
                      tau=self.tau, decay=self.decay, decay_input=self.decay_input,
                      soft_reset=self.soft_reset, v_threshold=self.v_threshold,
                      v_reset=self.v_reset, layout=self.layout)


class StatefulLIFNode(nn.Module):
    """LIF with carried membrane for T-chunked execution
    (snn_compiler/nn/modules.py:553-586)."""

    def __init__(self, *, tau: float = 2.0, decay: float | None = None,
                 decay_input: bool = True, soft_reset: bool = False,
                 v_threshold: float = 1.0, v_reset: float = 0.0, layout: str = "NCHW"):
        super().__init__()
        self.tau, self.decay, self.decay_input = tau, decay, decay_input
        self.soft_reset, self.v_threshold = soft_reset, float(v_threshold)
        self.v_reset, self.layout = v_reset, layout

    def forward(self, x_seq, v_init=None, return_v=False):
        return fused_bias_if_lif_stateful(
            x_seq if self.layout == "NHWC" else x_seq.contiguous(), None, v_init=v_init,
            return_v=return_v, neuron="lif", tau=self.tau, decay=self.decay,
            decay_input=self.decay_input, soft_reset=self.soft_reset,
            v_threshold=self.v_threshold, v_reset=self.v_reset, layout=self.layout)


class RateCodedLIFNode(nn.Module):
    """Spike count over T, fp32 [B, ...] (snn_compiler/nn/modules.py:487-522)."""

    def __init__(self, *, tau: float = 2.0, decay: float | None = None,
                 decay_input: bool = True, soft_reset: bool = False, v_threshold=1.0,
                 v_reset: float = 0.0, layout: str = "NCHW"):
        super().__init__()
        self.tau, self.decay, self.decay_input = tau, decay, decay_input
        self.soft_reset, self.v_reset, self.layout = soft_reset, v_reset, layout
        _thr(self, v_threshold)

    def forward(self, x_seq):
        return fused_bias_if_lif_rate(
            x_seq if self.layout == "NHWC" else x_seq.contiguous(), None, neuron="lif",
            tau=self.tau, decay=self.decay, decay_input=self.decay_input,
            soft_reset=self.soft_reset, v_threshold=self.v_threshold, v_reset=self.v_reset,
            layout=self.layout)


class RateCodedIFNode(nn.Module):
    """IF spike count over T (snn_compiler/nn/modules.py:525-547)."""

    def __init__(self, *, decay: float = 1.0, soft_reset: bool = False, v_threshold=1.0,
                 v_reset: float = 0.0, layout: str = "NCHW"):
        super().__init__()
        self.decay, self.soft_reset, self.v_reset, self.layout = decay, soft_reset, v_reset, layout
        _thr(self, v_threshold)

    def forward(self, x_seq):
        return fused_bias_if_lif_rate(
            x_seq if self.layout == "NHWC" else x_seq.contiguous(), None, neuron="if",
            decay=self.decay, soft_reset=self.soft_reset, v_threshold=self.v_threshold,
            v_reset=self.v_reset, layout=self.layout)


class _NeuronArgs:
    def _set_neuron(self, neuron, tau, decay, decay_input, soft_reset, v_threshold, v_reset,
                    layout):
        self.neuron, self.tau, self.decay, self.decay_input = neuron, tau, decay, decay_input
        self.soft_reset, self.v_reset, self.layout = soft_reset, v_reset, layout
        _thr(self, v_threshold)

    def _mfma_conv(self, x_seq, weight, bias):
        """conv3x3 + bias + neuron in one HIP kernel (bf16 MFMA, fp32
        accumulation) on bf16 spikes; returns [T, B, C, H, W] bf16, in
        channels-last memory for layout 'NHWC'.  The bf16 weight matrix is
        rebuilt whenever ``weight`` is replaced or changed in place."""
        stamp = (weight.device, weight.data_ptr(), weight._version)
        hit = self.__dict__.get("_w_prep_cache")
        if hit is None or hit[0] != stamp:
            hit = (stamp, prepare_conv3x3_weight(weight.detach().float()))
            self.__dict__["_w_prep_cache"] = hit
        df, sc = neuron_params(self.neuron, self.tau, self.decay, self.decay_input)
        b = None if bias is None else bias.detach().float().contiguous()
        s = conv3x3_bn_lif_nhwc(to_nhwc_bf16(x_seq), hit[1], b, pool=False, decay=df,
                                in_scale=sc, v_threshold=float(self.v_threshold),
                                v_reset=self.v_reset, soft_reset=self.soft_reset)
        s = s.permute(0, 1, 4, 2, 3)
        return s if self.layout == "NHWC" else s.contiguous()

    def _lif(self, y_seq, bias, residual=None):
        return fused_bias_if_lif(
            y_seq, bias, residual=residual, neuron=self.neuron, tau=self.tau,
            decay=self.decay, decay_input=self.decay_input, soft_reset=self.soft_reset,
            v_threshold=self.v_threshold, v_reset=self.v_reset, layout=self.layout)


def _mfma_conv_fits(x_seq, weight, conv, v_threshold) -> bool:
    """bf16 input to a 3x3 / stride 1 / padding 1 conv with channel counts
    that are multiples of 32 and a float threshold: what the HIP implicit-GEMM
    conv + neuron kernel covers."""
    return (x_seq.is_cuda and x_seq.dtype == torch.bfloat16 and x_seq.ndim == 5
            and tuple(weight.shape[2:]) == (3, 3) and conv["groups"] == 1
            and tuple(conv["stride"]) == (1, 1) and tuple(conv["padding"]) == (1, 1)
            and tuple(conv["dilation"]) == (1, 1)
            and weight.shape[0] % 32 == 0 and weight.shape[1] % 32 == 0
            and not isinstance(v_threshold, torch.Tensor))


def _conv_seq(x_seq, w, bias, conv, layout):
    """Vendor conv over [T*B, ...] returning [T, B, ...] in the module's layout."""
    T, B = x_seq.shape[0], x_seq.shape[1]
    x4 = x_seq.reshape(T * B, *x_seq.shape[2:])
    # the conv runs in the input's dtype (fp32 parameters meet a bf16 input)
    w = w.to(x4.dtype)
    bias = None if bias is None else bias.to(x4.dtype)
    if layout == "NHWC":
        x4 = x4.contiguous(memory_format=torch.channels_last)
        w = w.to(memory_format=torch.channels_last)
    else:
        x4 = x4.contiguous()
    y = F.conv2d(x4, w, bias=bias, stride=conv["stride"], padding=conv["padding"],
                 dilation=conv["dilation"], groups=conv["groups"])
    if layout == "NHWC":
        y = y.contiguous(memory_format=torch.channels_last)
    else:
        y = y.contiguous()
    return y.view(T, B, *y.shape[1:])


class FusedConvNeuron(nn.Module, _NeuronArgs):
    """Conv2d + bias + IF/LIF (snn_compiler/nn/modules.py:160-217).

    A bf16 input to a 3x3 / stride 1 / padding 1 conv with channel counts that
    are multiples of 32 (float threshold) runs the HIP implicit-GEMM conv with
    the bias and the neuron in its epilogue.  Other shapes -- and always fp32
    inputs, keeping the reference's precision -- run the vendor conv in the
    input's dtype, then the HIP neuron kernel."""

    def __init__(self, in_ch, out_ch, kernel_size, *, stride=1, padding=0, dilation=1,
                 groups=1, bias: bool = True, neuron: str = "if", tau: float = 2.0,
                 decay: float | None = None, decay_input: bool = True,
                 soft_reset: bool = False, v_threshold=1.0, v_reset: float = 0.0,
                 layout: str = "NCHW"):
        super().__init__()
        conv = nn.Conv2d(in_ch, out_ch, kernel_size, stride=stride, padding=padding,
                         dilation=dilation, groups=groups, bias=bias)
        self.weight = nn.Parameter(conv.weight.detach().clone())
        self.bias = nn.Parameter(conv.bias.detach().clone()) if bias else None
        self.conv = dict(stride=conv.stride, padding=conv.padding, dilation=conv.dilation,
                         groups=conv.groups)
        self._set_neuron(neuron, tau, decay, decay_input, soft_reset, v_threshold, v_reset,
                         layout)
        self.conv_mfma = True  # False: the vendor conv for every input

    def forward(self, x_seq):
        if self.conv_mfma and _mfma_conv_fits(x_seq, self.weight, self.conv, self.v_threshold):
            return self._mfma_conv(x_seq, self.weight, self.bias)
        y = _conv_seq(x_seq, self.weight, None, self.conv, self.layout)
        b = None if self.bias is None else self.bias.float().contiguous()
        return self._lif(y, b)


class FusedLinearNeuron(nn.Module, _NeuronArgs):
    """Linear + bias + IF/LIF (snn_compiler/nn/modules.py:220-255).

    A bf16 input runs the fused bf16-MFMA GEMM + LIF kernel (fp32
    accumulation) when the shape allows it (in_features % 32 == 0,
    out_features % 32 == 0, batch % 4 == 0, float threshold).  Otherwise --
    and always for fp32 inputs, keeping the reference's precision -- the
    vendor GEMM in the input's dtype runs first, then the HIP neuron kernel.
    """

    def __init__(self, in_features, out_features, *, bias: bool = True, neuron: str = "if",
                 tau: float = 2.0, decay: float | None = None, decay_input: bool = True,
                 soft_reset: bool = False, v_threshold=1.0, v_reset: float = 0.0):
        super().__init__()
        lin = nn.Linear(in_features, out_features, bias=bias)
        self.weight = nn.Parameter(lin.weight.detach().clone())
        self.bias = nn.Parameter(lin.bias.detach().clone()) if bias else None
        self._set_neuron(neuron, tau, decay, decay_input, soft_reset, v_threshold, v_reset,
                         "NCHW")
        self._w_bf16 = None

    def forward(self, x_seq):
        T, B = x_seq.shape[0], x_seq.shape[1]
        b = None if self.bias is None else self.bias.float().contiguous()
        if x_seq.dtype == torch.bfloat16 and linear_fusable(x_seq, self.weight,
                                                            self.v_threshold):
            if self._w_bf16 is None or self._w_bf16.device != x_seq.device:
                self._w_bf16 = self.weight.detach().to(torch.bfloat16).contiguous()
            df, sc = neuron_params(self.neuron, self.tau, self.decay, self.decay_input)
            s = linear_bias_lif(x_seq.reshape(T, B, -1).to(torch.bfloat16).contiguous(),
                                self._w_bf16, b, decay=df, in_scale=sc,
                                v_threshold=self.v_threshold, v_reset=self.v_reset,
                                soft_reset=self.soft_reset)
            return s.to(x_seq.dtype)
        y = F.linear(x_seq.reshape(T * B, -1), self.weight.to(x_seq.dtype), bias=None)
        return self._lif(y.view(T, B, -1), b)


class FusedConvBNNeuron(nn.Module, _NeuronArgs):
    """Conv2d + eval BN + IF/LIF (snn_compiler/nn/modules.py:258-357).

    fold_bn=True folds BN into the conv once; a bf16 input to a 3x3 / stride 1
    / padding 1 conv with channel counts that are multiples of 32 then runs
    the HIP implicit-GEMM conv with the folded bias and the neuron in its
    epilogue, other shapes and fp32 inputs the vendor conv then the HIP
    neuron kernel.  fold_bn=False keeps conv and BN as separate vendor ops
    (bit-exact with the unfused network) and fuses only the neuron.
    """

    def __init__(self, conv: nn.Conv2d, bn: nn.BatchNorm2d, *, fold_bn: bool = True,
                 neuron: str = "if", tau: float = 2.0, decay: float | None = None,
                 decay_input: bool = True, soft_reset: bool = False, v_threshold=1.0,
                 v_reset: float = 0.0, layout: str = "NCHW"):
        super().__init__()
        assert bn.running_mean is not None
        self.fold_bn = fold_bn
        if fold_bn:
            w, b = fold_conv_bn(conv.weight.detach(),
                                conv.bias.detach() if conv.bias is not None else None,
                                bn.weight.detach(), bn.bias.detach(),
                                bn.running_mean.detach(), bn.running_var.detach(), bn.eps)
            self.weight = nn.Parameter(w)
            self.bias = nn.Parameter(b)
        else:
            self.weight = nn.Parameter(conv.weight.detach().clone())
            self.register_parameter("conv_bias", nn.Parameter(conv.bias.detach().clone())
                                    if conv.bias is not None else None)
            for nm, t in (("bn_weight", bn.weight), ("bn_bias", bn.bias),
                          ("bn_mean", bn.running_mean), ("bn_var", bn.running_var)):
                self.register_buffer(nm, t.detach().clone())
            self.bn_eps = bn.eps
            self.bias = None
        self.conv = dict(stride=conv.stride, padding=conv.padding, dilation=conv.dilation,
                         groups=conv.groups)
        self._set_neuron(neuron, tau, decay, decay_input, soft_reset, v_threshold, v_reset,
                         layout)
        self.conv_mfma = True  # False: the vendor conv for every input

    def _conv_bn(self, x_seq):
        if self.fold_bn:
            y = _conv_seq(x_seq, self.weight, None, self.conv, self.layout)
            return y, self.bias.float().contiguous()
        y = _conv_seq(x_seq, self.weight, self.conv_bias, self.conv, self.layout)
        T, B = y.shape[:2]
        y4 = F.batch_norm(y.reshape(T * B, *y.shape[2:]), self.bn_mean, self.bn_var,
                          self.bn_weight, self.bn_bias, training=False, eps=self.bn_eps)
        if self.layout == "NHWC":
            y4 = y4.contiguous(memory_format=torch.channels_last)
        return y4.view(T, B, *y4.shape[1:]), None

    def forward(self, x_seq):
        if self.fold_bn and self.conv_mfma and \
                _mfma_conv_fits(x_seq, self.weight, self.conv, self.v_threshold):
            return self._mfma_conv(x_seq, self.weight, self.bias)
        y, bias = self._conv_bn(x_seq)
        return self._lif(y, bias)


class FusedConvBNAddNeuron(FusedConvBNNeuron):
    """Conv + BN + residual add + IF/LIF (snn_compiler/nn/modules.py:360-443)."""

    def forward(self, x_seq, residual_seq):
        y, bias = self._conv_bn(x_seq)
        return self._lif(y, bias, residual=residual_seq)


class FusedAddNeuron(nn.Module, _NeuronArgs):
    """a + b then IF/LIF (snn_compiler/nn/modules.py:446-481)."""

    def __init__(self, *, neuron: str = "if", tau: float = 2.0, decay: float | None = None,
                 decay_input: bool = True, soft_reset: bool = False, v_threshold=1.0,
                 v_reset: float = 0.0, layout: str = "NCHW"):
        super().__init__()
        self._set_neuron(neuron, tau, decay, decay_input, soft_reset, v_threshold, v_reset,
                         layout)

    def forward(self, a_seq, b_seq):
        a = a_seq if self.layout == "NHWC" else a_seq.contiguous()
        return self._lif(a, None, residual=b_seq)


class FusedConvBNLIFPool(nn.Module):
    """conv3x3 + eval BN (folded) + IF/LIF + optional 2x2 max-pool, one MFMA kernel.

    Replaces the reference's (FusedConvBNNeuron, nn.MaxPool2d) pair
    (snn_compiler/nn/modules.py:258-357 then snn_compiler/zoo/vgg.py:101-105).
    forward takes the reference's [T, B, C, H, W] (any memory format) and
    returns spikes [T, B, C, Ho, Wo] in channels-last memory, in ``out_dtype``
    (default: the input's dtype; spikes are exact in every float dtype);
    ``forward_nhwc`` chains layers on contiguous NHWC bf16 [T, B, H, W, C].
    """

    def __init__(self, conv: nn.Conv2d, bn: nn.BatchNorm2d | None, *, pool: str | None = "max",
                 neuron: str = "lif", tau: float = 2.0, decay: float | None = None,
                 decay_input: bool = True, soft_reset: bool = False, v_threshold: float = 1.0,
                 v_reset: float = 0.0, out_dtype: torch.dtype | None = None):
        super().__init__()
        self.out_dtype = out_dtype
        if tuple(conv.kernel_size) != (3, 3) or tuple(conv.stride) != (1, 1) or \
                tuple(conv.padding) != (1, 1) or tuple(conv.dilation) != (1, 1) or conv.groups != 1:
            raise ValueError("FusedConvBNLIFPool needs a 3x3 / stride 1 / padding 1 conv")
        if pool not in (None, "max"):
            raise ValueError(f"unsupported pool {pool!r}")
        w = conv.weight.detach().float()
        b = conv.bias.detach().float() if conv.bias is not None else None
        if bn is not None:
            w, b = fold_conv_bn(w, b, bn.weight.detach().float(), bn.bias.detach().float(),
                                bn.running_mean.detach().float(),
                                bn.running_var.detach().float(), bn.eps)
        if b is None:
            b = torch.zeros(w.shape[0], device=w.device)
        self.register_buffer("weight", w.contiguous())
        self.register_buffer("bias", b.float().contiguous())
        self.register_buffer("w_prep", prepare_conv3x3_weight(w))
        self.pool = pool
        self.decay_factor, self.input_scale = neuron_params(neuron, tau, decay, decay_input)
        self.soft_reset, self.v_threshold, self.v_reset = soft_reset, float(v_threshold), v_reset

    def _dense(self, H, W):
        """Dense-matrix form of the conv for a map of at most 2x2, built on the
        weights' device and rebuilt whenever ``weight`` or ``bias`` is replaced
        or changed in place (``load_state_dict``, ``.to()``, ``copy_``)."""
        stamp = tuple((t.device, t.data_ptr(), t._version) for t in (self.weight, self.bias))
        cache = self.__dict__.setdefault("_dense_cache", {})
        hit = cache.get((H, W))
        if hit is None or hit[0] != stamp:
            hit = (stamp, conv3x3_dense_weight(self.weight, self.bias, H, W, self.pool == "max"))
            cache[(H, W)] = hit
        return hit[1]

    def forward_nhwc(self, x_nhwc, out=None, tile_hint=-1, out_bits=False):
        """Spikes in, spikes out, channels last: ``x_nhwc`` is bf16 0/1
        ``[T, B, H, W, C]`` or int32 packed words ``[T, B, H, W, C // 32]``
        (bit c%32 of word c//32).  ``out_bits`` asks for packed words out; the
        2x2-map layer with pooling (column-pooled dense form) writes bf16."""
        packed = x_nhwc.dtype == torch.int32
        T, B, H, W = x_nhwc.shape[:4]
        lif = dict(decay=self.decay_factor, in_scale=self.input_scale,
                   v_threshold=self.v_threshold, v_reset=self.v_reset,
                   soft_reset=self.soft_reset)
        if H <= 2 and W <= 2 and B % 4 == 0 and tile_hint < 0 and \
                (self.pool != "max" or (H == 2 and W == 2)):
            # every output pixel sees the whole map: one dense Linear + LIF
            # (+ the pool as an OR of column groups), no padding taps
            w_d, b_d = self._dense(H, W)
            x2 = x_nhwc.reshape(T, B, -1)
            Cout = self.weight.shape[0]
            if self.pool == "max":
                o2 = None if out is None else out.view(T, B, Cout)
                y = (linear_bias_lif_act(x2, w_d, b_d, out_bits=False, col_pool=True, out=o2, **lif)
                     if packed else linear_bias_lif_pool4(x2, w_d, b_d, out=o2, **lif))
                return y.view(T, B, 1, 1, Cout)
            if packed or out_bits:
                o2 = None if out is None else out.view(T, B, -1)
                y = linear_bias_lif_act(x2, w_d, b_d, out_bits=out_bits, out=o2, **lif)
                return y.view(T, B, H, W, -1)
            o2 = None if out is None else out.view(T, B, H * W * Cout)
            y = linear_bias_lif(x2, w_d, b_d, out=o2, **lif)
            return y.view(T, B, H, W, Cout)
        if packed or out_bits:
            return conv3x3_bn_lif_act(x_nhwc, self.w_prep, self.bias, pool=self.pool == "max",
                                      out_bits=out_bits, out=out, tile_hint=tile_hint, **lif)
        return conv3x3_bn_lif_nhwc(x_nhwc, self.w_prep, self.bias, pool=self.pool == "max",
                                   out=out, tile_hint=tile_hint, **lif)

    def forward(self, x_seq):
        s = self.forward_nhwc(to_nhwc_bf16(x_seq)).permute(0, 1, 4, 2, 3)
        return s.to(self.out_dtype or x_seq.dtype)
