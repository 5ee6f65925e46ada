"""conv/linear output + bias (+ residual) + IF/LIF, in one HIP kernel.

Mirrors ``snn_compiler/kernels/fused.py``.  The bias of a conv or linear layer
is not added by the GEMM; the neuron kernel reads ``bias[c]`` into registers
and adds it to every step, as the reference does.
"""
from __future__ import annotations

import math

import torch
import torch.nn.functional as F

from .neurons import (
    check_flat, launch_lif, neuron_params,
    THR_SCALAR, THR_PER_CHANNEL, THR_PER_NEURON,
)


def _fused_C_HW(y_seq: torch.Tensor):
    """Channel count / spatial size used by the fused kernels
    (snn_compiler/kernels/fused.py:149-160): 2-D inputs treat every element
    of a step as its own channel."""
    if y_seq.ndim == 5:
        return y_seq.shape[2], y_seq.shape[3] * y_seq.shape[4]
    if y_seq.ndim == 4:
        return y_seq.shape[2], y_seq.shape[3]
    if y_seq.ndim == 3:
        return y_seq.shape[-1], 1
    return math.prod(y_seq.shape[1:]), 1


def _fused_threshold(v_threshold, C: int, NCL: int, like: torch.Tensor):
    if isinstance(v_threshold, torch.Tensor):
        assert v_threshold.is_cuda and v_threshold.dtype == torch.float32 \
            and v_threshold.is_contiguous()
        if v_threshold.numel() == C:
            return THR_PER_CHANNEL, v_threshold, 0.0
        if v_threshold.numel() == NCL:
            return THR_PER_NEURON, v_threshold, 0.0
        raise ValueError(f"v_threshold shape {tuple(v_threshold.shape)} unsupported")
    return THR_SCALAR, None, float(v_threshold)


def _check_bias(bias, C):
    if bias is not None:
        assert bias.is_cuda and bias.is_contiguous() and bias.dtype == torch.float32 \
            and bias.numel() == C, f"bias shape mismatch: {tuple(bias.shape)} vs C={C}"


def fused_bias_if_lif(
    y_seq: torch.Tensor,
    bias: torch.Tensor | None,
    *,
    residual: torch.Tensor | None = None,
    neuron: str = "if",
    tau: float = 2.0,
    decay: float | None = None,
    decay_input: bool = True,
    soft_reset: bool = False,
    v_threshold=1.0,
    v_reset: float = 0.0,
    layout: str = "NCHW",
    spike_dtype: torch.dtype | None = None,
) -> torch.Tensor:
    """``v = decay*v + scale*(y_t + bias[c] (+ residual_t))`` then spike/reset.

    Reference: snn_compiler/kernels/fused.py:117-226.
    """
    check_flat(y_seq, layout, "y_seq")
    assert y_seq.dtype in (torch.float32, torch.float16, torch.bfloat16)
    NCL = math.prod(y_seq.shape[1:])
    C, HW = _fused_C_HW(y_seq)
    df, sc = neuron_params(neuron, tau, decay, decay_input)
    thr = _fused_threshold(v_threshold, C, NCL, y_seq)
    _check_bias(bias, C)
    if residual is not None:
        assert residual.is_cuda and residual.dtype == y_seq.dtype \
            and residual.shape == y_seq.shape, \
            f"residual shape {tuple(residual.shape)} must match y_seq {tuple(y_seq.shape)}"
        check_flat(residual, layout, "residual")
        assert residual.stride() == y_seq.stride(), "residual memory layout must match y_seq"
    spike_seq = torch.empty_like(y_seq, dtype=spike_dtype or y_seq.dtype)
    launch_lif(y_seq, bias=bias, residual=residual, thr=thr, spikes=spike_seq,
               C=C, HW=HW, channel_last=(layout == "NHWC"), decay=df,
               in_scale=sc, v_reset=v_reset, soft_reset=soft_reset)
    return spike_seq


def fused_bias_if_lif_rate(
    y_seq: torch.Tensor,
    bias: torch.Tensor | None,
    *,
    neuron: str = "if",
    tau: float = 2.0,
    decay: float | None = None,
    decay_input: bool = True,
    soft_reset: bool = False,
    v_threshold=1.0,
    v_reset: float = 0.0,
    layout: str = "NCHW",
) -> torch.Tensor:
    """Spike count summed over T, fp32 ``[B, ...]``; no spike train is stored.

    Reference: snn_compiler/kernels/fused.py:303-382.
    """
    check_flat(y_seq, layout, "y_seq")
    assert y_seq.dtype in (torch.float32, torch.float16, torch.bfloat16)
    NCL = math.prod(y_seq.shape[1:])
    C, HW = _fused_C_HW(y_seq)
    df, sc = neuron_params(neuron, tau, decay, decay_input)
    thr = _fused_threshold(v_threshold, C, NCL, y_seq)
    _check_bias(bias, C)
    if y_seq.shape[0] == 0:  # no steps: no spikes
        return torch.zeros(y_seq.shape[1:], device=y_seq.device, dtype=torch.float32)
    count = torch.empty_like(y_seq[0], dtype=torch.float32)
    launch_lif(y_seq, bias=bias, thr=thr, count=count, C=C, HW=HW,
               channel_last=(layout == "NHWC"), decay=df, in_scale=sc,
               v_reset=v_reset, soft_reset=soft_reset)
    return count


def fused_bias_if_lif_stateful(
    y_seq: torch.Tensor,
    bias: torch.Tensor | None,
    *,
    v_init: torch.Tensor | None = None,
    return_v: bool = False,
    neuron: str = "if",
    tau: float = 2.0,
    decay: float | None = None,
    decay_input: bool = True,
    soft_reset: bool = False,
    v_threshold: float = 1.0,
    v_reset: float = 0.0,
    layout: str = "NCHW",
):
    """LIF with a carried membrane state, for T-chunked execution.

    Reference: snn_compiler/kernels/fused.py:444-507 (scalar threshold only).
    Returns ``spikes`` or ``(spikes, v_final)`` with ``v_final`` fp32
    ``[B, ...]``.
    """
    check_flat(y_seq, layout, "y_seq")
    assert y_seq.dtype in (torch.float32, torch.float16, torch.bfloat16)
    NCL = math.prod(y_seq.shape[1:])
    C, HW = _fused_C_HW(y_seq)
    df, sc = neuron_params(neuron, tau, decay, decay_input)
    _check_bias(bias, C)
    v_in = None
    if v_init is not None:
        assert v_init.numel() == NCL and v_init.dtype == torch.float32
        assert v_init.is_cuda and v_init.is_contiguous()
        v_in = v_init.reshape(-1)
    v_out = torch.empty(y_seq.shape[1:], device=y_seq.device, dtype=torch.float32) \
        if return_v else None
    spike = torch.empty_like(y_seq)
    if y_seq.shape[0] == 0:  # no steps: the membrane stays where it was
        if return_v:
            v_out.copy_(v_init.view(v_out.shape) if v_init is not None else torch.zeros_like(v_out))
            return spike, v_out
        return spike
    launch_lif(y_seq, bias=bias, thr=(THR_SCALAR, None, float(v_threshold)),
               v_init=v_in, v_out=v_out, spikes=spike, C=C, HW=HW,
               channel_last=(layout == "NHWC"), decay=df, in_scale=sc,
               v_reset=v_reset, soft_reset=soft_reset)
    if return_v:
        return spike, v_out
    return spike


def fold_conv_bn(conv_w, conv_b, bn_w, bn_b, bn_mean, bn_var, bn_eps):
    """Fold an eval-mode BatchNorm into the preceding conv.

    W' = W * gamma/sqrt(var+eps) (per output channel);
    b' = (b - mean) * gamma/sqrt(var+eps) + beta, with b = 0 when absent.
    Reference: snn_compiler/kernels/fused.py:585-599.
    """
    inv_std = bn_w / torch.sqrt(bn_var + bn_eps)
    view = [-1] + [1] * (conv_w.ndim - 1)
    new_w = conv_w * inv_std.view(*view).to(conv_w.dtype)
    if conv_b is None:
        conv_b = torch.zeros_like(bn_w)
    new_b = (conv_b - bn_mean) * inv_std + bn_b
    return new_w, new_b


def _pair(v) -> tuple:
    return tuple(v) if isinstance(v, (tuple, list)) else (v, v)


def conv_neuron(
    x_seq: torch.Tensor,
    weight: torch.Tensor,
    bias: torch.Tensor | None,
    *,
    stride=1, padding=0, dilation=1, groups=1,
    neuron: str = "if",
    tau: float = 2.0,
    decay: float | None = None,
    decay_input: bool = True,
    soft_reset: bool = False,
    v_threshold=1.0,
    v_reset: float = 0.0,
    layout: str = "NCHW",
) -> torch.Tensor:
    """Conv (no bias) then the fused bias+neuron HIP kernel.

    Reference: snn_compiler/kernels/fused.py:513-551.  A bf16 input to a 3x3 /
    stride 1 / padding 1 conv with channel counts that are multiples of 32
    (float threshold) runs the HIP implicit-GEMM conv with the bias and the
    neuron in its epilogue; otherwise the vendor conv (MIOpen) runs in the
    input's dtype.  The conv3x3 + BN + LIF + max-pool kernel is
    :func:`snnk.kernels.conv.conv_bn_lif_pool`.
    """
    T, B = x_seq.shape[0], x_seq.shape[1]
    if (x_seq.is_cuda and x_seq.dtype == torch.bfloat16 and x_seq.ndim == 5
            and tuple(weight.shape[2:]) == (3, 3) and groups == 1
            and _pair(stride) == (1, 1) and _pair(padding) == (1, 1) and _pair(dilation) == (1, 1)
            and weight.shape[0] % 32 == 0 and weight.shape[1] % 32 == 0
            and not isinstance(v_threshold, torch.Tensor)):
        from .conv import conv3x3_bn_lif_nhwc, prepare_conv3x3_weight, to_nhwc_bf16
        df, sc = neuron_params(neuron, tau, decay, decay_input)
        b = None if bias is None else bias.detach().float().contiguous()
        s = conv3x3_bn_lif_nhwc(to_nhwc_bf16(x_seq), prepare_conv3x3_weight(weight.float()), b,
                                pool=False, decay=df, in_scale=sc, v_threshold=float(v_threshold),
                                v_reset=v_reset, soft_reset=soft_reset).permute(0, 1, 4, 2, 3)
        return s if layout == "NHWC" else s.contiguous()
    weight = weight.to(x_seq.dtype)
    x_4d = x_seq.reshape(T * B, *x_seq.shape[2:])
    if layout == "NHWC":
        x_4d = x_4d.contiguous(memory_format=torch.channels_last)
    y = F.conv2d(x_4d, weight, bias=None, stride=stride, padding=padding,
                 dilation=dilation, groups=groups)
    if layout == "NCHW":
        y_seq = y.contiguous().view(T, B, *y.shape[1:])
    else:
        y_seq = y.contiguous(memory_format=torch.channels_last).view(T, B, *y.shape[1:])
    return fused_bias_if_lif(
        y_seq, bias, neuron=neuron, tau=tau, decay=decay,
        decay_input=decay_input, soft_reset=soft_reset,
        v_threshold=v_threshold, v_reset=v_reset, layout=layout)


def linear_neuron(
    x_seq: torch.Tensor,
    weight: torch.Tensor,
    bias: torch.Tensor | None,
    *,
    neuron: str = "if",
    tau: float = 2.0,
    decay: float | None = None,
    decay_input: bool = True,
    soft_reset: bool = False,
    v_threshold=1.0,
    v_reset: float = 0.0,
) -> torch.Tensor:
    """GEMM (no bias) then the fused bias+neuron HIP kernel.

    Reference: snn_compiler/kernels/fused.py:554-579.  A bf16 input whose
    shapes the fused kernel covers (features multiples of 32, batch a
    multiple of 4, float threshold) runs the bf16-MFMA GEMM with the bias and
    the neuron in its epilogue; otherwise the vendor GEMM runs in the input's
    dtype.
    """
    T, B = x_seq.shape[0], x_seq.shape[1]
    from .linear import linear_bias_lif, linear_fusable
    if x_seq.dtype == torch.bfloat16 and linear_fusable(x_seq, weight, v_threshold):
        df, sc = neuron_params(neuron, tau, decay, decay_input)
        b = None if bias is None else bias.detach().float().contiguous()
        return linear_bias_lif(x_seq.reshape(T, B, -1).contiguous(),
                               weight.detach().to(torch.bfloat16).contiguous(), b, decay=df,
                               in_scale=sc, v_threshold=float(v_threshold), v_reset=v_reset,
                               soft_reset=soft_reset)
    y = F.linear(x_seq.reshape(T * B, -1), weight.to(x_seq.dtype), bias=None)
    y_seq = y.view(T, B, y.shape[-1])
    return fused_bias_if_lif(
        y_seq, bias, neuron=neuron, tau=tau, decay=decay,
        decay_input=decay_input, soft_reset=soft_reset,
        v_threshold=v_threshold, v_reset=v_reset, layout="NCHW")


def conv_bn_neuron(x_seq, conv_w, conv_b, bn_w, bn_b, bn_mean, bn_var, bn_eps,
                   *, stride=1, padding=0, dilation=1, groups=1, **neuron_kwargs):
    """BN folded on the host, then :func:`conv_neuron`.

    Reference: snn_compiler/kernels/fused.py:602-611.
    """
    new_w, new_b = fold_conv_bn(conv_w, conv_b, bn_w, bn_b, bn_mean, bn_var, bn_eps)
    return conv_neuron(x_seq, new_w, new_b, stride=stride, padding=padding,
                       dilation=dilation, groups=groups, **neuron_kwargs)
