"""Conv block oracle (torch CPU, fp32) -- test infrastructure only.

Restates the reference's CPU-runnable pieces of the conv-BN-LIF(-pool) path:
  fold_conv_bn            snn_compiler/kernels/fused.py:585-599
  fold_conv1d_bn          snn_compiler/nn/attention.py:28-33
  conv (no bias) + fused bias LIF   snn_compiler/nn/modules.py:324-357 with
                          snn_compiler/kernels/fused.py:101-114
  max pool per step       snn_compiler/zoo/vgg.py:56,101-105 (nn.MaxPool2d(2,2))
  LIF-then-pool shape     snn_compiler/explore/large_T/pool_epilogue_proto.py:168-185
                          (avg there; max here)

Pins (tests/test_oracle_fused.py): the fold identity conv(x,W')+b' ==
BN(conv(x,W)+b) within 1e-4 (reference test_correctness.py:203-228); F.conv2d
padding/orientation against a float64 direct loop; max-pool of {0,1} spikes ==
OR of the window; the whole block against an independent composition
(direct conv + scalar LIF loop + OR) on tiny shapes.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F

from .neurons import lif_multistep, neuron_params


def fold_conv_bn(conv_w, conv_b, bn_w, bn_b, bn_mean, bn_var, bn_eps):
    """W' = W * g/sqrt(var+eps); b' = (b - mean) * g/sqrt(var+eps) + beta."""
    inv_std = bn_w / torch.sqrt(bn_var + bn_eps)
    new_w = conv_w * inv_std.view(-1, *([1] * (conv_w.ndim - 1))).to(conv_w.dtype)
    if conv_b is None:
        conv_b = torch.zeros_like(bn_w)
    new_b = (conv_b - bn_mean) * inv_std + bn_b
    return new_w, new_b


def conv3x3_seq(x_seq, w, bias=None):
    """[T,B,Cin,H,W] -> [T,B,Cout,H,W] per-step conv3x3, pad 1 (torch CPU fp32)."""
    T, B = x_seq.shape[:2]
    y = F.conv2d(x_seq.reshape(T * B, *x_seq.shape[2:]).float(), w.float(),
                 None if bias is None else bias.float(), padding=1)
    return y.view(T, B, *y.shape[1:])


def conv3x3_direct_f64(x, w):
    """Direct 7-loop conv3x3 pad 1 in float64 on [N,Cin,H,W] (tiny shapes only)."""
    x = x.double()
    w = w.double()
    N, Cin, H, W = x.shape
    Cout = w.shape[0]
    y = torch.zeros(N, Cout, H, W, dtype=torch.float64)
    for n in range(N):
        for co in range(Cout):
            for yy in range(H):
                for xx in range(W):
                    s = 0.0
                    for ci in range(Cin):
                        for kh in range(3):
                            for kw in range(3):
                                ys, xs = yy + kh - 1, xx + kw - 1
                                if 0 <= ys < H and 0 <= xs < W:
                                    s += float(x[n, ci, ys, xs]) * float(w[co, ci, kh, kw])
                    y[n, co, yy, xx] = s
    return y


def maxpool2x2_seq(s_seq):
    """Per-step 2x2 / stride 2 max pool on [T,B,C,H,W]."""
    T, B = s_seq.shape[:2]
    p = F.max_pool2d(s_seq.reshape(T * B, *s_seq.shape[2:]), 2, 2)
    return p.view(T, B, *p.shape[1:])


def conv_bn_lif_pool(x_seq, conv_w, conv_b, bn_w, bn_b, bn_mean, bn_var, bn_eps, *,
                     pool=True, neuron="lif", tau=2.0, decay=None, decay_input=True,
                     soft_reset=False, v_threshold=1.0, v_reset=0.0, weight_dtype=None):
    """The reference block on the CPU: returns (spikes [T,B,C,Ho,Wo] fp32,
    pre-reset membrane trace [T,B,C,H,W]).

    ``weight_dtype=torch.bfloat16`` rounds the folded weights (and the input)
    to bf16 before the fp32 conv, to model the GPU operand precision.
    """
    new_w, new_b = fold_conv_bn(conv_w, conv_b, bn_w, bn_b, bn_mean, bn_var, bn_eps)
    x = x_seq.float()
    if weight_dtype is not None:
        new_w = new_w.to(weight_dtype).float()
        x = x.to(weight_dtype).float()
    y = conv3x3_seq(x, new_w)
    spikes, _, _ = lif_multistep(y, bias=new_b, neuron=neuron, tau=tau, decay=decay,
                                 decay_input=decay_input, soft_reset=soft_reset,
                                 v_threshold=v_threshold, v_reset=v_reset)
    trace = membrane_trace(y, bias=new_b, neuron=neuron, tau=tau, decay=decay,
                           decay_input=decay_input, soft_reset=soft_reset,
                           v_threshold=v_threshold, v_reset=v_reset)
    if pool:
        spikes = maxpool2x2_seq(spikes)
    return spikes, trace


def membrane_trace(y_seq, *, bias=None, neuron="lif", tau=2.0, decay=None, decay_input=True,
                   soft_reset=False, v_threshold=1.0, v_reset=0.0):
    """Pre-reset membrane H_t of every step (same recurrence as lif_multistep)."""
    df, sc = neuron_params(neuron, tau, decay, decay_input)
    bb = None if bias is None else bias.float().view(1, -1, *([1] * (y_seq.ndim - 3)))
    v = torch.zeros_like(y_seq[0], dtype=torch.float32)
    hs = []
    for t in range(y_seq.shape[0]):
        u = y_seq[t].float() if bb is None else y_seq[t].float() + bb
        h = df * v + sc * u
        hs.append(h)
        s = h >= v_threshold
        v = torch.where(s, (h - v_threshold) if soft_reset else torch.full_like(h, v_reset), h)
    return torch.stack(hs, 0)
