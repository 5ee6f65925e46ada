"""VGG16-SNN oracle (torch CPU, fp32) -- test infrastructure only.

Restates the reference model and its layer semantics:
  VGG16_CFG                    snn_compiler/zoo/vgg.py:25-26
  VGGSNN layers / forward      snn_compiler/zoo/vgg.py:49-116 (MaxPool2d variant,
                               examples/vgg16_snn/vgg16_test.py:61-92)
  _maybe_init_bn               snn_compiler/zoo/vgg.py:118-126
  mean over T of the output    examples/vgg16_snn/vgg16_test.py:243
The reference sizes FC1 for 224x224 inputs (fc_in_dim = C*(224/32)^2,
snn_compiler/zoo/vgg.py:74); here fc_in_dim follows the actual input size
(32x32 -> 512).

Parameters come from ``make_params(seed)``: one CPU torch.Generator drawn in
layer order -- conv weight Kaiming-normal (fan_in, gain sqrt 2), conv bias
U(+-1/sqrt(fan_in)) (nn.Conv2d default), BN per _maybe_init_bn
(mean N(0,0.1^2), var U(0.5,1.5), gamma U(0.5,1.5), beta N(0,0.1^2)), FC
weight Kaiming-normal, FC bias U(+-1/sqrt(fan_in)).  ``gain`` scales every
weight (1.0 = BASELINE's init).
"""
from __future__ import annotations

import math

import torch
import torch.nn.functional as F

from .fused import fold_conv_bn, conv3x3_seq, maxpool2x2_seq
from .neurons import lif_multistep

VGG16_CFG = [64, 64, "P", 128, 128, "P", 256, 256, 256, "P",
             512, 512, 512, "P", 512, 512, 512, "P"]


def make_params(seed=0, *, cfg=VGG16_CFG, in_ch=3, input_size=32, fc_hidden=4096,
                num_classes=10, gain=1.0):
    g = torch.Generator().manual_seed(seed)
    convs = []
    ch = in_ch
    for v in cfg:
        if v == "P":
            continue
        fan_in = ch * 9
        w = torch.randn(v, ch, 3, 3, generator=g) * math.sqrt(2.0 / fan_in) * gain
        b = (torch.rand(v, generator=g) * 2 - 1) / math.sqrt(fan_in)
        mean = torch.randn(v, generator=g) * 0.1
        var = torch.rand(v, generator=g) + 0.5
        gamma = torch.rand(v, generator=g) + 0.5
        beta = torch.randn(v, generator=g) * 0.1
        convs.append(dict(w=w, b=b, mean=mean, var=var, gamma=gamma, beta=beta, eps=1e-5))
        ch = v
    n_pool = sum(1 for v in cfg if v == "P")
    fc_in = ch * (input_size // 2 ** n_pool) ** 2
    fcs = []
    for fi, fo in ((fc_in, fc_hidden), (fc_hidden, fc_hidden), (fc_hidden, num_classes)):
        w = torch.randn(fo, fi, generator=g) * math.sqrt(2.0 / fi) * gain
        b = (torch.rand(fo, generator=g) * 2 - 1) / math.sqrt(fi)
        fcs.append(dict(w=w, b=b))
    return dict(cfg=list(cfg), convs=convs, fcs=fcs, input_size=input_size)


def forward(params, image, T=4, *, tau=2.0, v_threshold=1.0, v_reset=0.0,
            soft_reset=False, return_rates=False):
    """image [B,3,H,W] fp32, repeated over T.  Returns [T,B,classes] (and the
    firing rate of every spiking block's output, after its pool if any, when
    return_rates)."""
    x = image.float().unsqueeze(0).expand(T, *image.shape).contiguous()
    lif = dict(neuron="lif", tau=tau, v_threshold=v_threshold, v_reset=v_reset,
               soft_reset=soft_reset)
    rates = []
    ci = 0
    for v in params["cfg"]:
        if v == "P":
            x = maxpool2x2_seq(x)
            rates[-1] = x.mean().item()   # a block's rate is taken after its pool
            continue
        p = params["convs"][ci]
        ci += 1
        w2, b2 = fold_conv_bn(p["w"], p["b"], p["gamma"], p["beta"], p["mean"], p["var"], p["eps"])
        y = conv3x3_seq(x, w2)
        x, _, _ = lif_multistep(y, bias=b2, **lif)
        rates.append(x.mean().item())
    T_, B = x.shape[:2]
    x = x.reshape(T_, B, -1)
    for i, p in enumerate(params["fcs"]):
        y = F.linear(x.reshape(T_ * B, -1), p["w"]).view(T_, B, -1)
        if i < 2:
            x, _, _ = lif_multistep(y, bias=p["b"], **lif)
            rates.append(x.mean().item())
        else:
            x = y + p["b"].view(1, 1, -1)
    return (x, rates) if return_rates else x


def forward_layers(params, image, T=4, *, tau=2.0, v_threshold=1.0, v_reset=0.0,
                   soft_reset=False):
    """Per-layer record of the forward: a list of dicts with the layer kind
    ('image', 'conv', 'fc_lif', 'fc_out'), its input, its output (spikes
    after any pool, or the FC3 logits) and the pre-reset membrane trace."""
    from .fused import membrane_trace
    x = image.float().unsqueeze(0).expand(T, *image.shape).contiguous()
    lif = dict(neuron="lif", tau=tau, v_threshold=v_threshold, v_reset=v_reset,
               soft_reset=soft_reset)
    rec = []
    cfg = params["cfg"]
    ci = 0
    k = 0
    while k < len(cfg):
        p = params["convs"][ci]
        w2, b2 = fold_conv_bn(p["w"], p["b"], p["gamma"], p["beta"], p["mean"], p["var"], p["eps"])
        y = conv3x3_seq(x, w2)
        s, _, _ = lif_multistep(y, bias=b2, **lif)
        tr = membrane_trace(y, bias=b2, **lif)
        pool = k + 1 < len(cfg) and cfg[k + 1] == "P"
        out = maxpool2x2_seq(s) if pool else s
        rec.append(dict(kind="image" if ci == 0 else "conv", input=x, output=out, trace=tr,
                        pool=pool, w=w2, b=b2))
        x = out
        ci += 1
        k += 2 if pool else 1
    T_, B = x.shape[:2]
    x = x.reshape(T_, B, -1)
    for i, p in enumerate(params["fcs"]):
        y = F.linear(x.reshape(T_ * B, -1), p["w"]).view(T_, B, -1)
        if i < 2:
            s, _, _ = lif_multistep(y, bias=p["b"], **lif)
            tr = membrane_trace(y, bias=p["b"], **lif)
            rec.append(dict(kind="fc_lif", input=x, output=s, trace=tr))
            x = s
        else:
            out = y + p["b"].view(1, 1, -1)
            rec.append(dict(kind="fc_out", input=x, output=out))
    return rec
