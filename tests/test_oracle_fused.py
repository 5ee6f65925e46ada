"""Pins for oracle/fused.py (BN folding, conv3x3, LIF + max-pool block)."""
import numpy as np
import torch
import torch.nn as nn
import torch.nn.functional as F

from oracle import fused as of
from oracle import neurons as on


def _bn(c, g):
    bn = nn.BatchNorm2d(c).eval()
    with torch.no_grad():
        bn.running_mean.copy_(torch.randn(c, generator=g))
        bn.running_var.copy_(torch.rand(c, generator=g) + 0.1)
        bn.weight.copy_(torch.rand(c, generator=g) + 0.5)
        bn.bias.copy_(torch.randn(c, generator=g) * 0.1)
    return bn


def test_fold_identity_reference_tolerance():
    """test_correctness.py:203-228: max|conv-bn(x) - conv'(x)| < 1e-4."""
    g = torch.Generator().manual_seed(3)
    conv = nn.Conv2d(8, 16, 3, padding=1, bias=True)
    with torch.no_grad():
        conv.weight.copy_(torch.randn(16, 8, 3, 3, generator=g) * 0.2)
        conv.bias.copy_(torch.randn(16, generator=g) * 0.1)
    bn = _bn(16, g)
    x = torch.randn(4, 8, 32, 32, generator=g)
    with torch.no_grad():
        ref = bn(conv(x))
        w2, b2 = of.fold_conv_bn(conv.weight, conv.bias, bn.weight, bn.bias,
                                 bn.running_mean, bn.running_var, bn.eps)
        got = F.conv2d(x, w2, b2, padding=1)
    assert (ref - got).abs().max().item() < 1e-4


def test_conv3x3_matches_direct_loop():
    g = torch.Generator().manual_seed(0)
    x = torch.randn(2, 3, 5, 4, generator=g)
    w = torch.randn(4, 3, 3, 3, generator=g)
    y = of.conv3x3_seq(x.view(1, 2, 3, 5, 4), w).view(2, 4, 5, 4)
    ref = of.conv3x3_direct_f64(x, w)
    assert (y.double() - ref).abs().max().item() < 1e-5


def test_maxpool_of_spikes_is_or():
    g = torch.Generator().manual_seed(1)
    s = (torch.rand(3, 2, 5, 6, 8, generator=g) < 0.3).float()
    p = of.maxpool2x2_seq(s)
    w = s.view(3, 2, 5, 3, 2, 4, 2)
    ref = (w.sum(dim=(4, 6)) > 0).float()
    assert torch.equal(p, ref)


def test_block_against_independent_composition():
    """conv (direct f64 loop) -> scalar LIF loop -> OR pool vs the oracle block."""
    g = torch.Generator().manual_seed(5)
    T, B, Cin, Cout, H, W = 3, 1, 2, 3, 4, 4
    x = (torch.rand(T, B, Cin, H, W, generator=g) < 0.4).float()
    w = torch.randn(Cout, Cin, 3, 3, generator=g)
    gamma, beta = torch.rand(Cout, generator=g) + 0.5, torch.randn(Cout, generator=g) * 0.1
    mean, var = torch.randn(Cout, generator=g) * 0.1, torch.rand(Cout, generator=g) + 0.5
    spikes, trace = of.conv_bn_lif_pool(x, w, None, gamma, beta, mean, var, 1e-5,
                                        pool=True, tau=2.0, v_threshold=0.5)
    w2, b2 = of.fold_conv_bn(w, None, gamma, beta, mean, var, 1e-5)
    y = of.conv3x3_direct_f64(x.view(T * B, Cin, H, W), w2).view(T, B, Cout, H, W)
    ref = np.zeros((T, B, Cout, H // 2, W // 2), np.float32)
    f = np.float32
    for b in range(B):
        for c in range(Cout):
            for yy in range(H):
                for xx in range(W):
                    v = f(0)
                    for t in range(T):
                        u = f(f(y[t, b, c, yy, xx]) + f(b2[c]))
                        h = f(f(f(0.5) * v) + f(f(0.5) * u))
                        s = h >= f(0.5)
                        v = f(0.0) if s else h
                        if s:
                            ref[t, b, c, yy // 2, xx // 2] = 1.0
    # conv sums may differ from F.conv2d in the last bit; spikes must agree
    # wherever the membrane is not within 1e-5 of threshold
    diff = spikes.numpy() != ref
    near = (trace - 0.5).abs().view(T, B, Cout, H // 2, 2, W // 2, 2).amin(dim=(4, 6)) < 1e-5
    assert not np.any(diff & ~near.numpy())
