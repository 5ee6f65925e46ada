"""Bit-packed activations through the fused conv3x3 / Linear + LIF kernels.

SNNK_ACT_BITS packs the channels of every pixel (row) into uint32 words, bit
c%32 of word c/32, LSB first -- the reference's _pack_N convention
(snn_compiler/kernels/attention.py:195-214) applied along the channel axis.
The packed input is expanded to the same bf16 0/1 operand values and the
packed output is taken from the same LIF results, so each packed path must
equal the bf16 path bit for bit:
  * out: words == oracle.bits.pack_rows(bf16 spikes of the same call plan);
  * in:  spikes from packed x == spikes from the bf16 x it packs;
and at the BASELINE conv config the words agree with the fp32 oracle block
(>= 99.9% of the spikes, as for the bf16 output).
"""
import numpy as np
import pytest
import torch

from oracle import bits as ob
from oracle import fused as of
from snnk.kernels import conv as kc
from snnk.kernels.linear import linear_bias_lif, linear_bias_lif_act
from snnk.kernels.neurons import if_lif, if_lif_packed

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _pack(s):
    """[..., C] 0/1 (any dtype, CPU) -> int32 words [..., C/32] (oracle packer)."""
    return torch.from_numpy(ob.pack_rows(s.float().numpy()).view(np.int32))


def _conv_case(T, B, Cin, Cout, H, W, seed, p=0.2):
    g = torch.Generator().manual_seed(seed)
    x = (torch.rand(T, B, H, W, Cin, generator=g) < p).to(torch.bfloat16)
    w = torch.randn(Cout, Cin, 3, 3, generator=g) * (2.0 / (Cin * 9)) ** 0.5 * 2.0
    b = torch.randn(Cout, generator=g) * 0.1
    return x, kc.prepare_conv3x3_weight(w.to(DEV)), b.to(DEV).float()


LIF = dict(decay=0.5, in_scale=0.5, v_threshold=1.0)
CONV = [  # T, B, Cin, Cout, H, W, tile
    (4, 2, 32, 64, 8, 8, -1), (3, 2, 96, 128, 6, 6, 2), (5, 1, 64, 256, 8, 8, 0),
    (4, 2, 128, 160, 4, 4, 8), (6, 1, 64, 96, 6, 6, 4), (3, 1, 32, 64, 2, 6, 3),
    (4, 3, 64, 128, 10, 6, 14), (2, 2, 64, 256, 8, 8, 21), (4, 2, 32, 64, 8, 8, 10),
    (3, 2, 96, 64, 6, 6, 13), (8, 1, 32, 64, 4, 4, 6),
]


@pytest.mark.parametrize("pool", [False, True])
@pytest.mark.parametrize("T,B,Cin,Cout,H,W,tile", CONV)
def test_conv_packed_paths_equal_bf16_path(T, B, Cin, Cout, H, W, tile, pool):
    if pool and (H % 2 or W % 2):
        pytest.skip("odd spatial size")
    x, wp, bd = _conv_case(T, B, Cin, Cout, H, W, seed=T * 31 + Cin + Cout)
    xd, xp = x.to(DEV), _pack(x).to(DEV)
    ref = kc.conv3x3_bn_lif_nhwc(xd, wp, bd, pool=pool, tile_hint=tile, **LIF).cpu()
    assert 0 < int(ref.float().sum()) < ref.numel()
    words = _pack(ref)
    got = kc.conv3x3_bn_lif_act(xd, wp, bd, pool=pool, tile_hint=tile, **LIF)
    assert got.dtype == torch.int32 and torch.equal(got.cpu(), words), "bf16 in, bits out"
    got = kc.conv3x3_bn_lif_act(xp, wp, bd, pool=pool, tile_hint=tile, out_bits=False, **LIF)
    assert torch.equal(got.cpu(), ref), "bits in, bf16 out"
    got = kc.conv3x3_bn_lif_act(xp, wp, bd, pool=pool, tile_hint=tile, **LIF)
    assert torch.equal(got.cpu(), words), "bits in, bits out"


@pytest.mark.parametrize("shape,splits", [((4, 32, 4, 4, 512, 512), None), ((4, 2, 4, 4, 512, 512), 3),
                                          ((5, 8, 8, 8, 256, 256), 2)])
@pytest.mark.parametrize("pool", [False, True])
def test_conv_packed_split_k(shape, splits, pool):
    """Cross-block split K (workspace reduction) with packed input and output."""
    T, B, H, W, Cin, Cout = shape
    x, wp, bd = _conv_case(T, B, Cin, Cout, H, W, seed=H * 7 + B, p=0.15)
    ref = kc.conv3x3_bn_lif_nhwc(x.to(DEV), wp, bd, pool=pool, splits=splits, **LIF).cpu()
    got = kc.conv3x3_bn_lif_act(_pack(x).to(DEV), wp, bd, pool=pool, splits=splits, **LIF)
    assert torch.equal(got.cpu(), _pack(ref))
    assert 0 < int(ref.float().sum()) < ref.numel()


def test_conv_baseline_config_bits_vs_oracle():
    """[4,32,128,16,16] Bernoulli(0.15) -> 256 ch, folded BN, LIF, 2x2 max, packed
    in and out: the words are the packed oracle block's spikes at >= 99.9%
    agreement (bf16 operands flip spikes near threshold), and exactly the
    packed bf16-path spikes."""
    g = torch.Generator().manual_seed(0)
    T, B, Cin, Cout, H, W = 4, 32, 128, 256, 16, 16
    x = (torch.rand(T, B, Cin, H, W, generator=g) < 0.15).float()
    w = torch.randn(Cout, Cin, 3, 3, generator=g) * (2.0 / (Cin * 9)) ** 0.5
    gamma, beta = torch.rand(Cout, generator=g) + 0.5, torch.randn(Cout, generator=g) * 0.1
    mean, var = torch.randn(Cout, generator=g) * 0.1, torch.rand(Cout, generator=g) + 0.5
    w2, b2 = of.fold_conv_bn(w, None, gamma, beta, mean, var, 1e-5)
    wp, bd = kc.prepare_conv3x3_weight(w2.to(DEV)), b2.to(DEV).float().contiguous()
    x_nhwc = x.permute(0, 1, 3, 4, 2).contiguous()
    xp = _pack(x_nhwc).to(DEV)
    assert xp.numel() * 4 == x.numel() // 8          # 16x fewer bytes than bf16
    words = kc.conv3x3_bn_lif_act(xp, wp, bd, pool=True, **LIF).cpu()
    assert words.shape == (T, B, 8, 8, Cout // 32) and words.numel() * 4 == 262144
    bf = kc.conv3x3_bn_lif_nhwc(x_nhwc.to(DEV, torch.bfloat16), wp, bd, pool=True, **LIF).cpu()
    assert torch.equal(words, _pack(bf))
    ref, _ = of.conv_bn_lif_pool(x, w, None, gamma, beta, mean, var, 1e-5, pool=True,
                                 tau=2.0, v_threshold=1.0)
    ref_words = _pack(ref.permute(0, 1, 3, 4, 2).contiguous())
    differ = (words ^ ref_words)
    flips = sum(bin(int(v) & 0xFFFFFFFF).count("1") for v in differ[differ != 0].tolist())
    assert flips <= 0.001 * ref.numel(), f"{flips} spike flips of {ref.numel()}"


def test_layer_chain_on_bits():
    """Two conv layers and a Linear chained on packed words equal the bf16 chain."""
    T, B = 4, 4
    x, w1, b1 = _conv_case(T, B, 64, 128, 8, 8, seed=5, p=0.3)
    _, w2, b2 = _conv_case(T, B, 128, 256, 4, 4, seed=6)
    g = torch.Generator().manual_seed(7)
    wl = (torch.randn(512, 4 * 4 * 256 // 4, generator=g) * 0.05).to(DEV, torch.bfloat16)
    bl = torch.zeros(512, device=DEV)
    xd = x.to(DEV)
    s1 = kc.conv3x3_bn_lif_nhwc(xd, w1, b1, pool=True, **LIF)               # [T,B,4,4,128]
    s2 = kc.conv3x3_bn_lif_nhwc(s1, w2, b2, pool=True, **LIF)               # [T,B,2,2,256]
    y = linear_bias_lif(s2.reshape(T, B, -1).contiguous(), wl, bl, **LIF)   # [T,B,512]
    p1 = kc.conv3x3_bn_lif_act(_pack(x).to(DEV), w1, b1, pool=True, **LIF)
    p2 = kc.conv3x3_bn_lif_act(p1, w2, b2, pool=True, **LIF)
    py = linear_bias_lif_act(p2.reshape(T, B, -1).contiguous(), wl, bl, **LIF)
    assert torch.equal(p1.cpu(), _pack(s1.cpu()))
    assert torch.equal(p2.cpu(), _pack(s2.cpu()))
    assert torch.equal(py.cpu(), _pack(y.cpu()))
    assert 0 < int(y.float().sum()) < y.numel()


@pytest.mark.parametrize("T,R,K,N,tile,splits", [(4, 32, 512, 4096, -1, None),
                                                 (4, 32, 4096, 4096, -1, None),
                                                 (3, 8, 1024, 96, 4, 1), (5, 12, 256, 512, 2, 1),
                                                 (4, 128, 2048, 1024, 10, 4)])
def test_linear_packed_paths(T, R, K, N, tile, splits):
    g = torch.Generator().manual_seed(K + N)
    x = (torch.rand(T, R, K, generator=g) < 0.25).to(torch.bfloat16)
    w = (torch.randn(N, K, generator=g) * (2.0 / K) ** 0.5 * 2.0).to(DEV, torch.bfloat16)
    b = (torch.randn(N, generator=g) * 0.1).to(DEV)
    ref = linear_bias_lif(x.to(DEV), w, b, tile_hint=tile, splits=splits, **LIF).cpu()
    assert 0 < int(ref.float().sum()) < ref.numel()
    xp = _pack(x).to(DEV)
    kw = dict(tile_hint=tile, splits=splits, **LIF)
    assert torch.equal(linear_bias_lif_act(x.to(DEV), w, b, **kw).cpu(), _pack(ref))
    assert torch.equal(linear_bias_lif_act(xp, w, b, out_bits=False, **kw).cpu(), ref)
    assert torch.equal(linear_bias_lif_act(xp, w, b, **kw).cpu(), _pack(ref))


def test_lif_packed_words_feed_conv():
    """The standalone LIF's packed spikes (SNNK_SPIKE_BITS on a channels-last map)
    are the conv's packed input layout."""
    T, B, H, W, C = 4, 2, 8, 8, 64
    g = torch.Generator().manual_seed(9)
    u = torch.randn(T, B, H, W, C, generator=g) * 1.5
    words = if_lif_packed(u.to(DEV).reshape(T, -1), neuron="lif", tau=2.0)
    s = if_lif(u.to(DEV).reshape(T, -1), neuron="lif", tau=2.0).cpu().reshape(T, B, H, W, C)
    assert torch.equal(words.cpu().reshape(T, B, H, W, C // 32), _pack(s))
    _, wp, bd = _conv_case(T, B, C, 128, H, W, seed=10)
    a = kc.conv3x3_bn_lif_act(words.reshape(T, B, H, W, C // 32).contiguous(), wp, bd,
                              pool=False, out_bits=False, **LIF)
    b = kc.conv3x3_bn_lif_nhwc(s.to(DEV, torch.bfloat16), wp, bd, pool=False, **LIF)
    assert torch.equal(a.cpu(), b.cpu())


@pytest.mark.parametrize("B,H,W,Cout", [(32, 32, 32, 64), (1, 32, 32, 64), (56, 32, 32, 64),
                                        (3, 12, 10, 96), (2, 7, 9, 32)])
def test_image_layer_packed_output(B, H, W, Cout):
    """The image layer's packed words are its bf16 spikes, packed (all three
    pixel-run widths: runs of 4 at B=56, 2 at B=32, 1 at odd widths)."""
    g = torch.Generator().manual_seed(B + H)
    img = torch.randn(B, 3, H, W, generator=g).to(DEV)
    w = (torch.randn(Cout, 3, 3, 3, generator=g) * 0.6).to(DEV)
    b = (torch.randn(Cout, generator=g) * 0.1).to(DEV)
    bf = kc.conv3x3_image_lif(img, w, b, 4, **LIF).cpu()
    words = kc.conv3x3_image_lif(img, w, b, 4, out_bits=True, **LIF).cpu()
    assert words.dtype == torch.int32 and words.shape == (4, B, H, W, Cout // 32)
    assert torch.equal(words, _pack(bf))
    assert 0 < int(bf.float().sum()) < bf.numel()
