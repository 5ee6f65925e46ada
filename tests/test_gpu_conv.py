"""GPU parity of the fused conv3x3 + BN + LIF (+ 2x2 max-pool) MFMA kernel.

Three layers of checks:
  1. pre-activation mode (conv + bias, fp32) against a float64 CPU conv of the
     same bf16-rounded operands: within fp32 accumulation error;
  2. the LIF + pool epilogue is exact: spikes equal the oracle's LIF + max-pool
     applied to the kernel's own pre-activations (same tile shape);
  3. BASELINE conv config against the fp32 reference path (oracle.fused:
     fold_conv_bn -> F.conv2d -> LIF -> max_pool2d): >= 99.9% spike agreement
     and every flip sits where the fp32 membrane is near threshold.
"""
import pytest
import torch
import torch.nn.functional as F

from oracle import fused as of
from oracle import neurons as on
from snnk.kernels import conv as kc

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _setup(T, B, Cin, Cout, H, W, seed, p=0.15):
    g = torch.Generator().manual_seed(seed)
    x = (torch.rand(T, B, Cin, H, W, generator=g) < p).float()
    w = torch.randn(Cout, Cin, 3, 3, generator=g) * (2.0 / (Cin * 9)) ** 0.5
    gamma = torch.rand(Cout, generator=g) + 0.5
    beta = torch.randn(Cout, generator=g) * 0.1
    mean = torch.randn(Cout, generator=g) * 0.1
    var = torch.rand(Cout, generator=g) + 0.5
    return x, w, gamma, beta, mean, var


def _gpu_operands(x, w, gamma, beta, mean, var):
    w2, b2 = of.fold_conv_bn(w, None, gamma, beta, mean, var, 1e-5)
    xd = kc.to_nhwc_bf16(x.to(DEV))
    wp = kc.prepare_conv3x3_weight(w2.to(DEV))
    return xd, wp, b2.to(DEV).float().contiguous(), w2, b2


def _preact_ref_f64(x, w2, b2):
    """float64 conv of the bf16-rounded operands, NHWC."""
    T, B = x.shape[:2]
    xb = x.to(torch.bfloat16).double()
    wb = w2.to(torch.bfloat16).double()
    y = F.conv2d(xb.reshape(T * B, *x.shape[2:]), wb, padding=1) + b2.double().view(1, -1, 1, 1)
    yabs = F.conv2d(xb.abs().reshape(T * B, *x.shape[2:]), wb.abs(), padding=1)
    to = lambda t: t.view(T, B, *t.shape[1:]).permute(0, 1, 3, 4, 2)  # noqa: E731
    return to(y), to(yabs)


SHAPES = [  # T, B, Cin, Cout, H, W, tile
    (4, 2, 32, 64, 8, 8, -1), (4, 2, 64, 64, 8, 8, 1), (3, 2, 32, 128, 8, 8, 2),
    (5, 1, 64, 256, 8, 8, 0), (4, 2, 128, 128, 4, 4, 3), (6, 1, 64, 96, 6, 6, 4),
    (1, 3, 32, 32, 4, 6, 5), (8, 1, 32, 64, 4, 4, 4), (4, 3, 64, 128, 10, 6, 2),
    (4, 2, 64, 64, 4, 4, 6), (3, 2, 64, 96, 4, 4, 7), (4, 1, 128, 160, 4, 4, 8),
    (5, 2, 64, 128, 8, 8, 9), (4, 2, 32, 64, 8, 8, 10), (2, 2, 64, 32, 4, 4, 11),
    (4, 2, 64, 128, 8, 8, 12), (3, 2, 96, 64, 6, 6, 13), (4, 3, 64, 128, 10, 6, 14),
    (5, 2, 64, 96, 8, 8, 15), (4, 2, 32, 128, 4, 6, 16), (6, 2, 64, 64, 8, 8, 17),
    (4, 1, 128, 160, 4, 4, 18), (4, 3, 64, 128, 10, 6, 19), (5, 2, 64, 96, 8, 8, 20),
    (2, 2, 64, 256, 8, 8, 21), (3, 2, 96, 256, 6, 6, 21), (4, 3, 32, 64, 10, 6, 22), (4, 2, 64, 160, 8, 8, 23),
    (3, 2, 64, 128, 6, 6, 24), (4, 2, 64, 96, 4, 4, 25), (3, 2, 96, 128, 6, 6, 26),
    (5, 2, 64, 128, 8, 8, 27), (4, 1, 128, 160, 4, 4, 28),
]


@pytest.mark.parametrize("T,B,Cin,Cout,H,W,tile", SHAPES)
def test_preact_matches_f64(T, B, Cin, Cout, H, W, tile):
    x, w, *bn = _setup(T, B, Cin, Cout, H, W, seed=T * 100 + Cin, p=0.3)
    x = x + torch.randn(x.shape, generator=torch.Generator().manual_seed(1)) * 0.5  # real-valued
    xd, wp, bd, w2, b2 = _gpu_operands(x, w, *bn)
    pre = kc.conv3x3_preact_nhwc(xd, wp, bd, tile_hint=tile).cpu().double()
    ref, absref = _preact_ref_f64(x, w2, b2)
    err = (pre - ref).abs()
    assert torch.all(err <= 3e-5 * absref + 1e-6), f"max err {err.max().item()}"


@pytest.mark.parametrize("pool", [True, False])
@pytest.mark.parametrize("T,B,Cin,Cout,H,W,tile", SHAPES)
def test_lif_pool_epilogue_exact(T, B, Cin, Cout, H, W, tile, pool):
    if pool and (H % 2 or W % 2):
        pytest.skip("odd spatial size")
    x, w, *bn = _setup(T, B, Cin, Cout, H, W, seed=T * 7 + Cout)
    xd, wp, bd, w2, b2 = _gpu_operands(x, w, *bn)
    for soft, vth in ((False, 1.0), (True, 0.3)):
        spk = kc.conv3x3_bn_lif_nhwc(xd, wp, bd, pool=pool, decay=0.5, in_scale=0.5,
                                     v_threshold=vth, soft_reset=soft, tile_hint=tile)
        pre = kc.conv3x3_preact_nhwc(xd, wp, bd, tile_hint=tile).cpu()
        y = pre.permute(0, 1, 4, 2, 3)                         # [T,B,C,H,W]
        s, _, _ = on.lif_multistep(y, neuron="lif", tau=2.0, soft_reset=soft, v_threshold=vth)
        if pool:
            s = of.maxpool2x2_seq(s)
        got = spk.cpu().float().permute(0, 1, 4, 2, 3)
        assert torch.equal(got, s), f"{int((got != s).sum())} spike mismatches"


def test_conv_block_baseline_config():
    """[4,32,128,16,16] Bernoulli(0.15) -> 256 ch, BN folded, LIF, 2x2 max."""
    x, w, gamma, beta, mean, var = _setup(4, 32, 128, 256, 16, 16, seed=0)
    out = kc.conv_bn_lif_pool(x.to(DEV), w.to(DEV), None, gamma.to(DEV), beta.to(DEV),
                              mean.to(DEV), var.to(DEV), 1e-5, pool="max", neuron="lif",
                              tau=2.0, v_threshold=1.0)
    assert out.shape == (4, 32, 256, 8, 8)
    ref, trace = of.conv_bn_lif_pool(x, w, None, gamma, beta, mean, var, 1e-5, pool=True,
                                     tau=2.0, v_threshold=1.0)
    got = out.float().cpu()
    agree = (got == ref).float().mean().item()
    assert agree >= 0.999, f"spike agreement {agree}"
    # flips must come from windows whose fp32 membrane was near threshold at
    # this step or an earlier one (a flip changes the later reset history)
    near = (trace - 1.0).abs().view(4, 32, 256, 8, 2, 8, 2).amin(dim=(4, 6)) < 2e-2
    near = torch.cummax(near.int(), dim=0).values.bool()
    assert not torch.any((got != ref) & ~near)


@pytest.mark.parametrize("B", [1, 32, 56])
def test_image_layer_run_lengths(B):
    """32x32 images at the batch sizes that select runs of 1, 2 and 4 pixels
    per thread: spikes match the fp64 conv + LIF except where the membrane
    came within 1e-5 of the threshold at this step or an earlier one (a flip
    there changes the neuron's later reset history)."""
    g = torch.Generator().manual_seed(40 + B)
    img = torch.randn(B, 3, 32, 32, generator=g)
    w = torch.randn(64, 3, 3, 3, generator=g) * (2.0 / 27) ** 0.5
    b = torch.randn(64, generator=g) * 0.1
    T = 4
    spk = kc.conv3x3_image_lif(img.to(DEV), w.to(DEV), b.to(DEV), T, decay=0.5,
                               in_scale=0.5, v_threshold=1.0)
    y = F.conv2d(img.double(), w.double(), b.double(), padding=1).float()
    yt = y.unsqueeze(0).expand(T, *y.shape).contiguous()
    ref, _, _ = on.lif_multistep(yt, neuron="lif")
    hs = of.membrane_trace(yt)
    got = spk.cpu().float().permute(0, 1, 4, 2, 3)
    near = torch.cummax(((hs - 1.0).abs() < 1e-5).int(), dim=0).values.bool()
    assert not torch.any((got != ref) & ~near)
    assert 0.01 < got.mean().item() < 0.99


@pytest.mark.parametrize("B,Cin,H,W,Cout", [(2, 1, 1, 1, 32), (1, 2, 2, 1, 32), (3, 4, 5, 7, 64),
                                             (2, 5, 3, 6, 32), (4, 6, 9, 3, 96), (2, 3, 1, 8, 64)])
def test_image_layer_borders_and_channel_chunks(B, Cin, H, W, Cout):
    """Maps of 1-9 pixels a side (every tap of a 1x1 image lies outside it),
    channel chunks of 4 (Cin % 3 != 0) and of 3, Cin short of a whole chunk
    (channels past Cin read as zeros): spikes match the fp64 conv + LIF away
    from the threshold, and the packed words are the bf16 spikes packed."""
    g = torch.Generator().manual_seed(100 + Cin * 7 + H)
    img = torch.randn(B, Cin, H, W, generator=g)
    w = torch.randn(Cout, Cin, 3, 3, generator=g) * (2.0 / (9 * Cin)) ** 0.5 * 2
    b = torch.randn(Cout, generator=g) * 0.1
    T = 4
    spk = kc.conv3x3_image_lif(img.to(DEV), w.to(DEV), b.to(DEV), T, decay=0.5,
                               in_scale=0.5, v_threshold=1.0)
    y = F.conv2d(img.double(), w.double(), b.double(), padding=1).float()
    yt = y.unsqueeze(0).expand(T, *y.shape).contiguous()
    ref, _, _ = on.lif_multistep(yt, neuron="lif")
    hs = of.membrane_trace(yt)
    got = spk.cpu().float().permute(0, 1, 4, 2, 3)
    near = torch.cummax(((hs - 1.0).abs() < 1e-5).int(), dim=0).values.bool()
    assert not torch.any((got != ref) & ~near)
    words = kc.conv3x3_image_lif(img.to(DEV), w.to(DEV), b.to(DEV), T, decay=0.5, in_scale=0.5,
                                 v_threshold=1.0, out_bits=True).cpu()
    bits = (words.unsqueeze(-1) >> torch.arange(32)) & 1
    assert torch.equal(bits.reshape(*words.shape[:-1], Cout).to(torch.bfloat16), spk.cpu())


def test_image_layer_and_layout():
    g = torch.Generator().manual_seed(4)
    img = torch.randn(3, 3, 12, 10, generator=g)
    w = torch.randn(64, 3, 3, 3, generator=g) * (2.0 / 27) ** 0.5
    b = torch.randn(64, generator=g) * 0.1
    T = 4
    spk = kc.conv3x3_image_lif(img.to(DEV), w.to(DEV), b.to(DEV), T, decay=0.5,
                               in_scale=0.5, v_threshold=1.0)
    y = F.conv2d(img.double(), w.double(), b.double(), padding=1).float()
    ref, _, _ = on.lif_multistep(y.unsqueeze(0).expand(T, *y.shape).contiguous(), neuron="lif")
    hs = of.membrane_trace(y.unsqueeze(0).expand(T, *y.shape).contiguous())
    got = spk.cpu().float().permute(0, 1, 4, 2, 3)
    assert not torch.any((got != ref) & ((hs - 1.0).abs() > 1e-5))
    # layout change: fp32 -> bf16 rounds like torch, u8 / bf16 exact
    x = torch.randn(2, 3, 40, 5, 7, generator=g)
    for src in (x, x.to(torch.bfloat16), (x > 0).to(torch.uint8)):
        got = kc.to_nhwc_bf16(src.to(DEV)).cpu()
        assert torch.equal(got, src.to(torch.bfloat16).permute(0, 1, 3, 4, 2))
