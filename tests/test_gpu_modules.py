"""GPU module tests for the residual and rate-coded neuron modules.

Restates the structure of the reference's own tests:
  residual kernel path bit-equal     snn_compiler/tests/test_residual_and_zoo.py:22-55
  FusedAddNeuron / FusedConvBNAddNeuron  test_residual_and_zoo.py:61-103
  RateCoded{LIF,IF}Node == sum over T    snn_compiler/tests/test_largeT_and_rate.py:71-103

The oracle is the CPU restatement ``oracle.neurons.lif_multistep``.  The
neuron part of every module is bit-equal to it.  FusedConvBNAddNeuron runs
its convolution on the vendor library (MIOpen), whose fp32 rounding differs
from the CPU's, so its neuron is checked teacher-forced (the oracle gets the
GPU's own conv output) and the whole module against an all-CPU pipeline at
>= 99.9% spike agreement.
"""
import pytest
import torch
import torch.nn as nn
import torch.nn.functional as F

from oracle import neurons as on
from snnk.nn import (FusedAddNeuron, FusedConvBNAddNeuron, RateCodedIFNode, RateCodedLIFNode,
                     LIFNode, IFNode)
from snnk.kernels.fused import fused_bias_if_lif

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _randn(shape, seed, scale=1.0):
    return torch.randn(*shape, generator=torch.Generator().manual_seed(seed)) * scale


MODES = [("if", True, 0.0), ("if", False, 0.0), ("if", False, 0.3),
         ("lif", True, 0.0), ("lif", False, 0.0), ("lif", False, 0.3)]


@pytest.mark.parametrize("neuron,soft,v_reset", MODES)
@pytest.mark.parametrize("layout", ["NCHW", "NHWC"])
def test_fused_bias_residual_kernel_bit_equal(neuron, soft, v_reset, layout):
    T, B, C, H, W = 4, 2, 16, 8, 8
    y, r, bias = _randn((T, B, C, H, W), 1), _randn((T, B, C, H, W), 2), _randn((C,), 3)
    ref, _, _ = on.lif_multistep(y, bias=bias, residual=r, neuron=neuron, tau=2.0,
                                 soft_reset=soft, v_threshold=1.0, v_reset=v_reset)
    yd, rd = y.to(DEV), r.to(DEV)
    if layout == "NHWC":
        yd = yd.reshape(T * B, C, H, W).contiguous(memory_format=torch.channels_last).view(
            T, B, C, H, W)
        rd = rd.reshape(T * B, C, H, W).contiguous(memory_format=torch.channels_last).view(
            T, B, C, H, W)
    out = fused_bias_if_lif(yd, bias.to(DEV), residual=rd, neuron=neuron, tau=2.0,
                            decay_input=True, soft_reset=soft, v_threshold=1.0,
                            v_reset=v_reset, layout=layout)
    assert torch.equal(out.cpu(), ref)


@pytest.mark.parametrize("neuron,soft,v_reset", MODES)
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_fused_add_neuron_module(neuron, soft, v_reset, dtype):
    a = _randn((4, 2, 16, 8, 8), 11).to(dtype)
    b = _randn((4, 2, 16, 8, 8), 12).to(dtype)
    m = FusedAddNeuron(neuron=neuron, tau=2.0, decay_input=True, soft_reset=soft,
                       v_threshold=1.0, v_reset=v_reset)
    out = m(a.to(DEV), b.to(DEV))
    ref, _, _ = on.lif_multistep(a, residual=b, neuron=neuron, tau=2.0, soft_reset=soft,
                                 v_threshold=1.0, v_reset=v_reset)
    assert out.dtype == dtype and torch.equal(out.cpu().float(), ref)


def _conv_bn(in_c, out_c, seed):
    g = torch.Generator().manual_seed(seed)
    conv = nn.Conv2d(in_c, out_c, 3, padding=1, bias=False)
    with torch.no_grad():
        conv.weight.copy_(torch.randn(conv.weight.shape, generator=g) * (2.0 / (9 * in_c)) ** 0.5)
    bn = nn.BatchNorm2d(out_c)
    with torch.no_grad():
        bn.running_mean.copy_(torch.randn(out_c, generator=g) * 0.1)
        bn.running_var.copy_(torch.rand(out_c, generator=g) + 0.5)
        bn.weight.copy_(torch.rand(out_c, generator=g) + 0.5)
        bn.bias.copy_(torch.randn(out_c, generator=g) * 0.1)
    return conv.eval(), bn.eval()


@pytest.mark.parametrize("fold_bn", [False, True])
@pytest.mark.parametrize("soft", [False, True])
def test_fused_conv_bn_add_neuron_module(fold_bn, soft):
    """conv(x) -> BN -> + r -> LIF, the residual block of snn_compiler/nn/modules.py:360-443."""
    T, B, Cin, Cout, H, W = 4, 2, 8, 16, 16, 16
    conv, bn = _conv_bn(Cin, Cout, 5)
    x, r = _randn((T, B, Cin, H, W), 6), _randn((T, B, Cout, H, W), 7)
    kw = dict(neuron="lif", tau=2.0, decay_input=True, soft_reset=soft, v_threshold=1.0,
              v_reset=0.0)
    mod = FusedConvBNAddNeuron(conv, bn, fold_bn=fold_bn, layout="NCHW", **kw).to(DEV)
    out = mod(x.to(DEV), r.to(DEV)).cpu()

    # teacher-forced: the oracle neuron on the GPU's own conv (+ BN) output
    with torch.no_grad():
        xd = x.to(DEV).reshape(T * B, Cin, H, W)
        if fold_bn:
            y = F.conv2d(xd, mod.weight, None, padding=1).view(T, B, Cout, H, W).cpu()
            ref_tf, _, _ = on.lif_multistep(y, bias=mod.bias.detach().cpu(), residual=r, **kw)
        else:
            y = F.batch_norm(F.conv2d(xd, mod.weight, None, padding=1), mod.bn_mean, mod.bn_var,
                             mod.bn_weight, mod.bn_bias, training=False, eps=mod.bn_eps)
            ref_tf, _, _ = on.lif_multistep(y.view(T, B, Cout, H, W).cpu(), residual=r, **kw)
    assert torch.equal(out, ref_tf)

    # end to end against an all-CPU pipeline (unfolded conv + BN)
    with torch.no_grad():
        y_cpu = bn(conv(x.reshape(T * B, Cin, H, W))).view(T, B, Cout, H, W)
    ref, _, _ = on.lif_multistep(y_cpu + r, **kw)
    agree = float((out == ref).float().mean())
    assert agree >= 0.999, agree


def test_fused_conv_bn_add_neuron_resnet_block():
    """A two-conv basic block wired like the reference's ResNet: the second
    neuron takes the block input as its residual, neuron2(conv2(s1), x)."""
    T, B, C, H, W = 4, 2, 16, 8, 8
    c1, b1 = _conv_bn(C, C, 21)
    c2, b2 = _conv_bn(C, C, 22)
    x = (torch.rand(T, B, C, H, W, generator=torch.Generator().manual_seed(23)) < 0.3).float()
    kw = dict(neuron="lif", tau=2.0, decay_input=True, soft_reset=False, v_threshold=1.0,
              v_reset=0.0)
    from snnk.nn import FusedConvBNNeuron
    n1 = FusedConvBNNeuron(c1, b1, fold_bn=False, **kw).to(DEV)
    n2 = FusedConvBNAddNeuron(c2, b2, fold_bn=False, **kw).to(DEV)
    xd = x.to(DEV)
    s1 = n1(xd)
    out = n2(s1, xd).cpu()
    with torch.no_grad():
        y2 = F.batch_norm(F.conv2d(s1.reshape(T * B, C, H, W), n2.weight, None, padding=1),
                          n2.bn_mean, n2.bn_var, n2.bn_weight, n2.bn_bias, training=False,
                          eps=n2.bn_eps).view(T, B, C, H, W).cpu()
    ref, _, _ = on.lif_multistep(y2, residual=x, **kw)
    assert torch.equal(out, ref)
    assert 0 < int(out.sum()) < out.numel()


@pytest.mark.parametrize("T", [4, 16, 64])
@pytest.mark.parametrize("soft", [True, False])
def test_rate_coded_lif_node(T, soft):
    x = _randn((T, 2, 8, 16, 16), 100 + T)
    mod = RateCodedLIFNode(tau=2.0, decay_input=True, soft_reset=soft, v_threshold=1.0,
                           v_reset=0.0, layout="NCHW")
    out = mod(x.to(DEV))
    _, _, count = on.lif_multistep(x, neuron="lif", tau=2.0, soft_reset=soft, v_threshold=1.0)
    assert out.shape == x.shape[1:] and out.dtype == torch.float32
    assert torch.equal(out.cpu(), count)
    # the count equals the sum over T of the spiking node's output
    s = LIFNode(tau=2.0, soft_reset=soft)(x.to(DEV))
    assert torch.equal(s.sum(0).cpu(), count)


@pytest.mark.parametrize("T", [4, 16, 64])
@pytest.mark.parametrize("decay", [1.0, 0.95])
@pytest.mark.parametrize("soft", [True, False])
def test_rate_coded_if_node(T, decay, soft):
    x = _randn((T, 2, 8, 16, 16), 200 + T)
    mod = RateCodedIFNode(decay=decay, soft_reset=soft, v_threshold=1.0, v_reset=0.0,
                          layout="NCHW")
    out = mod(x.to(DEV))
    _, _, count = on.lif_multistep(x, neuron="if", decay=decay, soft_reset=soft,
                                   v_threshold=1.0)
    assert torch.equal(out.cpu(), count)
    s = IFNode(decay=decay, soft_reset=soft)(x.to(DEV))
    assert torch.equal(s.sum(0).cpu(), count)


def test_rate_coded_per_channel_threshold_nhwc():
    T, B, C, H, W = 8, 2, 16, 6, 6
    x = _randn((T, B, C, H, W), 300)
    vth = torch.rand(C, generator=torch.Generator().manual_seed(301)) * 0.5 + 0.5
    xd = x.to(DEV).reshape(T * B, C, H, W).contiguous(memory_format=torch.channels_last)
    mod = RateCodedLIFNode(tau=3.0, v_threshold=vth.to(DEV), layout="NHWC")
    out = mod(xd.view(T, B, C, H, W))
    _, _, count = on.lif_multistep(x, neuron="lif", tau=3.0, v_threshold=vth)
    assert torch.equal(out.cpu().contiguous(), count)


def test_conv_pool_dense_weights_follow_state_dict():
    """The 2x2-map path caches a dense form of the weights; loading new
    weights after a first forward must change the output (no stale cache)."""
    from snnk.nn import FusedConvBNLIFPool
    C, T, B = 64, 4, 8
    g = torch.Generator().manual_seed(31)
    conv = nn.Conv2d(C, C, 3, padding=1)
    with torch.no_grad():
        conv.weight.copy_(torch.randn(conv.weight.shape, generator=g) * 0.2)
        conv.bias.zero_()
    mod = FusedConvBNLIFPool(conv.eval(), None, pool="max").to(DEV)
    x = (torch.rand(T, B, C, 2, 2, generator=g) < 0.5).float().to(DEV)
    y1 = mod(x).clone()
    sd = {k: v.clone() for k, v in mod.state_dict().items()}
    sd["weight"] = -sd["weight"]
    sd["w_prep"] = -sd["w_prep"]
    mod.load_state_dict(sd)
    y2 = mod(x)
    assert not torch.equal(y1, y2)
    # and equals a fresh module built with the negated weights
    conv2 = nn.Conv2d(C, C, 3, padding=1)
    with torch.no_grad():
        conv2.weight.copy_(-conv.weight)
        conv2.bias.zero_()
    fresh = FusedConvBNLIFPool(conv2.eval(), None, pool="max").to(DEV)
    assert torch.equal(fresh(x), y2)


def _spikes(shape, seed, p=0.2):
    return (torch.rand(*shape, generator=torch.Generator().manual_seed(seed)) < p).float()


def _membrane_near(y, bias, neuron, soft, v_reset, tol=2e-2):
    """Steps at which the fp32 membrane (CPU oracle, fed the conv output y) is
    within tol of the threshold, at that step or earlier."""
    from oracle.fused import membrane_trace
    tr = membrane_trace(y, bias=bias, neuron=neuron, tau=2.0, soft_reset=soft,
                        v_threshold=1.0, v_reset=v_reset)
    near = (tr - 1.0).abs() < tol
    return torch.cummax(near.int(), 0).values.bool()


@pytest.mark.parametrize("neuron,soft,v_reset", [("lif", False, 0.0), ("if", True, 0.0),
                                                 ("lif", True, 0.2)])
@pytest.mark.parametrize("layout", ["NCHW", "NHWC"])
def test_conv_bn_neuron_bf16_runs_the_hip_conv(neuron, soft, v_reset, layout):
    """FusedConvBNNeuron (BN folded) on bf16 spikes with a 3x3 conv runs the
    HIP implicit-GEMM conv with the neuron in its epilogue: the same spikes as
    FusedConvBNLIFPool without a pool (same kernel), >= 99.9% agreement with
    the fp32 conv + oracle neuron with every flip near threshold, and the
    module's layout contract (channels-last memory for 'NHWC')."""
    from snnk.nn import FusedConvBNNeuron, FusedConvBNLIFPool
    from oracle.fused import fold_conv_bn, conv3x3_seq
    torch.manual_seed(0)
    conv = nn.Conv2d(64, 96, 3, padding=1)
    bn = nn.BatchNorm2d(96).eval()
    with torch.no_grad():
        conv.weight.mul_(2.0)
        bn.running_mean.uniform_(-0.1, 0.1)
        bn.running_var.uniform_(0.5, 1.5)
    kw = dict(neuron=neuron, tau=2.0, soft_reset=soft, v_threshold=1.0, v_reset=v_reset)
    mod = FusedConvBNNeuron(conv, bn, fold_bn=True, layout=layout, **kw).to(DEV)
    x = _spikes((4, 2, 64, 10, 6), 21)
    got = mod(x.to(DEV, torch.bfloat16))
    assert got.dtype == torch.bfloat16 and got.shape == (4, 2, 96, 10, 6)
    if layout == "NHWC":
        assert got[0].is_contiguous(memory_format=torch.channels_last)
    else:
        assert got.is_contiguous()
    pool = FusedConvBNLIFPool(conv, bn, pool=None, **kw).to(DEV)
    assert torch.equal(got, pool(x.to(DEV, torch.bfloat16)))
    w2, b2 = fold_conv_bn(conv.weight.detach(), conv.bias.detach(), bn.weight.detach(),
                          bn.bias.detach(), bn.running_mean, bn.running_var, bn.eps)
    y = conv3x3_seq(x, w2)
    ref, _, _ = on.lif_multistep(y, bias=b2, neuron=neuron, tau=2.0, soft_reset=soft,
                                 v_threshold=1.0, v_reset=v_reset)
    g = got.float().cpu()
    assert (g == ref).float().mean().item() >= 0.999
    assert not torch.any((g != ref) & ~_membrane_near(y, b2, neuron, soft, v_reset))
    # fp32 input keeps the vendor conv in fp32, then the HIP neuron: the
    # oracle's neuron on the same conv output is bit-equal to it
    mod.conv_mfma = False
    got32 = mod(x.to(DEV)).cpu()
    assert (got32 == ref).float().mean().item() >= 0.999


def test_conv_neuron_bf16_runs_the_hip_conv_and_opt_out():
    """FusedConvNeuron with bias on bf16 spikes: the HIP conv path equals the
    vendor path (conv_mfma=False, bf16 conv + HIP neuron) up to near-threshold
    flips; shapes outside the kernel (5x5, Cin % 32 != 0) keep the vendor conv."""
    from snnk.nn import FusedConvNeuron
    torch.manual_seed(1)
    mod = FusedConvNeuron(32, 64, 3, padding=1, neuron="lif", tau=2.0).to(DEV)
    with torch.no_grad():
        mod.weight.mul_(3.0)
    x = _spikes((4, 4, 32, 8, 8), 31).to(DEV, torch.bfloat16)
    hip = mod(x).float()
    mod.conv_mfma = False
    vendor = mod(x).float()
    assert (hip == vendor).float().mean().item() >= 0.999
    odd = FusedConvNeuron(32, 64, 5, padding=2, neuron="lif").to(DEV)
    assert odd(x).shape == (4, 4, 64, 8, 8)
    narrow = FusedConvNeuron(3, 64, 3, padding=1, neuron="lif").to(DEV)
    assert narrow(_spikes((4, 2, 3, 8, 8), 32).to(DEV, torch.bfloat16)).shape == (4, 2, 64, 8, 8)


def test_functional_conv_and_linear_neuron_bf16_paths():
    """conv_neuron / linear_neuron (the reference's functional forms) on bf16
    spikes run the fused HIP kernels; against the same call in fp32 (vendor
    conv / GEMM in fp32, then the HIP neuron) >= 99.9% of the spikes agree."""
    from snnk.kernels.fused import conv_neuron, linear_neuron
    g = torch.Generator().manual_seed(41)
    x = _spikes((4, 2, 64, 8, 8), 42).to(DEV)
    w = (torch.randn(64, 64, 3, 3, generator=g) * (2.0 / 576) ** 0.5 * 3).to(DEV)
    b = (torch.randn(64, generator=g) * 0.1).to(DEV)
    kw = dict(stride=1, padding=1, neuron="lif", tau=2.0)
    s16 = conv_neuron(x.to(torch.bfloat16), w.to(torch.bfloat16), b, **kw)
    s32 = conv_neuron(x, w, b, **kw)
    assert s16.dtype == torch.bfloat16 and s16.shape == s32.shape
    assert (s16.float() == s32).float().mean().item() >= 0.999
    assert 0 < s32.sum().item() < s32.numel()
    xl = _spikes((4, 8, 256), 43).to(DEV)
    wl = (torch.randn(128, 256, generator=g) * (2.0 / 256) ** 0.5 * 3).to(DEV)
    bl = (torch.randn(128, generator=g) * 0.1).to(DEV)
    l16 = linear_neuron(xl.to(torch.bfloat16), wl, bl, neuron="lif", tau=2.0)
    l32 = linear_neuron(xl, wl, bl, neuron="lif", tau=2.0)
    assert l16.dtype == torch.bfloat16 and l16.shape == (4, 8, 128)
    assert (l16.float() == l32).float().mean().item() >= 0.999
