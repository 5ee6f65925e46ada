"""GPU parity of the fused Linear + bias + LIF kernel (1x1 mode of the conv kernel)."""
import pytest
import torch
import torch.nn.functional as F

import snnk.nn as snn
from snnk._abi import SnnkError
from oracle import neurons as on
from snnk.kernels.linear import linear_bias_lif, linear_preact

pytestmark = pytest.mark.gpu
DEV = "cuda"

SHAPES = [(4, 32, 512, 4096, -1), (4, 32, 4096, 4096, -1), (4, 2048, 384, 1152, -1),
          (5, 8, 64, 96, 4), (3, 12, 128, 64, 2), (1, 4, 32, 32, 5), (8, 16, 256, 128, 0)]


def _data(T, R, K, N, seed):
    g = torch.Generator().manual_seed(seed)
    x = (torch.rand(T, R, K, generator=g) < 0.2).float()
    w = torch.randn(N, K, generator=g) * (2.0 / K) ** 0.5
    b = torch.randn(N, generator=g) * 0.1
    return x, w, b


@pytest.mark.parametrize("T,R,K,N,tile", SHAPES)
def test_linear_preact_matches_f64(T, R, K, N, tile):
    x, w, b = _data(T, R, K, N, seed=K + N)
    y = linear_preact(x.to(DEV, torch.bfloat16), w.to(DEV, torch.bfloat16), b.to(DEV),
                      tile_hint=tile).cpu().double()
    wb = w.to(torch.bfloat16).double()
    ref = x.double() @ wb.t() + b.double()
    bound = x.double() @ wb.abs().t()
    assert torch.all((y - ref).abs() <= 3e-5 * bound + 1e-6)


@pytest.mark.parametrize("T,R,K,N,tile", SHAPES)
def test_linear_lif_epilogue_exact(T, R, K, N, tile):
    x, w, b = _data(T, R, K, N, seed=K * 3 + N)
    xd, wd, bd = x.to(DEV, torch.bfloat16), w.to(DEV, torch.bfloat16), b.to(DEV)
    for soft, vth in ((False, 1.0), (True, 0.25)):
        s = linear_bias_lif(xd, wd, bd, decay=0.5, in_scale=0.5, v_threshold=vth,
                            soft_reset=soft, tile_hint=tile).cpu().float()
        pre = linear_preact(xd, wd, bd, tile_hint=tile).cpu()
        ref, _, _ = on.lif_multistep(pre, neuron="lif", soft_reset=soft, v_threshold=vth)
        assert torch.equal(s, ref)


def test_fused_linear_neuron_module_paths():
    T, B, K, N = 4, 8, 256, 128
    x, w, b = _data(T, B, K, N, seed=1)
    mod = snn.FusedLinearNeuron(K, N, neuron="lif", tau=2.0, v_threshold=0.5).to(DEV)
    with torch.no_grad():
        mod.weight.copy_(w)
        mod.bias.copy_(b)
    # fp32 input keeps the reference's fp32 GEMM; bf16 input runs the MFMA kernel
    s32 = mod(x.to(DEV)).cpu()
    s16 = mod(x.to(DEV, torch.bfloat16)).cpu().float()
    y = F.linear(x.reshape(T * B, K).double(), w.double()).view(T, B, N).float()
    ref, _, _ = on.lif_multistep(y, bias=b, neuron="lif", v_threshold=0.5)
    tr = on.lif_membrane_trace(y + b.view(1, 1, -1), v_threshold=0.5)
    near = torch.cummax(((tr - 0.5).abs() < 1e-2).int(), 0).values.bool()
    assert s32.dtype == torch.float32 and not torch.any((s32 != ref) & ~near)
    assert (s16 == ref).float().mean().item() >= 0.999


@pytest.mark.parametrize("T,R,K,N,splits,tile", [(4, 32, 4096, 32, 0, -1), (6, 8, 512, 64, 1, -1),
                                                 (1, 12, 256, 96, 1, -1), (5, 32, 1024, 32, 4, -1),
                                                 # K-group tiles whose accumulator tiles are
                                                 # finished by different groups
                                                 (4, 32, 4096, 64, 1, 7), (5, 24, 1024, 128, 1, 9),
                                                 (4, 32, 2048, 96, 2, 41)])
def test_linear_mean_t_matches_f64(T, R, K, N, splits, tile):
    """snnk_linear_mean_t: the time average of x.w^T + b (the classifier head
    read as model(x).mean(0)) within fp32 accumulation error of float64,
    and equal to the mean of linear_preact's own per-step outputs within
    fp32 rounding of the 1/T average."""
    from snnk.kernels.linear import linear_mean_t
    g = torch.Generator().manual_seed(T * 1000 + K)
    x = (torch.rand(T, R, K, generator=g) < 0.2).to(torch.bfloat16)
    w = (torch.randn(N, K, generator=g) * K ** -0.5).to(torch.bfloat16)
    b = torch.randn(N, generator=g) * 0.1
    xd, wd, bd = x.to(DEV), w.to(DEV), b.to(DEV)
    kw = dict(splits=splits, tile_hint=tile)
    m = linear_mean_t(xd, wd, bd, **kw).cpu().double()
    ref = (x.double() @ w.double().t() + b.double()).mean(0)
    absref = (x.double() @ w.double().abs().t()).mean(0) + b.double().abs()
    assert m.shape == (R, N)
    assert torch.all((m - ref).abs() <= 3e-5 * absref + 1e-6)
    per_step = linear_preact(xd, wd, bd, **kw).cpu().double().mean(0)
    assert torch.allclose(m, per_step, rtol=1e-6, atol=1e-6)
    # repeated calls are bit-identical (fixed summation order)
    assert torch.equal(linear_mean_t(xd, wd, bd, **kw).cpu().double(), m)


@pytest.mark.parametrize("T,R,K,N,splits", [(4, 32, 2048, 2048, 0), (5, 8, 256, 128, 1),
                                            (3, 12, 512, 256, 2)])
def test_linear_pool4_epilogue_exact(T, R, K, N, splits):
    """snnk_linear_bias_lif_pool4_ws: the LIF runs per column and the output is
    the OR of each group of four adjacent columns; exact against the oracle's
    LIF + column max applied to the kernel's own pre-activations."""
    from snnk.kernels.linear import linear_bias_lif_pool4
    x, w, b = _data(T, R, K, N, seed=K + 7 * N)
    xd, wd, bd = x.to(DEV, torch.bfloat16), w.to(DEV, torch.bfloat16), b.to(DEV)
    for soft, vth in ((False, 0.5), (True, 0.25)):
        s = linear_bias_lif_pool4(xd, wd, bd, decay=0.5, in_scale=0.5, v_threshold=vth,
                                  soft_reset=soft, splits=splits).cpu().float()
        pre = linear_preact(xd, wd, bd, splits=splits).cpu()
        spk, _, _ = on.lif_multistep(pre, neuron="lif", soft_reset=soft, v_threshold=vth)
        ref = spk.view(T, R, N // 4, 4).amax(-1)
        assert s.shape == (T, R, N // 4) and torch.equal(s, ref)


@pytest.mark.parametrize("pool", [False, True])
@pytest.mark.parametrize("B,Cin,Cout", [(32, 512, 512), (8, 64, 96)])
def test_dense_small_map_conv_matches_conv_kernel(pool, B, Cin, Cout):
    """On a 2x2 map FusedConvBNLIFPool runs the conv as one dense Linear over
    (pixel, channel) (no padding taps; the 2x2 max-pool as an OR of column
    groups).  Its pre-activations equal a float64 conv of the same bf16
    operands within fp32 accumulation error, and its spikes agree with the
    direct conv kernel's (tile_hint forces that path) at >= 99.9%, every flip
    next to the threshold."""
    import torch.nn as nn
    from snnk.kernels.conv import conv3x3_dense_weight
    T, H, W = 4, 2, 2
    g = torch.Generator().manual_seed(B + Cin + Cout + pool)
    conv = nn.Conv2d(Cin, Cout, 3, padding=1)
    with torch.no_grad():
        conv.weight.copy_(torch.randn(Cout, Cin, 3, 3, generator=g) * (2.0 / (9 * Cin)) ** 0.5 * 3)
        conv.bias.copy_(torch.randn(Cout, generator=g) * 0.1)
    mod = snn.FusedConvBNLIFPool(conv, None, pool="max" if pool else None, neuron="lif",
                                 tau=2.0, v_threshold=1.0).to(DEV)
    x = (torch.rand(T, B, H, W, Cin, generator=g) < 0.3).to(torch.bfloat16)
    xd = x.to(DEV)
    dense = mod.forward_nhwc(xd).cpu().float()
    direct = mod.forward_nhwc(xd, tile_hint=3).cpu().float()
    assert dense.shape == direct.shape
    assert (dense == direct).float().mean().item() >= 0.999
    # pre-activations of the dense form against float64
    w_d, b_d = conv3x3_dense_weight(mod.weight, mod.bias, H, W, pool)
    pre = linear_preact(xd.reshape(T, B, -1), w_d, b_d).cpu().double()
    wb = mod.weight.cpu().to(torch.bfloat16).double()
    ref = F.conv2d(x.double().reshape(T * B, H, W, Cin).permute(0, 3, 1, 2), wb,
                   mod.bias.cpu().double(), padding=1)  # [TB, Cout, H, W]
    bound = F.conv2d(x.double().reshape(T * B, H, W, Cin).permute(0, 3, 1, 2), wb.abs(),
                     padding=1)
    if pool:
        ref = ref.reshape(T, B, Cout, H * W).reshape(T, B, -1)
        bound = bound.reshape(T, B, Cout, H * W).reshape(T, B, -1)
    else:
        ref = ref.permute(0, 2, 3, 1).reshape(T, B, -1)
        bound = bound.permute(0, 2, 3, 1).reshape(T, B, -1)
    assert torch.all((pre - ref).abs() <= 3e-5 * bound + 1e-6)
    # the dense path's spikes are exactly the LIF (+ column OR) of those sums
    spk, _, _ = on.lif_multistep(pre.float(), neuron="lif", v_threshold=1.0)
    if pool:
        spk = spk.view(T, B, Cout, 4).amax(-1).view(T, B, 1, 1, Cout)
    else:
        spk = spk.view(T, B, H, W, Cout)
    assert torch.equal(dense, spk)

@pytest.mark.parametrize("T,R,K,N,with_bias", [(4, 32, 4096, 10, True), (1, 5, 64, 1, True),
                                               (6, 12, 1024, 64, True), (3, 8, 8192, 33, False),
                                               (5, 3, 96, 16, True)])
def test_linear_mean_t_bits_matches_f64(T, R, K, N, with_bias):
    """snnk_linear_mean_t_bits: spike counts over T dotted with w, / T + bias,
    on packed words: within fp32 accumulation error of the float64 time
    average, close to the bf16-input head, and bit-identical on repeats."""
    from snnk.kernels.binary import pack_bits
    from snnk.kernels.linear import linear_mean_t, linear_mean_t_bits
    g = torch.Generator().manual_seed(T * 100 + K + N)
    x = (torch.rand(T, R, K, generator=g) < 0.3).to(torch.bfloat16)
    w = (torch.randn(N, K, generator=g) * K ** -0.5).to(torch.bfloat16)
    b = torch.randn(N, generator=g) * 0.1 if with_bias else None
    xd, wd = x.to(DEV), w.to(DEV)
    bd = b.to(DEV) if with_bias else None
    xp = pack_bits(xd, dim=-1)
    m = linear_mean_t_bits(xp, wd, bd).cpu().double()
    ref = (x.double() @ w.double().t()).mean(0)
    absref = (x.double() @ w.double().abs().t()).mean(0)
    if with_bias:
        ref = ref + b.double()
        absref = absref + b.double().abs()
    assert m.shape == (R, N)
    assert torch.all((m - ref).abs() <= 3e-5 * absref + 1e-6)
    assert torch.equal(linear_mean_t_bits(xp, wd, bd).cpu().double(), m)
    if N % 32 == 0 or N <= 32:
        wp = torch.zeros((N + 31) // 32 * 32, K, dtype=torch.bfloat16, device=DEV)
        wp[:N] = wd
        bp = torch.zeros(wp.shape[0], device=DEV)
        if with_bias:
            bp[:N] = bd
        R4 = (R + 3) // 4 * 4
        xr = torch.nn.functional.pad(xd, (0, 0, 0, R4 - R)).contiguous()
        mm = linear_mean_t(xr, wp, bp).cpu().double()[:R, :N]
        assert torch.all((m - mm).abs() <= 3e-5 * absref + 1e-6)


def test_linear_mean_t_bits_refuses_wide_heads():
    from snnk.kernels.binary import pack_bits
    from snnk.kernels.linear import linear_mean_t_bits
    xp = pack_bits(torch.zeros(2, 4, 64, dtype=torch.bfloat16, device=DEV), dim=-1)
    with pytest.raises(SnnkError):
        linear_mean_t_bits(xp, torch.zeros(65, 64, dtype=torch.bfloat16, device=DEV), None)
