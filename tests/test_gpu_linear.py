"""GPU parity of the fused Linear + bias + LIF kernel (1x1 mode of the conv kernel)."""
import pytest
import torch
import torch.nn.functional as F

import snnk.nn as snn
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


@pytest.mark.parametrize("T,R,K,N,splits", [(4, 32, 4096, 32, 0), (6, 8, 512, 64, 1),
                                            (1, 12, 256, 96, 1), (5, 32, 1024, 32, 4)])
def test_linear_mean_t_matches_f64(T, R, K, N, splits):
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
    m = linear_mean_t(xd, wd, bd, splits=splits).cpu().double()
    ref = (x.double() @ w.double().t() + b.double()).mean(0)
    absref = (x.double() @ w.double().abs().t()).mean(0) + b.double().abs()
    assert m.shape == (R, N)
    assert torch.all((m - ref).abs() <= 3e-5 * absref + 1e-6)
    per_step = linear_preact(xd, wd, bd, splits=splits).cpu().double().mean(0)
    assert torch.allclose(m, per_step, rtol=1e-6, atol=1e-6)
    # repeated calls are bit-identical (fixed summation order)
    assert torch.equal(linear_mean_t(xd, wd, bd, splits=splits).cpu().double(), m)
