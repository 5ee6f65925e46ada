"""HIP kernels against the committed golden fixtures (plain-Python loops,
tests/golden/make_golden.py): LIF spikes and final membrane bit for bit,
packed words and popcount GEMM counts bit for bit (both GEMM algorithms),
conv pre-activations within fp32 accumulation error of the exact sums and
spikes equal wherever the membrane is not within 1e-5 of the threshold,
attention counts bit for bit."""
import numpy as np
import pytest
import torch

import snnk
from golden_data import load
from snnk.kernels import conv as kc
from snnk.kernels.attention import spike_attention
from snnk.kernels.fused import fused_bias_if_lif_stateful
from oracle import fused as of

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.mark.parametrize("i", range(5))
def test_lif_kernel_matches_fixture(i):
    c = load("lif")["cases"][i]
    T, B, C, HW = c["shape"]
    x = torch.tensor(c["x"], dtype=torch.float32).view(T, B, C, HW).to(DEV)
    thr = c["v_threshold"]
    thr = torch.tensor(thr, dtype=torch.float32, device=DEV) if isinstance(thr, list) else thr
    s = snnk.if_lif(x, neuron=c["neuron"], tau=c["tau"], soft_reset=c["soft_reset"],
                    v_threshold=thr, v_reset=c["v_reset"])
    assert torch.equal(s.cpu(), torch.tensor(c["spikes"]).view(T, B, C, HW))
    if not isinstance(thr, torch.Tensor):   # the stateful entry takes a float threshold
        s2, v = fused_bias_if_lif_stateful(x, None, return_v=True, neuron=c["neuron"],
                                           tau=c["tau"], soft_reset=c["soft_reset"],
                                           v_threshold=thr, v_reset=c["v_reset"])
        assert torch.equal(s2.cpu(), s.cpu())
        assert torch.equal(v.cpu().reshape(-1), torch.tensor(c["v_final"], dtype=torch.float32))


@pytest.mark.parametrize("algo", ["popc", "mfma"])
def test_bits_kernels_match_fixture(algo):
    g = load("bits")
    A = torch.tensor(g["A"], dtype=torch.float32, device=DEV)
    W = torch.tensor(g["W"], dtype=torch.float32, device=DEV)
    Ap = snnk.pack_bits(A)
    assert np.array_equal(Ap.cpu().numpy().view(np.uint32), np.array(g["A_packed"], np.uint32))
    for signed, key in ((False, "C"), (True, "C_signed")):
        C = snnk.binary_gemm(A, W.t().contiguous(), signed=signed, algo=algo)
        assert np.array_equal(C.cpu().numpy(), np.array(g[key]))


@pytest.mark.parametrize("pool", [False, True])
def test_conv_kernel_matches_fixture(pool):
    g = load("conv")
    sh = g["shape"]
    x = torch.tensor(g["x_nhwc"], dtype=torch.bfloat16, device=DEV)          # [T,B,H,W,Cin]
    w = torch.tensor(g["w_khkwcin"])                                          # [Cout,3,3,Cin]
    wp = w.reshape(sh["Cout"], -1).to(torch.bfloat16).contiguous().to(DEV)    # k=(kh*3+kw)*Cin+c
    b = torch.tensor(g["bias"], dtype=torch.float32, device=DEV)
    pre_ref = torch.tensor(g["preact"], dtype=torch.float64)
    pre = kc.conv3x3_preact_nhwc(x, wp, b).cpu().double()
    bound = 3e-7 * (torch.tensor(g["w_khkwcin"]).abs().sum((1, 2, 3)).max() + 1)
    assert (pre - pre_ref).abs().max() <= bound
    s = kc.conv3x3_bn_lif_nhwc(x, wp, b, pool=pool, decay=0.5, in_scale=0.5,
                               v_threshold=1.0).cpu().float()
    want = torch.tensor(g["pooled" if pool else "spikes"])
    trace = of.membrane_trace(pre_ref.permute(0, 1, 4, 2, 3).float())       # [T,B,C,H,W]
    near = torch.cummax(((trace - 1.0).abs() < 1e-5).int(), 0).values.bool().permute(0, 1, 3, 4, 2)
    if pool:
        Tn, Bn, H, W_, Cn = near.shape
        near = near.view(Tn, Bn, H // 2, 2, W_ // 2, 2, Cn).any(4).any(2)
    assert not torch.any((s != want) & ~near)


def test_attention_kernel_matches_fixture():
    g = load("attention")
    Hh, N, d = g["heads"], g["N"], g["d"]
    q, k, v = (torch.tensor(g[n], dtype=torch.float32) for n in ("q", "k", "v"))  # [h,N,d]
    to_rows = lambda t: t.permute(1, 0, 2).reshape(1, N, Hh * d)  # noqa: E731  [T=1, B*N, D]
    qd, kd, vd = (to_rows(t).to(DEV, torch.bfloat16) for t in (q, k, v))
    _, S, O = spike_attention(qd, kd, vd, B=1, N=N, heads=Hh, scale=0.125, return_counts=True)
    assert torch.equal(S.cpu()[0, 0].long(), torch.tensor(g["S"]))
    assert torch.equal(O.cpu()[0, 0].long(), torch.tensor(g["O"]))
    kv = snnk.spike_ktv_popcount(k.view(1, 1, Hh, N, d).to(DEV), v.view(1, 1, Hh, N, d).to(DEV))
    assert torch.equal(kv.cpu()[0, 0].long(), torch.tensor(g["KtV"]))
