"""GPU edge cases of every operator: empty batches and time axes return empty
results without a launch, single steps and single rows run, and the smallest
legal shapes of each kernel agree with the oracle."""
import numpy as np
import pytest
import torch

import snnk
from oracle import bits as ob
from oracle import neurons as on
from snnk.kernels import conv as kc
from snnk.kernels.linear import linear_bias_lif, linear_preact

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.mark.parametrize("shape", [(0, 2, 8), (3, 0, 8), (2, 4, 0)])
def test_lif_empty(shape):
    x = torch.zeros(shape, device=DEV)
    s = snnk.if_lif(x, neuron="lif", tau=2.0)
    assert s.shape == x.shape


def test_lif_single_step_single_neuron():
    x = torch.tensor([[[1.5]], [[0.25]]], device=DEV)  # T=2, B=1, one neuron
    s = snnk.if_lif(x, neuron="lif", tau=2.0, v_threshold=0.5).cpu()
    ref, _, _ = on.lif_multistep(x.cpu(), neuron="lif", tau=2.0, v_threshold=0.5)
    assert torch.equal(s, ref)
    s1 = snnk.if_lif(x[:1], neuron="if", v_threshold=1.0).cpu()
    assert s1.flatten().tolist() == [1.0]


@pytest.mark.parametrize("M,N,K", [(0, 4, 32), (4, 0, 32), (1, 1, 1)])
def test_binary_gemm_degenerate(M, N, K):
    A = (torch.rand(M, K) < 0.5).to(torch.uint8)
    W = (torch.rand(K, N) < 0.5).to(torch.uint8)
    for algo in ("auto", "popc", "mfma", "mfma_f4"):
        C = snnk.binary_gemm(A.to(DEV), W.to(DEV), algo=algo)
        assert C.shape == (M, N)
        if M and N:
            assert np.array_equal(C.cpu().numpy(), ob.binary_gemm_closed_form(A.numpy(), W.numpy()))


def test_pack_bits_empty_and_single():
    assert snnk.pack_bits(torch.zeros(0, 40, device=DEV)).shape == (0, 2)
    one = torch.zeros(1, 1, device=DEV)
    one[0, 0] = 1
    assert snnk.pack_bits(one).cpu().tolist() == [[1]]


def test_conv_empty_batch_and_time():
    w = kc.prepare_conv3x3_weight(torch.randn(32, 32, 3, 3, device=DEV))
    b = torch.zeros(32, device=DEV)
    for T, B in ((0, 2), (2, 0)):
        x = torch.zeros(T, B, 4, 4, 32, device=DEV, dtype=torch.bfloat16)
        y = kc.conv3x3_bn_lif_nhwc(x, w, b, pool=True, decay=0.5, in_scale=0.5, v_threshold=1.0)
        assert y.shape == (T, B, 2, 2, 32)


def test_conv_single_step_2x2_map():
    """T=1, B=1, a 2x2 map (the smallest pooled case): conv kernel path."""
    g = torch.Generator().manual_seed(5)
    x = (torch.rand(1, 1, 2, 2, 32, generator=g) < 0.5).to(torch.bfloat16)
    w = torch.randn(64, 32, 3, 3, generator=g) * 0.3
    wp = kc.prepare_conv3x3_weight(w.to(DEV))
    b = torch.zeros(64, device=DEV)
    pre = kc.conv3x3_preact_nhwc(x.to(DEV), wp, b).cpu().double()
    ref = torch.nn.functional.conv2d(x.double().permute(0, 1, 4, 2, 3)[0],
                                     w.to(torch.bfloat16).double(), padding=1)
    assert torch.allclose(pre[0], ref.permute(0, 2, 3, 1), atol=1e-4)
    s = kc.conv3x3_bn_lif_nhwc(x.to(DEV), wp, b, pool=True, decay=0.5, in_scale=0.5,
                               v_threshold=0.25).cpu().float()
    spk, _, _ = on.lif_multistep(pre.float(), neuron="lif", v_threshold=0.25)
    assert torch.equal(s, spk.amax(dim=(2, 3), keepdim=True))


def test_linear_empty_rows_and_single_step():
    w = (torch.randn(64, 32) * 0.2).to(torch.bfloat16).to(DEV)
    b = torch.zeros(64, device=DEV)
    x0 = torch.zeros(2, 0, 32, device=DEV, dtype=torch.bfloat16)
    assert linear_bias_lif(x0, w, b, decay=0.5, in_scale=0.5, v_threshold=1.0).shape == (2, 0, 64)
    x = (torch.rand(1, 4, 32) < 0.5).to(torch.bfloat16)
    pre = linear_preact(x.to(DEV), w, b).cpu().double()
    ref = x.double() @ w.cpu().double().t()
    assert torch.allclose(pre, ref, atol=1e-5)


def test_spike_attention_single_token_and_step():
    """N=1 token, d=8, T=1: S = q.k, O = S v, LIF on the scaled count."""
    from snnk.kernels.attention import spike_attention
    q = torch.zeros(1, 1, 8, device=DEV, dtype=torch.bfloat16)
    k = torch.zeros_like(q)
    v = torch.zeros_like(q)
    q[0, 0, :3] = 1
    k[0, 0, :2] = 1
    v[0, 0, ::2] = 1
    spk, S, O = spike_attention(q, k, v, B=1, N=1, heads=1, scale=1.0, tau=2.0,
                                v_threshold=0.5, return_counts=True)
    assert S.flatten().tolist() == [2]
    assert O.flatten().tolist() == [2, 0, 2, 0, 2, 0, 2, 0]
    assert spk.float().flatten().tolist() == [1, 0, 1, 0, 1, 0, 1, 0]


def test_rate_and_stateful_with_no_steps():
    """T=0: the rate count is zero and the carried membrane is returned as is."""
    y = torch.zeros(0, 2, 4, 3, 3, device=DEV)
    c = snnk.fused_bias_if_lif_rate(y, None, neuron="lif", tau=2.0)
    assert c.shape == (2, 4, 3, 3) and not torch.any(c)
    v0 = torch.randn(2, 4, 3, 3, device=DEV)
    s, v = snnk.fused_bias_if_lif_stateful(y, None, v_init=v0, return_v=True, neuron="lif")
    assert s.shape == y.shape and torch.equal(v, v0)
    s, v = snnk.fused_bias_if_lif_stateful(y, None, return_v=True, neuron="lif")
    assert not torch.any(v)
