"""The oracle against the committed golden fixtures (CPU).

The fixtures come from plain-Python loops (tests/golden/make_golden.py) that
share no code with the oracle: fp32-rounded LIF steps in the reference's
operation order, LSB-first packing, popcount and integer matrix products,
exact double conv sums.  A dropped term, a swapped operand, a wrong reset or
bit order in the oracle fails one of these.
"""
import numpy as np
import pytest
import torch

from golden_data import load
from oracle import neurons as on, bits as ob, fused as of, clib


@pytest.mark.parametrize("i", range(5))
def test_lif_oracle_matches_fixture(i):
    c = load("lif")["cases"][i]
    T, B, C, HW = c["shape"]
    x = torch.tensor(c["x"], dtype=torch.float32).view(T, B, C, HW)
    thr = c["v_threshold"]
    thr = torch.tensor(thr, dtype=torch.float32) if isinstance(thr, list) else thr
    s, v, _ = on.lif_multistep(x, neuron=c["neuron"], tau=c["tau"], soft_reset=c["soft_reset"],
                               v_threshold=thr, v_reset=c["v_reset"])
    assert torch.equal(s, torch.tensor(c["spikes"]).view(T, B, C, HW))
    assert torch.equal(v, torch.tensor(c["v_final"], dtype=torch.float32).view(B, C, HW))
    # the C restatement
    df, sc = on.neuron_params(c["neuron"], c["tau"], None, True)
    per_c = isinstance(thr, torch.Tensor)
    sp, vf = clib.lif_f32(x.numpy().reshape(T, -1), C_=C, HW=HW,
                          vth=thr.view(1, C, 1).expand(B, C, HW).reshape(-1).numpy()
                          if per_c else None,                     # per-neuron array
                          vth_scalar=0.0 if per_c else float(thr), df=df, sc=sc,
                          soft_reset=c["soft_reset"], v_reset=c["v_reset"])
    assert np.array_equal(sp, np.array(c["spikes"], np.float32))
    assert np.array_equal(vf, np.array(c["v_final"], np.float32))


def test_bits_oracle_matches_fixture():
    g = load("bits")
    A, W = np.array(g["A"]), np.array(g["W"])
    Ap, Wp = ob.pack_rows(A), ob.pack_rows(W)
    assert np.array_equal(Ap, np.array(g["A_packed"], np.uint32))
    assert np.array_equal(Wp, np.array(g["W_packed"], np.uint32))
    assert np.array_equal(clib.pack_bits(A), Ap)
    assert np.array_equal(ob.popcount_gemm(Ap, Wp), np.array(g["C"]))
    assert np.array_equal(ob.popcount_gemm(Ap, Wp, signed=True), np.array(g["C_signed"]))
    assert np.array_equal(clib.popcount_gemm(Ap, Wp), np.array(g["C"]))
    assert np.array_equal(clib.popcount_gemm(Ap, Wp, signed=True), np.array(g["C_signed"]))
    assert ob.pack_rows(np.ones((1, 70)))[0].tolist() == g["all_ones_70"]
    for j, words in g["single_bits"].items():
        row = np.zeros((1, 70))
        row[0, int(j)] = 1
        assert ob.pack_rows(row)[0].tolist() == words


def test_conv_oracle_matches_fixture():
    g = load("conv")
    sh = g["shape"]
    x = torch.tensor(g["x_nhwc"]).permute(0, 1, 4, 2, 3)                  # [T,B,Cin,H,W]
    w = torch.tensor(g["w_khkwcin"]).permute(0, 3, 1, 2)                  # [Cout,Cin,3,3]
    b = torch.tensor(g["bias"])
    pre = torch.tensor(g["preact"], dtype=torch.float64).permute(0, 1, 4, 2, 3)
    # exact double path
    y64 = of.conv3x3_direct_f64(x[0], w) + b.double().view(1, -1, 1, 1)
    assert torch.allclose(y64, pre[0], rtol=0, atol=1e-12)
    # fp32 torch path, then LIF + pool on its output
    y = of.conv3x3_seq(x, w, b)
    assert torch.allclose(y.double(), pre, rtol=0, atol=2e-5)
    s, _, _ = on.lif_multistep(pre.float(), neuron="lif", tau=2.0, v_threshold=1.0)
    assert torch.equal(s, torch.tensor(g["spikes"]).permute(0, 1, 4, 2, 3))
    assert torch.equal(of.maxpool2x2_seq(s), torch.tensor(g["pooled"]).permute(0, 1, 4, 2, 3))


def test_attention_oracle_matches_fixture():
    g = load("attention")
    q, k, v = (np.array(g[n]) for n in ("q", "k", "v"))
    S = q @ k.transpose(0, 2, 1)
    assert np.array_equal(S, np.array(g["S"]))
    assert np.array_equal(S @ v, np.array(g["O"]))
    assert np.array_equal(ob.ktv_counts(k, v), np.array(g["KtV"]))
