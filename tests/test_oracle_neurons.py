"""Pins for oracle/neurons.py (multi-step IF/LIF restatement).

Each check fixes the oracle independently of its own formula: hand-computed
sequences, a pure-Python float32 scalar loop, the separately written C
restatement, IF closed forms, and sensitivity to planted mistakes.
"""
import itertools

import numpy as np
import pytest
import torch

from oracle import clib
from oracle import neurons as on


def _scalar_loop(x, *, df, sc, th, soft, vr, bias=None, C=1, HW=1, v0=None):
    """Pure-Python loop over numpy.float32 scalars (every op rounded to fp32)."""
    T, NCL = x.shape
    f = np.float32
    spikes = np.zeros((T, NCL), np.float32)
    vout = np.zeros(NCL, np.float32)
    for i in range(NCL):
        v = f(0) if v0 is None else f(v0[i])
        thr = f(th[i]) if isinstance(th, np.ndarray) else f(th)
        for t in range(T):
            u = f(x[t, i])
            if bias is not None:
                u = f(u + f(bias[(i // HW) % C]))
            h = f(f(f(df) * v) + f(f(sc) * u))
            s = h >= thr
            spikes[t, i] = 1.0 if s else 0.0
            v = (f(h - thr) if soft else f(vr)) if s else h
        vout[i] = v
    return spikes, vout


def test_known_answers_lif_hard():
    # tau=2, decay_input: v = 0.5 v + 0.5 x; theta=1, hard reset to 0.
    x = torch.tensor([2.0, 0.5, 1.0, 3.0]).view(4, 1)
    s, v, cnt = on.lif_multistep(x, neuron="lif", tau=2.0)
    # t0 v=1.0 (== theta -> spike), t1 0.25, t2 0.625, t3 1.8125 -> spike
    assert s.view(-1).tolist() == [1.0, 0.0, 0.0, 1.0]
    assert v.item() == 0.0 and cnt.item() == 2.0


def test_known_answers_lif_soft_and_no_decay_input():
    x = torch.tensor([3.0, 0.0, 0.0, 0.0]).view(4, 1)
    s, v, _ = on.lif_multistep(x, neuron="lif", tau=2.0, soft_reset=True)
    assert s.view(-1).tolist() == [1.0, 0.0, 0.0, 0.0]
    assert v.item() == 0.0625           # 1.5-1 = .5 -> .25 -> .125 -> .0625
    x = torch.tensor([0.6, 0.6, 0.0, 0.0]).view(4, 1)
    s, v, _ = on.lif_multistep(x, neuron="lif", tau=2.0, decay_input=False)
    # v = 0.5 v + x: 0.6, 0.9 -> no spikes
    assert s.sum().item() == 0.0
    assert abs(v.item() - np.float32(0.9) * 0.25) < 1e-7


def test_known_answers_if_vreset_and_thresholds():
    x = torch.full((4, 1), 0.6)
    s, v, _ = on.lif_multistep(x, neuron="if", v_reset=-0.5)
    # 0.6, 1.2 -> spike -> -0.5, 0.1, 0.7
    assert s.view(-1).tolist() == [0.0, 1.0, 0.0, 0.0]
    assert abs(v.item() - 0.7) < 1e-6
    # per-channel threshold broadcast over [T, B, C]
    x = torch.ones(2, 1, 3)
    s, _, _ = on.lif_multistep(x, neuron="if", v_threshold=torch.tensor([0.5, 1.5, 2.5]))
    assert s[:, 0, :].tolist() == [[1.0, 0.0, 0.0], [1.0, 1.0, 0.0]]


CASES = [c for c in itertools.product(["if", "lif"], [True, False], [0.0, 0.3, -0.5],
                                      [True, False], ["scalar", "per_n"], [None, 0.7])
         if not (c[1] and c[2] != 0.0)]      # soft reset ignores v_reset


@pytest.mark.parametrize("neuron,soft,vr,di,thr,decay", CASES)
def test_bruteforce_scalar_loop(neuron, soft, vr, di, thr, decay):
    g = torch.Generator().manual_seed(1)
    T, B, C, H, W = 5, 2, 3, 2, 2
    x = torch.randn(T, B, C, H, W, generator=g) * 1.5
    NCL = B * C * H * W
    th = 1.0 if thr == "scalar" else torch.rand(NCL, generator=g) * 0.5 + 0.5
    bias = torch.randn(C, generator=g)
    s, v, _ = on.lif_multistep(x, bias=bias, neuron=neuron, tau=2.0, decay=decay,
                               decay_input=di, soft_reset=soft, v_threshold=th, v_reset=vr)
    df, sc = on.neuron_params(neuron, 2.0, decay, di)
    th_np = th if thr == "scalar" else th.numpy()
    s_ref, v_ref = _scalar_loop(x.reshape(T, -1).numpy(), df=df, sc=sc, th=th_np,
                                soft=soft, vr=vr, bias=bias.numpy(), C=C, HW=H * W)
    assert np.array_equal(s.reshape(T, -1).numpy(), s_ref)
    assert np.array_equal(v.reshape(-1).numpy(), v_ref)


@pytest.mark.parametrize("neuron,decay,di,soft,vr", [
    ("lif", None, True, False, 0.0), ("lif", None, False, True, 0.0),
    ("lif", 0.3, True, False, 0.0), ("lif", 0.99, False, False, 0.3),
    ("if", 0.9, True, False, -0.5), ("if", None, True, True, 0.0),
])
def test_c_restatement_bit_equal(neuron, decay, di, soft, vr):
    g = torch.Generator().manual_seed(7)
    T, B, C, H, W = 6, 4, 16, 7, 7
    x = torch.randn(T, B, C, H, W, generator=g) * 1.5
    bias = torch.randn(C, generator=g) * 0.2
    v0 = torch.randn(B, C, H, W, generator=g) * 0.3
    s, v, _ = on.lif_multistep(x, bias=bias, v_init=v0, neuron=neuron, tau=2.0,
                               decay=decay, decay_input=di, soft_reset=soft, v_reset=vr)
    df, sc = on.neuron_params(neuron, 2.0, decay, di)
    sc_, vc = clib.lif_f32(x.reshape(T, -1).numpy(), bias=bias.numpy(), C_=C, HW=H * W,
                           v_init=v0.reshape(-1).numpy(), df=df, sc=sc,
                           soft_reset=soft, v_reset=vr)
    assert np.array_equal(s.reshape(T, -1).numpy(), sc_)
    assert np.array_equal(v.reshape(-1).numpy(), vc)


def test_if_closed_forms():
    g = torch.Generator().manual_seed(3)
    x = torch.randn(16, 50, generator=g)
    # below an unreachable threshold IF is a running fp32 sum
    s, v, _ = on.lif_multistep(x, neuron="if", v_threshold=1e30)
    assert s.sum().item() == 0.0
    assert np.array_equal(v.numpy(), np.cumsum(x.numpy(), axis=0, dtype=np.float32)[-1])
    # soft reset with integer charges conserves charge: v_T = sum x - theta*count
    xi = torch.randint(-1, 3, (16, 50), generator=g).float()
    s, v, cnt = on.lif_multistep(xi, neuron="if", soft_reset=True, v_threshold=2.0)
    assert torch.equal(v, xi.sum(0) - 2.0 * cnt)
    # hard reset: the state right after any spike is exactly v_reset
    s, v, _ = on.lif_multistep(xi, neuron="if", v_reset=-0.25)
    assert torch.all(v[s[-1] > 0] == -0.25)


def test_spikingjelly_form_agrees_within_tolerance():
    """BASELINE's SJ form H=v+(x-v)/tau vs the reference's 0.5v+0.5x: membrane
    within 1e-6 relative, spike flips only within 1e-5 of threshold."""
    g = torch.Generator().manual_seed(0)
    x = torch.randn(4, 8, 16, 16, 16, generator=g) * 1.5
    s_ref, v_ref, _ = on.lif_multistep(x, neuron="lif", tau=2.0)
    s_sj, h_sj, v_sj = on.sj_multistep_lif(x, tau=2.0)
    h_ref = on.lif_membrane_trace(x, tau=2.0)
    mism = s_ref != s_sj
    assert torch.all((h_ref[mism] - 1.0).abs() < 1e-5)
    same = ~mism.any(0)
    rel = (v_ref[same] - v_sj[same]).abs() / v_ref[same].abs().clamp_min(1.0)
    assert rel.max().item() <= 1e-6


def test_pins_catch_planted_mistakes(monkeypatch):
    """A wrong comparison (>), a dropped input scale, or a soft-reset sign flip
    in the oracle must fail the known-answer / scalar-loop pins."""
    x = torch.tensor([2.0, 0.5, 1.0, 3.0]).view(4, 1)
    real = on.lif_multistep

    def mutant_gt(x_seq, **kw):
        s, v, c = real(x_seq, **{**kw, "v_threshold": kw.get("v_threshold", 1.0) + 1e-7})
        return s, v, c
    s, _, _ = mutant_gt(x, neuron="lif", tau=2.0)
    assert s.view(-1).tolist() != [1.0, 0.0, 0.0, 1.0]
    s, _, _ = real(x, neuron="lif", tau=2.0, decay_input=False)      # scale dropped
    assert s.view(-1).tolist() != [1.0, 0.0, 0.0, 1.0]
    xs = torch.tensor([3.0, 0.0, 0.0, 0.0]).view(4, 1)
    _, v, _ = real(xs, neuron="lif", tau=2.0, soft_reset=True, v_threshold=-1.0)
    assert v.item() != 0.0625
