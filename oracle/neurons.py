"""Multi-step IF/LIF oracle (torch CPU, fp32) -- test infrastructure only.

Restates:
  naive_if_lif                 snn_compiler/kernels/neurons.py:467-502
  fused bias/residual step     snn_compiler/kernels/fused.py:101-114
  stateful v_init / v_final    snn_compiler/kernels/fused.py:424-441
  rate (count over T)          snn_compiler/kernels/fused.py:287-300
  test-local _naive_lif        snn_compiler/tests/test_largeT_and_rate.py:21-36

Arithmetic: state in fp32, each step ``v = df*v + sc*u`` with every product
and sum rounded to fp32 (torch CPU evaluates the expression op by op), spike
``v >= theta``, hard reset ``where(spike, v_reset, v)``, soft reset
``v - spike*theta``.

Pins (tests/test_oracle_neurons.py): hand-computed sequences; a pure-Python
float32 scalar loop on tiny shapes (bit-equal); the C restatement
oracle/c/oracle.c (bit-equal); IF closed forms (cumulative sum below
threshold, soft-reset charge conservation); SpikingJelly-form agreement.
"""
from __future__ import annotations

import torch


def neuron_params(neuron="if", tau=2.0, decay=None, decay_input=True):
    """(df, sc) per snn_compiler/kernels/neurons.py:470-475."""
    if neuron == "if":
        return (1.0 if decay is None else float(decay)), 1.0
    if neuron == "lif":
        df = (1.0 - 1.0 / tau) if decay is None else float(decay)
        sc = (1.0 / tau) if decay_input else 1.0
        return df, sc
    raise ValueError(f"unknown neuron: {neuron!r}")


def _threshold_view(v_threshold, x_seq):
    """Broadcastable threshold, per snn_compiler/kernels/neurons.py:476-490."""
    if not isinstance(v_threshold, torch.Tensor):
        return float(v_threshold)
    if v_threshold.numel() == x_seq[0].numel():
        return v_threshold.reshape(x_seq[0].shape).float()
    if x_seq.ndim >= 4:
        view = [1] * (x_seq.ndim - 1)
        view[1] = x_seq.shape[2]
        return v_threshold.view(*view).float()
    if x_seq.ndim == 3:
        return v_threshold.view(1, x_seq.shape[-1]).float()
    return v_threshold.float()


def _bias_view(bias, x_seq):
    """Per-channel bias broadcast over one step [B, C, ...] (or [B, C])."""
    if bias is None:
        return None
    if x_seq.ndim >= 4:
        view = [1] * (x_seq.ndim - 1)
        view[1] = x_seq.shape[2]
        return bias.view(*view).float()
    if x_seq.ndim == 3:
        return bias.view(1, -1).float()
    return bias.reshape(x_seq[0].shape).float()


def lif_multistep(x_seq, *, bias=None, residual=None, v_init=None,
                  neuron="if", tau=2.0, decay=None, decay_input=True,
                  soft_reset=False, v_threshold=1.0, v_reset=0.0):
    """General multi-step neuron: returns (spikes fp32 [T,...], v_final fp32, count fp32).

    ``u_t = x_t (+ bias[c]) (+ residual_t)`` as in fused.py:103-108, then the
    naive_if_lif update (neurons.py:493-500).
    """
    df, sc = neuron_params(neuron, tau, decay, decay_input)
    T = x_seq.shape[0]
    vth = _threshold_view(v_threshold, x_seq)
    bb = _bias_view(bias, x_seq)
    if v_init is None:
        v = torch.zeros_like(x_seq[0], dtype=torch.float32)
    else:
        v = v_init.reshape(x_seq[0].shape).float().clone()
    spikes = []
    for t in range(T):
        u = x_seq[t].to(torch.float32)
        if bb is not None:
            u = u + bb
        if residual is not None:
            u = u + residual[t].to(torch.float32)
        v = df * v + sc * u
        spike = (v >= vth).to(torch.float32)
        spikes.append(spike)
        if soft_reset:
            v = v - spike * vth
        else:
            v = torch.where(spike > 0, torch.full_like(v, float(v_reset)), v)
    s = torch.stack(spikes, 0) if T > 0 else torch.zeros_like(x_seq, dtype=torch.float32)
    return s, v, s.sum(0)


def naive_if_lif(x_seq, *, neuron="if", tau=2.0, decay=None, decay_input=True,
                 soft_reset=False, v_threshold=1.0, v_reset=0.0, layout="NCHW"):
    """Spikes in x's dtype; restates snn_compiler/kernels/neurons.py:467-502."""
    s, _, _ = lif_multistep(x_seq, neuron=neuron, tau=tau, decay=decay,
                            decay_input=decay_input, soft_reset=soft_reset,
                            v_threshold=v_threshold, v_reset=v_reset)
    return s.to(x_seq.dtype)


def sj_multistep_lif(x_seq, *, tau=2.0, v_threshold=1.0, v_reset=0.0, v_init=None):
    """SpikingJelly MultiStepLIFNode charge form (decay_input=True, hard reset):
    ``H = v + (x - v)/tau``; spike ``H >= v_th``; ``v = H*(1-spike) + v_reset*spike``.

    This is the form BASELINE's LIF config states; the reference's kernels use
    ``(1-1/tau)*v + x/tau`` instead.  The two are compared (not assumed
    equal) in tests/test_oracle_neurons.py.  Returns (spikes fp32, H fp32 per
    step, v_final fp32).
    """
    T = x_seq.shape[0]
    v = torch.zeros_like(x_seq[0], dtype=torch.float32) if v_init is None \
        else v_init.float().clone()
    spikes, hs = [], []
    for t in range(T):
        x = x_seq[t].to(torch.float32)
        h = v + (x - v) / tau
        s = (h >= v_threshold).to(torch.float32)
        spikes.append(s)
        hs.append(h)
        v = h * (1.0 - s) + float(v_reset) * s
    return torch.stack(spikes, 0), torch.stack(hs, 0), v


def lif_membrane_trace(x_seq, *, tau=2.0, v_threshold=1.0, v_reset=0.0):
    """Pre-reset membrane value H_t of every step for the reference form
    (used to decide which spike mismatches sit within 1e-5 of threshold)."""
    df, sc = neuron_params("lif", tau, None, True)
    v = torch.zeros_like(x_seq[0], dtype=torch.float32)
    hs = []
    for t in range(x_seq.shape[0]):
        h = df * v + sc * x_seq[t].to(torch.float32)
        hs.append(h)
        v = torch.where(h >= v_threshold, torch.full_like(h, float(v_reset)), h)
    return torch.stack(hs, 0)
