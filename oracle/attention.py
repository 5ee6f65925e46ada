"""Spike self-attention oracle (torch CPU fp32 + int64 counts) -- test infrastructure only.

Restates:
  _RefLIF / _RefSSA        snn_compiler/tests/test_spike_attention.py:23-80
  fold_conv1d_bn           snn_compiler/nn/attention.py:28-33
  spike_av_lif (linear order q @ (K^T V), scale folded into the LIF input
                           scale)  snn_compiler/kernels/attention.py:107-137
BASELINE's SSA takes tokens [T, B, N, D] that are already spikes, with
Linear (== Conv1d 1x1) projections and folded BN.

Pins (tests/test_oracle_attention.py): brute-force Q K^T and (Q K^T) V on tiny
shapes; (Q K^T) V == Q (K^T V) over integers; the quadratic-order block equals
the linear-order spike_av_lif path; the folded-Linear projection equals
Conv1d -> BatchNorm1d (tolerance 1e-5).
"""
from __future__ import annotations

import torch

from .neurons import lif_multistep


def fold_conv1d_bn(w, b, gamma, beta, mean, var, eps):
    inv = gamma / torch.sqrt(var + eps)
    w2 = w * inv.view(-1, *([1] * (w.ndim - 1)))
    cb = b if b is not None else torch.zeros_like(beta)
    return w2, (cb - mean) * inv + beta


def _lif(x, tau, vth):
    return lif_multistep(x, neuron="lif", tau=tau, v_threshold=vth)[0]


def ssa_forward(tokens, p, *, heads, scale=0.125, tau=2.0, vth_qkv=1.0, vth_attn=0.5,
                input_vth=None):
    """tokens [T,B,N,D]; p: wq,bq,wk,bk,wv,bv,wp,bp (BN folded, Linear layout [out,in]).

    Returns dict(x, q, k, v [T,B,N,D] spikes, S [T,B,H,N,N] int64, O
    [T,B,H,N,d] int64, attn [T,B,N,D] spikes, out [T,B,N,D] fp32).
    """
    T, B, N, D = tokens.shape
    d = D // heads
    x = tokens.float()
    if input_vth is not None:
        x = _lif(x, tau, input_vth)

    def proj(w, b, vth):
        y = x @ w.float().t() + b.float()          # bias over the feature (last) axis
        return lif_multistep(y, neuron="lif", tau=tau, v_threshold=vth)[0]

    q, k, v = proj(p["wq"], p["bq"], vth_qkv), proj(p["wk"], p["bk"], vth_qkv), \
        proj(p["wv"], p["bv"], vth_qkv)

    def heads_of(s):  # [T,B,N,D] -> [T,B,H,N,d]
        return s.view(T, B, N, heads, d).permute(0, 1, 3, 2, 4).long()

    qh, kh, vh = heads_of(q), heads_of(k), heads_of(v)
    S = qh @ kh.transpose(-1, -2)
    O = S @ vh
    a = O.float() * scale                                   # exact: power-of-two scale
    s = _lif(a, tau, vth_attn)                              # LIF over T per (b, h, n, d)
    attn = s.permute(0, 1, 3, 2, 4).reshape(T, B, N, D)
    out = attn @ p["wp"].float().t() + p["bp"].float()
    return dict(x=x, q=q, k=k, v=v, S=S, O=O, attn=attn, out=out)


def spike_av_lif(q, kv, *, scale, tau=2.0, v_threshold=0.5):
    """Linear order: a = q @ kv, v = (1-1/tau) v + (scale/tau) a, spike, hard reset 0."""
    a = q.double() @ kv.double()
    df, sc = 1.0 - 1.0 / tau, (1.0 / tau) * scale
    v = torch.zeros_like(a[0], dtype=torch.float32)
    out = []
    for t in range(a.shape[0]):
        h = df * v + sc * a[t].float()
        s = (h >= v_threshold).float()
        out.append(s)
        v = torch.where(s > 0, torch.zeros_like(h), h)
    return torch.stack(out, 0)
