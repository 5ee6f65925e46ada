"""Pins for oracle/attention.py (spike self-attention)."""
import torch
import torch.nn as nn

from oracle import attention as oa
from oracle import neurons as on


def _spikes(shape, p, seed):
    return (torch.rand(*shape, generator=torch.Generator().manual_seed(seed)) < p).float()


def test_counts_bruteforce_and_associativity():
    T, B, H, N, d = 2, 1, 2, 5, 3
    q, k, v = (_spikes((T, B, H, N, d), 0.5, s).long() for s in (1, 2, 3))
    S = q @ k.transpose(-1, -2)
    O = S @ v
    for t in range(T):
        for h in range(H):
            for i in range(N):
                for j in range(N):
                    assert S[t, 0, h, i, j] == sum(int(q[t, 0, h, i, c] * k[t, 0, h, j, c]) for c in range(d))
                for c in range(d):
                    assert O[t, 0, h, i, c] == sum(int(S[t, 0, h, i, j] * v[t, 0, h, j, c]) for j in range(N))
    assert torch.equal(O, q @ (k.transpose(-1, -2) @ v))


def test_quadratic_block_equals_linear_order_spike_av_lif():
    T, B, N, D, H = 4, 2, 16, 32, 4
    g = torch.Generator().manual_seed(0)
    p = {f"w{n}": torch.randn(D, D, generator=g) * (2.0 / D) ** 0.5 for n in "qkvp"}
    p.update({f"b{n}": torch.randn(D, generator=g) * 0.1 for n in "qkvp"})
    x = _spikes((T, B, N, D), 0.3, 5)
    r = oa.ssa_forward(x, p, heads=H, scale=0.125, vth_qkv=0.3, vth_attn=0.5)
    d = D // H
    hq = lambda s: s.view(T, B, N, H, d).permute(0, 1, 3, 2, 4)  # noqa: E731
    kv = hq(r["k"]).transpose(-1, -2) @ hq(r["v"])
    s_lin = oa.spike_av_lif(hq(r["q"]), kv, scale=0.125, tau=2.0, v_threshold=0.5)
    assert torch.equal(s_lin.permute(0, 1, 3, 2, 4).reshape(T, B, N, D), r["attn"])
    assert r["S"].max() <= d and r["O"].max() <= d * N


def test_folded_linear_equals_conv1d_bn():
    C = 16
    g = torch.Generator().manual_seed(1)
    conv = nn.Conv1d(C, C, 1, bias=False)
    bn = nn.BatchNorm1d(C).eval()
    with torch.no_grad():
        conv.weight.copy_(torch.randn(C, C, 1, generator=g))
        bn.running_mean.copy_(torch.randn(C, generator=g) * 0.2)
        bn.running_var.copy_(torch.rand(C, generator=g) + 0.5)
        bn.weight.copy_(torch.rand(C, generator=g) + 0.5)
        bn.bias.copy_(torch.randn(C, generator=g) * 0.2)
    x = torch.randn(6, C, 10, generator=g)
    with torch.no_grad():
        ref = bn(conv(x))
    w, b = oa.fold_conv1d_bn(conv.weight.detach(), None, bn.weight.detach(), bn.bias.detach(),
                             bn.running_mean, bn.running_var, bn.eps)
    got = torch.einsum("oc,bcn->bon", w.squeeze(-1), x) + b.view(1, -1, 1)
    assert (got - ref).abs().max().item() < 1e-5


def test_attention_lif_is_exact_dyadic():
    """0.5 * 0.125 * count keeps the membrane on a 2^-k grid: the fp32 LIF
    equals a float64 evaluation bit for bit."""
    O = torch.randint(0, 3073, (4, 1000))
    s32, v32, _ = on.lif_multistep((O.float() * 0.125), neuron="lif", v_threshold=0.5)
    v = torch.zeros(1000, dtype=torch.float64)
    for t in range(4):
        h = 0.5 * v + 0.5 * (O[t].double() * 0.125)
        s = h >= 0.5
        assert torch.equal(s.float(), s32[t])
        v = torch.where(s, torch.zeros_like(h), h)
    assert torch.equal(v.float(), v32)
