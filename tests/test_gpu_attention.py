"""GPU parity of the spike self-attention path.

The attention core (int8 MFMA) must reproduce the integer counts Q K^T and
(Q K^T) V bit for bit, and its LIF spikes exactly (power-of-two scales keep
the membrane exact).  Projections are bf16 GEMMs: checked teacher-forced
(>= 99.9% spike agreement, flips near threshold) and the output projection
within fp32-accumulation tolerance.  Restates snn_compiler/tests/
test_spike_attention.py:110-160 (block C=32, heads=4, x~B(0.3) [4,2,32,8,8],
thresholds 0.3 / 0.5, scale 0.125; popcount K^T V with N=70).
"""
import pytest
import torch
import torch.nn as nn

import snnk
from oracle import attention as oa
from oracle import neurons as on
from snnk.kernels.attention import spike_attention, spike_self_attention, spike_av_lif
from snnk.nn.attention import FusedSpikeAttention

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _spikes(shape, p, seed):
    return (torch.rand(*shape, generator=torch.Generator().manual_seed(seed)) < p).float()


@pytest.mark.parametrize("T,B,H,N,d", [(4, 32, 8, 64, 48), (4, 2, 4, 64, 8), (3, 3, 2, 49, 64),
                                       (1, 2, 3, 16, 32), (5, 1, 1, 33, 40), (4, 4, 6, 64, 16)])
def test_attention_core_counts_and_spikes_exact(T, B, H, N, d):
    D = H * d
    qkv = _spikes((T, B * N, 3 * D), 0.25, N + d)
    qd = qkv.to(DEV, torch.bfloat16)
    q, k, v = qd[..., :D], qd[..., D:2 * D], qd[..., 2 * D:]
    spk, S, O = spike_attention(q, k, v, B=B, N=N, heads=H, scale=0.125, tau=2.0,
                                v_threshold=0.5, return_counts=True)
    hq = lambda s: s.view(T, B, N, H, d).permute(0, 1, 3, 2, 4).long()  # noqa: E731
    qh, kh, vh = hq(qkv[..., :D]), hq(qkv[..., D:2 * D]), hq(qkv[..., 2 * D:])
    S_ref = qh @ kh.transpose(-1, -2)
    O_ref = S_ref @ vh
    assert torch.equal(S.cpu().long(), S_ref)
    assert torch.equal(O.cpu().long(), O_ref)
    a_ref, _, _ = on.lif_multistep(O_ref.float() * 0.125, neuron="lif", v_threshold=0.5)
    got = spk.cpu().float().view(T, B, N, H, d).permute(0, 1, 3, 2, 4)
    assert torch.equal(got, a_ref)


@pytest.mark.parametrize("T,B,H,N,d,soft,v_reset", [
    (3, 2, 2, 20, 48, True, 0.0),     # one token tile, two dim tiles, soft reset
    (4, 2, 2, 20, 48, False, 0.25),   # same tiling, hard reset to a non-zero value
    (2, 3, 2, 32, 64, True, 0.0),     # N = 32 exactly, d = 64
    (4, 1, 3, 17, 40, False, -0.5),   # ragged N and d, negative reset value
    (5, 2, 1, 50, 24, True, 0.0),     # two token tiles, one dim tile, soft reset
])
def test_attention_core_reset_modes_exact(T, B, H, N, d, soft, v_reset):
    """Every reset template of the core against oracle lif_multistep; with the
    power-of-two scale every membrane value is exact in fp32."""
    D = H * d
    qkv = _spikes((T, B * N, 3 * D), 0.3, 1000 + N * d)
    qd = qkv.to(DEV, torch.bfloat16)
    q, k, v = qd[..., :D], qd[..., D:2 * D], qd[..., 2 * D:]
    spk, S, O = spike_attention(q, k, v, B=B, N=N, heads=H, scale=0.125, tau=2.0,
                                v_threshold=0.5, v_reset=v_reset, soft_reset=soft,
                                return_counts=True)
    hq = lambda s: s.view(T, B, N, H, d).permute(0, 1, 3, 2, 4).long()  # noqa: E731
    qh, kh, vh = hq(qkv[..., :D]), hq(qkv[..., D:2 * D]), hq(qkv[..., 2 * D:])
    O_ref = (qh @ kh.transpose(-1, -2)) @ vh
    assert torch.equal(O.cpu().long(), O_ref)
    a_ref, _, _ = on.lif_multistep(O_ref.float() * 0.125, neuron="lif", tau=2.0,
                                   soft_reset=soft, v_threshold=0.5, v_reset=v_reset)
    got = spk.cpu().float().view(T, B, N, H, d).permute(0, 1, 3, 2, 4)
    assert torch.equal(got, a_ref)
    assert 0 < int(got.sum()) < got.numel()


def test_reference_api_linear_order_matches_core():
    """spike_ktv_popcount + spike_av_lif (reference linear order) == MFMA core."""
    T, B, H, N, d = 4, 2, 4, 70 - 6, 16
    D = H * d
    qkv = _spikes((T, B * N, 3 * D), 0.2, 7).to(DEV, torch.bfloat16)
    q, k, v = qkv[..., :D], qkv[..., D:2 * D], qkv[..., 2 * D:]
    core = spike_attention(q, k, v, B=B, N=N, heads=H, scale=0.125, v_threshold=0.5)
    hq = lambda s: s.reshape(T, B, N, H, d).permute(0, 1, 3, 2, 4).float().contiguous()  # noqa
    kv = snnk.spike_ktv_popcount(hq(k), hq(v))
    s = spike_av_lif(hq(q), kv, scale=0.125, tau=2.0, v_threshold=0.5)
    ref_lin = oa.spike_av_lif(hq(q).cpu(), kv.cpu(), scale=0.125, tau=2.0, v_threshold=0.5)
    assert torch.equal(s.cpu(), ref_lin)
    assert torch.equal(core.cpu().float(), s.permute(0, 1, 3, 2, 4).reshape(T, B * N, D).cpu())


def _block_params(D, seed):
    g = torch.Generator().manual_seed(seed)
    p = {f"w{n}": torch.randn(D, D, generator=g) * (2.0 / D) ** 0.5 for n in "qkvp"}
    p.update({f"b{n}": torch.randn(D, generator=g) * 0.1 for n in "qkvp"})
    return p


def test_ssa_baseline_block():
    """T=4, B=32, N=64, D=384, 8 heads, tokens ~ B(0.2), scale 0.125, attn theta 0.5."""
    T, B, N, D, H = 4, 32, 64, 384, 8
    p = _block_params(D, 0)
    x = _spikes((T, B, N, D), 0.2, 1)
    w_qkv = torch.cat([p["wq"], p["wk"], p["wv"]]).to(DEV, torch.bfloat16)
    b_qkv = torch.cat([p["bq"], p["bk"], p["bv"]]).to(DEV)
    out, mid = spike_self_attention(x.to(DEV), w_qkv, b_qkv, p["wp"].to(DEV, torch.bfloat16),
                                    p["bp"].to(DEV), heads=H, scale=0.125, vth_qkv=1.0,
                                    vth_attn=0.5, return_intermediates=True)
    ref = oa.ssa_forward(x, p, heads=H, scale=0.125, vth_qkv=1.0, vth_attn=0.5)
    # projections (bf16 weights): agreement with the fp32 reference
    qkv = mid["qkv"].cpu().float().view(T, B, N, 3 * D)
    qkv_ref = torch.cat([ref["q"], ref["k"], ref["v"]], -1)
    assert (qkv == qkv_ref).float().mean().item() >= 0.999
    # attention from the GPU's own Q, K, V: integer counts and spikes exact
    own = oa.ssa_forward(x, p, heads=H, scale=0.125, vth_qkv=1.0, vth_attn=0.5)
    d = D // H
    hq = lambda s: s.view(T, B, N, H, d).permute(0, 1, 3, 2, 4).long()  # noqa: E731
    S_ref = hq(qkv[..., :D]) @ hq(qkv[..., D:2 * D]).transpose(-1, -2)
    O_ref = S_ref @ hq(qkv[..., 2 * D:])
    assert torch.equal(mid["S"].cpu().long(), S_ref) and torch.equal(mid["O"].cpu().long(), O_ref)
    a_ref, _, _ = on.lif_multistep(O_ref.float() * 0.125, neuron="lif", v_threshold=0.5)
    attn = mid["attn"].cpu().float().view(T, B, N, H, d).permute(0, 1, 3, 2, 4)
    assert torch.equal(attn, a_ref)
    # output projection on the GPU's attention spikes
    a2 = mid["attn"].cpu().float().view(T, B, N, D)
    out_ref = a2.double() @ p["wp"].to(torch.bfloat16).double().t() + p["bp"].double()
    bound = a2.double() @ p["wp"].to(torch.bfloat16).double().abs().t()
    assert torch.all((out.cpu().double() - out_ref).abs() <= 3e-5 * bound + 1e-5)
    assert own["out"].shape == out.shape


class _LIF(nn.Module):
    def __init__(self, tau=2.0, v_threshold=1.0):
        super().__init__()
        self.tau, self.v_threshold = tau, v_threshold

    def forward(self, x):
        return on.naive_if_lif(x, neuron="lif", tau=self.tau, v_threshold=self.v_threshold)


def _bn1d(c, g):
    bn = nn.BatchNorm1d(c).eval()
    with torch.no_grad():
        bn.running_mean.copy_(torch.randn(c, generator=g) * 0.2)
        bn.running_var.copy_(torch.rand(c, generator=g) + 0.5)
        bn.weight.copy_(torch.rand(c, generator=g) + 0.5)
        bn.bias.copy_(torch.randn(c, generator=g) * 0.2)
    return bn


class _RefSSA(nn.Module):
    """Structure of snn_compiler/tests/test_spike_attention.py:55-80."""

    def __init__(self, C=32, heads=4, seed=0):
        super().__init__()
        g = torch.Generator().manual_seed(seed)
        self.num_heads, self.scale = heads, 0.125
        self.proj_lif = _LIF(v_threshold=0.3)
        for nm in ("q", "k", "v"):
            conv = nn.Conv1d(C, C, 1, bias=False)
            with torch.no_grad():
                conv.weight.copy_(torch.randn(C, C, 1, generator=g) * (1.0 / C) ** 0.5)
            setattr(self, f"{nm}_conv", conv)
            setattr(self, f"{nm}_bn", _bn1d(C, g))
            setattr(self, f"{nm}_lif", _LIF(v_threshold=0.3))
        self.attn_lif = _LIF(v_threshold=0.5)
        self.proj_conv = nn.Conv1d(C, C, 1)
        self.proj_bn = _bn1d(C, g)

    def forward(self, x):
        """Reference block forward (test_spike_attention.py:67-80)."""
        T, B, C, H, W = x.shape
        N, heads = H * W, self.num_heads
        d = C // heads
        x = self.proj_lif(x).flatten(3)
        xf = x.flatten(0, 1)

        def proj(nm):
            y = getattr(self, f"{nm}_bn")(getattr(self, f"{nm}_conv")(xf)).reshape(T, B, C, N)
            return _heads(getattr(self, f"{nm}_lif")(y), T, B, N, heads, d)
        q, k, v = proj("q"), proj("k"), proj("v")
        a = (q @ (k.transpose(-2, -1) @ v)) * self.scale
        s = self.attn_lif(a.transpose(3, 4).reshape(T, B, C, N)).flatten(0, 1)
        return self.proj_bn(self.proj_conv(s)).reshape(T, B, C, H, W)


def _heads(s, T, B, N, heads, d):
    return s.transpose(-1, -2).reshape(T, B, N, heads, d).permute(0, 1, 3, 2, 4).contiguous()


def _bn2d(c, g):
    bn = nn.BatchNorm2d(c).eval()
    with torch.no_grad():
        bn.running_mean.copy_(torch.randn(c, generator=g) * 0.2)
        bn.running_var.copy_(torch.rand(c, generator=g) + 0.5)
        bn.weight.copy_(torch.rand(c, generator=g) + 0.5)
        bn.bias.copy_(torch.randn(c, generator=g) * 0.2)
    return bn


class _RefMS(nn.Module):
    """Structure of snn_compiler/tests/test_spike_attention.py:83-107 (SDT-V2
    MS_Attention with plain 3x3 convs in place of RepConv)."""

    def __init__(self, C=32, heads=4, seed=1):
        super().__init__()
        g = torch.Generator().manual_seed(seed)
        self.num_heads, self.scale = heads, 0.125
        self.head_lif = _LIF(v_threshold=0.3)
        for nm in ("q", "k", "v", "proj"):
            conv = nn.Conv2d(C, C, 3, padding=1, bias=False)
            with torch.no_grad():
                conv.weight.copy_(torch.randn(C, C, 3, 3, generator=g) * (1.0 / (9 * C)) ** 0.5)
            setattr(self, f"{nm}_conv", nn.Sequential(conv, _bn2d(C, g)))
        for nm in ("q", "k", "v"):
            setattr(self, f"{nm}_lif", _LIF(v_threshold=0.3))
        self.attn_lif = _LIF(v_threshold=0.5)

    def forward(self, x):
        T, B, C, H, W = x.shape
        N, heads = H * W, self.num_heads
        d = C // heads
        x = self.head_lif(x)

        def proj(nm):
            y = getattr(self, f"{nm}_conv")(x.flatten(0, 1)).reshape(T, B, C, H, W)
            return _heads(getattr(self, f"{nm}_lif")(y).flatten(3), T, B, N, heads, d)
        q, k, v = proj("q"), proj("k"), proj("v")
        a = (q @ (k.transpose(-2, -1) @ v)) * self.scale
        s = self.attn_lif(a.transpose(3, 4).reshape(T, B, C, N)).reshape(T, B, C, H, W)
        return self.proj_conv(s.flatten(0, 1)).reshape(T, B, C, H, W)


def test_fused_spike_attention_from_reference_block():
    """from_reference on the reference test's block (test_spike_attention.py:110-117).

    Exact parts: the module equals the functional path on its folded buffers,
    and given the GPU's own Q/K/V the attention spikes are the oracle's bit
    for bit.  The bf16 projections flip a few near-threshold Q/K/V spikes, and
    each flip moves the counts of every query, so the end-to-end comparison
    with the fp32 block is statistical."""
    ref = _RefSSA(C=32, heads=4).eval()
    x = _spikes((4, 2, 32, 8, 8), 0.3, 0)
    fused = FusedSpikeAttention.from_reference(ref, ktv_mode="mfma").to(DEV)
    out = fused(x.to(DEV)).cpu()
    assert out.shape == x.shape
    p = {}
    for nm in ("q", "k", "v", "p"):
        conv = getattr(ref, f"{nm}_conv" if nm != "p" else "proj_conv")
        bn = getattr(ref, f"{nm}_bn" if nm != "p" else "proj_bn")
        w, b = oa.fold_conv1d_bn(conv.weight.detach().squeeze(-1),
                                 conv.bias.detach() if conv.bias is not None else None,
                                 bn.weight.detach(), bn.bias.detach(), bn.running_mean,
                                 bn.running_var, bn.eps)
        p[f"w{nm}"], p[f"b{nm}"] = w, b
    assert torch.equal(fused.w_qkv.cpu(), torch.cat([p["wq"], p["wk"], p["wv"]]).to(torch.bfloat16))
    tokens = x.reshape(4, 2, 32, 64).transpose(2, 3)
    out2, mid = spike_self_attention(tokens.to(DEV), fused.w_qkv, fused.b_qkv, fused.w_proj,
                                     fused.b_proj, heads=4, scale=0.125, vth_qkv=0.3,
                                     vth_attn=0.5, input_vth=0.3, return_intermediates=True)
    assert torch.equal(out2.cpu().transpose(2, 3).reshape(x.shape), out)
    T, B, N, D, H = 4, 2, 64, 32, 4
    qkv = mid["qkv"].cpu().float().view(T, B, N, 3 * D)
    hq = lambda s: s.view(T, B, N, H, D // H).permute(0, 1, 3, 2, 4).long()  # noqa: E731
    O_ref = (hq(qkv[..., :D]) @ hq(qkv[..., D:2 * D]).transpose(-1, -2)) @ hq(qkv[..., 2 * D:])
    a_ref, _, _ = on.lif_multistep(O_ref.float() * 0.125, neuron="lif", v_threshold=0.5)
    attn = mid["attn"].cpu().float().view(T, B, N, H, D // H).permute(0, 1, 3, 2, 4)
    assert torch.equal(attn, a_ref)
    r = oa.ssa_forward(tokens, p, heads=4, scale=0.125, vth_qkv=0.3, vth_attn=0.5, input_vth=0.3)
    qkv_ref = torch.cat([r["q"], r["k"], r["v"]], -1)
    assert (qkv == qkv_ref).float().mean().item() >= 0.995
    ref_out = r["out"].transpose(2, 3).reshape(x.shape)
    close = ((out - ref_out).abs() < 2e-2).float().mean().item()
    assert close >= 0.95, f"fraction of close outputs {close}"


@pytest.mark.parametrize("variant,ktv", [("ssa", "bmm"), ("ms", "bmm"), ("ssa", "popcount"),
                                         ("ms", "popcount")])
def test_reference_mode_bit_exact(variant, ktv):
    """from_reference(ref, fold_bn=False) reproduces the reference block bit for
    bit (test_spike_attention.py:110-160): the projections are the block's own
    conv + BN, every LIF is the HIP kernel (bit-exact neuron), K^T V and
    q (K^T V) are exact integer products and the scale folds exactly."""
    from snnk.verify import assert_equivalent
    ref = (_RefSSA(C=32, heads=4) if variant == "ssa" else _RefMS(C=32, heads=4)).to(DEV).eval()
    x = _spikes((4, 2, 32, 8, 8), 0.3, 3).to(DEV)
    fused = FusedSpikeAttention.from_reference(ref, fold_bn=False, ktv_mode=ktv).to(DEV)
    assert fused.variant == variant and fused.ktv_mode == ktv
    rep = assert_equivalent(ref, fused, x, verbose=False)
    assert rep["bit_exact"]


@pytest.mark.parametrize("variant,C,heads", [("ssa", 384, 6), ("ms", 384, 4)])
def test_reference_mode_spikformer_shapes(variant, C, heads):
    """Spikingformer / SDT-V2 block shapes: N = 14x14 = 196 tokens, d = 64 / 96."""
    from snnk.verify import assert_equivalent
    ref = (_RefSSA(C=C, heads=heads) if variant == "ssa" else _RefMS(C=C, heads=heads))
    ref = ref.to(DEV).eval()
    x = _spikes((4, 2, C, 14, 14), 0.2, 4).to(DEV)
    fused = FusedSpikeAttention.from_reference(ref, fold_bn=False, ktv_mode="popcount").to(DEV)
    rep = assert_equivalent(ref, fused, x, verbose=False)
    assert rep["bit_exact"]


def test_fuse_spiking_attention_pass():
    """fuse_spiking_attention swaps both block kinds inside a container
    (test_spike_attention.py:131-137)."""
    from snnk.passes import fuse_spiking_attention
    model = nn.ModuleList([_RefSSA(C=32, heads=4), _RefMS(C=32, heads=4)]).to(DEV).eval()
    x = _spikes((4, 2, 32, 8, 8), 0.3, 5).to(DEV)
    want = [m(x) for m in model]
    assert fuse_spiking_attention(model, fold_bn=False) == 2
    assert all(isinstance(m, FusedSpikeAttention) for m in model)
    for m, y in zip(model, want):
        assert torch.equal(m(x), y)


# ---- fused linear order: spike_av_lif and the large-shape core ----------------
def _kv_counts(k, v):
    return k.double().transpose(-1, -2) @ v.double()


def _mid_threshold(a, in_scale):
    """A threshold near the mean first-step input (a mix of spikes at any N)."""
    return float(torch.tensor(float((a[0] * in_scale).mean()) + 1e-3, dtype=torch.float32))


@pytest.mark.parametrize("T,B,H,N,d", [(4, 16, 8, 196, 96), (4, 2, 4, 70, 16), (3, 2, 3, 50, 40),
                                       (2, 1, 2, 33, 20), (5, 2, 1, 256, 128), (1, 3, 2, 7, 8)])
def test_spike_av_lif_fused_matches_oracle(T, B, H, N, d):
    """(q @ kv) * scale -> LIF in one kernel (snn_compiler/kernels/attention.py:49-137),
    bit-exact against the oracle on integer K^T V, for every q dtype and for
    kv given as fp32 or int32."""
    q = _spikes((T, B, H, N, d), 0.2, 400 + N)
    k = _spikes((T, B, H, N, d), 0.2, 401 + N)
    v = _spikes((T, B, H, N, d), 0.25, 402 + N)
    kv = _kv_counts(k, v)
    vth = _mid_threshold(q.double() @ kv, 0.0625)
    ref = oa.spike_av_lif(q, kv.float(), scale=0.125, tau=2.0, v_threshold=vth)
    assert 0 < int(ref.sum()) < ref.numel()
    for dt in (torch.float32, torch.bfloat16, torch.float16):
        for kv_dt in (torch.float32, torch.int32):
            s = spike_av_lif(q.to(DEV, dt), kv.to(DEV, kv_dt), scale=0.125, tau=2.0,
                             v_threshold=vth)
            assert s.dtype == dt and s.shape == q.shape
            assert torch.equal(s.cpu().float(), ref), (dt, kv_dt)


@pytest.mark.parametrize("soft,v_reset,decay_input", [(True, 0.0, True), (False, 0.25, True),
                                                       (False, 0.0, False)])
def test_spike_av_lif_reset_modes(soft, v_reset, decay_input):
    T, B, H, N, d = 4, 2, 3, 45, 24
    q = _spikes((T, B, H, N, d), 0.3, 11)
    kv = _kv_counts(_spikes((T, B, H, N, d), 0.3, 12), _spikes((T, B, H, N, d), 0.3, 13))
    a = q.double() @ kv
    sc = 0.125 if decay_input else 0.0625
    ref, _, _ = on.lif_multistep((a * sc).float(), neuron="lif", tau=2.0, decay_input=decay_input,
                                 soft_reset=soft, v_threshold=0.5, v_reset=v_reset)
    s = spike_av_lif(q.to(DEV), kv.float().to(DEV), scale=sc, tau=2.0, decay_input=decay_input,
                     v_threshold=0.5, v_reset=v_reset, soft_reset=soft)
    assert torch.equal(s.cpu(), ref)


def test_spike_av_lif_real_valued_kv():
    """kv with fractional values: the three bf16 parts make every product exact,
    so the kernel's pre-activation is an fp32 sum of exact terms; spikes agree
    with a float64 reference except within rounding distance of threshold."""
    T, B, H, N, d = 4, 2, 2, 64, 48
    g = torch.Generator().manual_seed(21)
    q = _spikes((T, B, H, N, d), 0.3, 22)
    kv = torch.randn(T, B, H, d, d, generator=g) * 3.0
    a = q.double() @ kv.double()
    v = torch.zeros(a.shape[1:], dtype=torch.float64)
    ref, near = [], []
    for t in range(T):
        h = 0.5 * v + 0.0625 * a[t]
        ref.append((h >= 0.5).float())
        near.append((h - 0.5).abs() < 1e-4)
        v = torch.where(h >= 0.5, torch.zeros_like(h), h)
    ref, near = torch.stack(ref), torch.stack(near)
    s = spike_av_lif(q.to(DEV), kv.to(DEV), scale=0.125, tau=2.0, v_threshold=0.5).cpu()
    bad = (s != ref)
    assert float(bad.float().mean()) <= 1e-3
    # a flip at t can only come from a near-threshold value at some step <= t
    assert bool((~bad[0] | near[0]).all())


@pytest.mark.parametrize("T,B,H,N,d", [(4, 16, 8, 196, 96), (4, 2, 2, 100, 64), (2, 3, 1, 65, 8),
                                       (3, 2, 2, 64, 72), (2, 1, 2, 300, 128), (3, 2, 2, 20, 104)])
def test_attention_core_large_shapes_exact(T, B, H, N, d):
    """Past 64 tokens / 64 dims the core runs Q (K^T V): O counts, S counts (binary
    GEMM) and spikes bit-exact against integer products and the oracle LIF."""
    D = H * d
    qkv = _spikes((T, B * N, 3 * D), 0.2, 7000 + N + d)
    qd = qkv.to(DEV, torch.bfloat16)
    q, k, v = qd[..., :D], qd[..., D:2 * D], qd[..., 2 * D:]
    hq = lambda s: s.view(T, B, N, H, d).permute(0, 1, 3, 2, 4).long()  # noqa: E731
    qh, kh, vh = hq(qkv[..., :D]), hq(qkv[..., D:2 * D]), hq(qkv[..., 2 * D:])
    S_ref = qh @ kh.transpose(-1, -2)
    O_ref = qh @ (kh.transpose(-1, -2) @ vh)
    vth = _mid_threshold(O_ref.double(), 0.0625)
    spk, S, O = spike_attention(q, k, v, B=B, N=N, heads=H, scale=0.125, tau=2.0,
                                v_threshold=vth, return_counts=True)
    assert torch.equal(O_ref, S_ref @ vh)
    assert torch.equal(O.cpu().long(), O_ref)
    assert torch.equal(S.cpu().long(), S_ref)
    a_ref = oa.spike_av_lif(qh.float(), (kh.transpose(-1, -2) @ vh).float(), scale=0.125,
                            tau=2.0, v_threshold=vth)
    got = spk.cpu().float().view(T, B, N, H, d).permute(0, 1, 3, 2, 4)
    assert torch.equal(got, a_ref)
    assert 0 < int(got.sum()) < got.numel()
