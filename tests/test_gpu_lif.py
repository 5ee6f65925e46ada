"""GPU parity of the HIP LIF kernel (snnk_lif_forward) against the CPU oracle.

Restates the structure of the reference's neuron tests on seeded CPU inputs:
  snn_compiler/tests/test_correctness.py:43-108   (mode matrix, bit-equal spikes)
  snn_compiler/tests/test_correctness.py:158-200  (bias fused into the neuron)
  snn_compiler/tests/test_correctness.py:231-329  (dtypes, decay overrides)
  snn_compiler/tests/test_largeT_and_rate.py:54-132 (i64 offsets, rate, stateful chunks)
Spikes must be bit-equal; the membrane state is compared exactly too (the
kernel rounds every operation as the oracle does).
"""
import itertools
import zlib

import numpy as np

import pytest
import torch

import snnk
from oracle import neurons as on

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _randn(shape, seed, scale=1.0, dtype=torch.float32):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * scale).to(dtype)


SHAPES = [(4, 2, 8, 4, 4), (4, 8, 64, 56, 56), (4, 8, 128)]


def _cases():
    for shape in SHAPES:
        for neuron, soft, vr in itertools.product(["if", "lif"], [True, False], [0.0, 0.3, -0.5]):
            if soft and vr != 0.0:
                continue
            for di in ([True, False] if neuron == "lif" else [True]):
                yield shape, neuron, soft, vr, di, "scalar", "NCHW"
                yield shape, neuron, soft, vr, di, "per_c", "NCHW"
                if len(shape) == 5:
                    yield shape, neuron, soft, vr, di, "per_c", "NHWC"
                yield shape, neuron, soft, vr, di, "per_n", "NCHW"


@pytest.mark.parametrize("shape,neuron,soft,vr,di,thr,layout", list(_cases()))
def test_if_lif_matrix_bit_equal(shape, neuron, soft, vr, di, thr, layout):
    x_cpu = _randn(shape, seed=zlib.crc32(repr((shape, neuron, soft, vr, di, thr, layout)).encode()))
    if layout == "NHWC":
        T, B, C, H, W = shape
        x = x_cpu.reshape(T * B, C, H, W).to(DEV).contiguous(
            memory_format=torch.channels_last).view(T, B, C, H, W)
    else:
        x = x_cpu.to(DEV)
    g = torch.Generator().manual_seed(11)
    if thr == "scalar":
        th_cpu = 1.0
    elif thr == "per_c":
        C = shape[2] if len(shape) == 5 else shape[-1]
        th_cpu = torch.rand(C, generator=g) * 0.5 + 0.5
    else:
        th_cpu = torch.rand(x_cpu[0].numel(), generator=g) * 0.5 + 0.5
    th = th_cpu.to(DEV) if isinstance(th_cpu, torch.Tensor) else th_cpu
    kw = dict(neuron=neuron, tau=2.0, decay_input=di, soft_reset=soft, v_reset=vr)
    out = snnk.if_lif(x, v_threshold=th, layout=layout, **kw)
    ref = on.naive_if_lif(x_cpu, v_threshold=th_cpu, **kw)
    assert out.shape == ref.shape and out.dtype == ref.dtype
    assert torch.equal(out.cpu(), ref)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_dtype_compat(dtype):
    x_cpu = _randn((4, 4, 32, 16, 16), seed=4, dtype=dtype)
    out = snnk.if_lif(x_cpu.to(DEV), neuron="lif", tau=2.0)
    ref = on.naive_if_lif(x_cpu, neuron="lif", tau=2.0)
    assert out.dtype == dtype and torch.equal(out.cpu(), ref)


@pytest.mark.parametrize("neuron,decay,di", [("if", 0.0, True), ("if", 0.5, True),
                                              ("if", 0.9, True), ("lif", 0.3, True),
                                              ("lif", 0.7, False), ("lif", 0.99, True)])
def test_decay_override(neuron, decay, di):
    x_cpu = _randn((4, 4, 16, 8, 8), seed=10)
    out = snnk.if_lif(x_cpu.to(DEV), neuron=neuron, tau=2.0, decay=decay, decay_input=di)
    ref = on.naive_if_lif(x_cpu, neuron=neuron, tau=2.0, decay=decay, decay_input=di)
    assert torch.equal(out.cpu(), ref)


@pytest.mark.parametrize("has_bias,neuron,soft,vr", [
    (True, "if", False, 0.0), (True, "lif", True, 0.0), (True, "lif", False, 0.2),
    (False, "lif", False, 0.0), (False, "if", True, 0.0)])
def test_fused_bias_matches_biased_naive(has_bias, neuron, soft, vr):
    """conv(no bias) + fused bias LIF == (conv + bias) + naive LIF
    (test_correctness.py:158-200), with the conv output fixed on the CPU."""
    T, B, C, H, W = 4, 2, 16, 16, 16
    y_cpu = _randn((T, B, C, H, W), seed=2)
    b_cpu = _randn((C,), seed=3) if has_bias else None
    out = snnk.fused_bias_if_lif(y_cpu.to(DEV), None if b_cpu is None else b_cpu.to(DEV),
                                 neuron=neuron, tau=2.0, soft_reset=soft, v_reset=vr)
    biased = y_cpu + (b_cpu.view(1, 1, C, 1, 1) if has_bias else 0.0)
    ref = on.naive_if_lif(biased, neuron=neuron, tau=2.0, soft_reset=soft, v_reset=vr)
    assert torch.equal(out.cpu(), ref)


def test_fused_bias_residual_nhwc():
    T, B, C, H, W = 4, 2, 16, 8, 8
    y_cpu, r_cpu = _randn((T, B, C, H, W), seed=5), _randn((T, B, C, H, W), seed=6)
    b_cpu = _randn((C,), seed=7)

    def cl(t):
        return t.reshape(T * B, C, H, W).to(DEV).contiguous(
            memory_format=torch.channels_last).view(T, B, C, H, W)
    out = snnk.fused_bias_if_lif(cl(y_cpu), b_cpu.to(DEV), residual=cl(r_cpu),
                                 neuron="lif", layout="NHWC")
    s, _, _ = on.lif_multistep(y_cpu, bias=b_cpu, residual=r_cpu, neuron="lif")
    assert torch.equal(out.cpu(), s)


def test_lif_config_final_state_and_tolerances():
    """BASELINE LIF config: x~N(0,1.5^2) [4,32,64,32,32], tau=2, theta=1, hard 0.
    Membrane within 1e-6 relative (here: exact), spikes bit-equal to the
    reference form and within the 1e-5 band of the SpikingJelly form."""
    x_cpu = _randn((4, 32, 64, 32, 32), seed=0, scale=1.5)
    s, v = snnk.fused_bias_if_lif_stateful(x_cpu.to(DEV), None, return_v=True,
                                           neuron="lif", tau=2.0)
    s_ref, v_ref, _ = on.lif_multistep(x_cpu, neuron="lif", tau=2.0)
    s, v = s.cpu(), v.cpu()
    assert torch.equal(s, s_ref)
    rel = ((v - v_ref).abs() / v_ref.abs().clamp_min(1e-30)).max().item()
    assert rel <= 1e-6
    s_sj, _, _ = on.sj_multistep_lif(x_cpu, tau=2.0)
    h_ref = on.lif_membrane_trace(x_cpu, tau=2.0)
    mism = s != s_sj
    assert torch.all((h_ref[mism] - 1.0).abs() < 1e-5)


def test_u8_spikes_and_rate():
    x_cpu = _randn((4, 8, 32, 8, 8), seed=8, scale=1.5)
    x = x_cpu.to(DEV)
    s8 = snnk.if_lif(x, neuron="lif", spike_dtype=torch.uint8)
    ref = on.naive_if_lif(x_cpu, neuron="lif")
    assert s8.dtype == torch.uint8 and torch.equal(s8.cpu().float(), ref)
    for T in (4, 16, 64):
        for soft in (True, False):
            xt = _randn((T, 2, 8, 16, 16), seed=T)
            cnt = snnk.fused_bias_if_lif_rate(xt.to(DEV), None, neuron="lif", soft_reset=soft)
            _, _, c_ref = on.lif_multistep(xt, neuron="lif", soft_reset=soft)
            assert torch.equal(cnt.cpu(), c_ref)


def test_stateful_chunks_equal_single_pass():
    """test_largeT_and_rate.py:106-132: chunked StatefulLIF == one pass."""
    T = 32
    x_cpu = _randn((T, 2, 16, 14, 14), seed=0)
    x = x_cpu.to(DEV)
    for soft in (True, False):
        ref, _, _ = on.lif_multistep(x_cpu, neuron="lif", soft_reset=soft)
        for chunk in (4, 8, 16, 32, 5):
            v, outs = None, []
            for i in range(0, T, chunk):
                s, v = snnk.fused_bias_if_lif_stateful(
                    x[i:i + chunk].contiguous(), None, v_init=v, return_v=True,
                    neuron="lif", soft_reset=soft)
                outs.append(s)
            assert torch.equal(torch.cat(outs).cpu(), ref)


def test_ragged_and_offset_views_use_scalar_path():
    # NCL = 3*5*7 = 105 is not a multiple of the vector width
    x_cpu = _randn((6, 3, 5, 7), seed=9, scale=1.5)
    out = snnk.if_lif(x_cpu.to(DEV), neuron="lif")
    assert torch.equal(out.cpu(), on.naive_if_lif(x_cpu, neuron="lif"))
    # a time slice starting 1 step in keeps each step contiguous
    big = _randn((5, 2, 3, 5, 5), seed=12).to(DEV)
    out = snnk.if_lif(big[1:], neuron="lif")
    assert torch.equal(out.cpu(), on.naive_if_lif(big[1:].cpu(), neuron="lif"))


def test_i64_offsets_large_T():
    """test_largeT_and_rate.py:54-68: (T-1)*NCL*2 B > 2^31 must not wrap.
    The tail neurons (highest offsets) are checked against the oracle."""
    T, B, C, H, W = 128, 4, 64, 224, 224
    assert (T - 1) * B * C * H * W * 2 > (2 << 30)
    g = torch.Generator(device=DEV).manual_seed(0)
    y = torch.randn(T, B, C, H, W, device=DEV, dtype=torch.bfloat16, generator=g)
    bias = torch.randn(C, device=DEV, generator=g)
    out = snnk.fused_bias_if_lif(y, bias, neuron="lif")
    torch.cuda.synchronize()
    assert out.shape == y.shape and not out.isnan().any().item()
    tail_y = y.view(T, -1)[:, -4096:].cpu()
    tail_s = out.view(T, -1)[:, -4096:].cpu()
    NCL = B * C * H * W
    ch = (torch.arange(NCL - 4096, NCL) // (H * W)) % C
    del out, y
    # bias[c] is added in fp32 before the charge, exactly as the kernel does
    u = tail_y.float() + bias.cpu()[ch].view(1, -1)
    ref, _, _ = on.lif_multistep(u, neuron="lif")
    assert torch.equal(tail_s.float(), ref)


def test_bf16_spike_output_from_fp32():
    x_cpu = _randn((4, 8, 32, 8, 8), seed=21, scale=1.5)
    for src in (x_cpu, x_cpu.half()):
        s = snnk.if_lif(src.to(DEV), neuron="lif", spike_dtype=torch.bfloat16)
        assert s.dtype == torch.bfloat16
        assert torch.equal(s.cpu().float(), on.naive_if_lif(src, neuron="lif").float())


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("layout", ["NCHW", "NHWC"])
def test_packed_spike_output(dtype, layout):
    """if_lif_packed: the words are the oracle's spikes packed LSB-first along
    the flat memory order (snn_compiler/kernels/attention.py:236-242 bit
    order), for every input dtype, per-channel thresholds and NHWC memory."""
    from oracle import bits as ob
    T, B, C, H, W = 4, 2, 64, 3, 5
    g = torch.Generator().manual_seed(11)
    x = (torch.randn(T, B, C, H, W, generator=g) * 1.5).to(dtype)
    thr = (torch.rand(C, generator=g) + 0.5)
    if layout == "NHWC":   # channels-last memory, NCHW labels
        xd = x.permute(0, 1, 3, 4, 2).contiguous().to(DEV).permute(0, 1, 4, 2, 3)
    else:
        xd = x.to(DEV)
    words = snnk.if_lif_packed(xd, neuron="lif", tau=3.0, v_threshold=thr.to(DEV), layout=layout)
    ref, _, _ = on.lif_multistep(x.float(), neuron="lif", tau=3.0, v_threshold=thr)
    flat = ref.permute(0, 1, 3, 4, 2) if layout == "NHWC" else ref
    want = ob.pack_rows(flat.reshape(T, -1, 32).numpy()).reshape(T, -1)
    assert np.array_equal(words.cpu().numpy().view(np.uint32), want)


def test_packed_spikes_feed_binary_gemm():
    """LIF -> packed words along K -> binary_gemm(a_packed=True) equals the
    GEMM of the unpacked spikes (no separate pack pass)."""
    T, R, K, N = 2, 64, 256, 96
    g = torch.Generator().manual_seed(12)
    x = (torch.randn(T, R, K, generator=g) * 1.5).to(DEV)
    Wb = (torch.rand(K, N, generator=g) < 0.5).float().to(DEV)
    words = snnk.if_lif_packed(x, neuron="lif", tau=2.0)
    spikes = snnk.if_lif(x, neuron="lif", tau=2.0)
    for signed in (False, True):
        got = snnk.binary_gemm(words.view(T, R, K // 32), Wb.expand(T, K, N).contiguous(),
                               a_packed=True, K=K, signed=signed)
        want = snnk.binary_gemm(spikes, Wb.expand(T, K, N).contiguous(), signed=signed)
        assert torch.equal(got, want)
    with pytest.raises(ValueError):
        snnk.if_lif_packed(torch.zeros(2, 3, 5, device=DEV))


class _TwoLayerStateful(torch.nn.Module):
    """conv -> StatefulLIF -> conv -> StatefulLIF, with the forward_chunked
    hook the chunked driver calls (membranes carried per layer)."""

    def __init__(self):
        super().__init__()
        g = torch.Generator().manual_seed(5)
        self.w1 = (torch.randn(8, 4, 3, 3, generator=g) * 0.6).to(DEV)
        self.w2 = (torch.randn(6, 8, 3, 3, generator=g) * 0.4).to(DEV)
        self.n1 = snnk.StatefulLIFNode(tau=2.0)
        self.n2 = snnk.StatefulLIFNode(tau=3.0, soft_reset=True)

    def _conv(self, x, w):
        T, B = x.shape[:2]
        y = torch.nn.functional.conv2d(x.flatten(0, 1), w, padding=1)
        return y.view(T, B, *y.shape[1:])

    def forward_chunked(self, x, state):
        state = state or {}
        s1, v1 = self.n1(self._conv(x, self.w1), v_init=state.get("n1"), return_v=True)
        s2, v2 = self.n2(self._conv(s1, self.w2), v_init=state.get("n2"), return_v=True)
        return s2, {"n1": v1, "n2": v2}

    def forward(self, x):
        return self.forward_chunked(x, None)[0]


def test_chunked_forward_equals_single_pass():
    """ChunkedForward / run_chunked (snn_compiler/nn/chunked.py:31-79) over a
    two-layer stateful network: every chunk size, including a ragged last
    chunk and chunk_t >= T, gives the single pass's spikes exactly."""
    net = _TwoLayerStateful()
    x = (_randn((12, 2, 4, 6, 6), seed=3) > 0.3).float().to(DEV)
    ref = net(x)
    assert 0.0 < ref.mean().item() < 1.0
    for chunk in (1, 4, 5, 12, 20):
        assert torch.equal(snnk.ChunkedForward(net, chunk_t=chunk)(x), ref), chunk
    plain = torch.nn.Sequential(torch.nn.Identity())
    assert snnk.ChunkedForward(plain, chunk_t=2)(x) is x     # no forward_chunked: plain call
