"""VGG16-SNN (32x32, T=4, FC 512-4096-4096-10) on the fused engine vs the CPU oracle.

Every spiking layer is checked teacher-forced (fed the oracle's own input)
at B=32: >= 99.9% spike agreement with the fp32 reference, flips only where
the fp32 membrane was near threshold.  Two inits: BASELINE's (Kaiming, the
network falls silent after a few layers) and an active one (weights x3,
every layer keeps firing).  End to end: the B=32 logits and their argmax,
graph replays equal to eager runs, and the batch curve shapes (B = 1, 56).
"""
import pytest
import torch

from oracle import vgg as ov
from oracle import fused as of
from snnk.kernels.conv import to_nhwc_bf16, conv3x3_image_lif
from snnk.kernels.linear import linear_bias_lif, linear_preact
from snnk.zoo import vgg16_snn

pytestmark = pytest.mark.gpu
DEV = "cuda"
T = 4


def _engine(gain):
    return vgg16_snn(num_classes=10, pool="max", input_size=32, seed=0, gain=gain,
                     engine=True).to(DEV)


def _image(B, seed=1):
    return torch.randn(B, 3, 32, 32, generator=torch.Generator().manual_seed(seed))


def _flips_ok(got, ref, trace, pool, tol):
    """Agreement >= 99.9% and flips only near threshold (this step or earlier)."""
    agree = (got == ref).float().mean().item()
    near = (trace - 1.0).abs() < tol
    if pool:
        Tn, B, C, H, W = near.shape
        near = near.view(Tn, B, C, H // 2, 2, W // 2, 2).any(dim=6).any(dim=4)
    near = torch.cummax(near.int(), 0).values.bool()
    return agree, bool(torch.any((got != ref) & ~near))


@pytest.mark.parametrize("B,gain", [(32, 1.0), (32, 3.0), (1, 3.0), (56, 3.0)])
def test_teacher_forced_layers(B, gain):
    """Every layer fed the oracle's input; B = 1 and 56 run the plans chosen
    for those batch sizes (32x32 tiles with K groups and splits at 1, larger
    tiles and other splits at 56, the 2x2 layers as dense Linear at 32 and 56)."""
    eng = _engine(gain)
    params = ov.make_params(0, gain=gain)
    img = _image(B)
    rec = ov.forward_layers(params, img, T)
    lif = eng._lif()
    convs = iter(eng.convs)
    fcs = [(eng.fc1_w, eng.fc1_b), (eng.fc2_w, eng.fc2_b)]
    for i, r in enumerate(rec):
        if r["kind"] == "image":
            out = conv3x3_image_lif(img.to(DEV), eng.w0, eng.b0, T, **lif)
            got = out.cpu().float().permute(0, 1, 4, 2, 3)
        elif r["kind"] == "conv":
            conv = next(convs)
            xin = to_nhwc_bf16(r["input"].to(DEV))
            out = conv.forward_nhwc(xin)
            got = out.cpu().float().permute(0, 1, 4, 2, 3)
            if xin.shape[2] <= 2 and B % 4 != 0:
                # the engine pads the batch to whole quads of rows before the
                # 2x2 layers, which then run in their dense Linear form
                xq = torch.nn.functional.pad(xin, (0, 0, 0, 0, 0, 0, 0, (B + 3) // 4 * 4 - B))
                dense = conv.forward_nhwc(xq)[:, :B].cpu().float().permute(0, 1, 4, 2, 3)
                agree, bad = _flips_ok(dense, r["output"], r["trace"], r.get("pool", False), 2e-2)
                assert agree >= 0.999 and not bad, f"layer {i} (padded batch): agreement {agree}"
        elif r["kind"] == "fc_lif":
            w, b = fcs.pop(0)
            x = r["input"]  # 1x1 spatial at 32x32: NCHW and NHWC flatten orders coincide
            R = (B + 3) // 4 * 4  # the kernel takes rows in fours, as the engine pads them
            xp = torch.nn.functional.pad(x, (0, 0, 0, R - B))
            got = linear_bias_lif(xp.to(DEV, torch.bfloat16).contiguous(), w, b, **lif)
            got = got[:, :B].cpu().float()
        else:
            xp = torch.nn.functional.pad(r["input"], (0, 0, 0, (B + 3) // 4 * 4 - B))
            y = linear_preact(xp.to(DEV, torch.bfloat16).contiguous(), eng.fc3_w,
                              eng.fc3_b).cpu()[:, :B, :10]
            err = (y - r["output"]).abs().max().item()
            assert err < 5e-2, f"fc3 max err {err}"
            continue
        agree, bad = _flips_ok(got, r["output"], r["trace"], r.get("pool", False), 2e-2)
        assert agree >= 0.999 and not bad, f"layer {i} ({r['kind']}): agreement {agree}"


def test_end_to_end_baseline_init_exact_logits():
    """BASELINE's init: the deep layers are silent, so the logits are fixed by
    the FC biases and must match closely, argmax included."""
    eng = _engine(1.0)
    img = _image(32)
    ref = ov.forward(ov.make_params(0, gain=1.0), img, T).mean(0)
    got = eng(img.to(DEV)).mean(0).cpu()
    assert got.shape == (32, 10)
    assert torch.equal(got.argmax(-1), ref.argmax(-1))
    assert ((got - ref).abs().max() / ref.abs().max()).item() < 1e-3


def test_end_to_end_active_firing_rates():
    """Active init: a single flipped spike decorrelates the output of this
    random network (tests/test_oracle_vgg.py shows it on the oracle alone), so
    the free-running comparison is statistical: every layer's firing rate
    within 10% (relative) of the oracle's."""
    eng = _engine(3.0)
    img = _image(32)
    _, ref_rates = ov.forward(ov.make_params(0, gain=3.0), img, T, return_rates=True)
    rates = []
    eng(img.to(DEV), rates=rates)
    got = [float(r) for r in rates]
    assert len(got) == len(ref_rates) == 15
    for i, (a, b) in enumerate(zip(got, ref_rates)):
        assert abs(a - b) <= 0.1 * b + 1e-3, f"layer {i}: rate {a:.4f} vs {b:.4f}"


def test_graph_replay_equals_eager():
    eng = _engine(3.0)
    img = _image(32).to(DEV)
    eager = eng(img).clone()
    for k in range(3):
        torch.cuda.synchronize()
        other = eng(_image(32, seed=10 + k).to(DEV))      # eager work between replays
        y = eng.run_graph(img).clone()
        torch.cuda.synchronize()
        assert torch.equal(y, eager), f"replay {k} differs"
        assert not torch.equal(other, eager)


def test_mean_over_t_head_and_graph():
    """forward(mean_t=True) folds the logits' mean over T into the last
    layer (what the bench times): with packed spikes between layers the head
    counts each input's spikes over T and takes one dot product, so it equals
    forward().mean(0) (T per-step dot products) within the fp32 rounding of
    the two summation orders; eager and replayed results are identical."""
    eng = _engine(3.0)
    img = _image(32, seed=4).to(DEV)
    full = eng(img)
    m = eng(img, mean_t=True)
    assert m.shape == (32, 10)
    scale = full.abs().max().item()
    assert torch.allclose(m, full.mean(0), rtol=1e-5, atol=1e-5 * scale)
    for _ in range(2):
        eng(_image(32, seed=9).to(DEV))
        assert torch.equal(eng.run_graph(img, mean_t=True), m)


@pytest.mark.parametrize("B", [1, 56])
def test_batch_curve(B):
    """B=1 pads the FC rows to 4; logits match the oracle (BASELINE init)."""
    eng = _engine(1.0)
    img = _image(B, seed=3)
    got = eng(img.to(DEV)).cpu()
    assert got.shape == (T, B, 10) and torch.isfinite(got).all()
    ref = ov.forward(ov.make_params(0, gain=1.0), img, T)
    assert torch.equal(got.mean(0).argmax(-1), ref.mean(0).argmax(-1))
    assert ((got - ref).abs().max() / ref.abs().max()).item() < 1e-3


def test_engine_rejects_time_varying_input():
    eng = _engine(1.0)
    x = torch.randn(T, 2, 3, 32, 32, device=DEV)
    with pytest.raises(ValueError):
        eng(x)
    same = x[:1].expand(T, -1, -1, -1, -1).contiguous()
    assert eng(same).shape == (T, 2, 10)


def test_fuse_snn_model_vgg_equivalent():
    """vgg16_snn(fused=True) = fuse_snn_model on the reference structure
    (snn_compiler/zoo/vgg.py:134-143): every 64+-channel conv block (and its
    max-pool) becomes one bf16-MFMA FusedConvBNLIFPool, layer 1 a
    FusedConvBNNeuron, FC1/FC2 FusedLinearNeuron.  Checked with the verify
    harness against the unfused model on a time-varying spike input."""
    from snnk.verify import compare_models, assert_equivalent
    from snnk.nn import FusedConvBNLIFPool, FusedConvBNNeuron, FusedLinearNeuron
    ref = vgg16_snn(num_classes=10, pool="max", input_size=32, seed=0).to(DEV)
    fused = vgg16_snn(num_classes=10, pool="max", input_size=32, seed=0, fused=True).to(DEV)
    kinds = [type(m) for m in fused.features]
    assert kinds.count(FusedConvBNLIFPool) == 12 and kinds.count(FusedConvBNNeuron) == 1
    assert sum(isinstance(m, FusedLinearNeuron) for m in fused.classifier) == 2
    assert fused._n_fused == 15
    g = torch.Generator().manual_seed(5)
    x = (torch.rand(T, 4, 3, 32, 32, generator=g) < 0.3).float().to(DEV)
    rep = compare_models(ref, fused, x)
    assert rep["shape_match"] and rep["argmax_agree"] is not None
    # silent deep layers at gain 1: logits are the FC3 bias on both sides
    assert_equivalent(ref, fused, x, require_bitexact=False, atol=1e-5, verbose=False)


def test_fused_pool_module_teacher_forced():
    """One FusedConvBNLIFPool from the pass (gain 3, active layer) against the
    reference layers Conv2d -> BatchNorm2d -> LIFNode -> MaxPool2d fed the same
    fp32 spike input: >= 99.9% agreement, flips only near threshold."""
    ref = vgg16_snn(num_classes=10, pool="max", input_size=32, seed=0, gain=3.0).to(DEV)
    fused = vgg16_snn(num_classes=10, pool="max", input_size=32, seed=0, gain=3.0,
                      fused=True).to(DEV)
    conv, bn, lif, pool = (ref.features[i] for i in range(3, 7))   # 64 -> 64, 32x32, pool
    blk = fused.features[1]
    assert blk.pool == "max"
    g = torch.Generator().manual_seed(6)
    x = (torch.rand(T, 4, 64, 32, 32, generator=g) < 0.2).float().to(DEV)
    got = blk(x)
    assert got.dtype == torch.float32
    with torch.no_grad():
        y = bn(conv(x.reshape(T * 4, 64, 32, 32))).view(T, 4, 64, 32, 32)
        s = lif(y)
        want = pool(s.reshape(T * 4, 64, 32, 32)).view(T, 4, 64, 16, 16)
    trace = of.membrane_trace(y.cpu())
    agree, bad = _flips_ok(got.cpu(), want.cpu(), trace, True, 5e-2)
    assert agree >= 0.999 and not bad, agree


def _unpack(words, C):
    """int32 packed words [..., C // 32] -> float 0/1 [..., C] (bit c%32 of word c//32)."""
    bits = (words.unsqueeze(-1) >> torch.arange(32, device=words.device)) & 1
    return bits.reshape(*words.shape[:-1], C).float()


@pytest.mark.parametrize("B,gain", [(32, 3.0), (1, 3.0), (56, 3.0)])
def test_teacher_forced_layers_on_packed_bits(B, gain):
    """The engine chains its conv layers on packed words: every conv layer fed
    the oracle's input as words gives exactly the spikes of the bf16 path (and
    so the same >= 99.9% agreement with the fp32 oracle)."""
    from snnk.kernels.binary import pack_bits
    eng = _engine(gain)
    assert eng.bits_between_layers
    rec = ov.forward_layers(ov.make_params(0, gain=gain), _image(B), T)
    convs = iter(eng.convs)
    n = 0
    for i, r in enumerate(rec):
        if r["kind"] != "conv":
            continue
        conv = next(convs)
        x = to_nhwc_bf16(r["input"].to(DEV))
        bf = conv.forward_nhwc(x).cpu().float()
        got = conv.forward_nhwc(pack_bits(x, dim=-1), out_bits=True)
        C = bf.shape[-1]
        got = _unpack(got, C).cpu() if got.dtype == torch.int32 else got.cpu().float()
        assert torch.equal(got, bf), f"layer {i}: packed path differs from bf16 path"
        agree, bad = _flips_ok(got.permute(0, 1, 4, 2, 3), r["output"], r["trace"],
                               r.get("pool", False), 2e-2)
        assert agree >= 0.999 and not bad, f"layer {i}: agreement {agree}"
        n += 1
    assert n == 12


def test_engine_bits_and_bf16_chains_agree():
    """Same network, activations as packed words or as bf16 between layers:
    identical logits (the formats carry the same spikes)."""
    eng = _engine(3.0)
    img = _image(32).to(DEV)
    y_bits = eng(img).clone()
    eng.bits_between_layers = False
    y_bf16 = eng(img)
    eng.bits_between_layers = True
    assert torch.equal(y_bits, y_bf16)
