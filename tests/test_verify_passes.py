"""Host logic of the verify harness and the fusion passes (CPU).

verify mirrors snn_compiler/verify.py:62-175: report keys, the spike and
logits heuristics and the pass/fail rules.  The passes mirror
snn_compiler/passes/fuse.py: the patterns they recognise, the neuron
arguments they carry over (including SpikingJelly-style look-alikes whose
v_reset=None means soft reset) and path-based fusion.  Running the fused
modules needs the GPU and is covered by test_gpu_vgg / test_gpu_attention.
"""
import pytest
import torch
import torch.nn as nn

from snnk.verify import compare_models, assert_equivalent
from snnk.passes import fuse_snn_model, fuse_modules_path, fuse_conv_bn_add_neuron_path
from snnk.passes.fuse import NeuronSpec
from snnk.nn import (
    LIFNode, IFNode, FusedConvBNNeuron, FusedConvNeuron, FusedLinearNeuron, FusedConvBNLIFPool,
    FusedConvBNAddNeuron,
)
from snnk.zoo.vgg import VGGSNN, VGG11_CFG


class _Const(nn.Module):
    def __init__(self, t):
        super().__init__()
        self.t = t

    def forward(self, x):
        return self.t


def test_compare_models_report():
    a = torch.tensor([[0.1, 2.0, -1.0], [3.0, 0.0, 1.0]])
    b = a.clone()
    b[0, 0] = 0.15
    rep = compare_models(_Const(a), _Const(b), torch.zeros(1))
    assert rep["shape_match"] and not rep["bit_exact"]
    assert rep["max_abs_diff"] == pytest.approx(0.05, abs=1e-6)
    assert rep["mean_abs_diff"] == pytest.approx(0.05 / 6, abs=1e-7)
    assert rep["rel_max"] == pytest.approx(0.05 / 3.0, rel=1e-5)
    assert rep["argmax_agree"] == 1.0          # logits-like: last dim >= 2
    assert rep["spike_mismatch_frac"] is None  # not 0/1 valued
    same = compare_models(_Const(a), _Const(a.clone()), torch.zeros(1))
    assert same["bit_exact"] and same["max_abs_diff"] == 0.0


def test_compare_models_spikes_and_shapes():
    s = (torch.arange(24).reshape(4, 6) % 3 == 0).float()
    s2 = s.clone()
    s2[0, 0] = 1 - s2[0, 0]
    rep = compare_models(_Const(s), _Const(s2), None)
    assert rep["spike_mismatch_frac"] == pytest.approx(1 / 24)
    bad = compare_models(_Const(s), _Const(s[:2]), None)
    assert not bad["shape_match"] and bad["max_abs_diff"] == float("inf")
    assert bad["bit_exact"] is False and bad["argmax_agree"] is None


def test_assert_equivalent_rules():
    a = torch.tensor([[0.0, 1.0], [2.0, 0.5]])
    assert assert_equivalent(_Const(a), _Const(a.clone()), None, verbose=False)["bit_exact"]
    b = a + 1e-4
    with pytest.raises(AssertionError, match="numeric"):
        assert_equivalent(_Const(a), _Const(b), None, verbose=False)       # bit-exact required
    assert_equivalent(_Const(a), _Const(b), None, atol=1e-3, require_bitexact=False,
                      verbose=False)
    c = a.clone()
    c[0] = torch.tensor([1.0, 0.0])                                         # top-1 flips
    with pytest.raises(AssertionError, match="topology"):
        assert_equivalent(_Const(a), _Const(c), None, atol=10.0, require_bitexact=False,
                          verbose=False)
    with pytest.raises(AssertionError, match="shapes differ"):
        assert_equivalent(_Const(a), _Const(a[:1]), None, verbose=False)


def test_assert_equivalent_resets_state():
    class _Stateful(nn.Module):
        def __init__(self):
            super().__init__()
            self.n = 0
            self.child = _Counter()

        def forward(self, x):
            return x + self.child.step()

    class _Counter(nn.Module):
        def __init__(self):
            super().__init__()
            self.v = 0.0

        def step(self):
            self.v += 1.0
            return self.v

        def reset(self):
            self.v = 0.0

    m = _Stateful()
    x = torch.zeros(2, 3)
    # both runs see fresh state, so the model equals itself
    assert assert_equivalent(m, m, x, verbose=False)["bit_exact"]


def _vgg11():
    return VGGSNN(VGG11_CFG, num_classes=10, pool="max", input_size=32).eval()


def test_fuse_snn_model_vgg_patterns():
    m, n = fuse_snn_model(_vgg11())
    feats = list(m.features)
    # conv 3->64 (Cin % 32 != 0) stays a FusedConvBNNeuron followed by its pool;
    # every other conv block (+ its pool) is one FusedConvBNLIFPool
    assert isinstance(feats[0], FusedConvBNNeuron) and isinstance(feats[1], nn.MaxPool2d)
    pools = [f for f in feats if isinstance(f, FusedConvBNLIFPool)]
    assert len(pools) == 7 and len(feats) == 9
    assert [p.pool for p in pools] == ["max", None, "max", None, "max", None, "max"]
    assert sum(isinstance(c, FusedLinearNeuron) for c in m.classifier) == 2
    assert n == 10


def test_fuse_snn_model_bit_exact_mode_keeps_fp32_convs():
    m, n = fuse_snn_model(_vgg11(), fold_bn=False)
    feats = list(m.features)
    assert not any(isinstance(f, FusedConvBNLIFPool) for f in feats)
    convs = [f for f in feats if isinstance(f, FusedConvBNNeuron)]
    assert len(convs) == 8 and all(not c.fold_bn for c in convs)
    assert sum(isinstance(f, nn.MaxPool2d) for f in feats) == 5
    assert n == 10


def test_fuse_snn_model_folded_weights_match():
    ref = _vgg11()
    m, _ = fuse_snn_model(_vgg11_copy(ref))
    conv, bn = ref.features[4], ref.features[5]             # conv 64->128, its BN
    blk = [f for f in m.features if isinstance(f, FusedConvBNLIFPool)][0]
    inv = bn.weight / torch.sqrt(bn.running_var + bn.eps)
    w = conv.weight * inv.view(-1, 1, 1, 1)
    b = (conv.bias - bn.running_mean) * inv + bn.bias
    assert torch.allclose(blk.weight, w.detach(), rtol=1e-6, atol=1e-7)
    assert torch.allclose(blk.bias, b.detach(), rtol=1e-6, atol=1e-7)
    assert blk.w_prep.dtype == torch.bfloat16 and blk.w_prep.shape == (128, 9 * 64)


def _vgg11_copy(ref):
    m = _vgg11()
    m.load_state_dict(ref.state_dict())
    return m.eval()


class _SJLif(nn.Module):
    """SpikingJelly look-alike: class name LIFNode, v_reset=None = soft reset."""
    def __init__(self):
        super().__init__()
        self.tau, self.v_threshold, self.v_reset, self.decay_input = 4.0, 0.7, None, False


_SJLif.__name__ = "LIFNode"


def test_neuron_spec_duck_typing():
    spec = NeuronSpec.of(_SJLif())
    assert spec.kwargs("NCHW") == dict(neuron="lif", decay=None, tau=4.0, decay_input=False,
                                       soft_reset=True, v_threshold=0.7, v_reset=0.0,
                                       layout="NCHW")
    kw = NeuronSpec.of(IFNode(v_threshold=0.5, soft_reset=True)).kwargs()
    assert kw["neuron"] == "if" and kw["soft_reset"] and kw["v_threshold"] == 0.5
    assert "tau" not in kw and "layout" not in kw
    assert NeuronSpec.kind_of(nn.ReLU()) is None
    with pytest.raises(TypeError):
        NeuronSpec.of(nn.ReLU())
    seq = nn.Sequential(nn.Conv2d(8, 8, 3, padding=1), nn.BatchNorm2d(8).eval(), _SJLif(),
                        nn.Flatten(), nn.Linear(8, 4), LIFNode(tau=3.0))
    m, n = fuse_snn_model(seq.eval())
    assert n == 2 and isinstance(m[0], FusedConvBNNeuron) and isinstance(m[2], FusedLinearNeuron)
    assert m[0].soft_reset and m[0].tau == 4.0 and m[2].tau == 3.0


def test_fuse_snn_model_recurses_into_non_sequential_containers():
    class Net(nn.Module):
        def __init__(self):
            super().__init__()
            self.stem = nn.Sequential(nn.Conv2d(3, 8, 3, padding=1), IFNode())
            self.blocks = nn.ModuleList([nn.Sequential(nn.Linear(8, 8), LIFNode()),
                                         nn.Sequential(nn.ReLU())])
    net = Net().eval()
    m, n = fuse_snn_model(net)
    assert m is net and n == 2
    assert isinstance(net.stem[0], FusedConvNeuron) and len(net.stem) == 1
    assert isinstance(net.blocks[0][0], FusedLinearNeuron)
    assert isinstance(net.blocks[1][0], nn.ReLU)


def test_fuse_modules_path_and_residual():
    class Block(nn.Module):
        def __init__(self):
            super().__init__()
            self.conv1, self.bn1, self.neuron1 = nn.Conv2d(4, 4, 3, padding=1), nn.BatchNorm2d(4), LIFNode()
            self.conv2, self.bn2, self.neuron2 = nn.Conv2d(4, 4, 3, padding=1), nn.BatchNorm2d(4), IFNode()
            self.fc, self.fc_neuron = nn.Linear(4, 4), IFNode()
            self.c3, self.n3 = nn.Conv2d(4, 4, 1), LIFNode()

    b = Block().eval()
    assert fuse_modules_path(b, [("conv1", "bn1", "neuron1"), ("fc", None, "fc_neuron"),
                                 ("c3", "", "n3")]) == 3
    assert isinstance(b.neuron1, FusedConvBNNeuron) and isinstance(b.conv1, nn.Identity)
    assert isinstance(b.bn1, nn.Identity) and isinstance(b.fc_neuron, FusedLinearNeuron)
    assert isinstance(b.n3, FusedConvNeuron) and isinstance(b.c3, nn.Identity)
    mod = fuse_conv_bn_add_neuron_path(b, "conv2", "bn2", "neuron2")
    assert isinstance(mod, FusedConvBNAddNeuron) and b.neuron2 is mod
    assert isinstance(b.conv2, nn.Identity) and isinstance(b.bn2, nn.Identity)
    with pytest.raises(ValueError):
        fuse_modules_path(b, [("a", "b")])
    with pytest.raises(TypeError):
        fuse_modules_path(b, [("fc", "bn1", "neuron1")])     # Linear is no Conv2d
