"""Pins for oracle/vgg.py (structure, seeded init, sensitivity)."""
import torch

from oracle import vgg as ov


def test_structure_and_init_distributions():
    p = ov.make_params(0)
    assert len(p["convs"]) == 13 and len(p["fcs"]) == 3
    assert sum(1 for v in p["cfg"] if v == "P") == 5
    assert p["fcs"][0]["w"].shape == (4096, 512)          # 32x32 input -> 1x1 x 512
    assert p["fcs"][2]["w"].shape == (10, 4096)
    w = p["convs"][5]["w"]                               # 256 -> 256
    assert abs(w.std().item() - (2.0 / (256 * 9)) ** 0.5) < 2e-3
    var = torch.cat([c["var"] for c in p["convs"]])
    assert var.min() >= 0.5 and var.max() <= 1.5
    assert torch.equal(ov.make_params(0)["convs"][3]["w"], p["convs"][3]["w"])


def test_forward_shapes_and_silent_baseline_init():
    img = torch.randn(2, 3, 32, 32, generator=torch.Generator().manual_seed(1))
    out, rates = ov.forward(ov.make_params(0), img, T=4, return_rates=True)
    assert out.shape == (4, 2, 10) and len(rates) == 15
    # Kaiming init with theta=1: the deep layers do not fire, the logits equal the FC3 bias
    assert max(rates[5:]) == 0.0
    assert torch.allclose(out, ov.make_params(0)["fcs"][2]["b"].view(1, 1, -1).expand_as(out))


def test_active_network_is_chaotic():
    """With weights x3 every layer fires, and flipping 0.01% of the layer-1
    spikes already scrambles the logits: end-to-end argmax agreement is not a
    usable parity measure for this network; per-layer checks are."""
    import torch.nn.functional as F
    from oracle import fused as of, neurons as on
    params = ov.make_params(0, gain=3.0)
    img = torch.randn(16, 3, 32, 32, generator=torch.Generator().manual_seed(1))
    T = 4

    def run(flip):
        x = img.unsqueeze(0).expand(T, *img.shape).contiguous()
        ci, k, cfg = 0, 0, params["cfg"]
        while k < len(cfg):
            p = params["convs"][ci]
            w2, b2 = of.fold_conv_bn(p["w"], p["b"], p["gamma"], p["beta"], p["mean"],
                                     p["var"], p["eps"])
            s, _, _ = on.lif_multistep(of.conv3x3_seq(x, w2), bias=b2, neuron="lif")
            pool = k + 1 < len(cfg) and cfg[k + 1] == "P"
            s = of.maxpool2x2_seq(s) if pool else s
            if ci == 0 and flip:
                m = torch.rand(s.shape, generator=torch.Generator().manual_seed(2)) < 1e-4
                s = torch.where(m, 1 - s, s)
            x, ci, k = s, ci + 1, k + (2 if pool else 1)
        x = x.reshape(T, img.shape[0], -1)
        for i, p in enumerate(params["fcs"]):
            y = F.linear(x, p["w"])
            x = on.lif_multistep(y, bias=p["b"], neuron="lif")[0] if i < 2 else y + p["b"]
        return x.mean(0)

    a, b = run(False), run(True)
    assert (a.argmax(-1) == b.argmax(-1)).float().mean().item() < 0.6


def _lif_t_loop(u, tau=2.0, v_th=1.0):
    """LIF written the SpikingJelly way, step by step over T:
    v += (u - v) / tau; spike = v >= v_th; hard reset to 0."""
    v = torch.zeros_like(u[0])
    spikes, trace = [], []
    for t in range(u.shape[0]):
        v = v + (u[t] - v) / tau
        s = (v >= v_th).float()
        trace.append(v.clone())
        spikes.append(s)
        v = v * (1.0 - s)
    return torch.stack(spikes), torch.stack(trace)


def _independent_layers(params, rec):
    """Each layer of the network rebuilt from torch.nn modules (nn.Conv2d with
    its bias, an eval-mode nn.BatchNorm2d kept separate, the T-loop LIF,
    nn.MaxPool2d, nn.Linear) and fed the oracle's input for that layer."""
    import torch.nn as nn
    out = []
    convs = iter(params["convs"])
    fcs = iter(params["fcs"])
    for r in rec:
        x = r["input"]
        T, B = x.shape[:2]
        if r["kind"] in ("image", "conv"):
            p = next(convs)
            Cout, Cin = p["w"].shape[:2]
            conv = nn.Conv2d(Cin, Cout, 3, padding=1)
            bn = nn.BatchNorm2d(Cout, eps=p["eps"]).eval()
            with torch.no_grad():
                conv.weight.copy_(p["w"])
                conv.bias.copy_(p["b"])
                bn.weight.copy_(p["gamma"])
                bn.bias.copy_(p["beta"])
                bn.running_mean.copy_(p["mean"])
                bn.running_var.copy_(p["var"])
                u = bn(conv(x.flatten(0, 1)))
            u = u.view(T, B, *u.shape[1:])
            s, tr = _lif_t_loop(u)
            if r["pool"]:
                H, W = s.shape[-2:]
                s = nn.MaxPool2d(2)(s.flatten(0, 1)).view(T, B, Cout, H // 2, W // 2)
            out.append((s, tr))
        else:
            p = next(fcs)
            lin = nn.Linear(p["w"].shape[1], p["w"].shape[0])
            with torch.no_grad():
                lin.weight.copy_(p["w"])
                lin.bias.copy_(p["b"])
                y = lin(x)
            out.append(_lif_t_loop(y) if r["kind"] == "fc_lif" else (y, None))
    return out


def test_forward_layers_match_independent_nn_composition_gain3():
    """At gain 3 (every layer fires) each oracle layer equals the same layer
    rebuilt from torch.nn modules with BN unfolded: >= 99.9% of the spikes
    agree and every flip sits where the membrane was within 1e-4 of the
    threshold (this step or earlier: a flipped reset shifts the later steps);
    the membrane traces agree to 1e-4; FC3's logits to 1e-4.  The chain is
    consistent (each layer's input is the previous layer's output) and its
    last entry equals forward()."""
    params = ov.make_params(0, gain=3.0)
    img = torch.randn(4, 3, 32, 32, generator=torch.Generator().manual_seed(5))
    T = 4
    rec = ov.forward_layers(params, img, T)
    assert [r["kind"] for r in rec] == ["image"] + ["conv"] * 12 + ["fc_lif"] * 2 + ["fc_out"]
    assert sum(r.get("pool", False) for r in rec) == 5
    for a, b in zip(rec[:-1], rec[1:]):
        assert torch.equal(a["output"].reshape(b["input"].shape), b["input"])
    assert torch.equal(rec[-1]["output"], ov.forward(params, img, T))
    ind = _independent_layers(params, rec)
    for i, (r, (s, tr)) in enumerate(zip(rec, ind)):
        if r["kind"] == "fc_out":
            assert (s - r["output"]).abs().max().item() < 1e-4
            continue
        assert r["output"].mean().item() > 0.0, f"layer {i} silent"
        assert (tr - r["trace"]).abs().max().item() < 1e-4, f"layer {i} trace"
        got = s
        agree = (got == r["output"]).float().mean().item()
        near = (tr - 1.0).abs() < 1e-4
        if r.get("pool", False):
            Tn, B, C, H, W = near.shape
            near = near.view(Tn, B, C, H // 2, 2, W // 2, 2).any(dim=6).any(dim=4)
        near = torch.cummax(near.int(), 0).values.bool()
        assert agree >= 0.999, f"layer {i}: agreement {agree}"
        assert not torch.any((got != r["output"]) & ~near), f"layer {i}: flip away from threshold"
