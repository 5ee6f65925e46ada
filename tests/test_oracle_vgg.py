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
