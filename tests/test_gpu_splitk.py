"""Cross-block split-K of the conv / linear MFMA kernel.

With a split the output tile's K range is shared by several workgroups that
store fp32 partial sums in the device workspace; the last workgroup of a tile
(per-tile ticket) adds them in split order and runs the epilogue.  Checked:
pre-activations within fp32 accumulation error of a float64 reference for
several split counts and tile shapes (T = 6 covers two 4-step chunks),
bit-identical results across repeated calls and graph replays (the
reduction order is fixed and the tickets reset themselves), the LIF epilogue
exact on the split path's own pre-activations, and the workspace-size
contract.
"""
import pytest
import torch
import torch.nn.functional as F

import snnk
from snnk import _abi
from snnk.kernels import conv as kc
from snnk.kernels.linear import linear_bias_lif, linear_preact
from oracle import neurons as on

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _conv_operands(T, B, H, W, Cin, Cout, seed):
    g = torch.Generator().manual_seed(seed)
    x = (torch.rand(T, B, Cin, H, W, generator=g) < 0.3).float()
    x = x + torch.randn(x.shape, generator=g) * 0.5
    w = torch.randn(Cout, Cin, 3, 3, generator=g) * (2.0 / (Cin * 9)) ** 0.5
    b = torch.randn(Cout, generator=g) * 0.1
    xd = kc.to_nhwc_bf16(x.to(DEV))
    wp = kc.prepare_conv3x3_weight(w.to(DEV))
    xb, wb = x.to(torch.bfloat16).double(), w.to(torch.bfloat16).double()
    y = F.conv2d(xb.reshape(T * B, Cin, H, W), wb, padding=1) + b.double().view(1, -1, 1, 1)
    ya = F.conv2d(xb.abs().reshape(T * B, Cin, H, W), wb.abs(), padding=1)
    nhwc = lambda t: t.view(T, B, Cout, H, W).permute(0, 1, 3, 4, 2)  # noqa: E731
    return xd, wp, b.to(DEV), nhwc(y), nhwc(ya)


@pytest.mark.parametrize("T,B,H,W,Cin,Cout,tile,splits", [
    (4, 32, 4, 4, 512, 512, 2, 4), (4, 32, 2, 2, 512, 512, 2, 8), (4, 32, 4, 4, 256, 512, 10, 3),
    (6, 8, 4, 4, 256, 256, 3, 5), (4, 8, 2, 2, 512, 512, -1, 0), (4, 4, 4, 4, 128, 96, 8, 2),
    (3, 8, 4, 4, 64, 64, 6, 2), (4, 32, 2, 2, 512, 512, 25, 2), (4, 32, 4, 4, 512, 512, 27, 3),
])
def test_conv_split_preact_matches_f64(T, B, H, W, Cin, Cout, tile, splits):
    xd, wp, bd, ref, absref = _conv_operands(T, B, H, W, Cin, Cout, seed=Cin + Cout + splits)
    n = _abi.size_call("snnk_conv3x3_bn_lif_ws_size", T, B, H, W, Cin, Cout, 0, 1, tile, splits)
    if splits not in (0, 1):
        assert n > 0
    pre = kc.conv3x3_preact_nhwc(xd, wp, bd, tile_hint=tile, splits=splits)
    err = (pre.cpu().double() - ref).abs()
    assert torch.all(err <= 3e-5 * absref + 1e-6), f"max err {err.max().item()}"
    # deterministic reduction, tickets reset between calls
    for _ in range(2):
        assert torch.equal(kc.conv3x3_preact_nhwc(xd, wp, bd, tile_hint=tile, splits=splits), pre)


@pytest.mark.parametrize("pool", [False, True])
def test_conv_split_lif_epilogue_exact(pool):
    T, B, H, W, Cin, Cout = 6, 16, 4, 4, 512, 256
    xd, wp, bd, _, _ = _conv_operands(T, B, H, W, Cin, Cout, seed=7)
    pre = kc.conv3x3_preact_nhwc(xd, wp, bd, tile_hint=2, splits=4).cpu()
    s = kc.conv3x3_bn_lif_nhwc(xd, wp, bd, pool=pool, decay=0.5, in_scale=0.5, v_threshold=1.0,
                               tile_hint=2, splits=4).cpu().float()
    ref, _, _ = on.lif_multistep(pre.permute(0, 1, 4, 2, 3), neuron="lif", tau=2.0)
    if pool:
        ref = ref.view(T, B, Cout, H // 2, 2, W // 2, 2).amax(dim=(4, 6))
    assert torch.equal(s.permute(0, 1, 4, 2, 3), ref)


def test_linear_split_matches_f64_and_graph_replays():
    T, R, K, N = 4, 32, 4096, 1024
    g = torch.Generator().manual_seed(3)
    x = (torch.rand(T, R, K, generator=g) < 0.2).to(torch.bfloat16)
    w = (torch.randn(N, K, generator=g) * K ** -0.5).to(torch.bfloat16)
    b = torch.randn(N, generator=g) * 0.1
    ref = x.double() @ w.double().t() + b.double()
    absref = x.double() @ w.double().abs().t()
    xd, wd, bd = x.to(DEV), w.to(DEV), b.to(DEV)
    for splits in (0, 2, 8):
        pre = linear_preact(xd, wd, bd, splits=splits).cpu().double()
        assert torch.all((pre - ref).abs() <= 3e-5 * absref + 1e-6)
    eager = linear_bias_lif(xd, wd, bd, decay=0.5, in_scale=0.5, v_threshold=0.05, splits=0)
    out = torch.empty_like(eager)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        linear_bias_lif(xd, wd, bd, decay=0.5, in_scale=0.5, v_threshold=0.05, splits=0, out=out)
        with torch.cuda.graph(graph, stream=s):
            linear_bias_lif(xd, wd, bd, decay=0.5, in_scale=0.5, v_threshold=0.05, splits=0,
                            out=out)
    torch.cuda.current_stream().wait_stream(s)
    for _ in range(3):
        out.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)
    assert 0.0 < eager.float().mean().item() < 1.0


def test_workspace_contract():
    T, B, H, W, Cin, Cout = 4, 32, 4, 4, 512, 512
    xd, wp, bd, _, _ = _conv_operands(T, B, H, W, Cin, Cout, seed=9)
    out = torch.empty(T, B, H, W, Cout, device=DEV, dtype=torch.bfloat16)
    need = _abi.size_call("snnk_conv3x3_bn_lif_ws_size", T, B, H, W, Cin, Cout, 0, 0, 2, 4)
    small = torch.zeros(need // 2, dtype=torch.uint8, device=DEV)
    st = _abi.lib().snnk_conv3x3_bn_lif_ws(
        xd.data_ptr(), wp.data_ptr(), bd.data_ptr(), out.data_ptr(), None, T, B, H, W, Cin, Cout,
        0, 0.5, 0.5, 1.0, 0.0, 0, 2, 4, small.data_ptr(), small.numel(), _abi.stream())
    assert st == _abi.EWORKSPACE
    st = _abi.lib().snnk_conv3x3_bn_lif_ws(
        xd.data_ptr(), wp.data_ptr(), bd.data_ptr(), out.data_ptr(), None, T, B, H, W, Cin, Cout,
        0, 0.5, 0.5, 1.0, 0.0, 0, 2, 4, None, 0, _abi.stream())
    assert st == _abi.EWORKSPACE
    # splits=1 needs no workspace and matches the plain entry point
    a = kc.conv3x3_bn_lif_nhwc(xd, wp, bd, pool=False, decay=0.5, in_scale=0.5,
                               v_threshold=1.0, tile_hint=2, splits=1)
    st = _abi.lib().snnk_conv3x3_bn_lif(
        xd.data_ptr(), wp.data_ptr(), bd.data_ptr(), out.data_ptr(), None, T, B, H, W, Cin, Cout,
        0, 0.5, 0.5, 1.0, 0.0, 0, 2, _abi.stream())
    assert st == _abi.OK
    torch.cuda.synchronize()
    assert torch.equal(a, out)
    assert snnk.__name__ == "snnk"


def test_workspace_shared_by_calls_of_different_shapes():
    """Calls with different tile counts share the device workspace: the ticket
    counters sit in a fixed region that no call uses for partial sums, so a
    call after a bigger or smaller one still reduces correctly."""
    shapes = [(4, 32, 4096, 4096, 13, 2), (4, 32, 4096, 1024, 10, 4), (4, 64, 2048, 2048, 2, 4),
              (4, 32, 4096, 4096, 13, 2), (4, 8, 1024, 512, 3, 4)]
    g = torch.Generator().manual_seed(21)
    for T, R, K, N, tile, sp in shapes * 2:
        x = (torch.rand(T, R, K, generator=g) < 0.2).to(torch.bfloat16)
        w = (torch.randn(N, K, generator=g) * K ** -0.5).to(torch.bfloat16)
        ref = x.double() @ w.double().t()
        absref = x.double() @ w.double().abs().t()
        pre = linear_preact(x.to(DEV), w.to(DEV), None, tile_hint=tile, splits=sp).cpu().double()
        assert torch.all((pre - ref).abs() <= 3e-5 * absref + 1e-6), (R, K, N, tile, sp)
