"""Resident-weight tiles (29-38) of the fused conv3x3 / Linear + LIF kernel.

These tiles keep all of K of a block's weight rows in LDS for the whole launch
and load the packed spike words of each lane's own rows straight into
registers, so their K loop has no LDS ring and no barrier.  Like every tile
without a K split they add the K stages in one fixed order, so on the same
operands they must equal the bf16-input path of tile 2 (128 x 128, one K
group, no split) bit for bit: fp32 pre-activations, spikes and packed words.
Cases cover partial row tiles, Cout past the last full column tile, T past a
multiple of 4 (several 4-step chunks), steps past T inside a chunk, the
largest K each tile holds, cross-block K splits, and the shapes they refuse.
"""
import numpy as np
import pytest
import torch

from oracle import bits as ob
from snnk._abi import SnnkError
from snnk.kernels import conv as kc
from snnk.kernels.linear import linear_bias_lif, linear_bias_lif_act, linear_preact, linear_preact_act

pytestmark = pytest.mark.gpu
DEV = "cuda"
LIF = dict(decay=0.5, in_scale=0.5, v_threshold=1.0)
REF = dict(tile_hint=2, splits=1)  # one K group, no split: the same K order


def _pack(s):
    """[..., C] 0/1 (any dtype, CPU) -> int32 words [..., C/32] (oracle packer)."""
    return torch.from_numpy(ob.pack_rows(s.float().numpy()).view(np.int32))


def _conv_case(T, B, Cin, Cout, H, W, seed, p=0.2):
    g = torch.Generator().manual_seed(seed)
    x = (torch.rand(T, B, H, W, Cin, generator=g) < p).to(torch.bfloat16)
    w = torch.randn(Cout, Cin, 3, 3, generator=g) * (2.0 / (Cin * 9)) ** 0.5 * 2.0
    b = torch.randn(Cout, generator=g) * 0.1
    return x, kc.prepare_conv3x3_weight(w.to(DEV)), b.to(DEV).float()


CONV = [  # T, B, Cin, Cout, H, W, tile
    (4, 4, 128, 256, 16, 16, 29),   # the conv config's shape at batch 4
    (4, 2, 64, 64, 8, 8, 29),       # K = 576
    (5, 2, 128, 96, 6, 6, 29),      # two 4-step chunks; Cout 96 = 1.5 column tiles
    (3, 1, 64, 128, 10, 6, 30),     # steps past T inside the chunk
    (4, 1, 128, 128, 4, 4, 29),     # 4 of the tile's 32 quads exist
    (4, 2, 256, 64, 8, 8, 31),      # K = 2304 on 32-column tiles
    (8, 1, 256, 256, 4, 4, 31),
    (4, 2, 64, 128, 8, 8, 32),      # K = 576 on 128-column tiles
    (2, 3, 64, 160, 6, 10, 32),
    (4, 4, 128, 256, 16, 16, 35),   # sixteen waves
    (5, 2, 64, 96, 6, 6, 35),
    (4, 2, 256, 64, 8, 8, 36),
    (3, 2, 256, 96, 4, 6, 37),
    (4, 2, 64, 160, 8, 8, 38),      # 128 columns per wave
]


@pytest.mark.parametrize("pool", [False, True])
@pytest.mark.parametrize("T,B,Cin,Cout,H,W,tile", CONV)
def test_resident_conv_equals_unsplit_bf16_tile(T, B, Cin, Cout, H, W, tile, pool):
    if pool and (H % 2 or W % 2):
        pytest.skip("odd spatial size")
    print(f"[resident conv] T{T} B{B} {Cin}->{Cout} {H}x{W} tile {tile} pool {pool}", flush=True)
    x, wp, bd = _conv_case(T, B, Cin, Cout, H, W, seed=T * 17 + Cin + Cout + tile)
    xd, xp = x.to(DEV), _pack(x).to(DEV)
    ref = kc.conv3x3_bn_lif_nhwc(xd, wp, bd, pool=pool, **REF, **LIF).cpu()
    assert 0 < int(ref.float().sum()) < ref.numel()
    got = kc.conv3x3_bn_lif_act(xp, wp, bd, pool=pool, tile_hint=tile, splits=1,
                                out_bits=False, **LIF)
    assert torch.equal(got.cpu(), ref), "bits in, bf16 out"
    got = kc.conv3x3_bn_lif_act(xp, wp, bd, pool=pool, tile_hint=tile, splits=1, **LIF)
    assert torch.equal(got.cpu(), _pack(ref)), "bits in, bits out"


LINEAR = [  # T, R, K, N, tile
    (4, 256, 384, 1152, 29),   # the SSA projection's K and N
    (4, 64, 512, 256, 30),
    (3, 40, 1280, 96, 29),     # K = 1280: the most a 64-column tile holds
    (5, 24, 2560, 64, 31),     # K = 2560: the most a 32-column tile holds
    (4, 128, 640, 384, 32),    # K = 640: the most a 128-column tile holds
    (4, 256, 384, 1152, 35),
    (4, 96, 384, 1152, 38),
    (3, 40, 2496, 64, 36),
]


@pytest.mark.parametrize("T,R,K,N,tile", LINEAR)
def test_resident_linear_equals_unsplit_bf16_tile(T, R, K, N, tile):
    print(f"[resident linear] T{T} R{R} K{K} N{N} tile {tile}", flush=True)
    g = torch.Generator().manual_seed(K + N + tile)
    x = (torch.rand(T, R, K, generator=g) < 0.25).to(torch.bfloat16)
    w = (torch.randn(N, K, generator=g) * (2.0 / K) ** 0.5 * 2.0).to(DEV, torch.bfloat16)
    b = (torch.randn(N, generator=g) * 0.1).to(DEV)
    xd, xp = x.to(DEV), _pack(x).to(DEV)
    pre = linear_preact(xd, w, b, **REF).cpu()
    assert torch.equal(linear_preact_act(xp, w, b, tile_hint=tile, splits=1).cpu(), pre)
    ref = linear_bias_lif(xd, w, b, **REF, **LIF).cpu()
    assert 0 < int(ref.float().sum()) < ref.numel()
    kw = dict(tile_hint=tile, splits=1, **LIF)
    assert torch.equal(linear_bias_lif_act(xp, w, b, out_bits=False, **kw).cpu(), ref)
    assert torch.equal(linear_bias_lif_act(xp, w, b, **kw).cpu(), _pack(ref))


SPLIT = [  # conv (T, B, Cin, Cout, H, W, pool) or Linear (T, R, K, N), tile, splits
    ((4, 8, 256, 512, 4, 4, False), 37, 2),   # VGG L8 at batch 8
    ((4, 8, 512, 512, 4, 4, True), 37, 2),    # L10: K = 4608 in two halves
    ((3, 4, 512, 256, 4, 4, False), 36, 3),
    ((5, 2, 256, 128, 4, 4, True), 35, 4),    # two chunks of 4 steps
    ((4, 32, 2048, 2048), 37, 4),             # L11 as a dense Linear over 2x2 pixels
    ((4, 32, 4096, 1024), 35, 4),             # FC2's K
    ((4, 20, 512, 4096), 34, 2),              # FC1's shape, partial row tile
]


@pytest.mark.parametrize("shape,tile,splits", SPLIT)
def test_resident_tiles_with_split_k_equal_bf16_split(shape, tile, splits):
    """Cross-block split K on resident tiles: each block holds its share of the
    K stages; the partial sums are reduced in split order, as in tile 2 with
    the same split, so the results agree bit for bit."""
    print(f"[resident split] {shape} tile {tile} splits {splits}", flush=True)
    ref_kw, kw = dict(tile_hint=2, splits=splits), dict(tile_hint=tile, splits=splits)
    if len(shape) == 7:
        T, B, Cin, Cout, H, W, pool = shape
        x, wp, bd = _conv_case(T, B, Cin, Cout, H, W, seed=Cin + Cout + splits, p=0.15)
        xd, xp = x.to(DEV), _pack(x).to(DEV)
        ref = kc.conv3x3_bn_lif_nhwc(xd, wp, bd, pool=pool, **ref_kw, **LIF).cpu()
        got = kc.conv3x3_bn_lif_act(xp, wp, bd, pool=pool, **kw, **LIF).cpu()
    else:
        T, R, K, N = shape
        g = torch.Generator().manual_seed(K + N + splits)
        x = (torch.rand(T, R, K, generator=g) < 0.2).to(torch.bfloat16)
        w = (torch.randn(N, K, generator=g) * (2.0 / K) ** 0.5 * 2.0).to(DEV, torch.bfloat16)
        b = (torch.randn(N, generator=g) * 0.1).to(DEV)
        xd, xp = x.to(DEV), _pack(x).to(DEV)
        pre = linear_preact(xd, w, b, **ref_kw).cpu()
        assert torch.equal(linear_preact_act(xp, w, b, **kw).cpu(), pre)
        ref = linear_bias_lif(xd, w, b, **ref_kw, **LIF).cpu()
        got = linear_bias_lif_act(xp, w, b, **kw, **LIF).cpu()
    assert 0 < int(ref.float().sum()) < ref.numel()
    assert torch.equal(got, _pack(ref))


def test_resident_tiles_refuse_what_they_do_not_hold():
    x, wp, bd = _conv_case(4, 1, 96, 64, 4, 4, seed=1)
    with pytest.raises(SnnkError):   # Cin % 64 != 0: a stage would span two taps
        kc.conv3x3_bn_lif_act(_pack(x).to(DEV), wp, bd, pool=False, tile_hint=29, splits=1, **LIF)
    x, wp, bd = _conv_case(4, 1, 256, 64, 4, 4, seed=2)
    with pytest.raises(SnnkError):   # K = 2304 > 1280 for 64-column tiles
        kc.conv3x3_bn_lif_act(_pack(x).to(DEV), wp, bd, pool=False, tile_hint=29, splits=1, **LIF)
    with pytest.raises(SnnkError):   # bf16 input
        kc.conv3x3_bn_lif_act(x.to(DEV), wp, bd, pool=False, tile_hint=31, splits=1, **LIF)
    with pytest.raises(SnnkError):   # 2304 / 2 = 1152 fits 64 columns, but 4608 / 2 does not
        x5, wp5, bd5 = _conv_case(4, 1, 512, 64, 4, 4, seed=3)
        kc.conv3x3_bn_lif_act(_pack(x5).to(DEV), wp5, bd5, pool=False, tile_hint=29, splits=2, **LIF)
