"""64-row ring tiles with K over 2-8 wave groups (tiles 39-41) on packed spikes.

The VGG layers with few rows and long K (the 4x4 maps, the FC layers at batch
56) run on these tiles.  Their bf16-input form does not fit LDS (refused with
SNNK_EUNSUPPORTED), so each is checked against a bf16 ring tile with the same
number of K groups and the same split: group g adds stages g, g + groups, ...
and the groups' sums are added in group order in both, so the fp32
pre-activations, the spikes and the packed words agree bit for bit.
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
# bf16 ring tiles with the same K groups: 4 -> tile 4 (32x32), 8 -> tile 6, 2 -> tile 13
SAME_GROUPS = {39: 4, 40: 6, 41: 13, 42: 4, 43: 4}


def _pack(s):
    """[..., C] 0/1 (any dtype, CPU) -> int32 words [..., C/32] (oracle packer)."""
    return torch.from_numpy(ob.pack_rows(s.float().numpy()).view(np.int32))


def _conv_case(T, B, Cin, Cout, H, W, seed, p=0.2):
    g = torch.Generator().manual_seed(seed)
    x = (torch.rand(T, B, H, W, Cin, generator=g) < p).to(torch.bfloat16)
    w = torch.randn(Cout, Cin, 3, 3, generator=g) * (2.0 / (Cin * 9)) ** 0.5 * 2.0
    b = torch.randn(Cout, generator=g) * 0.1
    return x, kc.prepare_conv3x3_weight(w.to(DEV)), b.to(DEV).float()


CONV = [  # T, B, Cin, Cout, H, W, pool, tile, splits
    (4, 8, 256, 512, 4, 4, False, 39, 1),    # VGG L8's shape at batch 8
    (4, 8, 512, 512, 4, 4, True, 39, 1),     # L10
    (4, 14, 512, 512, 4, 4, False, 41, 1),   # L9 at batch 14: rows not a multiple of the tile
    (5, 2, 256, 256, 4, 4, True, 40, 1),     # two 4-step chunks
    (3, 4, 512, 96, 2, 2, False, 39, 2),     # Cout 96, steps past T, split
    (4, 6, 256, 160, 4, 4, False, 41, 3),
    (4, 8, 256, 256, 4, 4, False, 42, 1),    # 64 x 32 tiles
    (5, 3, 256, 96, 4, 4, True, 42, 2),      # two chunks, pool, split
    (4, 14, 512, 512, 4, 4, False, 43, 1),   # L9 at batch 14 on 128 x 64 tiles
    (4, 10, 512, 512, 4, 4, True, 43, 1),    # L10, rows not a multiple of 128
    (5, 3, 256, 96, 4, 4, False, 43, 2),     # two chunks, Cout 96, split
]


@pytest.mark.parametrize("T,B,Cin,Cout,H,W,pool,tile,splits", CONV)
def test_tail_tile_conv_equals_bf16_tile_with_same_k_groups(T, B, Cin, Cout, H, W, pool, tile,
                                                           splits):
    print(f"[tail conv] T{T} B{B} {Cin}->{Cout} {H}x{W} pool {pool} tile {tile} splits {splits}",
          flush=True)
    x, wp, bd = _conv_case(T, B, Cin, Cout, H, W, seed=T * 7 + Cin + Cout + tile)
    xd, xp = x.to(DEV), _pack(x).to(DEV)
    ref = kc.conv3x3_bn_lif_nhwc(xd, wp, bd, pool=pool, tile_hint=SAME_GROUPS[tile], splits=splits,
                                 **LIF).cpu()
    assert 0 < int(ref.float().sum()) < ref.numel()
    kw = dict(tile_hint=tile, splits=splits, **LIF)
    got = kc.conv3x3_bn_lif_act(xp, wp, bd, pool=pool, out_bits=False, **kw)
    assert torch.equal(got.cpu(), ref), "bits in, bf16 out"
    got = kc.conv3x3_bn_lif_act(xp, wp, bd, pool=pool, **kw)
    assert torch.equal(got.cpu(), _pack(ref)), "bits in, bits out"


LINEAR = [  # T, R, K, N, tile, splits
    (4, 32, 4096, 1024, 39, 1),   # FC2's K at batch 32 rows (tile 4 is its plan there)
    (4, 56, 4096, 1024, 39, 1),   # FC2 at batch 56
    (4, 56, 512, 4096, 41, 1),    # FC1 at batch 56
    (4, 56, 2048, 2048, 40, 1),   # L11 as a dense Linear at batch 56
    (6, 20, 1024, 256, 41, 2),    # two chunks, split
    (4, 32, 4096, 1024, 42, 1),   # FC2's K at batch 32 on 64 x 32 tiles
    (4, 56, 2048, 2048, 42, 1),   # L11 as a dense Linear at batch 56
    (5, 20, 1024, 96, 42, 3),     # two chunks, partial tiles, split
    (4, 56, 4096, 512, 43, 1),    # 128 x 64 tiles on a Linear
]


@pytest.mark.parametrize("T,R,K,N,tile,splits", LINEAR)
def test_tail_tile_linear_equals_bf16_tile_with_same_k_groups(T, R, K, N, tile, splits):
    print(f"[tail linear] T{T} R{R} K{K} N{N} tile {tile} splits {splits}", flush=True)
    g = torch.Generator().manual_seed(K + N + tile + splits)
    x = (torch.rand(T, R, K, generator=g) < 0.2).to(torch.bfloat16)
    w = (torch.randn(N, K, generator=g) * (2.0 / K) ** 0.5 * 2.0).to(DEV, torch.bfloat16)
    b = (torch.randn(N, generator=g) * 0.1).to(DEV)
    xd, xp = x.to(DEV), _pack(x).to(DEV)
    ref_kw = dict(tile_hint=SAME_GROUPS[tile], splits=splits)
    kw = dict(tile_hint=tile, splits=splits)
    pre = linear_preact(xd, w, b, **ref_kw).cpu()
    assert torch.equal(linear_preact_act(xp, w, b, **kw).cpu(), pre)
    ref = linear_bias_lif(xd, w, b, **ref_kw, **LIF).cpu()
    assert 0 < int(ref.float().sum()) < ref.numel()
    assert torch.equal(linear_bias_lif_act(xp, w, b, out_bits=False, **kw, **LIF).cpu(), ref)
    assert torch.equal(linear_bias_lif_act(xp, w, b, **kw, **LIF).cpu(), _pack(ref))


def test_tail_tiles_bf16_form_refused():
    """Tiles 39, 40 and 43 need more LDS than a CU has with bf16 A: refused, not launched."""
    x, wp, bd = _conv_case(4, 2, 256, 128, 4, 4, seed=3)
    for tile in (39, 40, 43):
        with pytest.raises(SnnkError):
            kc.conv3x3_bn_lif_nhwc(x.to(DEV), wp, bd, pool=False, tile_hint=tile, splits=1, **LIF)


@pytest.mark.parametrize("pool", [False, True])
def test_tile_42_packed_equals_its_bf16_form(pool):
    """Tile 42 (64 x 32, 4 K groups) also runs bf16 input: both give the same spikes."""
    x, wp, bd = _conv_case(4, 8, 256, 256, 4, 4, seed=42)
    ref = kc.conv3x3_bn_lif_nhwc(x.to(DEV), wp, bd, pool=pool, tile_hint=42, splits=1, **LIF).cpu()
    assert 0 < int(ref.float().sum()) < ref.numel()
    got = kc.conv3x3_bn_lif_act(_pack(x).to(DEV), wp, bd, pool=pool, tile_hint=42, splits=1, **LIF)
    assert torch.equal(got.cpu(), _pack(ref))
