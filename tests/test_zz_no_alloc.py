"""snnk_conv3x3_bn_lif_noalloc against snnk_conv3x3_bn_lif_ws, through the C ABI.

The no-allocation entry point runs the same kernels as the workspace entry
point with its split-K tickets and partial sums in the library's fixed
device scratch region, so the two must agree bit for bit.  Two calls in a
row, the second on a smaller input, check that the region is reused (and its
ticket counters left at zero) between calls.
"""
import ctypes

import pytest
import torch

from snnk import _abi

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _operands(T, B, H, W, Cin, Cout, seed):
    g = torch.Generator().manual_seed(seed)
    x = (torch.rand(T, B, H, W, Cin, generator=g) < 0.2).to(torch.bfloat16)
    w = (torch.randn(Cout, 9 * Cin, generator=g) * (2.0 / (9 * Cin)) ** 0.5 * 3.0)
    bias = torch.randn(Cout, generator=g) * 0.1
    return x.to(DEV), w.to(DEV, torch.bfloat16), bias.to(DEV)


def _lif_args():
    return (0.5, 0.5, 1.0, 0.0, 0)  # decay, in_scale, v_threshold, v_reset, soft_reset


def _run_ws(x, w, bias, shape, pool, preact):
    T, B, H, W, Cin, Cout = shape
    Ho, Wo = (H // 2, W // 2) if pool else (H, W)
    lib = _abi.lib()
    n = lib.snnk_conv3x3_bn_lif_ws_size(T, B, H, W, Cin, Cout, pool, 1 if preact else 0, -1, 0)
    assert n > 0, "the case must use a cross-block split"
    ws = torch.zeros(n, dtype=torch.uint8, device=DEV)
    out = torch.zeros(T, B, Ho, Wo, Cout, dtype=torch.bfloat16, device=DEV)
    pre = torch.zeros(T, B, H, W, Cout, dtype=torch.float32, device=DEV) if preact else None
    st = lib.snnk_conv3x3_bn_lif_ws(x.data_ptr(), w.data_ptr(), bias.data_ptr(),
                                    None if preact else out.data_ptr(), _abi.ptr(pre),
                                    T, B, H, W, Cin, Cout, pool, *_lif_args(), -1, 0,
                                    ws.data_ptr(), n, _abi.stream())
    assert st == 0, lib.snnk_status_string(st)
    torch.cuda.synchronize()
    return pre if preact else out


def _run_noalloc(x, w, bias, shape, pool, preact):
    T, B, H, W, Cin, Cout = shape
    Ho, Wo = (H // 2, W // 2) if pool else (H, W)
    lib = _abi.lib()
    out = torch.zeros(T, B, Ho, Wo, Cout, dtype=torch.bfloat16, device=DEV)
    pre = torch.zeros(T, B, H, W, Cout, dtype=torch.float32, device=DEV) if preact else None
    st = lib.snnk_conv3x3_bn_lif_noalloc(x.data_ptr(), w.data_ptr(), bias.data_ptr(),
                                         None if preact else out.data_ptr(), _abi.ptr(pre),
                                         T, B, H, W, Cin, Cout, pool, *_lif_args(), -1, 0,
                                         _abi.stream())
    assert st == 0, lib.snnk_status_string(st)
    torch.cuda.synchronize()
    return pre if preact else out


# first a VGG L9-sized layer (4x4 map, 512 -> 512, B = 32: 16 MiB of partials),
# then smaller ones that reuse the region with other tile / split plans
CASES = [((4, 32, 4, 4, 512, 512), 0, False),
         ((4, 2, 4, 4, 512, 512), 1, False),
         ((3, 2, 4, 4, 512, 256), 0, True)]


def test_noalloc_matches_workspace_entry_point():
    for i, (shape, pool, preact) in enumerate(CASES):
        print(f"[no_alloc] case {i}: shape={shape} pool={pool} preact={preact}", flush=True)
        x, w, bias = _operands(*shape, seed=10 + i)
        ref = _run_ws(x, w, bias, shape, pool, preact)
        got = _run_noalloc(x, w, bias, shape, pool, preact)
        assert torch.equal(got, ref), f"case {i}: no-alloc result differs from the _ws result"
        if not preact:
            assert 0 < int(got.float().sum()) < got.numel(), "degenerate case: no or all spikes"
    # the region keeps the last call's contents; a repeat of the first case
    # must still agree (ticket counters were left at zero)
    shape, pool, preact = CASES[0]
    x, w, bias = _operands(*shape, seed=10)
    assert torch.equal(_run_noalloc(x, w, bias, shape, pool, preact),
                       _run_ws(x, w, bias, shape, pool, preact))


def test_noalloc_rejects_plans_beyond_the_scratch_region():
    """A forced plan whose partials exceed 32 MiB is refused before any launch."""
    lib = _abi.lib()
    shape = (4, 32, 16, 16, 512, 512)
    need = lib.snnk_conv3x3_bn_lif_ws_size(*shape, 0, 0, 2, 8)  # 128x128 tiles, 8 splits
    assert need > (32 << 20)
    x, w, bias = _operands(*shape, seed=1)
    out = torch.zeros(4, 32, 16, 16, 512, dtype=torch.bfloat16, device=DEV)
    st = lib.snnk_conv3x3_bn_lif_noalloc(x.data_ptr(), w.data_ptr(), bias.data_ptr(),
                                         out.data_ptr(), None, *shape, 0, *_lif_args(), 2, 8,
                                         _abi.stream())
    assert st == _abi.ESCRATCH
    assert b"no-alloc" in lib.snnk_status_string(st)
    assert ctypes.c_int(st).value == -5
