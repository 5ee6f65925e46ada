"""GPU parity of bit packing and the binary GEMM (popcount VALU and int8 MFMA).

Integer outputs must be bit-exact.  Small shapes are checked element-wise
against the numpy oracle; the BASELINE config (8192x4096x4096) is checked on
a bounded row sample against the C oracle, by two exact checksums that touch
every output, and by agreement of the two independent GPU algorithms.
Restates snn_compiler/tests/test_spike_attention.py:142-148 (popcount K^T V
with N=70, not a multiple of 32).
"""
import numpy as np
import pytest
import torch

import snnk
from oracle import bits as ob, clib

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _bern(shape, p, seed):
    g = torch.Generator().manual_seed(seed)
    return (torch.rand(*shape, generator=g) < p)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16, torch.uint8])
@pytest.mark.parametrize("shape,dim", [((37, 101), -1), ((3, 70, 5), 1), ((4, 64), 0),
                                       ((2, 3, 4096), -1), ((70, 33), -2)])
def test_pack_bits_vs_oracle(dtype, shape, dim):
    x = _bern(shape, 0.3, 1).to(dtype)
    got = snnk.pack_bits(x.to(DEV), dim=dim).cpu().numpy().view(np.uint32)
    ref = ob.pack_axis(x.to(torch.uint8).numpy(), dim % len(shape))
    assert got.shape == ref.shape and np.array_equal(got, ref)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16, torch.uint8])
@pytest.mark.parametrize("shape,dim", [((8, 4096), -1), ((5, 96), -1), ((3, 4, 160), -1),
                                       ((6, 48), -1), ((2, 112), -1), ((70, 8), 0),
                                       ((3, 100, 12), 1), ((64, 4096), 0)])
def test_pack_bits_aligned_rows_any_values(dtype, shape, dim):
    """Rows of 16-byte multiples packed along the last dim (one word per
    thread) and 4-aligned rows packed along an outer dim (4 rows per
    thread), with and without a partial last word: every nonzero element is
    a 1 bit, whatever its value (uint8 0..255; -0.0 is zero, NaN nonzero)."""
    g = torch.Generator().manual_seed(sum(shape))
    if dtype == torch.uint8:
        x = torch.randint(0, 256, shape, generator=g, dtype=torch.int32)
        x = torch.where(torch.rand(shape, generator=g) < 0.5, torch.zeros_like(x), x).to(torch.uint8)
    else:
        x = torch.randn(shape, generator=g) * 1e-3
        r = torch.rand(shape, generator=g)
        x = torch.where(r < 0.4, torch.zeros_like(x), x)
        x = torch.where((r >= 0.4) & (r < 0.5), torch.full_like(x, -0.0), x)
        x = torch.where((r >= 0.5) & (r < 0.55), torch.full_like(x, float("nan")), x)
        x = x.to(dtype)
    got = snnk.pack_bits(x.to(DEV), dim=dim).cpu().numpy().view(np.uint32)
    ref = ob.pack_axis((x != 0).to(torch.uint8).numpy(), dim % len(shape))
    assert got.shape == ref.shape and np.array_equal(got, ref)


def test_pack_known_answers():
    ones = torch.ones(1, 32, device=DEV)
    assert snnk.pack_bits(ones).cpu().numpy().view(np.uint32)[0, 0] == 0xFFFFFFFF
    x = torch.zeros(1, 70, device=DEV)
    x[0, 45] = 1.0
    w = snnk.pack_bits(x).cpu().numpy().view(np.uint32)
    assert w.tolist() == [[0, 1 << 13, 0]]


def test_spike_ktv_popcount_bit_exact():
    """test_spike_attention.py:142-148: N=70, d=16, k~B(0.1), v~B(0.15)."""
    T, B, H, N, d = 4, 2, 4, 70, 16
    k = _bern((T, B, H, N, d), 0.1, 3).float()
    v = _bern((T, B, H, N, d), 0.15, 4).float()
    out = snnk.spike_ktv_popcount(k.to(DEV), v.to(DEV))
    ref = torch.from_numpy(ob.ktv_counts(k.numpy(), v.numpy()).astype(np.float32))
    assert out.dtype == torch.float32 and torch.equal(out.cpu(), ref)
    # the reference's own oracle in that test: bmm of the fp32 spikes
    assert torch.equal(out.cpu(), k.transpose(-2, -1) @ v)


@pytest.mark.parametrize("algo", ["popc", "mfma", "mfma_f4"])
@pytest.mark.parametrize("signed", [False, True])
@pytest.mark.parametrize("M,N,K", [(5, 7, 33), (64, 48, 64), (130, 70, 70), (300, 257, 1000),
                                   (256, 256, 4096), (129, 384, 128)])
def test_binary_gemm_small_shapes(algo, signed, M, N, K):
    A = _bern((M, K), 0.1, M + K)
    W = _bern((K, N), 0.5, N + K)
    C = snnk.binary_gemm(A.to(DEV, torch.uint8), W.to(DEV, torch.uint8), signed=signed, algo=algo)
    ref = ob.binary_gemm_closed_form(A.numpy(), W.numpy(), signed=signed)
    assert C.dtype == torch.int32 and np.array_equal(C.cpu().numpy(), ref)


@pytest.mark.parametrize("algo", ["popc", "mfma", "mfma_f4"])
def test_binary_gemm_batched_and_float_out(algo):
    A = _bern((3, 200, 150), 0.2, 9)
    W = _bern((3, 150, 140), 0.5, 10)
    Ap = snnk.pack_bits(A.to(DEV).float(), dim=-1)
    Wp = snnk.pack_bits(W.to(DEV).float(), dim=-2)
    C = snnk.binary_gemm(Ap, Wp, a_packed=True, w_packed=True, K=150, algo=algo,
                         out_dtype=torch.float32)
    ref = np.stack([ob.binary_gemm_closed_form(A[i].numpy(), W[i].numpy()) for i in range(3)])
    assert torch.equal(C.cpu(), torch.from_numpy(ref.astype(np.float32)))


def test_garbage_bits_past_K_are_ignored():
    A = _bern((128, 40), 0.5, 1)
    W = _bern((40, 128), 0.5, 2)
    Ap = snnk.pack_bits(A.to(DEV).float())
    Wp = snnk.pack_bits(W.to(DEV).float(), dim=-2)
    Ap[:, 1] |= torch.tensor(-256, dtype=torch.int32, device=DEV)   # set bits 8..31 (k >= 40)
    Wp[:, 1] |= torch.tensor(-256, dtype=torch.int32, device=DEV)
    ref = ob.binary_gemm_closed_form(A.numpy(), W.numpy())
    for algo in ("popc", "mfma", "mfma_f4"):
        C = snnk.binary_gemm(Ap, Wp, a_packed=True, w_packed=True, K=40, algo=algo)
        assert np.array_equal(C.cpu().numpy(), ref)


@pytest.mark.parametrize("signed", [False, True])
def test_binary_gemm_baseline_config(signed):
    """M=8192, K=4096, N=4096, A~B(0.1), W~B(0.5), packed along K."""
    M, K, N = 8192, 4096, 4096
    A = _bern((M, K), 0.1, 0)
    W = _bern((K, N), 0.5, 1)
    Ad, Wd = A.to(DEV, torch.uint8), W.to(DEV, torch.uint8)
    Ap, Wp = snnk.pack_bits(Ad), snnk.pack_bits(Wd, dim=-2)
    # packing itself against the oracle on the whole operands
    A_np, W_np = A.numpy().astype(np.uint8), W.numpy().astype(np.uint8)
    Ap_ref, Wp_ref = ob.pack_rows(A_np), ob.pack_rows(W_np.T)
    assert np.array_equal(Ap.cpu().numpy().view(np.uint32), Ap_ref)
    assert np.array_equal(Wp.cpu().numpy().view(np.uint32), Wp_ref)
    C = snnk.binary_gemm(Ap, Wp, a_packed=True, w_packed=True, K=K, signed=signed, algo="mfma")
    C_popc = snnk.binary_gemm(Ap, Wp, a_packed=True, w_packed=True, K=K, signed=signed,
                              algo="popc")
    assert torch.equal(C, C_popc)
    C_f4 = snnk.binary_gemm(Ap, Wp, a_packed=True, w_packed=True, K=K, signed=signed,
                            algo="mfma_f4")
    assert torch.equal(C_f4, C_popc)
    Cn = C.cpu().numpy().astype(np.int64)
    # exact row sample (first, middle and last rows) against the C oracle
    for m0 in (0, 4064, M - 32):
        ref = clib.popcount_gemm(Ap_ref, Wp_ref, signed=signed, rows=(m0, m0 + 32))
        assert np.array_equal(Cn[m0:m0 + 32], ref)
    # checksums over every output: row sums and column sums in int64
    Wv = W_np.astype(np.int64) * (2 if signed else 1) - (1 if signed else 0)
    Ai = A_np.astype(np.int64)
    assert np.array_equal(Cn.sum(1), Ai @ Wv.sum(1))
    assert np.array_equal(Cn.sum(0), Ai.sum(0) @ Wv)
