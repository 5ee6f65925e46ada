"""Pins for oracle/bits.py (bit packing, popcount / binary GEMM)."""
import numpy as np
import pytest

from oracle import bits, clib


def test_pack_known_answers():
    assert bits.pack_rows(np.ones((1, 32), np.uint8))[0, 0] == 0xFFFFFFFF
    for k in (0, 1, 7, 31, 32, 45, 69):
        x = np.zeros((1, 70), np.uint8)
        x[0, k] = 1
        w = bits.pack_rows(x)
        assert w.shape == (1, 3)
        assert w[0, k // 32] == (1 << (k % 32)) and w.sum() == (1 << (k % 32))
    # tail of a ragged row (K=70) stays zero
    assert bits.pack_rows(np.ones((1, 70), np.uint8))[0, 2] == 0b111111


def test_pack_matches_c_and_roundtrips():
    rng = np.random.default_rng(0)
    x = (rng.random((37, 101)) < 0.3).astype(np.uint8)
    w = bits.pack_rows(x)
    assert np.array_equal(w, clib.pack_bits(x))
    assert np.array_equal(bits.unpack_rows(w, 101), x)


def test_pack_axis_is_bitpack_N_layout():
    """[TBH, N, D] packed along N -> [TBH, D, W] (phase6b_bitpack.py:35-46)."""
    rng = np.random.default_rng(1)
    k = (rng.random((3, 70, 5)) < 0.2).astype(np.uint8)
    p = bits.pack_axis(k, 1)
    assert p.shape == (3, 5, 3)
    for b in range(3):
        for d in range(5):
            for n in range(70):
                assert ((int(p[b, d, n // 32]) >> (n % 32)) & 1) == k[b, n, d]


@pytest.mark.parametrize("M,N,K", [(5, 7, 33), (16, 9, 64), (3, 4, 70)])
def test_popcount_gemm_bruteforce(M, N, K):
    rng = np.random.default_rng(M * N + K)
    A = (rng.random((M, K)) < 0.3).astype(np.uint8)
    Wkn = (rng.random((K, N)) < 0.5).astype(np.uint8)
    brute = np.zeros((M, N), np.int64)
    for m in range(M):
        for n in range(N):
            for k in range(K):
                brute[m, n] += int(A[m, k]) * int(Wkn[k, n])
    Ap, Bp = bits.pack_rows(A), bits.pack_rows(Wkn.T)
    assert np.array_equal(bits.popcount_gemm(Ap, Bp), brute)
    assert np.array_equal(bits.binary_gemm_closed_form(A, Wkn), brute)
    assert np.array_equal(clib.popcount_gemm(Ap, Bp), brute)
    signed = brute * 2 - A.sum(1, dtype=np.int64)[:, None]
    assert np.array_equal(bits.popcount_gemm(Ap, Bp, signed=True), signed)
    assert np.array_equal(bits.binary_gemm_closed_form(A, Wkn, signed=True), signed)
    assert np.array_equal(clib.popcount_gemm(Ap, Bp, signed=True), signed)


def test_popcount_gemm_large_vs_closed_form():
    rng = np.random.default_rng(5)
    A = (rng.random((128, 1000)) < 0.1).astype(np.uint8)
    Wkn = (rng.random((1000, 96)) < 0.5).astype(np.uint8)
    ref = bits.binary_gemm_closed_form(A, Wkn)
    Ap, Bp = bits.pack_rows(A), bits.pack_rows(Wkn.T)
    assert np.array_equal(clib.popcount_gemm(Ap, Bp), ref)
    assert np.array_equal(clib.popcount_gemm(Ap, Bp, rows=(10, 20)), ref[10:20])


def test_ktv_counts_is_kT_v():
    rng = np.random.default_rng(2)
    k = (rng.random((2, 70, 16)) < 0.1).astype(np.uint8)
    v = (rng.random((2, 70, 16)) < 0.15).astype(np.uint8)
    kv = bits.ktv_counts(k, v)
    kp, vp = bits.pack_axis(k, 1), bits.pack_axis(v, 1)
    for b in range(2):
        assert np.array_equal(bits.popcount_gemm(kp[b], vp[b]), kv[b])


def test_planted_mistake_msb_first_is_caught():
    x = np.zeros((1, 32), np.uint8)
    x[0, 0] = 1
    msb_first = np.uint32(1 << 31)
    assert bits.pack_rows(x)[0, 0] != msb_first
