"""Bit packing and binary (popcount) GEMM oracle (numpy) -- test infrastructure only.

Restates:
  bitpack_N              snn_compiler/explore/attention/phase6b_bitpack.py:35-46
                         (bit n%32 of word n//32, LSB first, zero-padded tail)
  _pack_N / _pack_N_kernel  snn_compiler/kernels/attention.py:195-214,236-242
  _ktv_popcount_kernel   snn_compiler/kernels/attention.py:217-233
                         C[i,j] = sum_w popc(Kp[i,w] & Vp[j,w])
  spike_ktv_popcount     snn_compiler/kernels/attention.py:245-258

The general binary GEMM C[m,n] = popcount(A_m AND W_n) (and its signed form
2*popc(A&W+) - popc(A)) is BASELINE's generalisation of the K^T V popcount.

Pins (tests/test_oracle_bits.py): known answers (all-ones word, single bits,
ragged tail); the C restatement (bit-equal); brute-force triple loop on tiny
shapes; the closed form C = A01 @ W01 in int64; the signed identity
A.(2W-1) = 2 A.W - rowsum(A).
"""
from __future__ import annotations

import numpy as np


def pack_rows(x01: np.ndarray) -> np.ndarray:
    """[..., K] {0,1} -> [..., ceil(K/32)] uint32, bit k%32 of word k//32."""
    x = np.asarray(x01)
    K = x.shape[-1]
    W = (K + 31) // 32
    pad = W * 32 - K
    xb = (x != 0).astype(np.uint64)
    if pad:
        xb = np.concatenate([xb, np.zeros(x.shape[:-1] + (pad,), np.uint64)], axis=-1)
    xb = xb.reshape(x.shape[:-1] + (W, 32))
    shifts = np.arange(32, dtype=np.uint64)
    return (xb << shifts).sum(-1).astype(np.uint32)


def pack_axis(x01: np.ndarray, axis: int) -> np.ndarray:
    """Pack along ``axis`` and move the word axis last.

    For k,v [TBH, N, D] and axis=1 this is bitpack_N's [TBH, D, W] output.
    """
    x = np.moveaxis(np.asarray(x01), axis, -1)
    return pack_rows(x)


def unpack_rows(words: np.ndarray, K: int) -> np.ndarray:
    """Inverse of pack_rows: [..., W] uint32 -> [..., K] uint8."""
    w = np.asarray(words, dtype=np.uint32)
    bits = ((w[..., None] >> np.arange(32, dtype=np.uint32)) & 1).astype(np.uint8)
    return bits.reshape(w.shape[:-1] + (w.shape[-1] * 32,))[..., :K]


def popcount_gemm(A_packed: np.ndarray, B_packed: np.ndarray, *, signed=False) -> np.ndarray:
    """A [M, W], B [N, W] uint32 -> int32 [M, N] via bitwise AND + popcount."""
    A = np.asarray(A_packed, dtype=np.uint32)
    B = np.asarray(B_packed, dtype=np.uint32)
    out = np.zeros((A.shape[0], B.shape[0]), np.int64)
    for w in range(A.shape[1]):
        out += np.bitwise_count(A[:, w][:, None] & B[:, w][None, :])
    if signed:
        rowpop = np.bitwise_count(A).astype(np.int64).sum(1)
        out = 2 * out - rowpop[:, None]
    return out.astype(np.int32)


def binary_gemm_closed_form(A01: np.ndarray, W01_kn: np.ndarray, *, signed=False) -> np.ndarray:
    """C = A01 @ W01 ([M,K] x [K,N]) in int64 arithmetic; signed uses 2W-1."""
    A = np.asarray(A01, dtype=np.int64)
    W = np.asarray(W01_kn, dtype=np.int64)
    if signed:
        W = 2 * W - 1
    return (A @ W).astype(np.int32)


def ktv_counts(k01: np.ndarray, v01: np.ndarray) -> np.ndarray:
    """K^T V for [..., N, d] spikes (int64), the exact value the reference's
    ``k.transpose(-2,-1) @ v`` bmm and spike_ktv_popcount both produce."""
    k = np.asarray(k01, dtype=np.int64)
    v = np.asarray(v01, dtype=np.int64)
    return np.swapaxes(k, -1, -2) @ v
