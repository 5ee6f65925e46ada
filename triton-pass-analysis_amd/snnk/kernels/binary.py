"""Bit packing and binary (popcount) GEMM on bit-packed spikes.

``pack_bits`` generalises the reference's token-axis packer
(snn_compiler/kernels/attention.py:195-214,236-242; bit n%32 of word n//32,
LSB first, int32 words).  ``binary_gemm`` generalises its popcount K^T V
(snn_compiler/kernels/attention.py:217-233,245-258) to any [M,K] x [K,N]
binary product, with int8- and fp4-MFMA algorithms for large shapes and the signed
{-1,+1}-weight form ``2*popc(A & W+) - popc(A)``.
"""
from __future__ import annotations

import math

import torch

from .. import _abi

_ALGOS = {"auto": _abi.BGEMM_AUTO, "popc": _abi.BGEMM_POPC, "mfma": _abi.BGEMM_MFMA_I8,
          "mfma_f4": _abi.BGEMM_MFMA_F4}


def packed_words(K: int) -> int:
    return (K + 31) // 32


def pack_bits(x01: torch.Tensor, dim: int = -1) -> torch.Tensor:
    """Pack a {0,1} tensor along ``dim`` into int32 words (word axis last).

    Output shape is ``x.shape`` without ``dim``, followed by ``ceil(K/32)``;
    element k lands in bit k%32 of word k//32; bits past K are zero.
    Nonzero elements count as 1.
    """
    assert x01.is_cuda, "pack_bits needs a GPU tensor"
    assert x01.dtype in (torch.float32, torch.bfloat16, torch.float16, torch.uint8), x01.dtype
    x = x01.contiguous()
    d = dim % x.ndim
    K = x.shape[d]
    batch = math.prod(x.shape[:d])
    rows = math.prod(x.shape[d + 1:])
    out_shape = tuple(x.shape[:d]) + tuple(x.shape[d + 1:]) + (packed_words(K),)
    out = torch.empty(out_shape, device=x.device, dtype=torch.int32)
    if out.numel() == 0:
        return out
    with torch.cuda.device(x.device):
        _abi.call("snnk_pack_bits", x.data_ptr(), _abi.dtype_code(x.dtype), out.data_ptr(),
                  batch, rows, K, K * rows, 1, rows, _abi.stream(x.device))
    return out


def _gemm_packed(Ap, Bp, K, *, signed, algo, out_dtype, out=None):
    """Ap [..., M, KW], Bp [..., N, KW] int32 words -> [..., M, N]."""
    assert Ap.is_cuda and Bp.is_cuda and Ap.device == Bp.device
    assert Ap.dtype == torch.int32 and Bp.dtype == torch.int32
    assert Ap.shape[:-2] == Bp.shape[:-2], "batch dims must match"
    assert Ap.shape[-1] >= packed_words(K) and Bp.shape[-1] >= packed_words(K)
    assert out_dtype in (torch.int32, torch.float32)
    Ap, Bp = Ap.contiguous(), Bp.contiguous()
    batch = math.prod(Ap.shape[:-2])
    M, lda = Ap.shape[-2], Ap.shape[-1]
    N, ldb = Bp.shape[-2], Bp.shape[-1]
    shape = tuple(Ap.shape[:-2]) + (M, N)
    if out is None:
        C = torch.empty(shape, device=Ap.device, dtype=out_dtype)
    else:
        assert out.shape == shape and out.dtype == out_dtype and out.is_contiguous() \
            and out.device == Ap.device, "out must be a contiguous tensor of the result shape"
        C = out
    if C.numel() == 0:
        return C
    with torch.cuda.device(Ap.device):
        _abi.call("snnk_binary_gemm", Ap.data_ptr(), Bp.data_ptr(), C.data_ptr(),
                  _abi.dtype_code(out_dtype), batch, M, N, K, lda, ldb, N,
                  M * lda, N * ldb, M * N, 1 if signed else 0, _ALGOS[algo],
                  _abi.stream(Ap.device))
    return C


def binary_gemm(A, W, *, signed: bool = False, a_packed: bool = False,
                w_packed: bool = False, K: int | None = None, algo: str = "auto",
                out_dtype: torch.dtype = torch.int32, out: torch.Tensor | None = None
                ) -> torch.Tensor:
    """Exact binary product ``C = A01 @ W01`` (counts), batched over leading dims.

    A: ``[..., M, K]`` {0,1} (fp32/bf16/fp16/uint8), or int32 words
       ``[..., M, ceil(K/32)]`` with ``a_packed=True``.
    W: ``[..., K, N]`` {0,1}, or int32 words ``[..., N, ceil(K/32)]`` (each
       output column packed along K) with ``w_packed=True``.
    signed: weights are -1 where W is 0 and +1 where W is 1:
       ``C = 2*popc(A & W) - popc(A)``.
    algo: 'auto' | 'popc' (VALU popcount) | 'mfma' (int8 MFMA) | 'mfma_f4'
       (MX fp4 MFMA, bits as e2m1 0/1.0, exact fp32 counts).
    out: optional preallocated contiguous result tensor.
    """
    if algo not in _ALGOS:
        raise ValueError(f"unknown algo {algo!r}")
    if not a_packed:
        K_a = A.shape[-1]
    if not w_packed:
        K_w = W.shape[-2]
    if K is None:
        if not a_packed:
            K = K_a
        elif not w_packed:
            K = K_w
        else:
            raise ValueError("K is required when both operands are packed")
    if not a_packed:
        assert K_a == K, f"A has K={K_a}, expected {K}"
        A = pack_bits(A, dim=-1)
    if not w_packed:
        assert K_w == K, f"W has K={K_w}, expected {K}"
        W = pack_bits(W, dim=-2)
    return _gemm_packed(A, W, K, signed=signed, algo=algo, out_dtype=out_dtype, out=out)
