"""Spike attention operators (mirror of snn_compiler/kernels/attention.py).

``spike_ktv_popcount``: bit-exact K^T V of binary spikes through bit packing
along the token axis and a popcount GEMM (reference
snn_compiler/kernels/attention.py:245-258).
"""
from __future__ import annotations

import torch

from .binary import pack_bits, _gemm_packed

# popcount is native on gfx950 (v_bcnt_u32_b32); kept for API parity with
# snn_compiler/kernels/attention.py:26-36.
HAS_POPC = True


def _pack_N(xf: torch.Tensor) -> torch.Tensor:
    """[TBH, N, D] {0,1} -> [TBH, D, ceil(N/32)] int32 (token axis packed).

    Reference: snn_compiler/kernels/attention.py:236-242.
    """
    return pack_bits(xf, dim=1)


def spike_ktv_popcount(k: torch.Tensor, v: torch.Tensor) -> torch.Tensor:
    """K^T V for spikes ``[T, B, heads, N, d]`` -> fp32 ``[T, B, heads, d, d]``.

    Reference: snn_compiler/kernels/attention.py:245-258 (fp32 counts).
    """
    T, B, H, N, D = k.shape
    assert v.shape == k.shape, f"k {tuple(k.shape)} and v {tuple(v.shape)} must match"
    TBH = T * B * H
    kp = _pack_N(k.reshape(TBH, N, D))
    vp = _pack_N(v.reshape(TBH, N, D))
    out = _gemm_packed(kp, vp, N, signed=False, algo="popc", out_dtype=torch.float32)
    return out.reshape(T, B, H, D, D)
