"""Spike attention operators (mirror of snn_compiler/kernels/attention.py).

* ``spike_ktv_popcount``: bit-exact K^T V through bit packing along the
  token axis and a popcount GEMM (reference attention.py:245-258).
* ``spike_av_lif``: the reference's fused ``(q @ kv) * scale -> LIF``
  (attention.py:107-137) in one HIP kernel (csrc/attention_linear.hip): the
  product runs on bf16 MFMA with kv split into exact bf16 parts, the
  membrane stays in registers across T and ``q @ kv`` is never stored.
* ``spike_attention``: the attention core straight from Q, K, V spikes: the
  quadratic order (Q K^T) V on int8 MFMA up to 64 tokens and 64 dims per
  head (csrc/attention.hip), the linear order Q (K^T V) on bf16 MFMA beyond
  (csrc/attention_linear.hip; equal counts over the integers), then the LIF,
  with the integer counts optionally returned.
* ``spike_self_attention``: the whole SSA block on tokens [T, B, N, D]:
  fused QKV Linear + BN + LIF, the attention core, and the output Linear + BN.
"""
from __future__ import annotations

import torch

from .. import _abi
from .binary import pack_bits, _gemm_packed
from .linear import linear_bias_lif_act, linear_preact_act, linear_bias_lif, linear_preact
from .neurons import if_lif, launch_lif, THR_SCALAR

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


def spike_ktv(k: torch.Tensor, v: torch.Tensor, *, algo: str = "auto") -> torch.Tensor:
    """K^T V for spikes ``[T, B, heads, N, d]`` -> fp32 ``[T, B, heads, d, d]``.

    Reference: snn_compiler/kernels/attention.py:177-187 (an fp32 dot product
    over the tokens).  Here an exact binary GEMM of the spikes packed along
    the token axis (nonzero counts as 1): the MFMA kernels where the shape
    allows, the VALU popcount kernel otherwise.
    """
    T, B, H, N, D = k.shape
    assert v.shape == k.shape, f"k {tuple(k.shape)} and v {tuple(v.shape)} must match"
    TBH = T * B * H
    kp = _pack_N(k.reshape(TBH, N, D))
    vp = _pack_N(v.reshape(TBH, N, D))
    out = _gemm_packed(kp, vp, N, signed=False, algo=algo, out_dtype=torch.float32)
    return out.reshape(T, B, H, D, D)


def _lif_scale(tau, decay, decay_input, scale):
    dec = (1.0 if tau is None else 1.0 - 1.0 / tau) if decay is None else float(decay)
    base = (1.0 / tau) if (decay_input and tau is not None) else 1.0
    return dec, base * float(scale)


def spike_av_lif(q, kv, *, scale, tau=2.0, decay=None, decay_input=True, v_threshold=0.5,
                 v_reset=0.0, soft_reset=False):
    """``(q @ kv) * scale -> LIF`` with q [T,B,heads,N,d] spikes and kv
    [T,B,heads,d,d] counts; returns spikes like q (same dtype).

    Reference: snn_compiler/kernels/attention.py:107-137 (the scale is folded
    into the LIF input scale, as there).  One HIP kernel: q @ kv on bf16 MFMA
    with kv as three bf16 parts whose sum is exact, fp32 accumulation (exact
    for integer kv), the LIF in registers across T.  q must hold spikes
    (0/1); kv may be fp32 or int32 (other dtypes are converted to fp32).
    """
    assert q.is_cuda and kv.is_cuda and q.device == kv.device
    assert q.ndim == 5 and kv.ndim == 5, "q [T,B,H,N,d] and kv [T,B,H,d,d]"
    T, B, H, N, D = q.shape
    assert tuple(kv.shape) == (T, B, H, D, D), \
        f"kv {tuple(kv.shape)} must be [T,B,H,d,d] = {(T, B, H, D, D)}"
    assert q.dtype in (torch.float32, torch.bfloat16, torch.float16), q.dtype
    if kv.dtype not in (torch.float32, torch.int32):
        kv = kv.float()
    qc, kvc = q.contiguous(), kv.contiguous()
    dec, in_scale = _lif_scale(tau, decay, decay_input, scale)
    out = torch.empty_like(qc)
    if out.numel() == 0:
        return out
    with torch.cuda.device(q.device):
        _abi.call("snnk_spike_av_lif", qc.data_ptr(), _abi.dtype_code(qc.dtype), kvc.data_ptr(),
                  _abi.dtype_code(kvc.dtype), out.data_ptr(), T, B * H, N, D, float(dec),
                  float(in_scale), float(v_threshold), float(v_reset), 1 if soft_reset else 0,
                  _abi.stream(q.device))
    return out


def _s_counts(q, k, *, B: int, N: int, heads: int) -> torch.Tensor:
    """Integer Q K^T [T, B, heads, N, N] from spike column slices [T, B*N, heads*d],
    through the bit-packed binary GEMM (the linear-order core forms no S)."""
    T = q.shape[0]
    d = q.shape[2] // heads

    def heads_major(s):  # [T, B*N, H*d] -> [T, B, H, N, d]
        return s.reshape(T, B, N, heads, d).permute(0, 1, 3, 2, 4)

    qp = pack_bits(heads_major(q), dim=-1)   # [T, B, H, N, words]
    kp = pack_bits(heads_major(k), dim=-1)
    return _gemm_packed(qp, kp, d, signed=False, algo="auto", out_dtype=torch.int32)


def spike_attention(q, k, v, *, B: int, N: int, heads: int, scale: float, tau: float = 2.0,
                    decay: float | None = None, decay_input: bool = True,
                    v_threshold: float = 0.5, v_reset: float = 0.0, soft_reset: bool = False,
                    out: torch.Tensor | None = None, return_counts: bool = False):
    """Attention core: the LIF of ``scale * (Q K^T) V`` per (batch, head).

    q, k, v: bf16 spikes ``[T, B*N, heads*d]`` (any row stride, e.g. column
    slices of one QKV projection output); d % 8 == 0 and d <= 128.  Returns
    spikes ``[T, B*N, heads*d]`` bf16, and with ``return_counts`` also int32
    ``S = Q K^T`` [T,B,heads,N,N] and ``O = (Q K^T) V`` [T,B,heads,N,d].
    Up to 64 tokens and 64 dims the core runs in the quadratic order on int8
    MFMA; beyond, in the linear order Q (K^T V) (equal integers), and S then
    comes from the bit-packed binary GEMM.
    """
    for t in (q, k, v):
        assert t.is_cuda and t.dtype == torch.bfloat16 and t.ndim == 3 and t.stride(2) == 1
    T, R, HD = q.shape
    assert R == B * N and HD % heads == 0 and k.shape == q.shape and v.shape == q.shape
    d = HD // heads
    dec, in_scale = _lif_scale(tau, decay, decay_input, scale)
    if out is None:
        out = torch.empty(T, R, HD, device=q.device, dtype=torch.bfloat16)
    linear = N > 64 or d > 64
    S = O = None
    if return_counts:
        if not linear:
            S = torch.empty(T, B, heads, N, N, device=q.device, dtype=torch.int32)
        O = torch.empty(T, B, heads, N, d, device=q.device, dtype=torch.int32)
    with torch.cuda.device(q.device):
        _abi.call("snnk_spike_attention", q.data_ptr(), k.data_ptr(), v.data_ptr(),
                  q.stride(1), k.stride(1), v.stride(1), q.stride(0), k.stride(0), v.stride(0),
                  out.data_ptr(), out.stride(1), out.stride(0), _abi.ptr(S), _abi.ptr(O),
                  T, B, heads, N, d, float(dec), float(in_scale), float(v_threshold),
                  float(v_reset), 1 if soft_reset else 0, _abi.stream(q.device))
        if return_counts and linear:
            S = _s_counts(q, k, B=B, N=N, heads=heads)
    return (out, S, O) if return_counts else out


def spike_attention_packed(q, k, v, *, B: int, N: int, heads: int, d: int, in_head_bits: int,
                           out_head_words: int, scale: float, tau: float = 2.0,
                           decay: float | None = None, decay_input: bool = True,
                           v_threshold: float = 0.5, v_reset: float = 0.0,
                           soft_reset: bool = False, out: torch.Tensor | None = None,
                           return_counts: bool = False):
    """:func:`spike_attention` on packed spikes.

    q, k, v: int32 words ``[T, B*N, W]`` (any row stride, e.g. column slices
    of one packed QKV projection output); head h starts at bit
    ``h*in_head_bits`` of a row (LSB first; ``in_head_bits = d`` for the rows
    a packed projection writes).  Returns packed spikes
    ``[T, B*N, heads*out_head_words]``, head h on words ``h*out_head_words ..``
    with its bits past d zero (and with ``return_counts`` the int32 S and O).
    N <= 64, d <= 64, d % 8 == 0.
    """
    for t in (q, k, v):
        assert t.is_cuda and t.dtype == torch.int32 and t.ndim == 3 and t.stride(2) == 1
    T, R, _ = q.shape
    assert R == B * N and k.shape[:2] == q.shape[:2] and v.shape[:2] == q.shape[:2]
    dec, in_scale = _lif_scale(tau, decay, decay_input, scale)
    if out is None:
        out = torch.empty(T, R, heads * out_head_words, device=q.device, dtype=torch.int32)
    S = O = None
    if return_counts:
        S = torch.empty(T, B, heads, N, N, device=q.device, dtype=torch.int32)
        O = torch.empty(T, B, heads, N, d, device=q.device, dtype=torch.int32)
    with torch.cuda.device(q.device):
        _abi.call("snnk_spike_attention_packed", q.data_ptr(), k.data_ptr(), v.data_ptr(),
                  q.stride(1), k.stride(1), v.stride(1), q.stride(0), k.stride(0), v.stride(0),
                  in_head_bits, out.data_ptr(), out.stride(1), out.stride(0), out_head_words,
                  _abi.ptr(S), _abi.ptr(O), T, B, heads, N, d, float(dec), float(in_scale),
                  float(v_threshold), float(v_reset), 1 if soft_reset else 0,
                  _abi.stream(q.device))
    return (out, S, O) if return_counts else out


def pad_heads_rows(w: torch.Tensor, b: torch.Tensor | None, heads: int, slot: int):
    """Rows of a [heads*d, K] projection (and its bias) spread to ``slot`` rows
    per head, the rows past d zero: its spikes come out with every head
    starting on a 32-bit word of a packed row (and never firing past d)."""
    d = w.shape[0] // heads
    wp = torch.zeros(heads, slot, w.shape[1], device=w.device, dtype=w.dtype)
    wp[:, :d] = w.view(heads, d, -1)
    bp = None
    if b is not None:
        bp = torch.zeros(heads, slot, device=b.device, dtype=b.dtype)
        bp[:, :d] = b.view(heads, d)
        bp = bp.reshape(-1).contiguous()
    return wp.reshape(heads * slot, -1).contiguous(), bp


def pad_heads_cols(w: torch.Tensor, heads: int, slot: int) -> torch.Tensor:
    """Columns of a [N, heads*d] projection spread to ``slot`` columns per
    head (zeros past d), to read head-padded packed spikes."""
    d = w.shape[1] // heads
    wp = torch.zeros(w.shape[0], heads, slot, device=w.device, dtype=w.dtype)
    wp[:, :, :d] = w.view(w.shape[0], heads, d)
    return wp.reshape(w.shape[0], heads * slot).contiguous()


def spike_self_attention(tokens, w_qkv, b_qkv, w_proj, b_proj, *, heads: int,
                         scale: float = 0.125, tau: float = 2.0, vth_qkv: float = 1.0,
                         vth_attn: float = 0.5, input_vth: float | None = None,
                         return_intermediates: bool = False):
    """Spikformer-style SSA block on tokens ``[T, B, N, D]``.

    w_qkv: bf16 [3D, D] (q, k, v Linear weights stacked, BN folded), b_qkv fp32
    [3D]; w_proj bf16 [D, D], b_proj fp32 [D].  Q, K, V = LIF(x W^T + b)
    (threshold vth_qkv), attention spikes = LIF(scale * (Q K^T) V) per head
    (threshold vth_attn), output = attn W_proj^T + b_proj (fp32).
    ``input_vth`` applies the reference block's input LIF first
    (snn_compiler/nn/attention.py:138).
    """
    T, B, N, D = tokens.shape
    x = tokens.reshape(T, B * N, D)
    if input_vth is not None:
        x = if_lif(x.contiguous(), neuron="lif", tau=tau, v_threshold=input_vth,
                   spike_dtype=torch.bfloat16)
    x = x.to(torch.bfloat16).contiguous()
    dec = 1.0 - 1.0 / tau
    qkv = linear_bias_lif(x, w_qkv, b_qkv, decay=dec, in_scale=1.0 / tau, v_threshold=vth_qkv)
    q, k, v = qkv[..., :D], qkv[..., D:2 * D], qkv[..., 2 * D:]
    res = spike_attention(q, k, v, B=B, N=N, heads=heads, scale=scale, tau=tau,
                          v_threshold=vth_attn, return_counts=return_intermediates)
    attn = res[0] if return_intermediates else res
    out = linear_preact(attn, w_proj, b_proj).view(T, B, N, D)
    if return_intermediates:
        return out, dict(qkv=qkv, attn=attn, S=res[1], O=res[2])
    return out


def prepare_ssa_packed(w_qkv, b_qkv, w_proj, *, heads: int) -> dict:
    """Weights of :func:`spike_self_attention` laid out for the packed block:
    the QKV projection as is (its packed output holds the heads back to back,
    ``d`` bits each), the output projection's input columns padded to whole
    32-bit words per head, the layout in which the packed attention core
    writes its spikes.  Built once per set of weights."""
    D = w_proj.shape[0]
    assert w_qkv.shape == (3 * D, D) and D % heads == 0 and D % 32 == 0
    d = D // heads
    slot = 32 * ((d + 31) // 32)
    return dict(w_qkv=w_qkv.to(torch.bfloat16).contiguous(),
                b_qkv=None if b_qkv is None else b_qkv.float().contiguous(),
                w_proj=pad_heads_cols(w_proj, heads, slot).to(torch.bfloat16).contiguous(),
                heads=heads, d=d, slot=slot, D=D)


def spike_self_attention_packed(x_words, prep: dict, b_proj, *, B: int, N: int,
                                scale: float = 0.125, tau: float = 2.0, vth_qkv: float = 1.0,
                                vth_attn: float = 0.5, return_intermediates: bool = False):
    """:func:`spike_self_attention` with the spikes packed end to end.

    x_words: int32 ``[T, B*N, D // 32]`` packed input spikes (bit c%32 of word
    c//32, as the LIF kernel writes them); ``prep`` from
    :func:`prepare_ssa_packed`.  Q, K and V leave the projection as packed
    words ``[T, B*N, 3D // 32]``, the attention core reads them and writes its
    spikes with every head on whole words, and the output projection reads
    those: output fp32 ``[T, B, N, D]``, the same spikes (and the output up to
    fp32 summation order) as the bf16 block.
    """
    T = x_words.shape[0]
    H, hw, D, d = prep["heads"], prep["slot"] // 32, prep["D"], prep["d"]
    dec = 1.0 - 1.0 / tau
    qkv = linear_bias_lif_act(x_words, prep["w_qkv"], prep["b_qkv"], decay=dec,
                              in_scale=1.0 / tau, v_threshold=vth_qkv, out_bits=True)
    Dw = D // 32
    q, k, v = qkv[..., :Dw], qkv[..., Dw:2 * Dw], qkv[..., 2 * Dw:]
    res = spike_attention_packed(q, k, v, B=B, N=N, heads=H, d=d, in_head_bits=d,
                                 out_head_words=hw, scale=scale, tau=tau, v_threshold=vth_attn,
                                 return_counts=return_intermediates)
    attn = res[0] if return_intermediates else res
    out = linear_preact_act(attn, prep["w_proj"], b_proj).view(T, B, N, D)
    if return_intermediates:
        return out, dict(qkv=qkv, attn=attn, S=res[1], O=res[2])
    return out
