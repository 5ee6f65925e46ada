"""Multi-step IF/LIF neuron operators (HIP, gfx950).

Mirrors ``snn_compiler/kernels/neurons.py``: same entry-point name, keyword
arguments, shape conventions and exception types.  Tensors are ``[T, B, ...]``
with the shape always labelled NCHW; ``layout='NHWC'`` only says the memory is
channels-last, which changes how the channel of a flat index is found.

The membrane recurrence itself runs in ``snnk_lif_forward`` (csrc/lif.hip).
"""
from __future__ import annotations

import math

import torch

from .. import _abi

NEURON_IF = 0
NEURON_LIF = 1

RESET_SOFT = 0
RESET_HARD = 1

THR_SCALAR = _abi.THR_SCALAR
THR_PER_CHANNEL = _abi.THR_PER_CHANNEL
THR_PER_NEURON = _abi.THR_PER_NEURON


def neuron_params(neuron: str, tau: float, decay, decay_input: bool):
    """(decay_factor, input_scale) of a neuron kind.

    Follows snn_compiler/kernels/neurons.py:349-356: IF has decay 1 (or the
    override) and input scale 1; LIF has decay 1-1/tau (or the override) and
    input scale 1/tau when ``decay_input`` else 1.
    """
    if neuron == "if":
        return (1.0 if decay is None else float(decay)), 1.0
    if neuron == "lif":
        df = (1.0 - 1.0 / tau) if decay is None else float(decay)
        sc = (1.0 / tau) if decay_input else 1.0
        return df, sc
    raise ValueError(f"unknown neuron: {neuron!r}")


def infer_C_HW(x_seq: torch.Tensor):
    """Channel count and spatial size of a ``[T, B, ...]`` tensor.

    Same rule as snn_compiler/kernels/neurons.py:295-308.
    """
    if x_seq.ndim == 5:
        return x_seq.shape[2], x_seq.shape[3] * x_seq.shape[4]
    if x_seq.ndim == 4:
        return x_seq.shape[2], x_seq.shape[3]
    if x_seq.ndim == 3:
        return x_seq.shape[-1], 1
    return 1, 1


def resolve_threshold(v_threshold, C: int, NCL: int):
    """(thr_mode, tensor_or_None, scalar) from a float or a [C]/[NCL] tensor.

    Follows snn_compiler/kernels/neurons.py:267-292: a tensor must be fp32,
    contiguous and on the GPU; its size picks per-channel (== C, checked
    first) or per-neuron (== NCL), anything else is a ValueError.
    """
    if isinstance(v_threshold, (int, float)):
        return THR_SCALAR, None, float(v_threshold)
    assert isinstance(v_threshold, torch.Tensor), type(v_threshold)
    assert (v_threshold.is_cuda and v_threshold.dtype == torch.float32
            and v_threshold.is_contiguous())
    if v_threshold.numel() == C:
        return THR_PER_CHANNEL, v_threshold, 0.0
    if v_threshold.numel() == NCL:
        return THR_PER_NEURON, v_threshold, 0.0
    raise ValueError(
        f"v_threshold shape {tuple(v_threshold.shape)} matches neither C={C} "
        f"nor NCL={NCL}")


def check_flat(x: torch.Tensor, layout: str, what: str = "x_seq") -> None:
    """The kernels index memory as ``t*NCL + i``: each time step must be one
    dense block of NCL elements, in NCHW order or (layout='NHWC') in
    channels-last order."""
    assert x.is_cuda, f"{what} must be a GPU tensor"
    if x.is_contiguous():
        return
    assert layout == "NHWC", \
        f"non-contiguous {what} requires layout='NHWC', got {layout}"
    ok = x.ndim == 5 and x.stride(0) == math.prod(x.shape[1:]) and \
        x[0].is_contiguous(memory_format=torch.channels_last)
    ok = ok or (x.ndim == 4 and x.stride(0) == math.prod(x.shape[1:])
                and x.permute(0, 1, 3, 2).is_contiguous())
    assert ok, f"{what} with layout='NHWC' must be dense channels-last per step"


def launch_lif(x, *, bias=None, residual=None, thr=(THR_SCALAR, None, 1.0),
               v_init=None, v_out=None, spikes=None, count=None,
               C=1, HW=1, channel_last=False, decay=1.0, in_scale=1.0,
               v_reset=0.0, soft_reset=False):
    """Enqueue snnk_lif_forward on the current stream of ``x``'s device.
    An int32 ``spikes`` tensor receives packed bits ([T, NCL/32] words)."""
    T = x.shape[0]
    NCL = math.prod(x.shape[1:])
    thr_mode, thr_t, thr_s = thr
    sfmt = _abi.SPIKE_SAME
    if spikes is not None and spikes.dtype != x.dtype:
        assert spikes.dtype in (torch.uint8, torch.bfloat16, torch.int32), spikes.dtype
        sfmt = {torch.uint8: _abi.SPIKE_U8, torch.bfloat16: _abi.SPIKE_BF16,
                torch.int32: _abi.SPIKE_BITS}[spikes.dtype]
    with torch.cuda.device(x.device):
        _abi.call(
            "snnk_lif_forward",
            _abi.ptr(x), _abi.dtype_code(x.dtype),
            _abi.ptr(bias), _abi.ptr(residual),
            _abi.ptr(thr_t), thr_mode, thr_s,
            _abi.ptr(v_init), _abi.ptr(v_out),
            _abi.ptr(spikes), sfmt, _abi.ptr(count),
            T, NCL, int(C), int(HW), 1 if channel_last else 0,
            float(decay), float(in_scale), float(v_reset),
            1 if soft_reset else 0, _abi.stream(x.device))


def if_lif(
    x_seq: torch.Tensor,
    *,
    neuron: str = "if",
    tau: float = 2.0,
    decay: float | None = None,
    decay_input: bool = True,
    soft_reset: bool = False,
    v_threshold=1.0,
    v_reset: float = 0.0,
    layout: str = "NCHW",
    spike_dtype: torch.dtype | None = None,
) -> torch.Tensor:
    """Multi-step IF/LIF forward; returns spikes shaped like ``x_seq``.

    Reference: snn_compiler/kernels/neurons.py:311-376 (``if_lif``).
    ``x_seq`` is ``[T, B, ...]`` fp32/bf16/fp16.  ``v_threshold`` is a float,
    a ``[C]`` or an ``[NCL]`` fp32 tensor.  ``spike_dtype`` (extension; default
    the input dtype, as in the reference) may be ``torch.uint8`` or
    ``torch.bfloat16``.
    """
    check_flat(x_seq, layout)
    assert x_seq.dtype in (torch.float32, torch.float16, torch.bfloat16)
    NCL = math.prod(x_seq.shape[1:])
    C, HW = infer_C_HW(x_seq)
    df, sc = neuron_params(neuron, tau, decay, decay_input)
    Cthr = x_seq.shape[2] if x_seq.ndim >= 4 else (x_seq.shape[-1] if x_seq.ndim == 3 else 1)
    thr = resolve_threshold(v_threshold, Cthr, NCL)
    spike_seq = torch.empty_like(x_seq, dtype=spike_dtype or x_seq.dtype)
    launch_lif(x_seq, thr=thr, spikes=spike_seq, C=C, HW=HW,
               channel_last=(layout == "NHWC"), decay=df, in_scale=sc,
               v_reset=v_reset, soft_reset=soft_reset)
    return spike_seq


def if_lif_packed(
    x_seq: torch.Tensor,
    *,
    neuron: str = "if",
    tau: float = 2.0,
    decay: float | None = None,
    decay_input: bool = True,
    soft_reset: bool = False,
    v_threshold=1.0,
    v_reset: float = 0.0,
    layout: str = "NCHW",
) -> torch.Tensor:
    """``if_lif`` writing bit-packed spikes: int32 words ``[T, NCL // 32]``.

    Extension of snn_compiler/kernels/neurons.py:311-376.  Neuron ``i`` of a
    step (flat memory order of ``x_seq[t]``) lands in bit ``i % 32`` of word
    ``i // 32`` -- LSB first, the convention of ``pack_bits`` and the
    reference's ``_pack_N``.  For channel-last activations (``[T, R, C]`` or
    NHWC ``[T, B, C, H, W]`` with ``layout='NHWC'``) the words are packed along
    C, so ``words.view(T, R, C // 32)`` is the ``a_packed`` operand of
    :func:`snnk.binary_gemm`.  Needs ``NCL % 32 == 0``; 1/8 of the bytes of
    uint8 spikes, 1/32 of fp32.
    """
    check_flat(x_seq, layout)
    assert x_seq.dtype in (torch.float32, torch.float16, torch.bfloat16)
    T = x_seq.shape[0]
    NCL = math.prod(x_seq.shape[1:])
    if NCL % 32 != 0:
        raise ValueError(f"packed spikes need NCL % 32 == 0, got NCL={NCL}")
    C, HW = infer_C_HW(x_seq)
    df, sc = neuron_params(neuron, tau, decay, decay_input)
    Cthr = x_seq.shape[2] if x_seq.ndim >= 4 else (x_seq.shape[-1] if x_seq.ndim == 3 else 1)
    thr = resolve_threshold(v_threshold, Cthr, NCL)
    words = torch.empty(T, NCL // 32, device=x_seq.device, dtype=torch.int32)
    launch_lif(x_seq, thr=thr, spikes=words, C=C, HW=HW, channel_last=(layout == "NHWC"),
               decay=df, in_scale=sc, v_reset=v_reset, soft_reset=soft_reset)
    return words
