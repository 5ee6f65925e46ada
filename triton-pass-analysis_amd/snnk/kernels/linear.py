"""Linear + bias + LIF over T on bf16 MFMA (csrc/conv.hip, 1x1 mode).

The reference runs F.linear (cuBLAS) and then its fused bias+LIF kernel
(snn_compiler/nn/modules.py:241-255, snn_compiler/kernels/fused.py:554-579).
Here the GEMM epilogue runs the neuron: each accumulator lane holds the four
time steps of one (row, feature), so only spikes leave the kernel.
"""
from __future__ import annotations

import torch

from .. import _abi, _workspace


def linear_fusable(x_seq: torch.Tensor, weight: torch.Tensor, v_threshold) -> bool:
    """Shapes and arguments the fused kernel covers."""
    if isinstance(v_threshold, torch.Tensor) or not x_seq.is_cuda:
        return False
    T, B = x_seq.shape[0], x_seq.shape[1]
    K = x_seq[0, 0].numel() if x_seq.ndim > 2 else 1
    N, Kw = weight.shape
    return K == Kw and K % 32 == 0 and N % 32 == 0 and B % 4 == 0 and T > 0


def _check(x, w, bias):
    assert x.is_cuda and x.dtype == torch.bfloat16 and x.ndim == 3 and x.is_contiguous(), \
        "x must be a contiguous bf16 [T, R, K] GPU tensor"
    assert w.dtype == torch.bfloat16 and w.ndim == 2 and w.is_contiguous() \
        and w.shape[1] == x.shape[2] and w.device == x.device
    if bias is not None:
        assert bias.dtype == torch.float32 and bias.numel() == w.shape[0] and bias.is_contiguous()


def linear_bias_lif(x: torch.Tensor, w: torch.Tensor, bias: torch.Tensor | None, *,
                    decay: float, in_scale: float, v_threshold: float, v_reset: float = 0.0,
                    soft_reset: bool = False, out: torch.Tensor | None = None,
                    tile_hint: int = -1, splits: int | None = None) -> torch.Tensor:
    """x [T, R, K] bf16, w [N, K] bf16 -> spikes [T, R, N] bf16.

    ``splits``: K split over workgroups per output tile (None: chosen from the
    shape, 1: never), reduced deterministically in the device workspace."""
    _check(x, w, bias)
    T, R, K = x.shape
    N = w.shape[0]
    if out is None:
        out = torch.empty(T, R, N, device=x.device, dtype=torch.bfloat16)
    else:
        assert out.shape == (T, R, N) and out.dtype == torch.bfloat16 and out.is_contiguous()
    _linear_call(x, w, bias, out, None, decay, in_scale, v_threshold, v_reset, soft_reset,
                 tile_hint, splits)
    return out


def _linear_call(x, w, bias, out, pre, decay, in_scale, v_threshold, v_reset, soft_reset,
                 tile_hint, splits):
    T, R, K = x.shape
    N = w.shape[0]
    sp = 0 if splits is None else int(splits)
    with torch.cuda.device(x.device):
        nbytes = _abi.size_call("snnk_linear_bias_lif_ws_size", T, R, K, N,
                                1 if pre is not None else 0, int(tile_hint), sp)
        ws = _workspace.get(x.device, nbytes)
        _abi.call("snnk_linear_bias_lif_ws", x.data_ptr(), w.data_ptr(), _abi.ptr(bias),
                  _abi.ptr(out), _abi.ptr(pre), T, R, K, N, float(decay), float(in_scale),
                  float(v_threshold), float(v_reset), 1 if soft_reset else 0, int(tile_hint),
                  sp, _abi.ptr(ws), 0 if ws is None else ws.numel(), _abi.stream(x.device))


def linear_bias_lif_act(x: torch.Tensor, w: torch.Tensor, bias: torch.Tensor | None, *,
                        decay: float, in_scale: float, v_threshold: float,
                        v_reset: float = 0.0, soft_reset: bool = False, out_bits: bool = True,
                        col_pool: bool = False, out: torch.Tensor | None = None,
                        tile_hint: int = -1, splits: int | None = None) -> torch.Tensor:
    """:func:`linear_bias_lif` with bit-packed activations on either side.

    x: bf16 0/1 ``[T, R, K]`` or int32 packed words ``[T, R, K // 32]``;
    returns int32 words ``[T, R, N // 32]`` (``out_bits=True``) or bf16
    ``[T, R, N]``, the same spikes as the bf16 path.  ``col_pool``: the OR of
    each group of four adjacent output columns (bf16 ``[T, R, N // 4]``, as
    :func:`linear_bias_lif_pool4`)."""
    assert x.is_cuda and x.ndim == 3 and x.is_contiguous()
    if x.dtype == torch.int32:
        x_fmt, K = _abi.ACT_BITS, x.shape[2] * 32
    else:
        assert x.dtype == torch.bfloat16, x.dtype
        x_fmt, K = _abi.ACT_BF16, x.shape[2]
    assert not (col_pool and out_bits), "the column-pooled output is bf16"
    T, R = x.shape[:2]
    N = w.shape[0]
    assert w.dtype == torch.bfloat16 and w.shape == (N, K) and w.is_contiguous() \
        and w.device == x.device
    if bias is not None:
        assert bias.dtype == torch.float32 and bias.numel() == N and bias.is_contiguous()
    shape = (T, R, N // 4 if col_pool else (N // 32 if out_bits else N))
    dt = torch.int32 if out_bits else torch.bfloat16
    if out is None:
        out = torch.empty(shape, device=x.device, dtype=dt)
    else:
        assert out.shape == shape and out.dtype == dt and out.is_contiguous()
    sp = 0 if splits is None else int(splits)
    with torch.cuda.device(x.device):
        nbytes = _abi.size_call("snnk_linear_bias_lif_act_ws_size", T, R, K, N, x_fmt,
                                1 if col_pool else 0, int(tile_hint), sp)
        ws = _workspace.get(x.device, nbytes)
        _abi.call("snnk_linear_bias_lif_act", x.data_ptr(), x_fmt, w.data_ptr(), _abi.ptr(bias),
                  out.data_ptr(), _abi.ACT_BITS if out_bits else _abi.ACT_BF16, T, R, K, N,
                  1 if col_pool else 0, float(decay), float(in_scale), float(v_threshold),
                  float(v_reset), 1 if soft_reset else 0, int(tile_hint), sp, _abi.ptr(ws),
                  0 if ws is None else ws.numel(), _abi.stream(x.device))
    return out


def linear_bias_lif_pool4(x: torch.Tensor, w: torch.Tensor, bias: torch.Tensor | None, *,
                          decay: float, in_scale: float, v_threshold: float,
                          v_reset: float = 0.0, soft_reset: bool = False,
                          out: torch.Tensor | None = None, tile_hint: int = -1,
                          splits: int | None = None) -> torch.Tensor:
    """x [T, R, K] bf16, w [N, K] bf16 -> spikes [T, R, N // 4] bf16: Linear +
    bias + LIF per column, then the OR (max) of each group of four adjacent
    columns, in one kernel."""
    _check(x, w, bias)
    T, R, K = x.shape
    N = w.shape[0]
    assert N % 4 == 0
    if out is None:
        out = torch.empty(T, R, N // 4, device=x.device, dtype=torch.bfloat16)
    else:
        assert out.shape == (T, R, N // 4) and out.dtype == torch.bfloat16 and out.is_contiguous()
    sp = 0 if splits is None else int(splits)
    with torch.cuda.device(x.device):
        nbytes = _abi.size_call("snnk_linear_bias_lif_ws_size", T, R, K, N, 0, int(tile_hint), sp)
        ws = _workspace.get(x.device, nbytes)
        _abi.call("snnk_linear_bias_lif_pool4_ws", x.data_ptr(), w.data_ptr(), _abi.ptr(bias),
                  out.data_ptr(), T, R, K, N, float(decay), float(in_scale), float(v_threshold),
                  float(v_reset), 1 if soft_reset else 0, int(tile_hint), sp, _abi.ptr(ws),
                  0 if ws is None else ws.numel(), _abi.stream(x.device))
    return out


def linear_preact(x: torch.Tensor, w: torch.Tensor, bias: torch.Tensor | None, *,
                  out: torch.Tensor | None = None, tile_hint: int = -1,
                  splits: int | None = None) -> torch.Tensor:
    """x [T, R, K] bf16, w [N, K] bf16 -> fp32 x.w^T + bias [T, R, N] (no neuron)."""
    _check(x, w, bias)
    T, R, K = x.shape
    N = w.shape[0]
    if out is None:
        out = torch.empty(T, R, N, device=x.device, dtype=torch.float32)
    else:
        assert out.shape == (T, R, N) and out.dtype == torch.float32 and out.is_contiguous()
    _linear_call(x, w, bias, None, out, 1.0, 1.0, 1.0, 0.0, False, tile_hint, splits)
    return out


def linear_preact_act(x: torch.Tensor, w: torch.Tensor, bias: torch.Tensor | None, *,
                      out: torch.Tensor | None = None, tile_hint: int = -1,
                      splits: int | None = None) -> torch.Tensor:
    """:func:`linear_preact` on bf16 ``[T, R, K]`` or int32 packed ``[T, R, K // 32]``
    spike rows: fp32 ``x.w^T + bias`` ``[T, R, N]`` (no neuron)."""
    assert x.is_cuda and x.ndim == 3 and x.is_contiguous()
    if x.dtype == torch.int32:
        x_fmt, K = _abi.ACT_BITS, x.shape[2] * 32
    else:
        assert x.dtype == torch.bfloat16, x.dtype
        x_fmt, K = _abi.ACT_BF16, x.shape[2]
    T, R = x.shape[:2]
    N = w.shape[0]
    assert w.dtype == torch.bfloat16 and w.shape == (N, K) and w.is_contiguous() \
        and w.device == x.device
    if bias is not None:
        assert bias.dtype == torch.float32 and bias.numel() == N and bias.is_contiguous()
    if out is None:
        out = torch.empty(T, R, N, device=x.device, dtype=torch.float32)
    else:
        assert out.shape == (T, R, N) and out.dtype == torch.float32 and out.is_contiguous()
    sp = 0 if splits is None else int(splits)
    with torch.cuda.device(x.device):
        nbytes = _abi.size_call("snnk_linear_bias_lif_act_ws_size", T, R, K, N, x_fmt, 0,
                                int(tile_hint), sp)
        ws = _workspace.get(x.device, nbytes)
        _abi.call("snnk_linear_preact_act", x.data_ptr(), x_fmt, w.data_ptr(), _abi.ptr(bias),
                  out.data_ptr(), T, R, K, N, int(tile_hint), sp, _abi.ptr(ws),
                  0 if ws is None else ws.numel(), _abi.stream(x.device))
    return out


def linear_mean_t(x: torch.Tensor, w: torch.Tensor, bias: torch.Tensor | None, *,
                  out: torch.Tensor | None = None, tile_hint: int = -1,
                  splits: int | None = None) -> torch.Tensor:
    """x [T, R, K] bf16, w [N, K] bf16 -> fp32 mean over T of x.w^T + bias, [R, N].

    A classifier head read as its time average (the reference's
    ``model(x_seq).mean(0)``, examples/vgg16_snn/benchmark_inference.py:68)
    in one kernel: the per-step sums stay in registers and only [R, N] is
    written."""
    _check(x, w, bias)
    T, R, K = x.shape
    N = w.shape[0]
    if out is None:
        out = torch.empty(R, N, device=x.device, dtype=torch.float32)
    else:
        assert out.shape == (R, N) and out.dtype == torch.float32 and out.is_contiguous()
    sp = 0 if splits is None else int(splits)
    with torch.cuda.device(x.device):
        nbytes = _abi.size_call("snnk_linear_bias_lif_ws_size", T, R, K, N, 1, int(tile_hint), sp)
        ws = _workspace.get(x.device, nbytes)
        _abi.call("snnk_linear_mean_t", x.data_ptr(), w.data_ptr(), _abi.ptr(bias), out.data_ptr(),
                  T, R, K, N, int(tile_hint), sp, _abi.ptr(ws), 0 if ws is None else ws.numel(),
                  _abi.stream(x.device))
    return out
def linear_mean_t_bits(x: torch.Tensor, w: torch.Tensor, bias: torch.Tensor | None, *,
                       out: torch.Tensor | None = None) -> torch.Tensor:
    """x int32 packed spike words [T, R, K // 32], w [N, K] bf16 (N <= 64) ->
    fp32 [R, N]: the time average of x.w^T + bias, computed as
    (spike counts over T) . w / T + bias in one pass over K (the spikes are
    0/1).  The classifier head of :func:`linear_mean_t` for a layer that
    writes packed spikes."""
    assert x.is_cuda and x.dtype == torch.int32 and x.ndim == 3 and x.is_contiguous()
    assert w.dtype == torch.bfloat16 and w.ndim == 2 and w.is_contiguous() and w.device == x.device
    T, R, KW = x.shape
    N, K = w.shape
    assert K == 32 * KW, f"K = {K} against {KW} words"
    if bias is not None:
        assert bias.dtype == torch.float32 and bias.shape == (N,) and bias.is_contiguous()
    if out is None:
        out = torch.empty(R, N, device=x.device, dtype=torch.float32)
    else:
        assert out.shape == (R, N) and out.dtype == torch.float32 and out.is_contiguous()
    with torch.cuda.device(x.device):
        _abi.call("snnk_linear_mean_t_bits", x.data_ptr(), w.data_ptr(), _abi.ptr(bias),
                  out.data_ptr(), T, R, K, N, _abi.stream(x.device))
    return out


