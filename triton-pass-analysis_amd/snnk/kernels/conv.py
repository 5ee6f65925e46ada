"""Fused conv3x3 + BN + LIF (+ 2x2 max-pool) on bf16 MFMA.

The reference runs this block as three passes -- F.conv2d (cuDNN), the fused
bias+LIF Triton kernel, then a separate nn.MaxPool2d
(snn_compiler/nn/modules.py:324-357, snn_compiler/zoo/vgg.py:101-105).  Here
it is one HIP kernel (csrc/conv.hip) that writes only spikes.

Activations flow between layers as NHWC bf16 ``[T, B, H, W, C]`` tensors;
``conv_bn_lif_pool`` accepts and returns the reference's ``[T, B, C, H, W]``
labelling (the returned tensor is a channels-last view of the NHWC result).
"""
from __future__ import annotations

import torch

from .. import _abi, _workspace
from .fused import fold_conv_bn
from .neurons import neuron_params


def prepare_conv3x3_weight(weight: torch.Tensor) -> torch.Tensor:
    """[Cout, Cin, 3, 3] (BN already folded) -> bf16 [Cout, 9*Cin], k = (kh*3+kw)*Cin + cin."""
    assert weight.ndim == 4 and weight.shape[2:] == (3, 3), tuple(weight.shape)
    Cout, Cin = weight.shape[:2]
    return weight.permute(0, 2, 3, 1).reshape(Cout, 9 * Cin).to(torch.bfloat16).contiguous()


def conv3x3_dense_weight(weight: torch.Tensor, bias: torch.Tensor | None, H: int, W: int,
                         pool: bool) -> tuple[torch.Tensor, torch.Tensor]:
    """A 3x3 / pad 1 conv on an H x W map (H, W <= 2) as one dense matrix.

    On such a map every output pixel sees every input pixel through one tap,
    so conv(x)[po, co] = sum_{pi, ci} x[pi, ci] * w[co, ci, yi - yo + 1,
    xi - xo + 1]: a Linear over the flattened NHWC map with K = H*W*Cin
    (the padding taps, zero by definition, drop out).  Returns bf16
    ``[N, H*W*Cin]`` and fp32 bias ``[N]`` with the output columns in
    (pixel, cout) order -- NHWC -- or, with ``pool`` (a 2x2 map), in (cout,
    pixel) order so that the 2x2 max-pool is the OR of four adjacent columns.
    """
    assert weight.ndim == 4 and weight.shape[2:] == (3, 3) and H <= 2 and W <= 2
    assert not pool or (H == 2 and W == 2)
    Cout, Cin = weight.shape[:2]
    P = H * W
    w = weight.float()
    dense = torch.empty(P, Cout, P, Cin, device=w.device, dtype=torch.float32)  # [po, co, pi, ci]
    for po in range(P):
        yo, xo = divmod(po, W)
        for pi in range(P):
            yi, xi = divmod(pi, W)
            dense[po, :, pi, :] = w[:, :, yi - yo + 1, xi - xo + 1]
    if pool:
        dense = dense.permute(1, 0, 2, 3)  # [co, po, pi, ci]
    b = bias.float() if bias is not None else torch.zeros(Cout, device=w.device)
    b_dense = b.repeat_interleave(P) if pool else b.repeat(P)
    return (dense.reshape(P * Cout, P * Cin).to(torch.bfloat16).contiguous(),
            b_dense.contiguous())


def to_nhwc_bf16(x_seq: torch.Tensor) -> torch.Tensor:
    """[T, B, C, H, W] (any memory format, fp32/bf16/fp16/uint8) -> contiguous NHWC bf16
    ``[T, B, H, W, C]``.  A bf16 channels-last input is returned as a view, any
    other channels-last input is cast in place of the transpose kernel."""
    assert x_seq.is_cuda and x_seq.ndim == 5, "expects a [T, B, C, H, W] GPU tensor"
    T, B, C, H, W = x_seq.shape
    nhwc = x_seq.permute(0, 1, 3, 4, 2)
    if nhwc.is_contiguous():  # channels-last memory already: a cast (RNE) or a view
        return nhwc if x_seq.dtype == torch.bfloat16 else nhwc.to(torch.bfloat16)
    src = x_seq.contiguous()
    out = torch.empty(T, B, H, W, C, device=x_seq.device, dtype=torch.bfloat16)
    with torch.cuda.device(x_seq.device):
        _abi.call("snnk_to_nhwc_bf16", src.data_ptr(), _abi.dtype_code(src.dtype),
                  out.data_ptr(), T * B, C, H * W, _abi.stream(x_seq.device))
    return out


def conv3x3_bn_lif_nhwc(x: torch.Tensor, w_prep: torch.Tensor, bias: torch.Tensor | None, *,
                        pool: bool, decay: float, in_scale: float, v_threshold: float,
                        v_reset: float = 0.0, soft_reset: bool = False,
                        out: torch.Tensor | None = None, tile_hint: int = -1,
                        splits: int | None = None) -> torch.Tensor:
    """NHWC bf16 spikes in, NHWC bf16 spikes out ([T, B, Ho, Wo, Cout]).

    ``splits``: K split over workgroups per output tile (None: chosen from the
    shape, 1: never), reduced deterministically in the device workspace."""
    assert x.is_cuda and x.dtype == torch.bfloat16 and x.ndim == 5 and x.is_contiguous()
    T, B, H, W, Cin = x.shape
    Cout = w_prep.shape[0]
    assert w_prep.dtype == torch.bfloat16 and w_prep.shape == (Cout, 9 * Cin) \
        and w_prep.is_contiguous() and w_prep.device == x.device
    if bias is not None:
        assert bias.dtype == torch.float32 and bias.numel() == Cout and bias.is_contiguous()
    Ho, Wo = (H // 2, W // 2) if pool else (H, W)
    if out is None:
        out = torch.empty(T, B, Ho, Wo, Cout, device=x.device, dtype=torch.bfloat16)
    else:
        assert out.shape == (T, B, Ho, Wo, Cout) and out.dtype == torch.bfloat16 \
            and out.is_contiguous()
    _conv_call(x, w_prep, bias, out, None, pool, decay, in_scale, v_threshold, v_reset,
               soft_reset, tile_hint, splits)
    return out


def _conv_call(x, w_prep, bias, out, pre, pool, decay, in_scale, v_threshold, v_reset,
               soft_reset, tile_hint, splits):
    T, B, H, W, Cin = x.shape
    Cout = w_prep.shape[0]
    sp = 0 if splits is None else int(splits)
    with torch.cuda.device(x.device):
        nbytes = _abi.size_call("snnk_conv3x3_bn_lif_ws_size", T, B, H, W, Cin, Cout,
                                1 if pool else 0, 1 if pre is not None else 0,
                                int(tile_hint), sp)
        ws = _workspace.get(x.device, nbytes)
        _abi.call("snnk_conv3x3_bn_lif_ws", x.data_ptr(), w_prep.data_ptr(), _abi.ptr(bias),
                  _abi.ptr(out), _abi.ptr(pre), T, B, H, W, Cin, Cout, 1 if pool else 0,
                  float(decay), float(in_scale), float(v_threshold), float(v_reset),
                  1 if soft_reset else 0, int(tile_hint), sp, _abi.ptr(ws),
                  0 if ws is None else ws.numel(), _abi.stream(x.device))


def _act_code(t: torch.Tensor) -> int:
    """Activation format of a tensor: bf16 0/1 values or int32 packed words."""
    if t.dtype == torch.bfloat16:
        return _abi.ACT_BF16
    if t.dtype == torch.int32:
        return _abi.ACT_BITS
    raise AssertionError(f"activations are bf16 0/1 or int32 packed words, not {t.dtype}")


def conv3x3_bn_lif_act(x: torch.Tensor, w_prep: torch.Tensor, bias: torch.Tensor | None, *,
                       pool: bool, decay: float, in_scale: float, v_threshold: float,
                       v_reset: float = 0.0, soft_reset: bool = False, out_bits: bool = True,
                       out: torch.Tensor | None = None, tile_hint: int = -1,
                       splits: int | None = None) -> torch.Tensor:
    """:func:`conv3x3_bn_lif_nhwc` with bit-packed activations on either side.

    x: NHWC bf16 0/1 ``[T, B, H, W, Cin]``, or int32 packed words
    ``[T, B, H, W, Cin // 32]`` (bit c%32 of word c//32, LSB first).  Returns
    int32 words ``[T, B, Ho, Wo, Cout // 32]`` (``out_bits=True``) or bf16
    ``[T, B, Ho, Wo, Cout]``.  The spikes are identical to the bf16 path's."""
    assert x.is_cuda and x.ndim == 5 and x.is_contiguous()
    x_fmt = _act_code(x)
    T, B, H, W, Cx = x.shape
    Cin = Cx * 32 if x_fmt == _abi.ACT_BITS else Cx
    Cout = w_prep.shape[0]
    assert w_prep.dtype == torch.bfloat16 and w_prep.shape == (Cout, 9 * Cin) \
        and w_prep.is_contiguous() and w_prep.device == x.device
    if bias is not None:
        assert bias.dtype == torch.float32 and bias.numel() == Cout and bias.is_contiguous()
    Ho, Wo = (H // 2, W // 2) if pool else (H, W)
    shape = (T, B, Ho, Wo, Cout // 32 if out_bits else Cout)
    dt = torch.int32 if out_bits else torch.bfloat16
    if out is None:
        out = torch.empty(shape, device=x.device, dtype=dt)
    else:
        assert out.shape == shape and out.dtype == dt and out.is_contiguous()
    sp = 0 if splits is None else int(splits)
    with torch.cuda.device(x.device):
        nbytes = _abi.size_call("snnk_conv3x3_bn_lif_act_ws_size", T, B, H, W, Cin, Cout,
                                1 if pool else 0, x_fmt, int(tile_hint), sp)
        ws = _workspace.get(x.device, nbytes)
        _abi.call("snnk_conv3x3_bn_lif_act", x.data_ptr(), x_fmt, w_prep.data_ptr(),
                  _abi.ptr(bias), out.data_ptr(), _abi.ACT_BITS if out_bits else _abi.ACT_BF16,
                  T, B, H, W, Cin, Cout, 1 if pool else 0, float(decay), float(in_scale),
                  float(v_threshold), float(v_reset), 1 if soft_reset else 0, int(tile_hint),
                  sp, _abi.ptr(ws), 0 if ws is None else ws.numel(), _abi.stream(x.device))
    return out


def conv3x3_preact_nhwc(x: torch.Tensor, w_prep: torch.Tensor, bias: torch.Tensor | None,
                        *, tile_hint: int = -1, splits: int | None = None) -> torch.Tensor:
    """fp32 conv + bias, NHWC ``[T, B, H, W, Cout]`` (the membrane input, no LIF)."""
    assert x.is_cuda and x.dtype == torch.bfloat16 and x.ndim == 5 and x.is_contiguous()
    T, B, H, W, Cin = x.shape
    Cout = w_prep.shape[0]
    assert w_prep.shape == (Cout, 9 * Cin) and w_prep.dtype == torch.bfloat16
    pre = torch.empty(T, B, H, W, Cout, device=x.device, dtype=torch.float32)
    _conv_call(x, w_prep, bias, None, pre, False, 1.0, 1.0, 1.0, 0.0, False, tile_hint, splits)
    return pre


def conv3x3_image_lif(image: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor | None,
                      T: int, *, decay: float, in_scale: float, v_threshold: float,
                      v_reset: float = 0.0, soft_reset: bool = False,
                      out: torch.Tensor | None = None, out_bits: bool = False) -> torch.Tensor:
    """Static image [B, Cin, H, W] fp32 shown at T steps -> NHWC bf16 spikes
    [T, B, H, W, Cout], or with ``out_bits`` int32 packed words [T, B, H, W, Cout // 32]."""
    assert image.is_cuda and image.dtype == torch.float32 and image.ndim == 4
    image = image.contiguous()
    B, Cin, H, W = image.shape
    Cout = weight.shape[0]
    w = weight.float().contiguous()
    assert w.shape == (Cout, Cin, 3, 3)
    if bias is not None:
        bias = bias.float().contiguous()
    if out is None:
        out = (torch.empty(T, B, H, W, Cout // 32, device=image.device, dtype=torch.int32)
               if out_bits else
               torch.empty(T, B, H, W, Cout, device=image.device, dtype=torch.bfloat16))
    with torch.cuda.device(image.device):
        _abi.call("snnk_conv3x3_image_lif_act", image.data_ptr(), w.data_ptr(), _abi.ptr(bias),
                  out.data_ptr(), _abi.ACT_BITS if out_bits else _abi.ACT_BF16, T, B, Cin, H,
                  W, Cout, float(decay), float(in_scale), float(v_threshold), float(v_reset),
                  1 if soft_reset else 0, _abi.stream(image.device))
    return out


def conv_bn_lif_pool(x_seq, conv_w, conv_b, bn_w, bn_b, bn_mean, bn_var, bn_eps, *,
                     pool: str | None = "max", neuron: str = "lif", tau: float = 2.0,
                     decay: float | None = None, decay_input: bool = True,
                     soft_reset: bool = False, v_threshold: float = 1.0,
                     v_reset: float = 0.0, stride=1, padding=1, dilation=1, groups=1):
    """conv3x3 + eval BN (folded) + IF/LIF + optional 2x2 max-pool, one kernel.

    Signature of ``conv_bn_neuron`` (snn_compiler/kernels/fused.py:602-611)
    plus ``pool``.  Only 3x3 / stride 1 / padding 1 / dilation 1 / groups 1,
    Cin % 32 == 0, Cout % 32 == 0 and a float threshold are fused; for any
    other conv use :func:`snnk.kernels.fused.conv_bn_neuron`.
    Returns bf16 spikes labelled ``[T, B, Cout, Ho, Wo]`` in channels-last memory.
    """
    if (stride, padding, dilation, groups) not in ((1, 1, 1, 1), ((1, 1), (1, 1), (1, 1), 1)):
        raise ValueError("conv_bn_lif_pool fuses 3x3 / stride 1 / padding 1 convs only")
    if pool not in (None, "max"):
        raise ValueError(f"unsupported pool {pool!r} (None or 'max')")
    if isinstance(v_threshold, torch.Tensor):
        raise ValueError("conv_bn_lif_pool takes a float threshold")
    df, sc = neuron_params(neuron, tau, decay, decay_input)
    new_w, new_b = fold_conv_bn(conv_w, conv_b, bn_w, bn_b, bn_mean, bn_var, bn_eps)
    x = to_nhwc_bf16(x_seq)
    out = conv3x3_bn_lif_nhwc(x, prepare_conv3x3_weight(new_w), new_b.float().contiguous(),
                              pool=pool == "max", decay=df, in_scale=sc,
                              v_threshold=float(v_threshold), v_reset=v_reset,
                              soft_reset=soft_reset)
    return out.permute(0, 1, 4, 2, 3)
