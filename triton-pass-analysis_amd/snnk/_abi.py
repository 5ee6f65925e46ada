"""ctypes boundary to libsnnk.so.

The library exposes a plain C ABI (``include/snnk.h``): raw device pointers,
int64 sizes, an ``int`` status and the HIP stream as ``void*``.  This module
loads it, declares every prototype once, and turns a non-zero status into a
Python exception.  It never falls back to another implementation: if the
library is missing the first call raises.
"""
from __future__ import annotations

import ctypes as C
import pathlib
import threading

import torch

LIB_PATH = pathlib.Path(__file__).resolve().parent / "libsnnk.so"

# status codes (include/snnk.h)
OK, EINVAL, EUNSUPPORTED, EALIGN, EWORKSPACE, ESCRATCH = 0, -1, -2, -3, -4, -5
# element types
F32, BF16, F16, U8, I32 = 0, 1, 2, 3, 4
# spike formats
SPIKE_SAME, SPIKE_U8, SPIKE_BF16, SPIKE_BITS = 0, 1, 2, 3
# threshold modes
THR_SCALAR, THR_PER_CHANNEL, THR_PER_NEURON = 0, 1, 2
# activation formats of the _act entry points
ACT_BF16, ACT_BITS = 0, 1
# binary GEMM algorithms
BGEMM_AUTO, BGEMM_POPC, BGEMM_MFMA_I8, BGEMM_MFMA_F4 = 0, 1, 2, 3

_p = C.c_void_p
_i32 = C.c_int32
_i64 = C.c_int64
_f32 = C.c_float

# name -> argtypes (restype is int for every entry point except the two
# informational ones declared below).
PROTOTYPES: dict[str, list] = {
    "snnk_lif_forward": [
        _p, _i32,              # x, x_dtype
        _p, _p,                # bias, residual
        _p, _i32, _f32,        # vth, thr_mode, vth_scalar
        _p, _p,                # v_init, v_out
        _p, _i32, _p,          # spikes, spike_fmt, count_out
        _i64, _i64, _i64, _i64,  # T, NCL, C, HW
        _i32,                  # channel_last
        _f32, _f32, _f32,      # decay, in_scale, v_reset
        _i32, _p,              # soft_reset, stream
    ],
    "snnk_pack_bits": [
        _p, _i32, _p,          # src, src_dtype, dst
        _i64, _i64, _i64,      # batch, rows, K
        _i64, _i64, _i64,      # stride_b, stride_r, stride_k
        _p,                    # stream
    ],
    "snnk_binary_gemm": [
        _p, _p, _p, _i32,      # A, B, C, c_dtype
        _i64, _i64, _i64, _i64,  # batch, M, N, K
        _i64, _i64, _i64,      # lda, ldb, ldc
        _i64, _i64, _i64,      # stride_a, stride_b, stride_c
        _i32, _i32, _p,        # signed_w, algo, stream
    ],
    "snnk_conv3x3_bn_lif": [
        _p, _p, _p,            # x, w, bias
        _p, _p,                # spikes_out, preact_out
        _i64, _i64, _i64, _i64,  # T, B, H, W
        _i64, _i64, _i32,      # Cin, Cout, pool
        _f32, _f32, _f32,      # decay, in_scale, v_threshold
        _f32, _i32, _i32,      # v_reset, soft_reset, tile_hint
        _p,                    # stream
    ],
    "snnk_linear_bias_lif": [
        _p, _p, _p,            # x, w, bias
        _p, _p,                # spikes_out, preact_out
        _i64, _i64, _i64, _i64,  # T, R, K, N
        _f32, _f32, _f32, _f32,  # decay, in_scale, v_threshold, v_reset
        _i32, _i32, _p,        # soft_reset, tile_hint, stream
    ],
    "snnk_conv3x3_bn_lif_ws": [
        _p, _p, _p,            # x, w, bias
        _p, _p,                # spikes_out, preact_out
        _i64, _i64, _i64, _i64,  # T, B, H, W
        _i64, _i64, _i32,      # Cin, Cout, pool
        _f32, _f32, _f32,      # decay, in_scale, v_threshold
        _f32, _i32, _i32,      # v_reset, soft_reset, tile_hint
        _i32, _p, _i64,        # splits, workspace, workspace_bytes
        _p,                    # stream
    ],
    "snnk_conv3x3_bn_lif_noalloc": [
        _p, _p, _p,            # x, w, bias
        _p, _p,                # spikes_out, preact_out
        _i64, _i64, _i64, _i64,  # T, B, H, W
        _i64, _i64, _i32,      # Cin, Cout, pool
        _f32, _f32, _f32,      # decay, in_scale, v_threshold
        _f32, _i32, _i32,      # v_reset, soft_reset, tile_hint
        _i32, _p,              # splits, stream
    ],
    "snnk_linear_bias_lif_ws": [
        _p, _p, _p,            # x, w, bias
        _p, _p,                # spikes_out, preact_out
        _i64, _i64, _i64, _i64,  # T, R, K, N
        _f32, _f32, _f32, _f32,  # decay, in_scale, v_threshold, v_reset
        _i32, _i32,            # soft_reset, tile_hint
        _i32, _p, _i64,        # splits, workspace, workspace_bytes
        _p,                    # stream
    ],
    "snnk_conv3x3_bn_lif_act": [
        _p, _i32, _p, _p,      # x, x_fmt, w, bias
        _p, _i32,              # spikes_out, out_fmt
        _i64, _i64, _i64, _i64,  # T, B, H, W
        _i64, _i64, _i32,      # Cin, Cout, pool
        _f32, _f32, _f32,      # decay, in_scale, v_threshold
        _f32, _i32, _i32,      # v_reset, soft_reset, tile_hint
        _i32, _p, _i64,        # splits, workspace, workspace_bytes
        _p,                    # stream
    ],
    "snnk_linear_bias_lif_act": [
        _p, _i32, _p, _p,      # x, x_fmt, w, bias
        _p, _i32,              # spikes_out, out_fmt
        _i64, _i64, _i64, _i64,  # T, R, K, N
        _i32,                  # col_pool
        _f32, _f32, _f32, _f32,  # decay, in_scale, v_threshold, v_reset
        _i32, _i32,            # soft_reset, tile_hint
        _i32, _p, _i64,        # splits, workspace, workspace_bytes
        _p,                    # stream
    ],
    "snnk_linear_bias_lif_pool4_ws": [
        _p, _p, _p, _p,        # x, w, bias, spikes_out
        _i64, _i64, _i64, _i64,  # T, R, K, N
        _f32, _f32, _f32, _f32,  # decay, in_scale, v_threshold, v_reset
        _i32, _i32,            # soft_reset, tile_hint
        _i32, _p, _i64,        # splits, workspace, workspace_bytes
        _p,                    # stream
    ],
    "snnk_linear_mean_t": [
        _p, _p, _p, _p,        # x, w, bias, out
        _i64, _i64, _i64, _i64,  # T, R, K, N
        _i32, _i32,            # tile_hint, splits
        _p, _i64,              # workspace, workspace_bytes
        _p,                    # stream
    ],
    "snnk_linear_mean_t_bits": [
        _p, _p, _p, _p,        # x words, w, bias, out
        _i64, _i64, _i64, _i64,  # T, R, K, N
        _p,                    # stream
    ],
    "snnk_spike_attention": [
        _p, _p, _p,            # q, k, v
        _i64, _i64, _i64,      # q_row, k_row, v_row
        _i64, _i64, _i64,      # q_step, k_step, v_step
        _p, _i64, _i64,        # spikes_out, out_row, out_step
        _p, _p,                # s_counts, o_counts
        _i64, _i64, _i64, _i64, _i64,  # T, B, H, N, d
        _f32, _f32, _f32, _f32,  # decay, in_scale, v_threshold, v_reset
        _i32, _p,              # soft_reset, stream
    ],
    "snnk_spike_attention_packed": [
        _p, _p, _p,            # q, k, v (uint32 words)
        _i64, _i64, _i64,      # q_row, k_row, v_row (words)
        _i64, _i64, _i64,      # q_step, k_step, v_step (words)
        _i64,                  # in_head_bits
        _p, _i64, _i64, _i64,  # spikes_out, out_row, out_step (words), out_head_words
        _p, _p,                # s_counts, o_counts
        _i64, _i64, _i64, _i64, _i64,  # T, B, H, N, d
        _f32, _f32, _f32, _f32,  # decay, in_scale, v_threshold, v_reset
        _i32, _p,              # soft_reset, stream
    ],
    "snnk_linear_preact_act": [
        _p, _i32, _p, _p,      # x, x_fmt, w, bias
        _p,                    # out (fp32)
        _i64, _i64, _i64, _i64,  # T, R, K, N
        _i32, _i32,            # tile_hint, splits
        _p, _i64,              # workspace, workspace_bytes
        _p,                    # stream
    ],
    "snnk_spike_av_lif": [
        _p, _i32, _p, _i32,    # q, q_dtype, kv, kv_dtype
        _p,                    # spikes_out
        _i64, _i64, _i64, _i64,  # T, BH, N, d
        _f32, _f32, _f32, _f32,  # decay, in_scale, v_threshold, v_reset
        _i32, _p,              # soft_reset, stream
    ],
    "snnk_conv3x3_image_lif": [
        _p, _p, _p, _p,        # image, w, bias, spikes_out
        _i64, _i64, _i64,      # T, B, Cin
        _i64, _i64, _i64,      # H, W, Cout
        _f32, _f32, _f32, _f32,  # decay, in_scale, v_threshold, v_reset
        _i32, _p,              # soft_reset, stream
    ],
    "snnk_conv3x3_image_lif_act": [
        _p, _p, _p, _p, _i32,  # image, w, bias, spikes_out, out_fmt
        _i64, _i64, _i64,      # T, B, Cin
        _i64, _i64, _i64,      # H, W, Cout
        _f32, _f32, _f32, _f32,  # decay, in_scale, v_threshold, v_reset
        _i32, _p,              # soft_reset, stream
    ],
    "snnk_to_nhwc_bf16": [
        _p, _i32, _p,          # src, src_dtype, dst
        _i64, _i64, _i64,      # N, C, HW
        _p,                    # stream
    ],
}

# entry points returning int64 (workspace bytes, or a negative status)
SIZE_PROTOTYPES: dict[str, list] = {
    "snnk_conv3x3_bn_lif_ws_size": [_i64, _i64, _i64, _i64, _i64, _i64,  # T, B, H, W, Cin, Cout
                                    _i32, _i32, _i32, _i32],           # pool, preact, tile, splits
    "snnk_linear_bias_lif_ws_size": [_i64, _i64, _i64, _i64,            # T, R, K, N
                                     _i32, _i32, _i32],                 # preact, tile, splits
    "snnk_conv3x3_bn_lif_act_ws_size": [_i64, _i64, _i64, _i64, _i64, _i64,  # T, B, H, W, Cin, Cout
                                        _i32, _i32, _i32, _i32],        # pool, x_fmt, tile, splits
    "snnk_linear_bias_lif_act_ws_size": [_i64, _i64, _i64, _i64,        # T, R, K, N
                                         _i32, _i32, _i32, _i32],       # x_fmt, col_pool, tile, splits
}

_lib = None
_lock = threading.Lock()


class SnnkError(RuntimeError):
    """A libsnnk entry point returned a non-zero status."""


def lib():
    """Load libsnnk.so once; raise if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with `python -m snnk.build` "
                "(or __graft_entry__.build()); snnk has no fallback path")
        h = C.CDLL(str(LIB_PATH))
        h.snnk_version.restype = C.c_int
        h.snnk_version.argtypes = []
        h.snnk_status_string.restype = C.c_char_p
        h.snnk_status_string.argtypes = [C.c_int]
        for name, argtypes in PROTOTYPES.items():
            fn = getattr(h, name)
            fn.restype = C.c_int
            fn.argtypes = argtypes
        for name, argtypes in SIZE_PROTOTYPES.items():
            fn = getattr(h, name)
            fn.restype = C.c_int64
            fn.argtypes = argtypes
        _lib = h
    return _lib


def check(status: int, what: str) -> None:
    if status != OK:
        msg = lib().snnk_status_string(status).decode()
        raise SnnkError(f"{what}: libsnnk status {status} ({msg})")


def call(name: str, *args) -> None:
    check(getattr(lib(), name)(*args), name)


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def stream(device: torch.device | None = None) -> int:
    """The current torch stream on ``device`` as a raw hipStream_t."""
    return torch.cuda.current_stream(device).cuda_stream


_DT = {torch.float32: F32, torch.bfloat16: BF16, torch.float16: F16,
       torch.uint8: U8, torch.int32: I32}


def dtype_code(dt: torch.dtype) -> int:
    try:
        return _DT[dt]
    except KeyError:
        raise AssertionError(f"unsupported dtype {dt}") from None


def size_call(name: str, *args) -> int:
    """Call an int64-returning entry point; negative results raise SnnkError."""
    n = getattr(lib(), name)(*args)
    if n < 0:
        check(int(n), name)
    return int(n)
