"""ctypes access to the C restatement (oracle/c/oracle.c) -- test infrastructure only."""
from __future__ import annotations

import ctypes as C
import pathlib
import subprocess

import numpy as np

_DIR = pathlib.Path(__file__).resolve().parent
LIB = _DIR / "_build" / "liboracle.so"
_lib = None


def build() -> pathlib.Path:
    subprocess.run(["make", "-B", "-C", str(_DIR)], check=True,
                   capture_output=True, text=True)
    return LIB


def lib():
    global _lib
    if _lib is None:
        if not LIB.exists():
            build()
        h = C.CDLL(str(LIB))
        p, i64, f32, i32 = C.c_void_p, C.c_int64, C.c_float, C.c_int
        h.oracle_lif_f32.argtypes = [p, i64, i64, p, i64, i64, p, f32, p, f32, f32,
                                     i32, f32, p, p]
        h.oracle_lif_f32.restype = None
        h.oracle_pack_bits.argtypes = [p, i64, i64, p]
        h.oracle_pack_bits.restype = None
        h.oracle_popcount_gemm.argtypes = [p, p, i64, i64, i64, i64, i32, p]
        h.oracle_popcount_gemm.restype = None
        _lib = h
    return _lib


def _p(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


def lif_f32(x, *, bias=None, C_=1, HW=1, vth=None, vth_scalar=1.0, v_init=None,
            df=0.5, sc=0.5, soft_reset=False, v_reset=0.0):
    """x: float32 [T, NCL] -> (spikes [T, NCL] float32, v_final [NCL])."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    T, NCL = x.shape
    spikes = np.empty_like(x)
    v_out = np.empty(NCL, np.float32)
    args = [np.ascontiguousarray(a, dtype=np.float32) if a is not None else None
            for a in (bias, vth, v_init)]
    lib().oracle_lif_f32(_p(x), T, NCL, _p(args[0]), int(C_), int(HW), _p(args[1]),
                         float(vth_scalar), _p(args[2]), float(df), float(sc),
                         1 if soft_reset else 0, float(v_reset), _p(spikes), _p(v_out))
    return spikes, v_out


def pack_bits(src01):
    """src01: [rows, K] {0,1} -> [rows, ceil(K/32)] uint32 (LSB first)."""
    src = np.ascontiguousarray(src01, dtype=np.uint8)
    rows, K = src.shape
    out = np.empty((rows, (K + 31) // 32), np.uint32)
    lib().oracle_pack_bits(_p(src), rows, K, _p(out))
    return out


def popcount_gemm(A_packed, B_packed, *, signed=False, rows=None):
    """A [M, W], B [N, W] uint32 -> int32 [m1-m0, N] for rows (m0, m1)."""
    A = np.ascontiguousarray(A_packed, dtype=np.uint32)
    B = np.ascontiguousarray(B_packed, dtype=np.uint32)
    M, W = A.shape
    N = B.shape[0]
    m0, m1 = rows if rows is not None else (0, M)
    out = np.empty((m1 - m0, N), np.int32)
    lib().oracle_popcount_gemm(_p(A), _p(B), m0, m1, N, W, 1 if signed else 0, _p(out))
    return out
