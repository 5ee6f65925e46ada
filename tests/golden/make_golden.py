"""Write the golden fixtures of this directory (run: python tests/golden/make_golden.py).

Every value is computed by plain Python loops, independently of the oracle's
vectorised torch code, from inputs drawn with ``random.Random(seed)``:

* lif.json      -- multi-step IF/LIF (snn_compiler/kernels/neurons.py:467-502):
                   fp32 state, every product and sum rounded to fp32 in the
                   reference's order ``df*v + sc*x``, hard/soft reset, scalar
                   and per-channel thresholds; spikes and final membrane.
* bits.json     -- LSB-first bit packing (bit k%32 of word k//32, explore/
                   attention/phase6b_bitpack.py:35-46) with K = 70 (ragged tail)
                   and the popcount GEMM C[m,n] = popc(A_m & W_n), unsigned and
                   signed (W in {-1,+1}: 2*popc(A & W+) - popc(A)).
* conv.json     -- conv3x3 / pad 1 over NHWC spikes with bf16-representable
                   weights, exact double sums + bias, the LIF over T on those
                   pre-activations and the 2x2 max (OR) pool.
* attention.json -- integer Q K^T and (Q K^T) V counts of 0/1 Q, K, V.
"""
from __future__ import annotations

import json
import math
import os
import random
import struct

HERE = os.path.dirname(os.path.abspath(__file__))


def f32(x: float) -> float:
    """Round a double to the nearest fp32 (ties to even)."""
    return struct.unpack("<f", struct.pack("<f", x))[0]


def bf16(x: float) -> float:
    """Round to the nearest bf16 (ties to even) via its fp32 bit pattern."""
    u = struct.unpack("<I", struct.pack("<f", f32(x)))[0]
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    return struct.unpack("<f", struct.pack("<I", u))[0]


# -- LIF -----------------------------------------------------------------------
def lif_case(rng, T, B, C, HW, neuron, tau, soft, thr, v_reset):
    x = [[f32(rng.gauss(0.0, 1.5)) for _ in range(B * C * HW)] for _ in range(T)]
    if neuron == "lif":
        df, sc = f32(1.0 - 1.0 / tau), f32(1.0 / tau)
    else:
        df, sc = 1.0, 1.0
    per_c = isinstance(thr, list)
    v = [0.0] * (B * C * HW)
    spikes = []
    for t in range(T):
        st = []
        for i in range(B * C * HW):
            c = (i // HW) % C
            vth = thr[c] if per_c else thr
            h = f32(f32(df * v[i]) + f32(sc * x[t][i]))
            s = 1.0 if h >= vth else 0.0
            if s:
                v[i] = f32(h - vth) if soft else v_reset
            else:
                v[i] = h
            st.append(s)
        spikes.append(st)
    return dict(shape=[T, B, C, HW], neuron=neuron, tau=tau, soft_reset=soft,
                v_threshold=thr, v_reset=v_reset, x=x, spikes=spikes, v_final=v)


def make_lif():
    rng = random.Random(101)
    thr_c = [f32(v) for v in (0.6, 1.0, 1.4)]
    return {"cases": [
        lif_case(rng, 4, 2, 3, 4, "lif", 2.0, False, 1.0, 0.0),
        lif_case(rng, 5, 2, 3, 4, "lif", 3.0, False, 1.0, 0.0),     # inexact decay 2/3
        lif_case(rng, 4, 2, 3, 4, "lif", 3.0, True, 1.0, 0.0),      # soft reset
        lif_case(rng, 6, 1, 3, 5, "if", 2.0, False, 1.0, -0.25),    # IF, v_reset != 0
        lif_case(rng, 4, 2, 3, 4, "lif", 2.0, False, thr_c, 0.0),   # per-channel threshold
    ]}


# -- bits ----------------------------------------------------------------------
def pack_row(bits):
    words = [0] * ((len(bits) + 31) // 32)
    for k, b in enumerate(bits):
        if b:
            words[k // 32] |= 1 << (k % 32)
    return words


def popc(x):
    return bin(x).count("1")


def make_bits():
    rng = random.Random(202)
    M, N, K = 5, 7, 70
    A = [[1 if rng.random() < 0.3 else 0 for _ in range(K)] for _ in range(M)]
    W = [[1 if rng.random() < 0.5 else 0 for _ in range(K)] for _ in range(N)]
    Ap, Wp = [pack_row(r) for r in A], [pack_row(r) for r in W]
    C = [[sum(popc(a & w) for a, w in zip(Ap[m], Wp[n])) for n in range(N)] for m in range(M)]
    rowpop = [sum(popc(a) for a in Ap[m]) for m in range(M)]
    Cs = [[2 * C[m][n] - rowpop[m] for n in range(N)] for m in range(M)]
    # direct integer check of both identities
    for m in range(M):
        for n in range(N):
            assert C[m][n] == sum(A[m][k] * W[n][k] for k in range(K))
            assert Cs[m][n] == sum(A[m][k] * (2 * W[n][k] - 1) for k in range(K))
    # known answers of the packing convention
    ones = pack_row([1] * 64 + [1] * 6)
    single = [pack_row([1 if k == j else 0 for k in range(70)]) for j in (0, 31, 32, 69)]
    return dict(M=M, N=N, K=K, A=A, W=W, A_packed=Ap, W_packed=Wp, C=C, C_signed=Cs,
                all_ones_70=ones, single_bits={"0": single[0], "31": single[1],
                                               "32": single[2], "69": single[3]})


# -- conv ----------------------------------------------------------------------
def make_conv():
    rng = random.Random(303)
    T, B, H, W, Cin, Cout = 2, 1, 4, 4, 32, 32
    x = [[[[[1.0 if rng.random() < 0.3 else 0.0 for _ in range(Cin)] for _ in range(W)]
           for _ in range(H)] for _ in range(B)] for _ in range(T)]
    # weights [Cout][kh][kw][cin], bf16 values so the GPU operand is exact
    w = [[[[bf16(rng.gauss(0.0, 0.3)) for _ in range(Cin)] for _ in range(3)] for _ in range(3)]
         for _ in range(Cout)]
    bias = [f32(rng.gauss(0.0, 0.2)) for _ in range(Cout)]
    pre = [[[[[0.0] * Cout for _ in range(W)] for _ in range(H)] for _ in range(B)] for _ in range(T)]
    for t in range(T):
        for b in range(B):
            for y in range(H):
                for xx in range(W):
                    for n in range(Cout):
                        acc = 0.0
                        for kh in range(3):
                            ys = y + kh - 1
                            if not 0 <= ys < H:
                                continue
                            for kw in range(3):
                                xs = xx + kw - 1
                                if not 0 <= xs < W:
                                    continue
                                row, wr = x[t][b][ys][xs], w[n][kh][kw]
                                for c in range(Cin):
                                    if row[c]:
                                        acc += wr[c]
                        pre[t][b][y][xx][n] = acc + bias[n]      # exact in double
    # LIF (tau 2, theta 1, hard reset 0) on the fp32-rounded pre-activations
    spk = [[[[[0.0] * Cout for _ in range(W)] for _ in range(H)] for _ in range(B)] for _ in range(T)]
    for b in range(B):
        for y in range(H):
            for xx in range(W):
                for n in range(Cout):
                    v = 0.0
                    for t in range(T):
                        h = f32(f32(0.5 * v) + f32(0.5 * f32(pre[t][b][y][xx][n])))
                        s = h >= 1.0
                        v = 0.0 if s else h
                        spk[t][b][y][xx][n] = 1.0 if s else 0.0
    pooled = [[[[[max(spk[t][b][2 * py + dy][2 * px + dx][n] for dy in (0, 1) for dx in (0, 1))
                  for n in range(Cout)] for px in range(W // 2)] for py in range(H // 2)]
               for b in range(B)] for t in range(T)]
    return dict(shape=dict(T=T, B=B, H=H, W=W, Cin=Cin, Cout=Cout), x_nhwc=x,
                w_khkwcin=w, bias=bias, preact=pre, spikes=spk, pooled=pooled,
                lif=dict(tau=2.0, v_threshold=1.0, v_reset=0.0))


# -- attention -----------------------------------------------------------------
def make_attention():
    rng = random.Random(404)
    heads, N, d = 2, 16, 8
    q, k, v = ([[[1 if rng.random() < 0.3 else 0 for _ in range(d)] for _ in range(N)]
                for _ in range(heads)] for _ in range(3))
    S = [[[sum(q[h][i][c] * k[h][j][c] for c in range(d)) for j in range(N)] for i in range(N)]
         for h in range(heads)]
    O = [[[sum(S[h][i][j] * v[h][j][c] for j in range(N)) for c in range(d)] for i in range(N)]
         for h in range(heads)]
    KtV = [[[sum(k[h][j][a] * v[h][j][c] for j in range(N)) for c in range(d)] for a in range(d)]
           for h in range(heads)]
    for h in range(heads):  # associativity over the integers
        for i in range(N):
            for c in range(d):
                assert O[h][i][c] == sum(q[h][i][a] * KtV[h][a][c] for a in range(d))
    return dict(heads=heads, N=N, d=d, q=q, k=k, v=v, S=S, O=O, KtV=KtV)


def main():
    for name, fn in (("lif", make_lif), ("bits", make_bits), ("conv", make_conv),
                     ("attention", make_attention)):
        path = os.path.join(HERE, f"{name}.json")
        with open(path, "w") as f:
            json.dump(fn(), f, separators=(",", ":"))
        print(f"{path}: {os.path.getsize(path)} bytes")


if __name__ == "__main__":
    assert math.isclose(bf16(1.0 + 2 ** -9), 1.0) and bf16(1.0 + 2 ** -7) == 1.0 + 2 ** -7
    main()
