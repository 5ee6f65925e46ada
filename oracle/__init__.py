"""CPU oracle for the snnk parity tests -- TEST INFRASTRUCTURE ONLY.

Restatements of the reference's own CPU algorithms for the hot path of
Xarlley/Triton-Pass-Analysis (``snn_compiler/kernels``), each function citing
the reference file:line it follows.  Only ``tests/``, ``__graft_entry__.smoke``
and the ``cpu_baseline`` leg of ``bench.py`` may import this package, and only
as the checker / the timed CPU baseline; the product (``snnk`` + libsnnk.so)
never calls it.

Modules
  neurons   multi-step IF/LIF (naive_if_lif and the fused/stateful/rate forms),
            plus the SpikingJelly ``H = v + (x - v)/tau`` form      (torch CPU)
  fused     BN folding, conv3x3 + BN + LIF + 2x2 max-pool block    (torch CPU)
  bits      LSB-first bit packing and popcount / binary GEMM       (numpy)
  attention spike self-attention with integer QK^T and (QK^T)V     (torch CPU + int64)
  vgg       VGG16-SNN at 32x32 with seeded init                     (torch CPU)
  clib      ctypes access to the C restatement in oracle/c/oracle.c

Parity pins (what fixes each function independently of its own formula) are
listed in the module docstrings; every function is pinned by at least one
known-answer, brute-force or closed-form check in tests/test_oracle_*.py.
"""
