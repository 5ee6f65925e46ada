"""snnk -- MI355X-native (gfx950) SNN inference kernels.

Drop-in for the operator layer of ``snn_compiler`` (Xarlley/Triton-Pass-Analysis,
snn_compiler/__init__.py:21-38): the same entry points and module classes,
backed by hand-written HIP kernels in ``libsnnk.so`` behind a C ABI
(``include/snnk.h``).  There is no fallback: an operator whose library is
missing raises.
"""
from .kernels import (
    if_lif, pack_bits, binary_gemm, spike_ktv_popcount, HAS_POPC,
    fused_bias_if_lif, fused_bias_if_lif_rate, fused_bias_if_lif_stateful,
    conv_neuron, linear_neuron, conv_bn_neuron, fold_conv_bn,
)

__all__ = [
    "if_lif", "pack_bits", "binary_gemm", "spike_ktv_popcount", "HAS_POPC",
    "fused_bias_if_lif", "fused_bias_if_lif_rate", "fused_bias_if_lif_stateful",
    "conv_neuron", "linear_neuron", "conv_bn_neuron", "fold_conv_bn",
]
