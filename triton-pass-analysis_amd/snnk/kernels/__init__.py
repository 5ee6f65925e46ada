"""Operator entry points (mirror of snn_compiler/kernels/__init__.py:1-15)."""
from .neurons import if_lif
from .binary import pack_bits, binary_gemm
from .attention import spike_ktv_popcount, HAS_POPC
from .fused import (
    fused_bias_if_lif, fused_bias_if_lif_rate, fused_bias_if_lif_stateful,
    conv_neuron, linear_neuron, conv_bn_neuron, fold_conv_bn,
)

__all__ = [
    "if_lif", "pack_bits", "binary_gemm", "spike_ktv_popcount", "HAS_POPC",
    "fused_bias_if_lif", "fused_bias_if_lif_rate", "fused_bias_if_lif_stateful",
    "conv_neuron", "linear_neuron", "conv_bn_neuron", "fold_conv_bn",
]
