"""Operator entry points (mirror of snn_compiler/kernels/__init__.py:1-15)."""
from .neurons import if_lif
from .fused import (
    fused_bias_if_lif, fused_bias_if_lif_rate, fused_bias_if_lif_stateful,
    conv_neuron, linear_neuron, conv_bn_neuron, fold_conv_bn,
)

__all__ = [
    "if_lif",
    "fused_bias_if_lif", "fused_bias_if_lif_rate", "fused_bias_if_lif_stateful",
    "conv_neuron", "linear_neuron", "conv_bn_neuron", "fold_conv_bn",
]
