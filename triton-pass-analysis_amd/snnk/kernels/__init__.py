"""Operator entry points (mirror of snn_compiler/kernels/__init__.py:1-15, plus
the fused conv / linear / attention operators of this library)."""
from .neurons import if_lif, if_lif_packed
from .binary import pack_bits, binary_gemm
from .attention import (spike_ktv, spike_ktv_popcount, spike_av_lif, spike_attention,
                        spike_attention_packed, spike_self_attention,
                        spike_self_attention_packed, prepare_ssa_packed, HAS_POPC)
from .conv import (conv_bn_lif_pool, conv3x3_bn_lif_nhwc, conv3x3_bn_lif_act,
                   conv3x3_image_lif, to_nhwc_bf16)
from .linear import (linear_bias_lif, linear_bias_lif_act, linear_preact, linear_preact_act,
                     linear_mean_t)
from .fused import (
    fused_bias_if_lif, fused_bias_if_lif_rate, fused_bias_if_lif_stateful,
    conv_neuron, linear_neuron, conv_bn_neuron, fold_conv_bn,
)

__all__ = [
    "if_lif", "if_lif_packed", "pack_bits", "binary_gemm",
    "spike_ktv", "spike_ktv_popcount", "spike_av_lif", "spike_attention", "spike_self_attention", "HAS_POPC",
    "spike_attention_packed", "spike_self_attention_packed", "prepare_ssa_packed",
    "conv_bn_lif_pool", "conv3x3_bn_lif_nhwc", "conv3x3_bn_lif_act", "conv3x3_image_lif",
    "to_nhwc_bf16", "linear_bias_lif", "linear_bias_lif_act", "linear_preact", "linear_preact_act",
    "linear_mean_t",
    "fused_bias_if_lif", "fused_bias_if_lif_rate", "fused_bias_if_lif_stateful",
    "conv_neuron", "linear_neuron", "conv_bn_neuron", "fold_conv_bn",
]
