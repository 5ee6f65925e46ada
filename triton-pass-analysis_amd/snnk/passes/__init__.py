"""Model-level fusion passes (mirror of snn_compiler/passes)."""
from .fuse import fuse_snn_model, fuse_modules_path, fuse_conv_bn_add_neuron_path
from .attention_fuse import fuse_spiking_attention

__all__ = ["fuse_snn_model", "fuse_modules_path", "fuse_conv_bn_add_neuron_path",
           "fuse_spiking_attention"]
