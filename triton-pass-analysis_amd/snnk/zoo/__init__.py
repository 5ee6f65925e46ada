"""Model zoo (mirror of snn_compiler/zoo, VGG family)."""
from .vgg import (VGGSNN, FusedVGGSNN, vgg11_snn, vgg13_snn, vgg16_snn, vgg19_snn,
                  seeded_init_, VGG16_CFG)

__all__ = ["VGGSNN", "FusedVGGSNN", "vgg11_snn", "vgg13_snn", "vgg16_snn", "vgg19_snn",
           "seeded_init_", "VGG16_CFG"]
