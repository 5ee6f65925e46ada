"""Module layer (mirror of snn_compiler/nn/__init__.py)."""
from .modules import (
    IFNode, LIFNode, StatefulLIFNode, RateCodedLIFNode, RateCodedIFNode,
    FusedConvNeuron, FusedLinearNeuron, FusedConvBNNeuron, FusedConvBNAddNeuron,
    FusedAddNeuron, FusedConvBNLIFPool,
)
from .chunked import ChunkedForward, run_chunked

__all__ = [
    "IFNode", "LIFNode", "StatefulLIFNode", "RateCodedLIFNode", "RateCodedIFNode",
    "FusedConvNeuron", "FusedLinearNeuron", "FusedConvBNNeuron", "FusedConvBNAddNeuron",
    "FusedAddNeuron", "FusedConvBNLIFPool", "ChunkedForward", "run_chunked",
]
