"""snnk -- MI355X-native (gfx950) SNN inference kernels.

Drop-in for the operator layer of ``snn_compiler`` (Xarlley/Triton-Pass-Analysis,
snn_compiler/__init__.py:21-38): the same entry points and module classes,
backed by hand-written HIP kernels in ``libsnnk.so`` behind a C ABI
(``include/snnk.h``).  There is no fallback: an operator whose library is
missing raises.
"""
from .kernels import *  # noqa: F401,F403
from .kernels import __all__ as _kernels_all
from .nn import (  # noqa: F401
    IFNode, LIFNode, StatefulLIFNode, RateCodedLIFNode, RateCodedIFNode,
    FusedConvNeuron, FusedLinearNeuron, FusedConvBNNeuron, FusedConvBNAddNeuron,
    FusedAddNeuron, FusedConvBNLIFPool, ChunkedForward, run_chunked,
)
from .nn.attention import FusedSpikeAttention  # noqa: F401
from .verify import assert_equivalent, compare_models  # noqa: F401
from . import passes  # noqa: F401

__all__ = list(_kernels_all) + [
    "IFNode", "LIFNode", "StatefulLIFNode", "RateCodedLIFNode", "RateCodedIFNode",
    "FusedConvNeuron", "FusedLinearNeuron", "FusedConvBNNeuron", "FusedConvBNAddNeuron",
    "ChunkedForward", "run_chunked",
    "FusedAddNeuron", "FusedConvBNLIFPool", "FusedSpikeAttention",
    "assert_equivalent", "compare_models",
]
