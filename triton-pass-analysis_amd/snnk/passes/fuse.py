"""Rewrite passes that put fused modules in place of layer runs.

Public API of ``snn_compiler/passes/fuse.py``: :func:`fuse_snn_model`
(182-209), :func:`fuse_modules_path` (236-318) and
:func:`fuse_conv_bn_add_neuron_path` (321-350).

Design.  A network is rewritten by a table of rules.  A rule looks at the
children of an ``nn.Sequential`` from some position on, says how many of
them it consumes, and builds the one module that replaces them; the first
rule that matches wins, and containers that are not Sequential are entered
recursively.  The rules, in order:

  ``conv3x3_mfma``  Conv2d(3x3, stride 1, pad 1, Cin and Cout multiples of 32)
                    [-> BatchNorm2d] -> neuron with a scalar threshold
                    [-> MaxPool2d(2, 2)]          -> FusedConvBNLIFPool
                    (bf16 MFMA; only with fold_bn=True and conv_mfma=True)
  ``conv_bn``       Conv2d -> BatchNorm2d -> neuron -> FusedConvBNNeuron
  ``conv``          Conv2d -> neuron              -> FusedConvNeuron
  ``linear``        Linear -> neuron              -> FusedLinearNeuron

A neuron is this package's IFNode / LIFNode or a look-alike of the same
class name carrying ``v_threshold`` (and ``tau`` for LIF), such as
SpikingJelly's nodes, whose ``v_reset=None`` means soft reset.
:class:`NeuronSpec` turns any of them into the constructor arguments of the
fused modules.  Path-based fusion addresses modules by dotted name through
``nn.Module.get_submodule`` and reuses the same builders.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Callable, Optional, Sequence, Tuple, Union

import torch
import torch.nn as nn

from ..nn.modules import (
    IFNode, LIFNode, FusedConvNeuron, FusedConvBNNeuron, FusedLinearNeuron,
    FusedConvBNAddNeuron, FusedConvBNLIFPool,
)

Threshold = Union[float, torch.Tensor]


# ---- neurons -----------------------------------------------------------------
@dataclass(frozen=True)
class NeuronSpec:
    """Normalised description of a multi-step IF / LIF neuron module."""
    kind: str                      # "if" or "lif"
    v_threshold: Threshold
    soft_reset: bool = False
    v_reset: float = 0.0
    tau: float = 2.0
    decay: Optional[float] = None
    decay_input: bool = True
    layout: str = "NCHW"

    @staticmethod
    def kind_of(m: nn.Module) -> Optional[str]:
        """'if' / 'lif' for a neuron module, None for anything else."""
        if isinstance(m, LIFNode):
            return "lif"
        if isinstance(m, IFNode):
            return "if"
        name = type(m).__name__
        if name == "LIFNode" and hasattr(m, "v_threshold") and hasattr(m, "tau"):
            return "lif"
        if name == "IFNode" and hasattr(m, "v_threshold"):
            return "if"
        return None

    @classmethod
    def of(cls, m: nn.Module) -> "NeuronSpec":
        kind = cls.kind_of(m)
        if kind is None:
            raise TypeError(f"{type(m).__name__} is not an IF / LIF neuron module")
        if isinstance(m, (IFNode, LIFNode)):       # this package's own nodes
            return cls(kind=kind, v_threshold=m.v_threshold, soft_reset=bool(m.soft_reset),
                       v_reset=float(m.v_reset), tau=float(getattr(m, "tau", 2.0)),
                       decay=m.decay, decay_input=bool(getattr(m, "decay_input", True)),
                       layout=m.layout)
        reset = getattr(m, "v_reset", 0.0)         # look-alike: None = soft reset
        return cls(kind=kind, v_threshold=getattr(m, "v_threshold", 1.0),
                   soft_reset=reset is None, v_reset=0.0 if reset is None else float(reset),
                   tau=float(getattr(m, "tau", 2.0)),
                   decay=1.0 if kind == "if" else None,
                   decay_input=bool(getattr(m, "decay_input", True)))

    def kwargs(self, layout: Optional[str] = None) -> dict:
        """Neuron keyword arguments of the fused modules; ``layout`` is added
        for the modules that take one."""
        kw = dict(neuron=self.kind, decay=self.decay, soft_reset=self.soft_reset,
                  v_threshold=self.v_threshold, v_reset=self.v_reset)
        if self.kind == "lif":
            kw.update(tau=self.tau, decay_input=self.decay_input)
        if layout is not None:
            kw["layout"] = layout
        return kw

    @property
    def scalar_threshold(self) -> bool:
        return not isinstance(self.v_threshold, torch.Tensor)


def _is_neuron(m: nn.Module) -> bool:
    return NeuronSpec.kind_of(m) is not None


# ---- builders shared by the rules and the path fusion ---------------------
def _placed(mod: nn.Module, like: nn.Module) -> nn.Module:
    """``mod`` on the device and in the dtype of ``like``'s weight."""
    return mod.to(device=like.weight.device, dtype=like.weight.dtype)


def _with_weights(mod: nn.Module, src: nn.Module) -> nn.Module:
    with torch.no_grad():
        mod.weight.copy_(src.weight)
        if src.bias is not None:
            mod.bias.copy_(src.bias)
    return mod


def build_conv_neuron(conv: nn.Conv2d, spec: NeuronSpec, layout: str) -> FusedConvNeuron:
    mod = FusedConvNeuron(conv.in_channels, conv.out_channels, conv.kernel_size,
                          stride=conv.stride, padding=conv.padding, dilation=conv.dilation,
                          groups=conv.groups, bias=conv.bias is not None,
                          **spec.kwargs(layout))
    return _with_weights(_placed(mod, conv), conv)


def build_linear_neuron(lin: nn.Linear, spec: NeuronSpec) -> FusedLinearNeuron:
    mod = FusedLinearNeuron(lin.in_features, lin.out_features, bias=lin.bias is not None,
                            **spec.kwargs())
    return _with_weights(_placed(mod, lin), lin)


def build_conv_bn_neuron(conv: nn.Conv2d, bn: nn.BatchNorm2d, spec: NeuronSpec, layout: str,
                         fold_bn: bool, cls=FusedConvBNNeuron) -> FusedConvBNNeuron:
    return _placed(cls(conv.eval(), bn.eval(), fold_bn=fold_bn, **spec.kwargs(layout)), conv)


def build_conv_lif_pool(conv: nn.Conv2d, bn: Optional[nn.BatchNorm2d], spec: NeuronSpec,
                        pool: bool) -> FusedConvBNLIFPool:
    kw = spec.kwargs()
    mod = FusedConvBNLIFPool(conv.eval(), None if bn is None else bn.eval(),
                             pool="max" if pool else None, **kw)
    return mod.to(device=conv.weight.device)


# ---- the rule table ----------------------------------------------------------
@dataclass(frozen=True)
class Options:
    layout: str = "NCHW"
    fold_bn: bool = True
    conv_mfma: bool = True


def _pair(v) -> tuple:
    return tuple(v) if isinstance(v, (tuple, list)) else (v, v)


def _is_pool_2x2(m: nn.Module) -> bool:
    return (isinstance(m, nn.MaxPool2d) and _pair(m.kernel_size) == (2, 2)
            and _pair(m.stride) == (2, 2) and _pair(m.padding) == (0, 0)
            and _pair(m.dilation) == (1, 1) and not m.ceil_mode and not m.return_indices)


def _mfma_shape(conv: nn.Conv2d) -> bool:
    return (_pair(conv.kernel_size) == (3, 3) and _pair(conv.stride) == (1, 1)
            and _pair(conv.padding) == (1, 1) and _pair(conv.dilation) == (1, 1)
            and conv.groups == 1 and conv.in_channels % 32 == 0 and conv.out_channels % 32 == 0)


def _at(layers: Sequence[nn.Module], i: int, kind) -> bool:
    return i < len(layers) and (kind(layers[i]) if callable(kind) and not isinstance(kind, type)
                                else isinstance(layers[i], kind))


@dataclass(frozen=True)
class Rule:
    name: str
    match: Callable[[Sequence[nn.Module], int, Options], int]   # children consumed, 0 = none
    build: Callable[[Sequence[nn.Module], Options], nn.Module]


def _match_conv3x3_mfma(layers, i, opt):
    if not (opt.fold_bn and opt.conv_mfma and _at(layers, i, nn.Conv2d)
            and _mfma_shape(layers[i])):
        return 0
    j = i + 1 + (1 if _at(layers, i + 1, nn.BatchNorm2d) else 0)
    if not _at(layers, j, _is_neuron) or not NeuronSpec.of(layers[j]).scalar_threshold:
        return 0
    return j - i + 1 + (1 if _at(layers, j + 1, _is_pool_2x2) else 0)


def _build_conv3x3_mfma(run, opt):
    conv = run[0]
    bn = run[1] if isinstance(run[1], nn.BatchNorm2d) else None
    k = 2 if bn is not None else 1
    return build_conv_lif_pool(conv, bn, NeuronSpec.of(run[k]), pool=len(run) > k + 1)


def _mfma_opt(mod: nn.Module, opt: Options) -> nn.Module:
    """conv_mfma=False keeps the module's bf16 path on the vendor conv too."""
    mod.conv_mfma = opt.conv_mfma
    return mod


RULES: Tuple[Rule, ...] = (
    Rule("conv3x3_mfma", _match_conv3x3_mfma, _build_conv3x3_mfma),
    Rule("conv_bn",
         lambda L, i, o: 3 if (_at(L, i, nn.Conv2d) and _at(L, i + 1, nn.BatchNorm2d)
                               and _at(L, i + 2, _is_neuron)) else 0,
         lambda r, o: _mfma_opt(build_conv_bn_neuron(r[0], r[1], NeuronSpec.of(r[2]), o.layout,
                                                     o.fold_bn), o)),
    Rule("conv",
         lambda L, i, o: 2 if (_at(L, i, nn.Conv2d) and _at(L, i + 1, _is_neuron)) else 0,
         lambda r, o: _mfma_opt(build_conv_neuron(r[0], NeuronSpec.of(r[1]), o.layout), o)),
    Rule("linear",
         lambda L, i, o: 2 if (_at(L, i, nn.Linear) and _at(L, i + 1, _is_neuron)) else 0,
         lambda r, o: build_linear_neuron(r[0], NeuronSpec.of(r[1]))),
)


def _rewrite(module: nn.Module, opt: Options) -> Tuple[nn.Module, int]:
    """Apply the rules inside ``module``; returns the (possibly new) module and
    the number of runs replaced."""
    if not isinstance(module, nn.Sequential):
        total = 0
        for name, child in list(module.named_children()):
            new, k = _rewrite(child, opt)
            if new is not child:
                setattr(module, name, new)
            total += k
        return module, total
    layers = list(module.children())
    out, total, i = [], 0, 0
    while i < len(layers):
        for rule in RULES:
            n = rule.match(layers, i, opt)
            if n:
                out.append(rule.build(layers[i:i + n], opt))
                i, total = i + n, total + 1
                break
        else:
            new, k = _rewrite(layers[i], opt)
            out.append(new)
            i, total = i + 1, total + k
    return nn.Sequential(*out), total


def fuse_snn_model(model: nn.Module, *, layout: str = "NCHW", fold_bn: bool = True,
                   conv_mfma: bool = True) -> Tuple[nn.Module, int]:
    """Replace every Conv/Linear -> (BN) -> neuron (-> MaxPool) run inside the
    network's Sequential containers by a fused module; returns
    ``(model, n_fused)``.

    ``fold_bn=False`` keeps conv and BN as separate fp32 ops (bit-identical to
    the unfused network) and never uses the bf16 conv kernel; ``conv_mfma=False``
    keeps the vendor conv even when folding.  Check the result with
    :func:`snnk.verify.assert_equivalent` before trusting it.
    """
    return _rewrite(model, Options(layout=layout, fold_bn=fold_bn, conv_mfma=conv_mfma))


# ---- fusion by module path -----------------------------------------------------
def replace_module(model: nn.Module, path: str, new: nn.Module) -> None:
    """Put ``new`` at dotted ``path`` (Sequential / ModuleList indices are names too)."""
    parent_path, _, leaf = path.rpartition(".")
    parent = model.get_submodule(parent_path) if parent_path else model
    setattr(parent, leaf, new)


def fuse_modules_path(model: nn.Module, fusion_groups, *, layout: str = "NCHW",
                      fold_bn: bool = True) -> int:
    """Fuse explicitly named modules; returns the number of groups fused.

    Each group is ``(conv_path, bn_path or None/"", neuron_path)`` or the same
    with a fourth ``target_path`` (default: the neuron's path).  The fused
    module goes to the target; the conv and BN it absorbed become
    ``nn.Identity``, so a forward that still calls them passes its input
    through.  A Linear in the conv slot (with no BN) gives FusedLinearNeuron.
    """
    fused = 0
    for group in fusion_groups:
        if len(group) not in (3, 4):
            raise ValueError(f"a fusion group names (conv, bn, neuron[, target]); got {group!r}")
        conv_p, bn_p, neuron_p = group[:3]
        target_p = group[3] if len(group) == 4 else neuron_p
        layer = model.get_submodule(conv_p)
        spec = NeuronSpec.of(model.get_submodule(neuron_p))
        if bn_p:
            bn = model.get_submodule(bn_p)
            if not (isinstance(layer, nn.Conv2d) and isinstance(bn, nn.BatchNorm2d)):
                raise TypeError(f"({conv_p!r}, {bn_p!r}) must be a Conv2d and a BatchNorm2d, "
                                f"not {type(layer).__name__} and {type(bn).__name__}")
            new = build_conv_bn_neuron(layer, bn, spec, layout, fold_bn)
        elif isinstance(layer, nn.Conv2d):
            new = build_conv_neuron(layer, spec, layout)
        elif isinstance(layer, nn.Linear):
            new = build_linear_neuron(layer, spec)
        else:
            raise TypeError(f"{conv_p!r} must be a Conv2d or Linear, not {type(layer).__name__}")
        _install(model, new, target_p, absorbed=(conv_p, bn_p))
        fused += 1
    return fused


def _install(model: nn.Module, new: nn.Module, target_p: str, absorbed) -> None:
    replace_module(model, target_p, new)
    for p in absorbed:
        if p and p != target_p:
            replace_module(model, p, nn.Identity())


def fuse_conv_bn_add_neuron_path(model: nn.Module, conv_p: str, bn_p: str, neuron_p: str, *,
                                 target_p: str | None = None, layout: str = "NCHW",
                                 fold_bn: bool = True) -> nn.Module:
    """Fuse (conv, BN, neuron) into a FusedConvBNAddNeuron at ``target_p``
    (default: the neuron's path) and return it.  The module's forward takes
    ``(x, residual)``: the caller's forward passes the skip connection to it
    instead of adding it before the neuron."""
    target_p = target_p or neuron_p
    conv, bn = model.get_submodule(conv_p), model.get_submodule(bn_p)
    new = build_conv_bn_neuron(conv, bn, NeuronSpec.of(model.get_submodule(neuron_p)), layout,
                               fold_bn, cls=FusedConvBNAddNeuron)
    _install(model, new, target_p, absorbed=(conv_p, bn_p))
    return new
