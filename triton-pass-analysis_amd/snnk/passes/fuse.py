"""Model-level fusion pass (mirror of snn_compiler/passes/fuse.py).

Walks ``nn.Sequential`` containers (recursing into children of anything
else) and replaces adjacent layer runs by fused modules, like
snn_compiler/passes/fuse.py:107-203:

1. Conv2d -> BatchNorm2d -> Neuron            -> FusedConvBNNeuron
2. Conv2d -> Neuron                            -> FusedConvNeuron
3. Linear -> Neuron                            -> FusedLinearNeuron

and, new here, with ``fold_bn=True`` and ``conv_mfma=True`` (the defaults):

0. Conv2d(3x3, s1, p1) -> [BatchNorm2d] -> LIF/IF [-> MaxPool2d(2, 2)]
   -> FusedConvBNLIFPool: conv + folded BN + neuron (+ 2x2 max-pool) in one
   bf16-MFMA kernel, when Cin % 32 == 0, Cout % 32 == 0 and the threshold is
   a float.  The conv runs on bf16 operands with fp32 accumulation, so this
   pattern is never used when ``fold_bn=False`` (the bit-exact mode).

Neurons are this package's IFNode / LIFNode or look-alikes with
``v_threshold`` (and ``tau`` for LIF), e.g. SpikingJelly nodes, whose
``v_reset=None`` means soft reset (fuse.py:46-101).
"""
from __future__ import annotations

from typing import List, Tuple

import torch
import torch.nn as nn

from ..nn.modules import (
    IFNode, LIFNode, FusedConvNeuron, FusedConvBNNeuron, FusedLinearNeuron,
    FusedConvBNAddNeuron, FusedConvBNLIFPool,
)


def _is_if_node(m: nn.Module) -> bool:
    return isinstance(m, IFNode) or (type(m).__name__ == "IFNode" and hasattr(m, "v_threshold"))


def _is_lif_node(m: nn.Module) -> bool:
    return isinstance(m, LIFNode) or (type(m).__name__ == "LIFNode" and hasattr(m, "v_threshold")
                                      and hasattr(m, "tau"))


def _is_neuron(m: nn.Module) -> bool:
    return _is_if_node(m) or _is_lif_node(m)


def _neuron_kwargs(m: nn.Module) -> dict:
    """Constructor arguments of the fused module from a neuron module."""
    if isinstance(m, IFNode):
        return dict(neuron="if", decay=m.decay, soft_reset=m.soft_reset,
                    v_threshold=m.v_threshold, v_reset=m.v_reset, layout=m.layout)
    if isinstance(m, LIFNode):
        return dict(neuron="lif", tau=m.tau, decay=m.decay, decay_input=m.decay_input,
                    soft_reset=m.soft_reset, v_threshold=m.v_threshold, v_reset=m.v_reset,
                    layout=m.layout)
    v_th = getattr(m, "v_threshold", 1.0)
    v_reset = getattr(m, "v_reset", 0.0)
    soft = v_reset is None
    if soft:
        v_reset = 0.0
    if _is_lif_node(m):
        return dict(neuron="lif", tau=getattr(m, "tau", 2.0),
                    decay_input=getattr(m, "decay_input", True), soft_reset=soft,
                    v_threshold=v_th, v_reset=v_reset, layout="NCHW")
    return dict(neuron="if", decay=1.0, soft_reset=soft, v_threshold=v_th, v_reset=v_reset,
                layout="NCHW")


def _is_max_pool_2x2(m: nn.Module) -> bool:
    if not isinstance(m, nn.MaxPool2d):
        return False
    ks = m.kernel_size if isinstance(m.kernel_size, tuple) else (m.kernel_size,) * 2
    st = m.stride if isinstance(m.stride, tuple) else (m.stride,) * 2
    pd = m.padding if isinstance(m.padding, tuple) else (m.padding,) * 2
    dl = m.dilation if isinstance(m.dilation, tuple) else (m.dilation,) * 2
    return ks == (2, 2) and st == (2, 2) and pd == (0, 0) and dl == (1, 1) and not m.ceil_mode \
        and not m.return_indices


def _mfma_conv_ok(conv: nn.Conv2d, neuron: nn.Module) -> bool:
    return (tuple(conv.kernel_size) == (3, 3) and tuple(conv.stride) == (1, 1)
            and tuple(conv.padding) == (1, 1) and tuple(conv.dilation) == (1, 1)
            and conv.groups == 1 and conv.in_channels % 32 == 0 and conv.out_channels % 32 == 0
            and not isinstance(getattr(neuron, "v_threshold", 1.0), torch.Tensor))


def _pool_fused(conv, bn, neuron, pool: bool) -> FusedConvBNLIFPool:
    kw = _neuron_kwargs(neuron)
    kw.pop("layout", None)
    mod = FusedConvBNLIFPool(conv.eval(), bn.eval() if bn is not None else None,
                             pool="max" if pool else None, **kw)
    return mod.to(device=conv.weight.device)


def _fuse_seq(seq: nn.Sequential, *, layout: str, fold_bn: bool,
              conv_mfma: bool) -> Tuple[nn.Sequential, int]:
    out: List[nn.Module] = []
    layers = list(seq.children())
    n, i, count = len(layers), 0, 0
    while i < n:
        a = layers[i]
        if isinstance(a, nn.Conv2d):
            has_bn = i + 1 < n and isinstance(layers[i + 1], nn.BatchNorm2d)
            j = i + (2 if has_bn else 1)
            if j < n and _is_neuron(layers[j]):
                neuron = layers[j]
                bn = layers[i + 1] if has_bn else None
                if fold_bn and conv_mfma and _mfma_conv_ok(a, neuron):
                    pool = j + 1 < n and _is_max_pool_2x2(layers[j + 1])
                    out.append(_pool_fused(a, bn, neuron, pool))
                    i, count = j + (2 if pool else 1), count + 1
                    continue
                kw = _neuron_kwargs(neuron)
                kw["layout"] = layout
                if has_bn:
                    mod = FusedConvBNNeuron(a.eval(), bn.eval(), fold_bn=fold_bn, **kw)
                else:
                    mod = FusedConvNeuron(a.in_channels, a.out_channels, a.kernel_size,
                                          stride=a.stride, padding=a.padding,
                                          dilation=a.dilation, groups=a.groups,
                                          bias=a.bias is not None, **kw)
                    with torch.no_grad():
                        mod.weight.copy_(a.weight)
                        if a.bias is not None:
                            mod.bias.copy_(a.bias)
                out.append(mod.to(device=a.weight.device, dtype=a.weight.dtype))
                i, count = j + 1, count + 1
                continue
        if isinstance(a, nn.Linear) and i + 1 < n and _is_neuron(layers[i + 1]):
            kw = _neuron_kwargs(layers[i + 1])
            kw.pop("layout", None)
            mod = FusedLinearNeuron(a.in_features, a.out_features, bias=a.bias is not None, **kw)
            mod = mod.to(device=a.weight.device, dtype=a.weight.dtype)
            with torch.no_grad():
                mod.weight.copy_(a.weight)
                if a.bias is not None:
                    mod.bias.copy_(a.bias)
            out.append(mod)
            i, count = i + 2, count + 1
            continue
        if isinstance(a, nn.Sequential):
            sub, k = _fuse_seq(a, layout=layout, fold_bn=fold_bn, conv_mfma=conv_mfma)
            out.append(sub)
            count += k
        else:
            out.append(a)
        i += 1
    return nn.Sequential(*out), count


def fuse_snn_model(model: nn.Module, *, layout: str = "NCHW", fold_bn: bool = True,
                   conv_mfma: bool = True) -> Tuple[nn.Module, int]:
    """Replace every Conv/Linear -> (BN) -> Neuron (-> MaxPool) run by a fused
    module; returns ``(model, n_fused)``.  Reference: fuse.py:182-203.

    ``fold_bn=False`` keeps conv and BN as separate ops (bit-exact with the
    unfused network) and never uses the bf16 conv kernel.  Check the result
    with :func:`snnk.verify.assert_equivalent` before trusting it."""
    if not isinstance(model, nn.Sequential):
        total = 0
        for name, child in list(model.named_children()):
            new_child, k = fuse_snn_model(child, layout=layout, fold_bn=fold_bn,
                                          conv_mfma=conv_mfma)
            setattr(model, name, new_child)
            total += k
        return model, total
    return _fuse_seq(model, layout=layout, fold_bn=fold_bn, conv_mfma=conv_mfma)


def _get_submodule(model: nn.Module, path: str) -> nn.Module:
    cur = model
    for part in path.split("."):
        cur = cur[int(part)] if part.isdigit() else getattr(cur, part)
    return cur


def _set_submodule(model: nn.Module, path: str, mod: nn.Module) -> None:
    parts = path.split(".")
    cur = model
    for part in parts[:-1]:
        cur = cur[int(part)] if part.isdigit() else getattr(cur, part)
    if parts[-1].isdigit():
        cur[int(parts[-1])] = mod
    else:
        setattr(cur, parts[-1], mod)


def fuse_modules_path(model: nn.Module, fusion_groups, *, layout: str = "NCHW",
                      fold_bn: bool = True) -> int:
    """Fuse explicit module paths (reference fuse.py:225-323).

    Each group is ``(conv_path, bn_path_or_None, neuron_path[, target_path])``;
    the fused module goes to ``target_path`` (default: the neuron's path) and
    the consumed conv / BN become ``nn.Identity``.  Returns the group count."""
    done = 0
    for grp in fusion_groups:
        if len(grp) == 3:
            conv_p, bn_p, neuron_p = grp
            target_p = neuron_p
        elif len(grp) == 4:
            conv_p, bn_p, neuron_p, target_p = grp
        else:
            raise ValueError(f"fusion group must have 3 or 4 elements, got {grp}")
        conv = _get_submodule(model, conv_p)
        kw = _neuron_kwargs(_get_submodule(model, neuron_p))
        kw["layout"] = layout
        if not bn_p:
            if isinstance(conv, nn.Conv2d):
                mod = FusedConvNeuron(conv.in_channels, conv.out_channels, conv.kernel_size,
                                      stride=conv.stride, padding=conv.padding,
                                      dilation=conv.dilation, groups=conv.groups,
                                      bias=conv.bias is not None, **kw)
            elif isinstance(conv, nn.Linear):
                kw.pop("layout", None)
                mod = FusedLinearNeuron(conv.in_features, conv.out_features,
                                        bias=conv.bias is not None, **kw)
            else:
                raise TypeError(f"{conv_p} is not Conv2d or Linear: {type(conv)}")
            mod = mod.to(device=conv.weight.device, dtype=conv.weight.dtype)
            with torch.no_grad():
                mod.weight.copy_(conv.weight)
                if conv.bias is not None:
                    mod.bias.copy_(conv.bias)
        else:
            bn = _get_submodule(model, bn_p)
            if not isinstance(conv, nn.Conv2d) or not isinstance(bn, nn.BatchNorm2d):
                raise TypeError(f"{conv_p}/{bn_p}: expected Conv2d/BatchNorm2d")
            mod = FusedConvBNNeuron(conv.eval(), bn.eval(), fold_bn=fold_bn, **kw).to(
                device=conv.weight.device, dtype=conv.weight.dtype)
        _set_submodule(model, target_p, mod)
        if conv_p != target_p:
            _set_submodule(model, conv_p, nn.Identity())
        if bn_p and bn_p != target_p:
            _set_submodule(model, bn_p, nn.Identity())
        done += 1
    return done


def fuse_conv_bn_add_neuron_path(model: nn.Module, conv_p: str, bn_p: str, neuron_p: str, *,
                                 target_p: str | None = None, layout: str = "NCHW",
                                 fold_bn: bool = True) -> nn.Module:
    """(conv, bn, neuron) -> FusedConvBNAddNeuron at ``target_p`` (default the
    neuron's path); conv / BN become Identity (reference fuse.py:326-352).
    The caller's forward passes the residual: ``neuron(x, residual)``."""
    target_p = target_p or neuron_p
    conv = _get_submodule(model, conv_p)
    bn = _get_submodule(model, bn_p)
    kw = _neuron_kwargs(_get_submodule(model, neuron_p))
    kw["layout"] = layout
    mod = FusedConvBNAddNeuron(conv.eval(), bn.eval(), fold_bn=fold_bn, **kw).to(
        device=conv.weight.device, dtype=conv.weight.dtype)
    _set_submodule(model, target_p, mod)
    if conv_p != target_p:
        _set_submodule(model, conv_p, nn.Identity())
    if bn_p != target_p:
        _set_submodule(model, bn_p, nn.Identity())
    return mod
