"""Equivalence check between a reference network and its accelerated version.

Mirrors ``snn_compiler/verify.py:62-175``: :func:`compare_models` runs both
models on one input and reports ``shape_match``, ``max_abs_diff``,
``mean_abs_diff``, ``rel_max``, ``argmax_agree`` (None when the output is not
logits-like), ``spike_mismatch_frac`` (None unless both outputs look like 0/1
spikes) and ``bit_exact``; :func:`assert_equivalent` raises AssertionError
when the accelerated model is not equivalent within the requested tolerance,
with a hint at the likely cause (a small numeric difference points at BN
folding or bf16 operands flipping near-threshold spikes, a large one at a
mis-wired topology).
"""
from __future__ import annotations

from typing import Any

import torch


def _reset(model) -> None:
    """Reset neuron state of every submodule that keeps one (``reset()``)."""
    root = getattr(model, "_orig_mod", model)
    if not isinstance(root, torch.nn.Module):
        return
    for m in root.modules():
        fn = getattr(m, "reset", None)
        if callable(fn) and m is not root:
            fn()


def _as_tensor(out) -> torch.Tensor:
    if isinstance(out, (tuple, list)):
        out = out[0]
    if not isinstance(out, torch.Tensor):
        raise TypeError(f"model output is not a tensor (got {type(out)})")
    return out


@torch.no_grad()
def _run(model, x) -> torch.Tensor:
    _reset(model)
    out = _as_tensor(model(x))
    _reset(model)
    return out.float()


def _looks_like_spikes(t: torch.Tensor) -> bool:
    u = torch.unique(t)
    return u.numel() <= 3 and float(u.abs().max()) <= 1.0 + 1e-6


@torch.no_grad()
def compare_models(reference, fast, example_input, *, reduce_logits: bool = True) -> dict[str, Any]:
    """Run both models on ``example_input`` and return the difference report.

    Reference: snn_compiler/verify.py:62-121 (same keys; never raises on a
    mismatch).
    """
    y_ref = _run(reference, example_input)
    y_fast = _run(fast, example_input)
    rep: dict[str, Any] = {
        "ref_shape": tuple(y_ref.shape),
        "fast_shape": tuple(y_fast.shape),
        "shape_match": tuple(y_ref.shape) == tuple(y_fast.shape),
    }
    if not rep["shape_match"]:
        rep.update(max_abs_diff=float("inf"), mean_abs_diff=float("inf"), rel_max=float("inf"),
                   argmax_agree=None, spike_mismatch_frac=None, bit_exact=False)
        return rep
    y_fast = y_fast.to(y_ref.device)
    d = (y_ref - y_fast).abs()
    max_abs = float(d.max()) if d.numel() else 0.0
    rep["max_abs_diff"] = max_abs
    rep["mean_abs_diff"] = float(d.mean()) if d.numel() else 0.0
    rep["rel_max"] = max_abs / (float(y_ref.abs().max()) + 1e-12 if y_ref.numel() else 1.0)
    rep["bit_exact"] = max_abs == 0.0
    rep["argmax_agree"] = None
    if reduce_logits and y_ref.ndim >= 2 and y_ref.shape[-1] >= 2:
        rep["argmax_agree"] = float((y_ref.argmax(-1) == y_fast.argmax(-1)).float().mean())
    rep["spike_mismatch_frac"] = (
        float((y_ref != y_fast).float().mean())
        if y_ref.numel() and _looks_like_spikes(y_ref) and _looks_like_spikes(y_fast) else None)
    return rep


def _format(rep: dict[str, Any]) -> str:
    parts = [f"shape_match={rep['shape_match']}",
             f"max|d|={rep['max_abs_diff']:.3e}",
             f"rel={rep['rel_max']:.3e}"]
    if rep.get("argmax_agree") is not None:
        parts.append(f"top1-agree={rep['argmax_agree'] * 100:.2f}%")
    if rep.get("spike_mismatch_frac") is not None:
        parts.append(f"spike-mismatch={rep['spike_mismatch_frac'] * 100:.2f}%")
    return "  ".join(parts)


@torch.no_grad()
def assert_equivalent(reference, fast, example_input, *, atol: float = 0.0,
                      require_bitexact: bool = True, min_argmax_agree: float = 1.0,
                      verbose: bool = True) -> dict[str, Any]:
    """Assert that ``fast`` reproduces ``reference`` on ``example_input``.

    Reference: snn_compiler/verify.py:124-175.  By default the outputs must
    be bit-identical; with ``require_bitexact=False`` the max abs difference
    must be <= ``atol``.  Whenever the output is logits-like the top-1
    agreement must also reach ``min_argmax_agree``.  Returns the report.
    """
    rep = compare_models(reference, fast, example_input)
    if verbose:
        print("[snnk.verify] " + _format(rep))
    if not rep["shape_match"]:
        raise AssertionError(
            f"output shapes differ: reference={rep['ref_shape']} vs fast={rep['fast_shape']}; "
            "the accelerated topology almost certainly differs (residual/downsample wiring or "
            "the final reduction over time)")
    ok = rep["bit_exact"] if require_bitexact else rep["max_abs_diff"] <= atol
    if rep["argmax_agree"] is not None and rep["argmax_agree"] < min_argmax_agree:
        ok = False
    if not ok:
        agree = rep["argmax_agree"]
        small = (rep["max_abs_diff"] > 0 and rep["rel_max"] <= 0.05
                 and (agree is None or agree >= 0.9))
        if small:
            hint = ("the difference is small and top-1 barely moves: most likely numeric "
                    "(folded BN or bf16 operands flipping spikes that sit on the threshold); "
                    "use require_bitexact=False with a suitable atol if that is acceptable")
        else:
            hint = ("the difference is large: most likely a topology error (residual added "
                    "before vs after the neuron, downsample with or without its own neuron, "
                    "or a different reduction over time); compare_models with forward hooks "
                    "localises the first diverging layer")
        raise AssertionError("accelerated model is not equivalent: " + _format(rep) + "\n  -> " + hint)
    return rep
