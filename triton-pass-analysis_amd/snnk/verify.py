"""Check that an accelerated network computes what the original one does.

Public API of ``snn_compiler/verify.py:62-175``: :func:`compare_models`
returns a report with the keys ``ref_shape``, ``fast_shape``,
``shape_match``, ``max_abs_diff``, ``mean_abs_diff``, ``rel_max``,
``argmax_agree`` (None unless the output ends in a class axis),
``spike_mismatch_frac`` (None unless both outputs are spike trains) and
``bit_exact``; :func:`assert_equivalent` raises AssertionError when the
accelerated network is not equivalent at the requested tolerance.

Design.  Both networks run on the same input through one driver
(:class:`_Probe`) that clears neuron state before and after the call and
reduces the output to a single float64 tensor on the reference's device;
:class:`Report` gathers every statistic in one pass.  A failure is explained
by the *shape* of the error rather than its size alone: a handful of flipped
threshold-crossings (folded BN, bf16 operands) leaves the normalised RMS
error small and the class decision intact, while a wiring mistake (residual
on the wrong side of a neuron, a different reduction over T) disturbs most
of the output.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field
from typing import Any, Iterator, Optional

import torch

# normalised RMS error below which a failed check is called numeric drift
_NUMERIC_RMS = 0.1
# and the class agreement it must keep
_NUMERIC_AGREE = 0.9


def _state_holders(model) -> Iterator[Any]:
    root = getattr(model, "_orig_mod", model)   # torch.compile wrapper
    if isinstance(root, torch.nn.Module):
        yield from (m for m in root.modules() if m is not root)


def reset_states(model) -> None:
    """Clear the membrane state of every submodule that keeps one: any module
    with a ``reset()`` method (this package's stateful nodes, SpikingJelly's
    memory modules)."""
    for m in _state_holders(model):
        fn = getattr(m, "reset", None)
        if callable(fn):
            fn()


class _Probe:
    """Runs one network on one input with fresh neuron state."""

    def __init__(self, model):
        self.model = model

    @staticmethod
    def _single(out) -> torch.Tensor:
        while isinstance(out, (tuple, list)) and out:
            out = out[0]
        if isinstance(out, dict) and out:
            out = next(iter(out.values()))
        if not isinstance(out, torch.Tensor):
            raise TypeError(f"model output is not a tensor (got {type(out)})")
        return out

    @torch.no_grad()
    def __call__(self, x) -> torch.Tensor:
        reset_states(self.model)
        try:
            return self._single(self.model(x)).detach()
        finally:
            reset_states(self.model)


def _is_spike_train(t: torch.Tensor) -> bool:
    """Every value is -1, 0 or 1 (binary or ternary spikes)."""
    if t.numel() == 0:
        return False
    return bool(((t == 0) | (t == 1) | (t == -1)).all())


@dataclass
class Report:
    ref_shape: tuple
    fast_shape: tuple
    shape_match: bool
    max_abs_diff: float = math.inf
    mean_abs_diff: float = math.inf
    rel_max: float = math.inf
    argmax_agree: Optional[float] = None
    spike_mismatch_frac: Optional[float] = None
    bit_exact: bool = False
    rms_rel: float = math.inf              # ||fast - ref||_2 / ||ref||_2
    extra: dict = field(default_factory=dict)

    @classmethod
    def of(cls, ref: torch.Tensor, fast: torch.Tensor, logits: bool) -> "Report":
        rep = cls(tuple(ref.shape), tuple(fast.shape), tuple(ref.shape) == tuple(fast.shape))
        if not rep.shape_match:
            return rep
        a = ref.double()
        b = fast.to(device=ref.device).double()
        err = (b - a).abs()
        n = a.numel()
        peak = float(a.abs().max()) if n else 0.0
        rep.max_abs_diff = float(err.max()) if n else 0.0
        rep.mean_abs_diff = float(err.mean()) if n else 0.0
        rep.rel_max = rep.max_abs_diff / (peak + 1e-12)
        rep.bit_exact = bool(torch.equal(ref, fast.to(device=ref.device, dtype=ref.dtype)))
        norm = float(a.norm()) if n else 0.0
        rep.rms_rel = float(err.norm()) / norm if norm > 0 else (0.0 if rep.bit_exact else math.inf)
        if logits and a.ndim >= 2 and a.shape[-1] >= 2:
            rep.argmax_agree = float((a.argmax(-1) == b.argmax(-1)).double().mean())
        if _is_spike_train(ref) and _is_spike_train(fast):
            rep.spike_mismatch_frac = float((a != b).double().mean())
        return rep

    def as_dict(self) -> dict[str, Any]:
        d = {k: getattr(self, k) for k in ("ref_shape", "fast_shape", "shape_match",
                                           "max_abs_diff", "mean_abs_diff", "rel_max",
                                           "argmax_agree", "spike_mismatch_frac", "bit_exact",
                                           "rms_rel")}
        d.update(self.extra)
        return d

    def summary(self) -> str:
        words = [f"shape_match={self.shape_match}", f"max|d|={self.max_abs_diff:.3e}",
                 f"rel={self.rel_max:.3e}", f"rms_rel={self.rms_rel:.3e}"]
        if self.argmax_agree is not None:
            words.append(f"top1-agree={100 * self.argmax_agree:.2f}%")
        if self.spike_mismatch_frac is not None:
            words.append(f"spike-mismatch={100 * self.spike_mismatch_frac:.2f}%")
        return "  ".join(words)

    def diagnosis(self) -> str:
        """Most likely cause of a failed check, from the shape of the error."""
        keeps_class = self.argmax_agree is None or self.argmax_agree >= _NUMERIC_AGREE
        if self.rms_rel <= _NUMERIC_RMS and keeps_class:
            return ("numeric drift: the error is a small fraction of the output and the class "
                    "decision holds, as when folded BN or bf16 operands move a few spikes across "
                    "the threshold; pass require_bitexact=False with an atol if that is "
                    "acceptable, or build the fused network with fold_bn=False")
        return ("topology: the error is a large fraction of the output, as when a residual is "
                "added on the other side of a neuron, a downsample path gains or loses its "
                "neuron, or the output is reduced over T differently; compare the networks "
                "layer by layer to find the first divergence")


@torch.no_grad()
def compare_models(reference, fast, example_input, *, reduce_logits: bool = True) -> dict[str, Any]:
    """Run both networks on ``example_input`` and report how their outputs
    differ; never raises on a mismatch.  Reference API:
    snn_compiler/verify.py:62-109."""
    ref = _Probe(reference)(example_input)
    out = _Probe(fast)(example_input)
    return Report.of(ref, out, reduce_logits).as_dict()


@torch.no_grad()
def assert_equivalent(reference, fast, example_input, *, atol: float = 0.0,
                      require_bitexact: bool = True, min_argmax_agree: float = 1.0,
                      verbose: bool = True) -> dict[str, Any]:
    """Raise AssertionError unless ``fast`` reproduces ``reference``.

    Reference API: snn_compiler/verify.py:124-175.  The outputs must be
    bit-identical, or (``require_bitexact=False``) within ``atol`` element by
    element; a class axis must also keep ``min_argmax_agree`` of its top-1
    decisions.  Returns the report of :func:`compare_models`.
    """
    ref = _Probe(reference)(example_input)
    out = _Probe(fast)(example_input)
    rep = Report.of(ref, out, True)
    if verbose:
        print("[snnk.verify] " + rep.summary())
    if not rep.shape_match:
        raise AssertionError(
            f"output shapes differ: reference={rep.ref_shape} vs fast={rep.fast_shape}; the "
            "accelerated network is wired differently (residual or downsample path, or the "
            "reduction over time)")
    within = rep.bit_exact if require_bitexact else rep.max_abs_diff <= atol
    agrees = rep.argmax_agree is None or rep.argmax_agree >= min_argmax_agree
    if not (within and agrees):
        raise AssertionError(f"accelerated model is not equivalent: {rep.summary()}\n"
                             f"  likely cause -> {rep.diagnosis()}")
    return rep.as_dict()
