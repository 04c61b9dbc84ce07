"""The accuracy rule that ranks two 16-bit programs of one model.

Two bf16 (or fp16) programs of the same Transformer round their residual
streams at different points, so an elementwise gate between them measures
their combined rounding noise, not a defect: one ulp of a residual-stream
value of magnitude 4-8 is 0.03, above the 2e-2 gate.  This rule compares each
program with the same model run in fp32 instead and asks that the candidate be
no less accurate than the incumbent (the reference-order program, or the
deployed default) up to the spread of two 16-bit pipelines:

* every candidate element is finite;
* its max-abs error is within 1.25x of the incumbent's, or within the 2e-2
  gate itself;
* its mean-abs error is within 1.25x of the incumbent's (+1e-4);
* at most 1.25x as many of its elements fail the elementwise gate
  ``|err| <= 2e-2 or |err| <= 1e-2 * |ref|`` (+1e-4 of the elements).

The elementwise gate is the OR rule of the reference's comparator
(official/torch_transformer_benchmark.py:289-356, ``abs(err) <= atol`` or
``abs(err) <= rtol * abs(ref)``) at the bf16 tolerances of this build.

One rule serves two callers: the launch search's publication gate
(``autotune.hip_launch_search``) and the model-level parity tests, which
summarize their comparisons into :class:`ErrorSummary` and call
:func:`summary_no_less_accurate`.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

GATE_ATOL = 2e-2
GATE_RTOL = 1e-2
# Spread allowed between two 16-bit programs' errors against fp32.
SPREAD = 1.25
MEAN_FLOOR = 1e-4
OUTSIDE_FLOOR = 1e-4  # fraction of the elements


@dataclass(frozen=True)
class ErrorSummary:
    """Errors of one output against an fp32 reference of the same model."""

    max_abs: float  # +inf when an element is not finite
    mean_abs: float
    outside: int  # elements failing the elementwise gate (non-finite ones included)
    total: int
    finite: bool


def summarize_errors(
    output: torch.Tensor, reference: torch.Tensor, *, atol: float = GATE_ATOL, rtol: float = GATE_RTOL
) -> ErrorSummary:
    """Errors of ``output`` against ``reference`` (same shape)."""

    if output.shape != reference.shape:
        raise ValueError(f"shape mismatch: {tuple(output.shape)} vs {tuple(reference.shape)}")
    out = output.detach().float()
    ref = reference.detach().float().to(out.device)
    finite_mask = torch.isfinite(out) & torch.isfinite(ref)
    err = (out - ref).abs()
    ok = finite_mask & ((err <= atol) | (err <= rtol * ref.abs()))
    finite = bool(finite_mask.all())
    total = out.numel()
    if total == 0:
        return ErrorSummary(0.0, 0.0, 0, 0, True)
    safe = torch.where(finite_mask, err, torch.zeros_like(err))
    return ErrorSummary(
        max_abs=float(safe.max()) if finite else float("inf"),
        mean_abs=float(safe.mean()) if finite else float("inf"),
        outside=int((~ok).sum()),
        total=total,
        finite=finite,
    )


def gate_ratio(output: torch.Tensor, reference: torch.Tensor, *, atol: float, rtol: float) -> float:
    """How far ``output`` is from failing the elementwise OR gate: the largest
    over elements of min(|err| / atol, |err| / (rtol |ref|)), so the gate
    passes exactly when the ratio is at most 1 (the continuous figure the
    reference reports with its measurements,
    benchmarking/measurement_core.py:182-224).  An element with a zero
    allowance counts 0 when its error is 0 and infinity otherwise; a
    non-finite element makes the ratio infinite."""

    out = output.detach().float()
    ref = reference.detach().float().to(out.device)
    if out.shape != ref.shape:
        return float("inf")
    if out.numel() == 0:
        return 0.0
    if not bool((torch.isfinite(out) & torch.isfinite(ref)).all()):
        return float("inf")
    err = (out - ref).abs()
    zero_rule = torch.where(err == 0, torch.zeros_like(err), torch.full_like(err, float("inf")))
    absolute = err / atol if atol > 0 else zero_rule
    allowance = rtol * ref.abs()
    relative = torch.where(allowance > 0, err / allowance.clamp_min(torch.finfo(torch.float32).tiny), zero_rule)
    return float(torch.minimum(absolute, relative).max())


def summary_no_less_accurate(candidate: ErrorSummary, incumbent: ErrorSummary) -> bool:
    """The rule above on precomputed summaries (same reference, same shape)."""

    if candidate.total != incumbent.total:
        raise ValueError("summaries of different outputs")
    if not candidate.finite:
        return False
    return (
        candidate.max_abs <= max(GATE_ATOL, SPREAD * incumbent.max_abs)
        and candidate.mean_abs <= SPREAD * incumbent.mean_abs + MEAN_FLOOR
        and candidate.outside <= SPREAD * incumbent.outside + OUTSIDE_FLOOR * candidate.total
    )


def no_less_accurate(candidate: torch.Tensor, incumbent: torch.Tensor, reference: torch.Tensor) -> bool:
    """``candidate`` is no less accurate than ``incumbent`` against the fp32
    ``reference`` of the same model and input."""

    return summary_no_less_accurate(
        summarize_errors(candidate, reference), summarize_errors(incumbent, reference)
    )


__all__ = [
    "ErrorSummary",
    "GATE_ATOL",
    "GATE_RTOL",
    "gate_ratio",
    "no_less_accurate",
    "summarize_errors",
    "summary_no_less_accurate",
]
