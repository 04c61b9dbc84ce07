"""Comparators (test infrastructure).

official_compare restates compare_outputs of
official/torch_transformer_benchmark.py:289-356: an element passes when
``abs(err) <= atol`` OR ``abs(err) <= rtol * abs(ref)`` (not torch.isclose's
sum), both values must be finite.  The official defaults are rtol 0.02 and
atol 0.002 (official :618-619).

The parity gates of this build use the same OR rule with the tolerances of
the project brief: bf16/fp16 outputs pass with atol 2e-2 / rtol 1e-2, fp32
outputs with atol 1e-4 / rtol 1e-4.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

OFFICIAL_RTOL = 0.02
OFFICIAL_ATOL = 0.002
BF16_ATOL = 2e-2
BF16_RTOL = 1e-2
FP32_ATOL = 1e-4
FP32_RTOL = 1e-4


@dataclass(frozen=True)
class Comparison:
    passed: bool
    total_elements: int
    failed_elements: int
    max_abs_error: float
    max_relative_error: float
    mean_abs_error: float
    worst_index: tuple[int, ...]

    @property
    def failed_ratio(self) -> float:
        return self.failed_elements / max(self.total_elements, 1)


def official_compare(
    reference: torch.Tensor, candidate: torch.Tensor, *, rtol: float, atol: float
) -> Comparison:
    if reference.shape != candidate.shape:
        raise AssertionError(
            f"shape mismatch: reference={tuple(reference.shape)}, candidate={tuple(candidate.shape)}"
        )
    ref = reference.detach().float().cpu()
    opt = candidate.detach().float().cpu()
    finite = torch.isfinite(ref) & torch.isfinite(opt)
    err = (opt - ref).abs()
    ok = finite & ((err <= atol) | (err <= rtol * ref.abs()))
    failed = int((~ok).sum().item())
    safe_err = torch.where(finite, err, torch.full_like(err, float("inf")))
    flat = int(safe_err.reshape(-1).argmax().item()) if safe_err.numel() else 0
    index = []
    for size in reversed(ref.shape):
        index.append(flat % size)
        flat //= size
    rel = err / ref.abs().clamp_min(1e-12)
    return Comparison(
        passed=failed == 0,
        total_elements=ref.numel(),
        failed_elements=failed,
        max_abs_error=float(safe_err.max().item()) if safe_err.numel() else 0.0,
        max_relative_error=float(rel.max().item()) if rel.numel() else 0.0,
        mean_abs_error=float(err.mean().item()) if err.numel() else 0.0,
        worst_index=tuple(reversed(index)),
    )


def gate_tolerances(dtype: torch.dtype) -> tuple[float, float]:
    """(atol, rtol) of the parity gate for an output dtype."""

    if dtype in (torch.bfloat16, torch.float16):
        return BF16_ATOL, BF16_RTOL
    return FP32_ATOL, FP32_RTOL


def parity_gate(reference: torch.Tensor, candidate: torch.Tensor, dtype: torch.dtype) -> Comparison:
    atol, rtol = gate_tolerances(dtype)
    return official_compare(reference, candidate, rtol=rtol, atol=atol)


@dataclass(frozen=True)
class ModelParity:
    """End-to-end parity of a 16-bit model output.

    ``candidate`` and ``reference_path`` (the official op order run in the
    same 16-bit dtype) are both compared with ``exact`` (the same forward in
    fp32 from the same rounded weights and inputs).  The candidate passes when
    it is no less accurate than the reference path, up to the run-to-run
    spread of two 16-bit pipelines: max-abs within 1.25x of the reference
    path's (or within the 2e-2 gate), mean-abs within 1.25x (+1e-4), and at
    most 1.25x as many elements outside the elementwise 2e-2 / 1e-2 gate
    (+1e-4 of the elements).
    A strict elementwise gate between two 16-bit pipelines is below the noise
    floor: a one-ulp rounding flip of a residual-stream value of magnitude
    4-8 is 0.03-0.06 before the final LayerNorm.
    """

    candidate: Comparison
    reference_path: Comparison
    candidate_vs_reference_path: Comparison

    @property
    def passed(self) -> bool:
        c, r = self.candidate, self.reference_path
        return (
            c.max_abs_error <= max(BF16_ATOL, 1.25 * r.max_abs_error)
            and c.mean_abs_error <= 1.25 * r.mean_abs_error + 1e-4
            and c.failed_elements <= 1.25 * r.failed_elements + 1e-4 * c.total_elements
        )

    def summary(self) -> str:
        c, r, x = self.candidate, self.reference_path, self.candidate_vs_reference_path
        return (
            f"vs fp32: candidate max_abs={c.max_abs_error:.4g} mean_abs={c.mean_abs_error:.3g} "
            f"gate_failures={c.failed_elements}/{c.total_elements}; reference path max_abs="
            f"{r.max_abs_error:.4g} mean_abs={r.mean_abs_error:.3g} gate_failures={r.failed_elements}; "
            f"candidate vs reference path max_abs={x.max_abs_error:.4g} gate_failures={x.failed_elements}"
        )


def model_parity(
    exact: torch.Tensor, reference_path: torch.Tensor, candidate: torch.Tensor
) -> ModelParity:
    atol, rtol = BF16_ATOL, BF16_RTOL
    return ModelParity(
        candidate=official_compare(exact, candidate, rtol=rtol, atol=atol),
        reference_path=official_compare(exact, reference_path, rtol=rtol, atol=atol),
        candidate_vs_reference_path=official_compare(reference_path, candidate, rtol=rtol, atol=atol),
    )


__all__ = [
    "ModelParity",
    "model_parity",
    "BF16_ATOL",
    "BF16_RTOL",
    "Comparison",
    "FP32_ATOL",
    "FP32_RTOL",
    "OFFICIAL_ATOL",
    "OFFICIAL_RTOL",
    "gate_tolerances",
    "official_compare",
    "parity_gate",
]
