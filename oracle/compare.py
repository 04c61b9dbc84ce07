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


__all__ = [
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
