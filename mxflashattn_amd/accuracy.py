"""Error summaries for parity reports (mxflashattn/accuracy.py:9-51)."""

from __future__ import annotations

from dataclasses import asdict, dataclass
from typing import Any

import torch


@dataclass(frozen=True)
class ErrorSummary:
    sample_count: int
    finite: bool
    max_abs: float
    mean_abs: float
    p95_abs: float
    p99_abs: float
    max_relative: float

    def as_dict(self) -> dict[str, Any]:
        return asdict(self)


def summarize_error(actual: torch.Tensor, expected: torch.Tensor) -> ErrorSummary:
    """Absolute/relative error statistics; non-finite errors count as +inf."""
    if not isinstance(actual, torch.Tensor) or not isinstance(expected, torch.Tensor):
        raise TypeError("actual and expected must be torch.Tensor values")
    if actual.shape != expected.shape:
        raise ValueError("actual and expected must have identical shapes")
    if actual.numel() == 0:
        raise ValueError("cannot summarize an empty tensor")
    a = actual.detach().float().reshape(-1)
    e = expected.detach().float().reshape(-1)
    finite = bool(torch.isfinite(a).all() and torch.isfinite(e).all())
    inf = float("inf")
    abs_err = torch.nan_to_num((a - e).abs(), nan=inf, posinf=inf, neginf=inf)
    rel_err = torch.nan_to_num((a - e).abs() / e.abs().clamp_min(1e-6), nan=inf, posinf=inf,
                               neginf=inf)
    q95, q99 = torch.quantile(abs_err, torch.tensor([0.95, 0.99])).tolist()
    return ErrorSummary(
        sample_count=abs_err.numel(),
        finite=finite,
        max_abs=float(abs_err.max().item()),
        mean_abs=float(abs_err.mean().item()),
        p95_abs=float(q95),
        p99_abs=float(q99),
        max_relative=float(rel_err.max().item()),
    )
