"""Tensor-free candidate policy: which backend a workload shape would get.

Same interface and rule as the reference's ``mxflashattn/policy.py:11-111``
(``WorkloadShape``, ``DispatchPolicyConfig``, ``DispatchDecision``,
``AdaptiveDispatchPolicy.select``), kept so code that imports these names keeps
working. As in the reference, nothing at run time consults it: ``dispatch``
routes by argument checks alone. It is off by default, and when enabled it
still answers "vendor" until the thresholds are marked calibrated.

Two differences, both because of what this package contains:

- the decode candidate is ``mi355x_split_decode`` (the reference names its
  ``m1_split_kv`` kernel), eligible for the reference's decode contract: GQ in
  (2, 4, 8), head dim in (64, 128), batch and length above the thresholds;
- there is no prefill kernel here, so a prefill shape that passes the
  reference's prefill thresholds is handed to the vendor with the reason
  ``prefill_not_on_this_path`` instead of naming a chunked-prefill backend.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Literal

from .dispatch import BACKEND_MI355X
from .native import SUPPORTED_GQA, SUPPORTED_HEAD_DIMS

Phase = Literal["prefill", "decode"]
Backend = Literal["vendor", "mi355x_split_decode"]


@dataclass(frozen=True)
class WorkloadShape:
    """Shape metadata only: no tensors, no device queries."""

    phase: Phase
    batch_size: int
    query_len: int
    kv_len: int
    head_dim: int
    gqa_ratio: int

    def __post_init__(self) -> None:
        if self.phase not in ("prefill", "decode"):
            raise ValueError("phase must be 'prefill' or 'decode'")
        if min(self.batch_size, self.query_len, self.kv_len) <= 0:
            raise ValueError("batch_size, query_len, and kv_len must be positive")
        if self.head_dim <= 0 or self.gqa_ratio <= 0:
            raise ValueError("head_dim and gqa_ratio must be positive")


@dataclass(frozen=True)
class DispatchPolicyConfig:
    """Candidate thresholds (the reference's defaults); disabled by default."""

    enabled: bool = False
    calibrated: bool = False
    prefill_batch_min: int = 4
    prefill_kv_len_min: int = 512
    decode_batch_min: int = 16
    decode_kv_len_min: int = 256


@dataclass(frozen=True)
class DispatchDecision:
    backend: Backend
    reason: str
    eligible: bool
    policy_enabled: bool
    thresholds_calibrated: bool


class AdaptiveDispatchPolicy:
    def __init__(self, config: DispatchPolicyConfig | None = None) -> None:
        self.config = config if config is not None else DispatchPolicyConfig()

    def _vendor(self, reason: str, enabled: bool = True) -> DispatchDecision:
        return DispatchDecision("vendor", reason, False, enabled, self.config.calibrated)

    def select(self, shape: WorkloadShape) -> DispatchDecision:
        cfg = self.config
        if not cfg.enabled:
            return self._vendor("policy_disabled", enabled=False)
        if not cfg.calibrated:
            return self._vendor("thresholds_not_calibrated")
        if shape.phase == "prefill":
            above = (shape.batch_size >= cfg.prefill_batch_min
                     and shape.kv_len >= cfg.prefill_kv_len_min)
            return self._vendor("prefill_not_on_this_path" if above else "prefill_below_threshold")
        eligible = (shape.batch_size >= cfg.decode_batch_min
                    and shape.kv_len >= cfg.decode_kv_len_min
                    and shape.gqa_ratio in SUPPORTED_GQA
                    and shape.head_dim in SUPPORTED_HEAD_DIMS)
        if not eligible:
            return self._vendor("decode_shape_or_threshold_miss")
        return DispatchDecision(BACKEND_MI355X, "decode_threshold_match", True, True, True)
