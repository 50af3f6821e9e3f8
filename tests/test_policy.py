"""The tensor-free candidate policy (mirrors tests/test_policy.py of the
reference; the decode candidate is this package's backend, and prefill shapes
stay with the vendor since no prefill kernel exists here)."""

import pytest

from mxflashattn_amd import AdaptiveDispatchPolicy, DispatchPolicyConfig, WorkloadShape
from mxflashattn_amd.dispatch import BACKEND_MI355X


def shape(**overrides):
    values = dict(phase="prefill", batch_size=8, query_len=512, kv_len=1024, head_dim=128,
                  gqa_ratio=4)
    values.update(overrides)
    return WorkloadShape(**values)


def calibrated():
    return AdaptiveDispatchPolicy(DispatchPolicyConfig(enabled=True, calibrated=True))


def test_policy_is_safe_by_default():
    decision = AdaptiveDispatchPolicy().select(shape(phase="decode", query_len=1))
    assert (decision.backend, decision.reason) == ("vendor", "policy_disabled")
    assert not decision.eligible and not decision.policy_enabled


def test_enabled_policy_falls_back_until_thresholds_are_calibrated():
    decision = AdaptiveDispatchPolicy(DispatchPolicyConfig(enabled=True)).select(
        shape(phase="decode", query_len=1, batch_size=32))
    assert (decision.backend, decision.reason) == ("vendor", "thresholds_not_calibrated")
    assert decision.policy_enabled and not decision.thresholds_calibrated


def test_calibrated_policy_selects_decode_candidate_only_for_supported_shapes():
    policy = calibrated()
    decision = policy.select(shape(phase="decode", batch_size=32, query_len=1, kv_len=1024))
    assert (decision.backend, decision.reason, decision.eligible) == (
        BACKEND_MI355X, "decode_threshold_match", True)
    for miss in (dict(gqa_ratio=7), dict(gqa_ratio=1), dict(head_dim=256), dict(batch_size=15),
                 dict(kv_len=255)):
        got = policy.select(shape(**{**dict(phase="decode", batch_size=32, query_len=1,
                                            kv_len=1024), **miss}))
        assert (got.backend, got.reason) == ("vendor", "decode_shape_or_threshold_miss"), miss
    # The thresholds are inclusive.
    assert policy.select(shape(phase="decode", batch_size=16, kv_len=256)).eligible


def test_calibrated_policy_keeps_prefill_with_the_vendor():
    policy = calibrated()
    assert policy.select(shape()).reason == "prefill_not_on_this_path"
    assert policy.select(shape(batch_size=1)).reason == "prefill_below_threshold"
    assert policy.select(shape(kv_len=128)).reason == "prefill_below_threshold"
    assert all(policy.select(s).backend == "vendor" for s in (shape(), shape(batch_size=1)))


@pytest.mark.parametrize("kwargs", [
    {"phase": "other"}, {"batch_size": 0}, {"query_len": 0}, {"kv_len": 0}, {"head_dim": 0},
    {"gqa_ratio": -1},
])
def test_workload_shape_rejects_invalid_metadata(kwargs):
    with pytest.raises(ValueError):
        shape(**kwargs)
