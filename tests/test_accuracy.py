"""ErrorSummary / summarize_error: the statistics behind the parity reports.

Each statistic is checked against numpy computed independently on the same
errors, over seeded random tensors of several shapes and dtypes, plus the
edge cases the contract names (non-finite values, empty or mismatched inputs,
inputs that are not tensors). The error texts are the reference's contract
(mxflashattn/accuracy.py).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from mxflashattn_amd.accuracy import ErrorSummary, summarize_error


def numpy_stats(actual: torch.Tensor, expected: torch.Tensor) -> dict:
    a = actual.double().numpy().ravel()
    e = expected.double().numpy().ravel()
    err = np.abs(a - e)
    return {
        "max_abs": err.max(),
        "mean_abs": err.mean(),
        "p95_abs": np.quantile(err, 0.95),
        "p99_abs": np.quantile(err, 0.99),
        "max_relative": (err / np.maximum(np.abs(e), 1e-6)).max(),
    }


@pytest.mark.parametrize("shape", [(7,), (3, 5), (2, 4, 8, 16)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
def test_statistics_equal_numpy_on_random_tensors(shape, dtype):
    g = torch.Generator().manual_seed(hash((shape, str(dtype))) % 10_000)
    expected = torch.randn(shape, generator=g).to(dtype)
    actual = (expected.float() + 0.01 * torch.randn(shape, generator=g)).to(dtype)
    got = summarize_error(actual, expected)
    ref = numpy_stats(actual.float(), expected.float())
    assert got.sample_count == expected.numel()
    assert got.finite
    for key, value in ref.items():
        assert getattr(got, key) == pytest.approx(value, rel=1e-5, abs=1e-7), key
    assert got.mean_abs <= got.p95_abs <= got.p99_abs <= got.max_abs


def test_identical_tensors_have_zero_error():
    x = torch.linspace(-3, 3, 101)
    got = summarize_error(x, x.clone())
    assert (got.max_abs, got.mean_abs, got.p95_abs, got.p99_abs, got.max_relative) == (
        0.0, 0.0, 0.0, 0.0, 0.0)


def test_relative_error_uses_a_floor_on_tiny_expected_values():
    # |e| below 1e-6 is treated as 1e-6, so a zero expectation gives a large
    # but finite relative error.
    got = summarize_error(torch.tensor([1e-3, 2.0]), torch.tensor([0.0, 2.0]))
    assert got.max_relative == pytest.approx(1e-3 / 1e-6)
    assert got.finite


@pytest.mark.parametrize("bad", [float("nan"), float("inf"), float("-inf")])
@pytest.mark.parametrize("where", ["actual", "expected"])
def test_non_finite_values_count_as_infinite_error(bad, where):
    clean = torch.tensor([0.5, -1.0, 2.0])
    dirty = clean.clone()
    dirty[1] = bad
    actual, expected = (dirty, clean) if where == "actual" else (clean, dirty)
    got = summarize_error(actual, expected)
    assert not got.finite
    assert got.max_abs == float("inf")
    assert got.sample_count == 3


def test_summary_is_a_frozen_record_with_a_dict_view():
    got = summarize_error(torch.tensor([1.0, 3.0]), torch.tensor([1.5, 3.0]))
    assert isinstance(got, ErrorSummary)
    as_dict = got.as_dict()
    assert set(as_dict) == {"sample_count", "finite", "max_abs", "mean_abs", "p95_abs",
                            "p99_abs", "max_relative"}
    assert as_dict["max_abs"] == pytest.approx(0.5)
    with pytest.raises(AttributeError):
        got.max_abs = 0.0  # frozen


@pytest.mark.parametrize("actual,expected,error,text", [
    (torch.empty(0, 3), torch.empty(0, 3), ValueError, "empty"),
    (torch.zeros(4), torch.zeros(2, 2), ValueError, "identical shapes"),
    (torch.zeros(2), torch.zeros(3), ValueError, "identical shapes"),
    ([0.0, 1.0], torch.zeros(2), TypeError, "torch.Tensor"),
    (torch.zeros(2), np.zeros(2), TypeError, "torch.Tensor"),
])
def test_inputs_outside_the_contract_are_rejected(actual, expected, error, text):
    with pytest.raises(error, match=text):
        summarize_error(actual, expected)
