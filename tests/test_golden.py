"""The oracle against the committed golden vectors (CPU).

tests/golden/reference_vectors.npz holds inputs and outputs of the
reference's own ATen build (csrc/mxmac: paged_kv.cpp:53-126,
attention_forward.cpp) on small seeded decode cases, written by
tests/golden/make_golden.py. These tests need neither the reference nor its
build: the restatement in oracle/reference_port.py and the fp64 C oracle must
reproduce every output to one rounding step of the output type, and the
restated append must rewrite exactly the cache rows the reference rewrote,
bit for bit. Where oracle/_ref is built, it must regenerate the file bit for
bit (the fixture is current).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from golden import make_golden, vectors
from oracle import c_oracle, ref_aten, reference_port

CASES = vectors.load()

# One rounding step of each output type at |x| < 4 (the two fp32 computations
# agree to ~1e-6 before the final rounding).
ULP = {torch.float32: 2e-5, torch.float16: 4e-3, torch.bfloat16: 3.2e-2}


def port_output(case: dict, block_table=None):
    """Runs the restatement on a case; returns (output, k_cache, v_cache, seqlens)."""
    kind = case["kind"]
    if kind == "varlen":
        out = reference_port.attention_varlen(
            case["q"], case["k"], case["v"], case["cu_seqlens_q"].tolist(),
            case["cu_seqlens_k"].tolist(), softmax_scale=case["scale"], causal=case["causal"])
        return out, None, None, None
    if kind == "func":
        out = reference_port.attention_batched(case["q"], case["k"], case["v"],
                                               softmax_scale=case["scale"],
                                               causal=case["causal"])
        return out, None, None, None
    kc, vc = case["k_cache"].clone(), case["v_cache"].clone()
    sl = case["cache_seqlens"].clone()
    bt = case.get("block_table") if block_table is None else block_table
    out = reference_port.attention_kvcache(case["q"], kc, vc, k=case.get("k"), v=case.get("v"),
                                           cache_seqlens=sl, block_table=bt,
                                           softmax_scale=case["scale"], causal=case["causal"])
    return out, kc, vc, sl


def rewritten_rows(before: torch.Tensor, after: torch.Tensor) -> torch.Tensor:
    diff = (before.view(torch.int16) != after.view(torch.int16)).flatten(2).any(-1)
    return diff.nonzero().to(torch.int64)


def test_the_vectors_cover_every_route():
    kinds = {case["kind"] for case in CASES.values()}
    assert kinds == {"kvcache", "varlen", "func"}
    assert {case["dtype"] for case in CASES.values()} == {torch.float16, torch.bfloat16}
    assert any("k" in case and case["kind"] == "kvcache" for case in CASES.values())
    assert any(case["scale"] == 0.0 for case in CASES.values())


@pytest.mark.parametrize("name", vectors.names())
def test_port_reproduces_reference_vectors(name):
    case = CASES[name]
    out, kc, vc, sl = port_output(case)
    want = case["out"]
    assert out.shape == want.shape and out.dtype == want.dtype
    err = (out.float() - want.float()).abs().max().item()
    assert err <= ULP[case["dtype"]], f"max-abs {err:.3e}"
    if "k" in case and case["kind"] == "kvcache":
        # The append rewrote exactly the reference's rows, with its values.
        for cache, before, key in ((kc, case["k_cache"], "k"), (vc, case["v_cache"], "v")):
            index = case[f"{key}_cache_after_index"]
            assert torch.equal(rewritten_rows(before, cache), index)
            rows = cache[index[:, 0], index[:, 1]]
            assert torch.equal(rows.view(torch.int16),
                               case[f"{key}_cache_after_rows"].view(torch.int16))
        assert torch.equal(sl, case["cache_seqlens_after"])


@pytest.mark.parametrize("name", [n for n in vectors.names()
                                  if CASES[n]["kind"] == "kvcache" and "k" not in CASES[n]
                                  and "block_table" in CASES[n]])
def test_fp64_c_oracle_reproduces_reference_vectors(name):
    case = CASES[name]
    got = c_oracle.paged_decode_f64(case["q"], case["k_cache"], case["v_cache"],
                                    case["block_table"], case["cache_seqlens"], case["scale"])
    want = case["out"][:, 0].double().numpy()
    np.testing.assert_allclose(got, want, atol=ULP[case["dtype"]] / 2, rtol=0)


def test_a_wrong_page_order_misses_the_vectors():
    """The comparison sees a gather through the table in the wrong order."""
    case = CASES["table_order"]
    out, *_ = port_output(case, block_table=case["block_table"].flip(1).contiguous())
    assert (out.float() - case["out"].float()).abs().max().item() > 0.05


@pytest.mark.skipif(ref_aten.load() is None, reason="oracle/_ref not built (no reference checkout)")
def test_reference_build_regenerates_the_vectors():
    fresh = make_golden.flatten(make_golden.cases(ref_aten.load()))
    stored = vectors._raw()
    assert sorted(fresh) == sorted(stored)
    for key, value in fresh.items():
        assert value.dtype == stored[key].dtype and np.array_equal(value, stored[key]), key
