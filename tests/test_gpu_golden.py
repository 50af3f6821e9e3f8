"""The HIP path against the committed golden vectors of the reference's own
ATen build (tests/golden/reference_vectors.npz), through the public API.

Every case goes through flash_attn_with_kvcache, flash_attn_varlen_func or
flash_attn_func on the GPU and must be served by the MI355X backend. Outputs
are written into NaN-filled buffers where the API takes one, so a row the
kernels never write fails. Tolerances: max-abs 2e-3 for
fp16 and 1.6e-2 for bf16 against the reference's outputs; the append is
bit-exact: the same cache rows rewritten with the same bytes, every other
row untouched, and the lengths advanced.
"""

from __future__ import annotations

import pytest
import torch

import mxflashattn_amd as mx
from golden import vectors

pytestmark = pytest.mark.gpu

CASES = vectors.load()
TOL = {torch.float16: 2e-3, torch.bfloat16: 1.6e-2}


def rewritten_rows(before: torch.Tensor, after: torch.Tensor) -> torch.Tensor:
    diff = (before.view(torch.int16) != after.view(torch.int16)).flatten(2).any(-1)
    return diff.nonzero().to(torch.int64)


@pytest.mark.parametrize("name", vectors.names())
def test_hip_path_reproduces_reference_vectors(device, name):
    case = CASES[name]
    dev = {k: (v.to(device) if isinstance(v, torch.Tensor) else v) for k, v in case.items()}
    kind = case["kind"]
    if kind == "varlen":
        got = mx.flash_attn_varlen_func(dev["q"], dev["k"], dev["v"], dev["cu_seqlens_q"],
                                        dev["cu_seqlens_k"], case["max_seqlen_q"],
                                        case["max_seqlen_k"], softmax_scale=case["scale"],
                                        causal=case["causal"])
    elif kind == "func":
        got = mx.flash_attn_func(dev["q"], dev["k"], dev["v"], softmax_scale=case["scale"],
                                 causal=case["causal"])
    else:
        out = torch.full_like(dev["q"], float("nan"))
        got = mx.flash_attn_with_kvcache(dev["q"], dev["k_cache"], dev["v_cache"],
                                         k=dev.get("k"), v=dev.get("v"),
                                         cache_seqlens=dev["cache_seqlens"],
                                         block_table=dev.get("block_table"),
                                         softmax_scale=case["scale"], causal=case["causal"],
                                         out=out)
        assert got is out
    torch.cuda.synchronize()
    info = mx.get_last_dispatch_info()
    assert info is not None and info.backend == "mi355x_split_decode", info
    want = case["out"]
    assert got.shape == want.shape and got.dtype == want.dtype
    assert torch.isfinite(got.float()).all(), "an output row was left unwritten"
    err = (got.float().cpu() - want.float()).abs().max().item()
    assert err <= TOL[case["dtype"]], f"max-abs {err:.3e}"
    if "k" in case and kind == "kvcache":
        for key in ("k", "v"):
            cache = dev[f"{key}_cache"].cpu()
            index = case[f"{key}_cache_after_index"]
            assert torch.equal(rewritten_rows(case[f"{key}_cache"], cache), index)
            assert torch.equal(cache[index[:, 0], index[:, 1]].view(torch.int16),
                               case[f"{key}_cache_after_rows"].view(torch.int16))
        assert torch.equal(dev["cache_seqlens"].cpu(), case["cache_seqlens_after"])
