"""The oracle against the reference's own ATen build (CPU).

oracle/build_ref.py compiles the reference's csrc/mxmac sources
(attention_forward.cpp, paged_kv.cpp, workspace.cpp) into oracle/_ref/; these
tests run the restatement in oracle/reference_port.py and the fp64 C oracle
against that build on the same seeded inputs: paged and dense caches,
appends with the causal mask, GQA, packed varlen segments and batched dense
attention. They skip where the build is absent (no reference checkout).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from mxflashattn_amd.workloads import make_paged_batch
from oracle import c_oracle, ref_aten, reference_port

REF = ref_aten.load()
pytestmark = pytest.mark.skipif(REF is None, reason="oracle/_ref not built (no reference checkout)")

# One unit in the last place of each output type at |x| <~ 4: outputs of the
# two fp32 computations agree to ~1e-6 before the final rounding, so they may
# differ by one rounding step.
ULP = {torch.float32: 2e-5, torch.float16: 4e-3, torch.bfloat16: 3.2e-2}


def _close(a: torch.Tensor, b: torch.Tensor, dtype: torch.dtype) -> float:
    err = (a.float() - b.float()).abs().max().item()
    assert err <= ULP[dtype], f"max-abs {err:.3e} > {ULP[dtype]:.1e}"
    return err


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("hq,hkv,hd,ps", [(8, 2, 64, 16), (32, 8, 128, 16), (16, 8, 64, 1),
                                          (8, 1, 128, 64), (6, 6, 64, 4)])
def test_paged_decode_matches_reference_build(dtype, hq, hkv, hd, ps):
    lengths = torch.tensor([1, 17, 300, 64, 129])
    b = make_paged_batch(5, hq, hkv, hd, dtype, lengths, page_size=ps, seed=hq * 7 + hd + ps)
    want = REF.flash_attn_with_kvcache(b.q, b.k_cache, b.v_cache, None, None,
                                       b.cache_seqlens.clone(), b.block_table, b.scale, False)
    got = reference_port.attention_kvcache(b.q, b.k_cache, b.v_cache,
                                           cache_seqlens=b.cache_seqlens.clone(),
                                           block_table=b.block_table, softmax_scale=b.scale)
    assert got.shape == want.shape and got.dtype == want.dtype
    _close(got, want, dtype)


def test_fp64_c_oracle_matches_reference_build():
    lengths = torch.tensor([1, 2, 255, 1000, 33, 7])
    b = make_paged_batch(6, 16, 4, 128, torch.float32, lengths, seed=11)
    want = REF.flash_attn_with_kvcache(b.q, b.k_cache, b.v_cache, None, None,
                                       b.cache_seqlens.clone(), b.block_table, b.scale, False)
    got = c_oracle.paged_decode_f64(b.q, b.k_cache, b.v_cache, b.block_table, b.cache_seqlens,
                                    b.scale)
    np.testing.assert_allclose(got, want[:, 0].double().numpy(), atol=2e-5, rtol=0)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
@pytest.mark.parametrize("new_tokens", [1, 3])
def test_append_and_causal_match_reference_build(dtype, new_tokens):
    """Append at cache_seqlens, causal attention over the grown sequences,
    cache bytes and lengths after the call (paged_kv.cpp:80-123)."""
    lengths = torch.tensor([0, 15, 16, 40])
    b = make_paged_batch(4, 8, 2, 64, dtype, lengths, page_size=16, seed=5,
                         block_table_width=8)
    g = torch.Generator().manual_seed(9)
    k_new = torch.randn(4, new_tokens, 2, 64, generator=g).to(dtype)
    v_new = torch.randn(4, new_tokens, 2, 64, generator=g).to(dtype)
    q = torch.randn(4, new_tokens, 8, 64, generator=g).to(dtype)
    kc_r, vc_r, sl_r = b.k_cache.clone(), b.v_cache.clone(), b.cache_seqlens.clone()
    want = REF.flash_attn_with_kvcache(q, kc_r, vc_r, k_new, v_new, sl_r, b.block_table,
                                       b.scale, True)
    kc_p, vc_p, sl_p = b.k_cache.clone(), b.v_cache.clone(), b.cache_seqlens.clone()
    got = reference_port.attention_kvcache(q, kc_p, vc_p, k=k_new, v=v_new, cache_seqlens=sl_p,
                                           block_table=b.block_table, softmax_scale=b.scale,
                                           causal=True)
    _close(got, want, dtype)
    assert torch.equal(kc_p, kc_r) and torch.equal(vc_p, vc_r)
    assert torch.equal(sl_p, sl_r) and torch.equal(sl_r, b.cache_seqlens + new_tokens)


def test_dense_cache_matches_reference_build():
    g = torch.Generator().manual_seed(3)
    kc = torch.randn(3, 50, 4, 64, generator=g)
    vc = torch.randn(3, 50, 4, 64, generator=g)
    q = torch.randn(3, 1, 16, 64, generator=g)
    sl = torch.tensor([1, 49, 20], dtype=torch.int32)
    want = REF.flash_attn_with_kvcache(q, kc, vc, None, None, sl.clone(), None, 0.125, False)
    got = reference_port.attention_kvcache(q, kc, vc, cache_seqlens=sl.clone(), block_table=None,
                                           softmax_scale=0.125)
    _close(got, want, torch.float32)


@pytest.mark.parametrize("causal", [False, True])
def test_varlen_matches_reference_build(causal):
    g = torch.Generator().manual_seed(4)
    cu_q, cu_k = [0, 1, 1, 4, 5], [0, 7, 9, 30, 31]  # an empty query segment among them
    q = torch.randn(cu_q[-1], 8, 64, generator=g)
    k = torch.randn(cu_k[-1], 2, 64, generator=g)
    v = torch.randn(cu_k[-1], 2, 64, generator=g)
    want = REF.flash_attn_varlen_func(q, k, v, torch.tensor(cu_q, dtype=torch.int32),
                                      torch.tensor(cu_k, dtype=torch.int32), 3, 21, causal, 0.2)
    got = reference_port.attention_varlen(q, k, v, cu_q, cu_k, softmax_scale=0.2, causal=causal)
    _close(got, want, torch.float32)


@pytest.mark.parametrize("causal", [False, True])
def test_batched_matches_reference_build(causal):
    g = torch.Generator().manual_seed(6)
    q = torch.randn(2, 3, 8, 64, generator=g)
    k = torch.randn(2, 11, 4, 64, generator=g)
    v = torch.randn(2, 11, 4, 64, generator=g)
    want = REF.flash_attn_func(q, k, v, causal, 0.3)
    got = reference_port.attention_batched(q, k, v, softmax_scale=0.3, causal=causal)
    _close(got, want, torch.float32)


def test_a_planted_mistake_is_caught():
    """The comparison is sharp enough to see a one-off error in the gather:
    reading a sequence one page-table column late changes the output."""
    lengths = torch.tensor([40, 40])
    b = make_paged_batch(2, 8, 2, 64, torch.float32, lengths, page_size=16, seed=8,
                         block_table_width=5)
    want = REF.flash_attn_with_kvcache(b.q, b.k_cache, b.v_cache, None, None,
                                       b.cache_seqlens.clone(), b.block_table, b.scale, False)
    shifted = torch.roll(b.block_table, shifts=-1, dims=1)
    wrong = reference_port.attention_kvcache(b.q, b.k_cache, b.v_cache,
                                             cache_seqlens=b.cache_seqlens.clone(),
                                             block_table=shifted, softmax_scale=b.scale)
    assert (wrong - want).abs().max().item() > 1e-2
