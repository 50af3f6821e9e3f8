"""Public API contract on the CPU (mirrors the reference's tests/test_api.py).

Host tensors never qualify for the MI355X decode backend, so these calls go
through the rest of the dispatch chain: the explicit PyTorch path behind
MXFLASHATTN_ALLOW_FALLBACK=1, or BackendUnavailableError without it. The
decode routes' own qualification logic is checked at the end without a GPU.
"""

import pytest
import torch

import mxflashattn_amd.dispatch as dispatch
from mxflashattn_amd import (
    BackendUnavailableError,
    decode,
    fallback,
    flash_attn_func,
    flash_attn_varlen_func,
    flash_attn_with_kvcache,
    get_last_dispatch_info,
)

pytestmark = pytest.mark.filterwarnings(
    "ignore:MXFlashAttn is using the PyTorch reference path:RuntimeWarning")


def tensors(batch=1, q_len=2, kv_len=3, q_heads=2, kv_heads=1, head_dim=64):
    q = torch.randn(batch, q_len, q_heads, head_dim, dtype=torch.float32)
    k = torch.randn(batch, kv_len, kv_heads, head_dim, dtype=torch.float32)
    v = torch.randn_like(k)
    return q, k, v


def test_native_backend_is_required_unless_fallback_is_explicit(monkeypatch):
    q, k, v = tensors()
    monkeypatch.delenv("MXFLASHATTN_ALLOW_FALLBACK", raising=False)
    monkeypatch.setattr(dispatch, "_flash_attn_function", lambda operation: None)
    monkeypatch.setattr(dispatch, "_native_extension", lambda: None)
    with pytest.raises(BackendUnavailableError, match="MXFLASHATTN_ALLOW_FALLBACK=1"):
        flash_attn_func(q, k, v)


def test_explicit_reference_fallback_runs_and_records_reason(monkeypatch):
    q, k, v = tensors()
    monkeypatch.setenv("MXFLASHATTN_ALLOW_FALLBACK", "1")
    monkeypatch.setattr(dispatch, "_flash_attn_function", lambda operation: None)
    monkeypatch.setattr(dispatch, "_native_extension", lambda: None)
    with pytest.warns(RuntimeWarning, match="native_backend_requires_accelerator_tensor"):
        output = flash_attn_func(q, k, v, causal=True)
    assert output.shape == q.shape
    assert torch.isfinite(output).all()
    info = get_last_dispatch_info()
    assert info.backend == "reference"
    assert info.fallback_reason
    # The MI355X route names why it declined the call.
    assert "mi355x_split_decode:requires_accelerator_tensor" in info.fallback_reason


def test_causal_attention_handles_query_longer_than_key_without_nan(monkeypatch):
    monkeypatch.setenv("MXFLASHATTN_ALLOW_FALLBACK", "1")
    q = torch.randn(1, 3, 2, 64)
    k = torch.randn(1, 1, 1, 64)
    v = torch.randn_like(k)
    output = flash_attn_func(q, k, v, causal=True)
    assert torch.isfinite(output).all()
    torch.testing.assert_close(output[:, :2], torch.zeros_like(output[:, :2]))
    torch.testing.assert_close(output[:, 2:], v.expand(-1, -1, 2, -1))


def test_varlen_attention_supports_gqa_and_unequal_sequences(monkeypatch):
    monkeypatch.setenv("MXFLASHATTN_ALLOW_FALLBACK", "1")
    q = torch.randn(3, 2, 64)
    k = torch.randn(5, 1, 64)
    v = torch.randn_like(k)
    cu_q = torch.tensor([0, 2, 3], dtype=torch.int32)
    cu_k = torch.tensor([0, 3, 5], dtype=torch.int32)
    output = flash_attn_varlen_func(q, k, v, cu_q, cu_k, max_seqlen_q=2, max_seqlen_k=3)
    assert output.shape == q.shape
    assert torch.isfinite(output).all()
    # Row 2 is sequence 1's only query: attention over keys 3..4.
    expected = fallback.attention_batched(q[None, 2:3], k[None, 3:5], v[None, 3:5])[0]
    torch.testing.assert_close(output[2:3], expected)


def test_varlen_rejects_cumulative_lengths_that_do_not_cover_tokens(monkeypatch):
    monkeypatch.setenv("MXFLASHATTN_ALLOW_FALLBACK", "1")
    q = torch.randn(2, 1, 64)
    k = torch.randn(2, 1, 64)
    cu = torch.tensor([0, 1], dtype=torch.int32)
    with pytest.raises(ValueError, match="cover all tokens"):
        flash_attn_varlen_func(q, k, k, cu, cu, max_seqlen_q=1, max_seqlen_k=1)


def test_varlen_rejects_empty_key_sequences(monkeypatch):
    monkeypatch.setenv("MXFLASHATTN_ALLOW_FALLBACK", "1")
    q = torch.randn(2, 1, 64)
    k = torch.randn(1, 1, 64)
    cu_q = torch.tensor([0, 1, 2], dtype=torch.int32)
    cu_k = torch.tensor([0, 0, 1], dtype=torch.int32)
    with pytest.raises(ValueError, match="key/value sequences must be non-empty"):
        flash_attn_varlen_func(q, k, k, cu_q, cu_k, max_seqlen_q=1, max_seqlen_k=1)


def test_varlen_rejects_cumulative_lengths_on_a_different_device(monkeypatch):
    monkeypatch.setenv("MXFLASHATTN_ALLOW_FALLBACK", "1")
    q = torch.randn(1, 1, 64)
    k = torch.randn(1, 1, 64)
    cu = torch.tensor([0, 1], device="meta", dtype=torch.int32)
    with pytest.raises(ValueError, match="same device as q"):
        flash_attn_varlen_func(q, k, k, cu, cu, max_seqlen_q=1, max_seqlen_k=1)


def test_varlen_rejects_sequences_longer_than_max_seqlen(monkeypatch):
    monkeypatch.setenv("MXFLASHATTN_ALLOW_FALLBACK", "1")
    q = torch.randn(1, 1, 64)
    k = torch.randn(3, 1, 64)
    with pytest.raises(ValueError, match="longer than max_seqlen"):
        flash_attn_varlen_func(q, k, k, torch.tensor([0, 1], dtype=torch.int32),
                               torch.tensor([0, 3], dtype=torch.int32), max_seqlen_q=1,
                               max_seqlen_k=2)


def test_kvcache_rejects_zero_page_size(monkeypatch):
    monkeypatch.setenv("MXFLASHATTN_ALLOW_FALLBACK", "1")
    q = torch.randn(1, 1, 1, 64)
    k_cache = torch.empty(1, 0, 1, 64)
    v_cache = torch.empty_like(k_cache)
    with pytest.raises(ValueError, match="page size must be positive"):
        flash_attn_with_kvcache(q, k_cache, v_cache,
                                cache_seqlens=torch.tensor([1], dtype=torch.int32),
                                block_table=torch.tensor([[0]], dtype=torch.int32))


def test_paged_kv_cache_reads_blocks_in_table_order(monkeypatch):
    monkeypatch.setenv("MXFLASHATTN_ALLOW_FALLBACK", "1")
    q = torch.randn(1, 1, 2, 64)
    k_cache = torch.randn(2, 2, 1, 64)
    v_cache = torch.randn_like(k_cache)
    output = flash_attn_with_kvcache(q, k_cache, v_cache,
                                     cache_seqlens=torch.tensor([3], dtype=torch.int32),
                                     block_table=torch.tensor([[1, 0]], dtype=torch.int32))
    expected_k = torch.cat((k_cache[1], k_cache[0, :1]), dim=0).unsqueeze(0)
    expected_v = torch.cat((v_cache[1], v_cache[0, :1]), dim=0).unsqueeze(0)
    torch.testing.assert_close(output, flash_attn_func(q, expected_k, expected_v))


def test_paged_kv_cache_appends_and_advances_sequence_length(monkeypatch):
    monkeypatch.setenv("MXFLASHATTN_ALLOW_FALLBACK", "1")
    q, k_new, v_new = tensors(q_len=1, kv_len=1)
    k_cache = torch.zeros(2, 2, 1, 64)
    v_cache = torch.zeros_like(k_cache)
    k_cache[0] = torch.randn_like(k_cache[0])
    v_cache[0] = torch.randn_like(v_cache[0])
    cache_seqlens = torch.tensor([2], dtype=torch.int32)
    output = flash_attn_with_kvcache(q, k_cache, v_cache, k=k_new, v=v_new,
                                     cache_seqlens=cache_seqlens,
                                     block_table=torch.tensor([[0, 1]], dtype=torch.int32))
    assert output.shape == q.shape
    assert cache_seqlens.tolist() == [3]
    torch.testing.assert_close(k_cache[1, 0], k_new[0, 0])
    torch.testing.assert_close(v_cache[1, 0], v_new[0, 0])


def test_dense_kv_cache_appends_and_advances_sequence_length(monkeypatch):
    monkeypatch.setenv("MXFLASHATTN_ALLOW_FALLBACK", "1")
    q, k_new, v_new = tensors(q_len=1, kv_len=1)
    k_cache = torch.zeros(1, 4, 1, 64)
    v_cache = torch.zeros_like(k_cache)
    k_cache[:, :2] = torch.randn(1, 2, 1, 64)
    v_cache[:, :2] = torch.randn(1, 2, 1, 64)
    cache_seqlens = torch.tensor([2], dtype=torch.int32)
    flash_attn_with_kvcache(q, k_cache, v_cache, k=k_new, v=v_new, cache_seqlens=cache_seqlens)
    assert cache_seqlens.tolist() == [3]
    torch.testing.assert_close(k_cache[0, 2], k_new[0, 0])
    torch.testing.assert_close(v_cache[0, 2], v_new[0, 0])


def test_unsupported_flash_attention_options_fail_clearly(monkeypatch):
    monkeypatch.setenv("MXFLASHATTN_ALLOW_FALLBACK", "1")
    q, k, v = tensors()
    with pytest.raises(NotImplementedError, match="dropout"):
        flash_attn_func(q, k, v, dropout_p=0.1)
    q1, kc, vc = tensors(q_len=1)
    sl = torch.tensor([2], dtype=torch.int32)
    with pytest.raises(NotImplementedError, match="rotary"):
        flash_attn_with_kvcache(q1, kc, vc, cache_seqlens=sl, rotary_cos=torch.zeros(1))
    with pytest.raises(NotImplementedError, match="return_softmax_lse"):
        flash_attn_with_kvcache(q1, kc, vc, cache_seqlens=sl, return_softmax_lse=True)


def test_explicit_zero_scale_is_preserved_and_nonfinite_scale_is_rejected(monkeypatch):
    monkeypatch.setenv("MXFLASHATTN_ALLOW_FALLBACK", "1")
    q, k, v = tensors()
    zero_scale = flash_attn_func(q, k, v, softmax_scale=0.0)
    expected = fallback.attention_batched(q, k, v, softmax_scale=0.0)
    default_scale = flash_attn_func(q, k, v)
    torch.testing.assert_close(zero_scale, expected)
    assert not torch.allclose(zero_scale, default_scale)
    with pytest.raises(ValueError, match="softmax_scale must be finite"):
        flash_attn_func(q, k, v, softmax_scale=float("nan"))


def test_kvcache_requires_cache_seqlens_and_matching_table(monkeypatch):
    monkeypatch.setenv("MXFLASHATTN_ALLOW_FALLBACK", "1")
    q, kc, vc = tensors(q_len=1)
    with pytest.raises(ValueError, match="cache_seqlens is required"):
        flash_attn_with_kvcache(q, kc, vc)
    with pytest.raises(ValueError, match="one row per batch item"):
        flash_attn_with_kvcache(q, kc, vc, cache_seqlens=torch.tensor([1], dtype=torch.int32),
                                block_table=torch.zeros(2, 1, dtype=torch.int32))


def test_strict_validation_reads_lengths_back(monkeypatch):
    monkeypatch.setenv("MXFLASHATTN_ALLOW_FALLBACK", "1")
    monkeypatch.setenv("MXFLASHATTN_STRICT_VALIDATION", "1")
    q, kc, vc = tensors(q_len=1)
    with pytest.raises(ValueError, match="exceeds dense cache capacity"):
        flash_attn_with_kvcache(q, kc, vc, cache_seqlens=torch.tensor([4], dtype=torch.int32))
    with pytest.raises(ValueError, match="out-of-range page index"):
        flash_attn_with_kvcache(q, kc, vc, cache_seqlens=torch.tensor([2], dtype=torch.int32),
                                block_table=torch.tensor([[5]], dtype=torch.int32))


# --- qualification of the MI355X decode route (no kernel runs here) --------

def meta(*shape, dtype=torch.bfloat16):
    return torch.empty(*shape, dtype=dtype, device="meta")


def fake_cuda(t):
    """A tensor whose .device reads as cuda:0 without a GPU, for route checks."""

    class FakeDevice(torch.Tensor):
        @property
        def device(self):
            return torch.device("cuda", 0)

    return t.as_subclass(FakeDevice)


@pytest.mark.parametrize("hq,hkv,hd,dtype,reason", [
    (32, 8, 128, torch.bfloat16, None),
    (32, 16, 64, torch.float16, None),
    (32, 4, 128, torch.bfloat16, None),
    (32, 8, 256, torch.bfloat16, "head_dim_256"),
    # Any 1..16 query heads per kv head runs on the kernels (GQ 3, 1, 16).
    (24, 8, 128, torch.bfloat16, None),
    (32, 32, 128, torch.bfloat16, None),
    (64, 4, 64, torch.float16, None),
    (34, 2, 128, torch.bfloat16, "gqa_ratio_34/2"),
    (64, 2, 128, torch.bfloat16, "gqa_ratio_64/2"),
    (32, 8, 128, torch.float32, "supports_only_float16_and_bfloat16"),
])
def test_kvcache_route_qualification(hq, hkv, hd, dtype, reason):
    q = fake_cuda(torch.empty(4, 1, hq, hd, dtype=dtype))
    cache = fake_cuda(torch.empty(10, 16, hkv, hd, dtype=dtype))
    route = decode.route_kvcache(q, cache, cache, None, None, None, torch.empty(4, 2), 0.1, False)
    if reason is None:
        assert route.reason is None and route.run is not None
    else:
        assert route.reason.startswith(reason)


def test_kvcache_route_declines_prefill_and_odd_pages():
    cache = fake_cuda(torch.empty(10, 16, 8, 128, dtype=torch.bfloat16))
    # A few draft tokens per sequence fit the 16 kernel columns (QL x GQ <= 16);
    # longer queries (prefill) are declined.
    for ql in (2, 4):
        q = fake_cuda(torch.empty(4, ql, 32, 128, dtype=torch.bfloat16))
        route = decode.route_kvcache(q, cache, cache, None, None, None, torch.empty(4, 2), 0.1,
                                     True)
        assert route.reason is None and route.run is not None
    q = fake_cuda(torch.empty(4, 5, 32, 128, dtype=torch.bfloat16))
    assert decode.route_kvcache(q, cache, cache, None, None, None, torch.empty(4, 2), 0.1,
                                False).reason.startswith("query_length_5_times_gqa_4")
    # Causal: up to four launches of token chunks (64 columns), not a prefill.
    assert decode.route_kvcache(q, cache, cache, None, None, None, torch.empty(4, 2), 0.1,
                                True).reason is None
    q17 = fake_cuda(torch.empty(4, 17, 32, 128, dtype=torch.bfloat16))
    assert decode.route_kvcache(q17, cache, cache, None, None, None, torch.empty(4, 2), 0.1,
                                True).reason.startswith("query_length_17_times_gqa_4_exceeds_64")
    q = fake_cuda(torch.empty(4, 2, 32, 128, dtype=torch.bfloat16))
    q16 = fake_cuda(torch.empty(4, 2, 32, 128, dtype=torch.bfloat16))
    cache2 = fake_cuda(torch.empty(10, 16, 2, 128, dtype=torch.bfloat16))  # GQ 16
    assert decode.route_kvcache(q16, cache2, cache2, None, None, None, torch.empty(4, 2), 0.1,
                                False).reason.startswith("query_length_2_times_gqa_16")
    q1 = fake_cuda(torch.empty(4, 1, 32, 128, dtype=torch.bfloat16))
    odd = fake_cuda(torch.empty(10, 12, 8, 128, dtype=torch.bfloat16))
    assert decode.route_kvcache(q1, odd, odd, None, None, None, torch.empty(4, 2), 0.1,
                                False).reason.startswith("page_size_12")


def test_host_tensors_never_take_the_decode_route():
    q = torch.empty(4, 1, 32, 128, dtype=torch.bfloat16)
    cache = torch.empty(10, 16, 8, 128, dtype=torch.bfloat16)
    route = decode.route_kvcache(q, cache, cache, None, None, None, torch.empty(4, 2), 0.1, False)
    assert route.reason == "requires_accelerator_tensor"


@pytest.mark.parametrize("seq,page", [(1, 1), (16, 16), (48, 16), (256, 256), (1024, 256),
                                      (7, 1), (6, 2)])
def test_dense_cache_page_view(seq, page):
    assert decode._dense_page_size(seq) == page
    cache = torch.arange(2 * seq * 3 * 8, dtype=torch.float32).view(2, seq, 3, 8)
    pages = decode._dense_as_pages(cache)
    table = decode._dense_table(2, seq // page, torch.device("cpu"))
    for b in range(2):
        for t in range(seq):
            assert torch.equal(pages[table[b, t // page], t % page], cache[b, t])


def test_varlen_route_declines_multi_token_queries():
    q = fake_cuda(torch.empty(3, 8, 64, dtype=torch.float16))
    k = fake_cuda(torch.empty(5, 2, 64, dtype=torch.float16))
    assert decode.route_varlen(q, k, k, k, [0, 2, 3], [0, 3, 5], 3, 0.1,
                               False).reason == "varlen_query_length_above_one"
    assert decode.route_varlen(q, k, k, k, [0, 1, 2, 3], [0, 1, 3, 5], 3, 0.1, False).reason is None
