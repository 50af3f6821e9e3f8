"""Public API on the CPU: the argument contract, the explicit fallback, and
the MI355X route's qualification.

Host tensors never take the MI355X route, so a valid call here goes down the
rest of the chain: with MXFLASHATTN_ALLOW_FALLBACK=1 to the PyTorch path (its
results are checked against properties and the oracle port), without it to
BackendUnavailableError. The messages matched below are the reference's
(mxflashattn/api.py, mxflashattn/validation.py), which callers match on.
"""

import math

import pytest
import torch

import mxflashattn_amd.dispatch as dispatch
from mxflashattn_amd import (
    BackendUnavailableError,
    decode,
    flash_attn_func,
    flash_attn_varlen_func,
    flash_attn_with_kvcache,
    get_last_dispatch_info,
)
from oracle import reference_port

pytestmark = pytest.mark.filterwarnings(
    "ignore:MXFlashAttn is using the PyTorch reference path:RuntimeWarning")


@pytest.fixture
def fallback(monkeypatch):
    """The PyTorch path is the only backend: no vendor wheel, no extension."""
    monkeypatch.setenv("MXFLASHATTN_ALLOW_FALLBACK", "1")
    monkeypatch.setattr(dispatch, "_flash_attn_function", lambda operation: None)
    monkeypatch.setattr(dispatch, "_native_extension", lambda: None)
    return monkeypatch


def rand(*shape, seed=0, dtype=torch.float32):
    return torch.randn(*shape, generator=torch.Generator().manual_seed(seed)).to(dtype)


def i32(values):
    return torch.tensor(values, dtype=torch.int32)


# --- argument contract ------------------------------------------------------

Q4, K4 = rand(2, 3, 4, 64), rand(2, 5, 2, 64)
QD, KD = rand(2, 1, 4, 64), rand(2, 6, 2, 64)  # decode against a dense cache
SL = i32([3, 4])

CONTRACT = [
    ("dropout", lambda: flash_attn_func(Q4, K4, K4, dropout_p=0.2), NotImplementedError,
     "dropout is not supported"),
    ("window", lambda: flash_attn_func(Q4, K4, K4, window_size=(8, 0)), NotImplementedError,
     "local window attention is not supported"),
    ("softcap", lambda: flash_attn_func(Q4, K4, K4, softcap=30.0), NotImplementedError,
     "soft-capping is not supported"),
    ("alibi", lambda: flash_attn_func(Q4, K4, K4, alibi_slopes=torch.ones(4)),
     NotImplementedError, "alibi_slopes are not supported"),
    ("probs", lambda: flash_attn_func(Q4, K4, K4, return_attn_probs=True), NotImplementedError,
     "return_attn_probs is not supported"),
    ("deterministic", lambda: flash_attn_func(Q4, K4, K4, deterministic=True),
     NotImplementedError, "deterministic mode"),
    ("nan scale", lambda: flash_attn_func(Q4, K4, K4, softmax_scale=math.nan), ValueError,
     "softmax_scale must be finite"),
    ("text scale", lambda: flash_attn_func(Q4, K4, K4, softmax_scale="x"), TypeError,
     "finite number or None"),
    ("rank", lambda: flash_attn_func(Q4[0], K4, K4), ValueError, "rank 4"),
    ("head dim", lambda: flash_attn_func(rand(1, 1, 2, 96), rand(1, 2, 1, 96),
                                         rand(1, 2, 1, 96)), ValueError, "head dimension"),
    ("gqa", lambda: flash_attn_func(rand(1, 1, 3, 64), rand(1, 2, 2, 64), rand(1, 2, 2, 64)),
     ValueError, "divisible by the number of kv heads"),
    ("int dtype", lambda: flash_attn_func(Q4.int(), K4.int(), K4.int()), TypeError,
     "supported dtypes"),
    ("rotary", lambda: flash_attn_with_kvcache(QD, KD, KD, cache_seqlens=SL,
                                               rotary_cos=torch.zeros(1)),
     NotImplementedError, "rotary embeddings are not supported"),
    ("lse", lambda: flash_attn_with_kvcache(QD, KD, KD, cache_seqlens=SL,
                                            return_softmax_lse=True),
     NotImplementedError, "return_softmax_lse is not supported"),
    ("no lengths", lambda: flash_attn_with_kvcache(QD, KD, KD), ValueError,
     "cache_seqlens is required"),
    ("lengths shape", lambda: flash_attn_with_kvcache(QD, KD, KD, cache_seqlens=i32([3])),
     ValueError, "one value per batch item"),
    ("lengths dtype", lambda: flash_attn_with_kvcache(QD, KD, KD, cache_seqlens=SL.float()),
     TypeError, "int32 or int64"),
    ("table rows", lambda: flash_attn_with_kvcache(QD, KD, KD, cache_seqlens=SL,
                                                   block_table=torch.zeros(3, 1,
                                                                           dtype=torch.int32)),
     ValueError, "one row per batch item"),
    ("page size", lambda: flash_attn_with_kvcache(QD, torch.empty(2, 0, 2, 64),
                                                  torch.empty(2, 0, 2, 64),
                                                  cache_seqlens=SL,
                                                  block_table=i32([[0], [1]])),
     ValueError, "page size must be positive"),
    ("half append", lambda: flash_attn_with_kvcache(QD, KD, KD, k=rand(2, 1, 2, 64),
                                                    cache_seqlens=SL),
     ValueError, "both be provided"),
    ("out shape", lambda: flash_attn_with_kvcache(QD, KD, KD, cache_seqlens=SL,
                                                  out=torch.empty(2, 1, 4, 32)),
     ValueError, "out must match"),
    ("varlen coverage", lambda: flash_attn_varlen_func(rand(3, 2, 64), rand(3, 1, 64),
                                                       rand(3, 1, 64), i32([0, 2]), i32([0, 3]),
                                                       2, 3), ValueError, "cover all tokens"),
    ("varlen empty keys", lambda: flash_attn_varlen_func(rand(2, 2, 64), rand(2, 1, 64),
                                                         rand(2, 1, 64), i32([0, 1, 2]),
                                                         i32([0, 2, 2]), 1, 2),
     ValueError, "key/value sequences must be non-empty"),
    ("varlen too long", lambda: flash_attn_varlen_func(rand(1, 2, 64), rand(4, 1, 64),
                                                       rand(4, 1, 64), i32([0, 1]),
                                                       i32([0, 4]), 1, 3),
     ValueError, "longer than max_seqlen"),
    ("varlen decreasing", lambda: flash_attn_varlen_func(rand(2, 2, 64), rand(3, 1, 64),
                                                         rand(3, 1, 64), i32([0, 2, 2]),
                                                         i32([0, 3, 2, 3]), 2, 3),
     ValueError, "same batch size|non-decreasing"),
    ("varlen device", lambda: flash_attn_varlen_func(
        rand(1, 2, 64), rand(1, 1, 64), rand(1, 1, 64),
        torch.tensor([0, 1], dtype=torch.int32, device="meta"), i32([0, 1]), 1, 1),
     ValueError, "same device as q"),
]


@pytest.mark.parametrize("name,call,error,text", CONTRACT, ids=[c[0] for c in CONTRACT])
def test_contract_errors(fallback, name, call, error, text):
    with pytest.raises(error, match=text):
        call()


# --- the fallback switch ------------------------------------------------------

def test_without_the_switch_the_chain_refuses(monkeypatch):
    monkeypatch.delenv("MXFLASHATTN_ALLOW_FALLBACK", raising=False)
    monkeypatch.setattr(dispatch, "_flash_attn_function", lambda operation: None)
    monkeypatch.setattr(dispatch, "_native_extension", lambda: None)
    for call in (lambda: flash_attn_func(Q4, K4, K4),
                 lambda: flash_attn_with_kvcache(QD, KD, KD, cache_seqlens=SL)):
        with pytest.raises(BackendUnavailableError, match="MXFLASHATTN_ALLOW_FALLBACK=1"):
            call()


def test_with_the_switch_the_reference_path_runs_and_says_why(fallback):
    with pytest.warns(RuntimeWarning, match="native_backend_requires_accelerator_tensor"):
        out = flash_attn_with_kvcache(QD, KD, KD, cache_seqlens=SL)
    info = get_last_dispatch_info()
    assert (info.backend, info.operation) == ("reference", "flash_attn_with_kvcache")
    reasons = info.fallback_reason.split(";")
    assert "native_backend_requires_accelerator_tensor" in reasons
    assert "mi355x_split_decode:requires_accelerator_tensor" in reasons
    assert out.shape == QD.shape and torch.isfinite(out).all()


# --- results of the fallback path -------------------------------------------

@pytest.mark.parametrize("seed", range(4))
def test_paged_cache_equals_the_gathered_dense_cache(fallback, seed):
    # Random tables over a shuffled pool: the paged call equals the dense call
    # on the rows gathered in table order.
    g = torch.Generator().manual_seed(seed)
    ps, pages, hkv = 4, 13, 2
    lengths = torch.randint(1, 4 * ps + 1, (3,), generator=g)
    k_cache, v_cache = rand(pages, ps, hkv, 64, seed=seed), rand(pages, ps, hkv, 64, seed=99)
    table = torch.randperm(pages, generator=g)[:12].view(3, 4).to(torch.int32)
    q = rand(3, 1, 6, 64, seed=seed + 7)
    paged = flash_attn_with_kvcache(q, k_cache, v_cache, cache_seqlens=lengths.to(torch.int32),
                                    block_table=table)
    for b in range(3):
        n = int(lengths[b])
        rows = [k_cache[table[b, t // ps], t % ps] for t in range(n)]
        vrows = [v_cache[table[b, t // ps], t % ps] for t in range(n)]
        dense = flash_attn_func(q[b:b + 1], torch.stack(rows)[None], torch.stack(vrows)[None])
        torch.testing.assert_close(paged[b:b + 1], dense)


@pytest.mark.parametrize("paged", [True, False])
def test_append_writes_the_new_rows_then_attends_over_them(fallback, paged):
    q, k_new, v_new = rand(2, 1, 4, 64, seed=1), rand(2, 2, 2, 64, seed=2), rand(2, 2, 2, 64,
                                                                                   seed=3)
    lengths = i32([3, 5])
    if paged:
        k_cache, v_cache = rand(6, 4, 2, 64, seed=4), rand(6, 4, 2, 64, seed=5)
        table = i32([[5, 0], [2, 4]])
    else:
        k_cache, v_cache = rand(2, 8, 2, 64, seed=4), rand(2, 8, 2, 64, seed=5)
        table = None
    k_before, v_before = k_cache.clone(), v_cache.clone()
    out = flash_attn_with_kvcache(q, k_cache, v_cache, k=k_new, v=v_new, cache_seqlens=lengths,
                                  block_table=table)
    assert lengths.tolist() == [5, 7]
    # The port on the untouched caches does the same append and attention.
    expected = reference_port.attention_kvcache(q, k_before, v_before, k=k_new, v=v_new,
                                                cache_seqlens=i32([3, 5]), block_table=table)
    torch.testing.assert_close(out, expected)
    torch.testing.assert_close(k_cache, k_before)  # the port appended the same rows
    for b, old in enumerate((3, 5)):
        for t in range(2):
            pos = old + t
            row = k_cache[table[b, pos // 4], pos % 4] if paged else k_cache[b, pos]
            assert torch.equal(row, k_new[b, t])


def test_causal_rows_without_a_visible_key_are_zero(fallback):
    # Four queries at the end of three keys: query i sits at key position
    # i - 1, so query 0 sees nothing and query j > 0 sees keys 0..j-1.
    q, k, v = rand(1, 4, 2, 64, seed=8), rand(1, 3, 1, 64, seed=9), rand(1, 3, 1, 64, seed=10)
    out = flash_attn_func(q, k, v, causal=True)
    assert torch.equal(out[0, 0], torch.zeros_like(out[0, 0]))
    for j in range(1, 4):
        alone = flash_attn_func(q[:, j:j + 1], k[:, :j], v[:, :j])
        torch.testing.assert_close(out[:, j:j + 1], alone)


def test_varlen_segments_are_independent_calls(fallback):
    cu_q, cu_k = [0, 1, 4, 6], [0, 5, 7, 12]
    q, k, v = rand(6, 4, 128, seed=11), rand(12, 2, 128, seed=12), rand(12, 2, 128, seed=13)
    out = flash_attn_varlen_func(q, k, v, i32(cu_q), i32(cu_k), max_seqlen_q=3, max_seqlen_k=5,
                                 causal=True)
    for i in range(3):
        qs, ks = slice(cu_q[i], cu_q[i + 1]), slice(cu_k[i], cu_k[i + 1])
        alone = flash_attn_func(q[None, qs], k[None, ks], v[None, ks], causal=True)[0]
        torch.testing.assert_close(out[qs], alone)


def test_an_explicit_zero_scale_averages_v(fallback):
    q, k, v = rand(1, 1, 2, 64, seed=14), rand(1, 5, 1, 64, seed=15), rand(1, 5, 1, 64, seed=16)
    out = flash_attn_func(q, k, v, softmax_scale=0.0)
    torch.testing.assert_close(out[0, 0, 0], v[0, :, 0].mean(dim=0))
    assert not torch.allclose(out, flash_attn_func(q, k, v))  # 0.0 is not "default"


def test_out_receives_the_result(fallback):
    out = torch.full_like(QD, math.nan)
    got = flash_attn_with_kvcache(QD, KD, KD, cache_seqlens=SL, out=out)
    assert got is out
    torch.testing.assert_close(out, flash_attn_with_kvcache(QD, KD, KD, cache_seqlens=SL))


@pytest.mark.parametrize("lengths,table,text", [
    ([7, 1], None, "exceeds dense cache capacity"),
    ([0, 2], None, "at least one cached or appended"),
    ([-1, 2], None, "non-negative"),
    ([2, 5], [[0, 1], [1, 2]], "enough pages"),
    ([2, 1], [[9, 0], [1, 2]], "out-of-range page index"),
])
def test_strict_validation_reads_lengths_and_tables_back(fallback, lengths, table, text):
    fallback.setenv("MXFLASHATTN_STRICT_VALIDATION", "1")
    caches = (KD, KD) if table is None else (rand(3, 2, 2, 64), rand(3, 2, 2, 64))
    with pytest.raises(ValueError, match=text):
        flash_attn_with_kvcache(QD, *caches, cache_seqlens=i32(lengths),
                                block_table=None if table is None else i32(table))


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


@pytest.mark.parametrize("case,reason", [
    ("batch", "batch_16001_exceeds_16000"),
    ("misaligned cache", "cache_not_16_byte_aligned"),
    ("cache strides", "cache_strides_not_multiples_of_16_bytes"),
    ("table capacity", "block_table_capacity_exceeds_kernel_limit"),
])
def test_kvcache_route_declines_what_the_kernels_cannot_address(case, reason):
    # Calls the C ABI would reject are handed down the chain with a reason,
    # before any launch (the ABI's limits: csrc/split_decode.hip).
    batch, width = (16001, 2) if case == "batch" else (4, 2)
    if case == "table capacity":
        width = (1 << 30) // 16 + 1
    q = fake_cuda(torch.empty(batch, 1, 8, 64, dtype=torch.float16))
    base = torch.empty(10 * 16 * 2 * 64 + 8, dtype=torch.float16)
    if case == "misaligned cache":
        cache = base[4:4 + 10 * 16 * 2 * 64].view(10, 16, 2, 64)  # 8-byte offset
    elif case == "cache strides":
        cache = torch.empty(10, 16, 2, 68, dtype=torch.float16)[..., :64]  # 136-byte rows
    else:
        cache = base[:10 * 16 * 2 * 64].view(10, 16, 2, 64)
    cache = fake_cuda(cache)
    table = torch.empty(batch, 1, dtype=torch.int32).expand(batch, width)  # shape only
    route = decode.route_kvcache(q, cache, cache, None, None, None, table, 0.1, False)
    assert route.reason == reason
