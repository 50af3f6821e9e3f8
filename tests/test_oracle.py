"""Pins of the CPU oracle (oracle/) before it is trusted as the parity checker.

The reference ships no golden vectors for this path (its kernel tests compare
against the closed MetaX wheel on a C500). Each oracle function is pinned by
checks that a plausible mistake would fail:

  reference_port.attention_kvcache / attention_single
    - paged read order through block table [1, 0] equals attention over the
      manually gathered rows (reference tests/test_api.py:136-155)
    - append writes the new row into page table[b][pos // PS], row pos % PS,
      and advances cache_seqlens (tests/test_api.py:158-197, tests/test_c500.py:84-126)
    - one key: output is the V row exactly (csrc_native/debug_m1.py:25-28)
    - scale 0: output is the mean of the V rows
    - causal with q longer than k: zeros, then V (tests/test_api.py:52-62)
    - agreement with torch's scaled_dot_product_attention (a library routine)
      on independently gathered K/V, per query head against kv head h // GQ
    - GQA mapping: kv heads with constant, distinct V rows give every query head
      exactly its group's constant
  reference_port.attention_varlen
    - each packed segment, an empty-query segment among them, equals float64
      library attention over that segment's keys with an independently built
      bottom-right causal mask (rows that see no key are zeros); moving a
      segment boundary by one key changes the result
  c_oracle.paged_decode_f64
    - agreement with reference_port (fp32) and with a float64 SDPA
    - a peaked query (q = 40 * k_j) returns V_j
    - permuting physical pages together with the block table changes nothing
  c_oracle.append_kv / reshape_and_cache
    - bitwise against torch index assignment; slot < 0 and positions beyond
      the table are skipped
  split_model
    - the LSE merge of any split of the keys, empty splits included, equals
      unsplit attention (the invariant behind csrc_native/m1_kernel.cpp:861-888)
  c_oracle.e4m3fn_decode / e4m3fn_encode (fp8 caches; no reference counterpart)
    - decode of all 256 codes equals torch's float8_e4m3fn -> float32
    - encode equals torch's round-to-nearest-even conversion on in-range values,
      exact midpoints (ties) included, and is the nearest finite code by brute
      force; saturation to +-448 and NaN are fixed by hand-picked cases
  c_oracle.reshape_and_cache_fp8 / paged_decode_fp8_f64
    - the append equals torch index assignment of (x / scale).to(e4m3fn)
    - fp8 decode equals the fp64 oracle on caches dequantised exactly
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from mxflashattn_amd.workloads import make_paged_batch
from oracle import c_oracle, reference_port, split_model


def gather_dense(cache: torch.Tensor, table_row: list[int], length: int) -> torch.Tensor:
    """Rows 0..length-1 of a paged sequence by explicit per-token indexing."""
    ps = cache.shape[1]
    return torch.stack([cache[table_row[t // ps], t % ps] for t in range(length)])


def sdpa_reference(q_row: torch.Tensor, keys: torch.Tensor, values: torch.Tensor,
                   scale: float) -> torch.Tensor:
    """Library attention for one query token: q_row [HQ, D], keys/values [L, HKV, D]."""
    hq, hkv = q_row.shape[0], keys.shape[1]
    group = hq // hkv
    outs = []
    for h in range(hq):
        qh = q_row[h].double().view(1, 1, 1, -1)
        kh = keys[:, h // group].double().unsqueeze(0).unsqueeze(0)
        vh = values[:, h // group].double().unsqueeze(0).unsqueeze(0)
        outs.append(F.scaled_dot_product_attention(qh, kh, vh, scale=scale).view(-1))
    return torch.stack(outs)


def test_paged_read_order_matches_manual_gather():
    torch.manual_seed(0)
    q = torch.randn(1, 1, 2, 64)
    k_cache = torch.randn(2, 2, 1, 64)
    v_cache = torch.randn_like(k_cache)
    table = torch.tensor([[1, 0]], dtype=torch.int32)
    seqlens = torch.tensor([3], dtype=torch.int32)
    out = reference_port.attention_kvcache(q, k_cache, v_cache, cache_seqlens=seqlens,
                                           block_table=table)
    keys = torch.cat((k_cache[1], k_cache[0, :1]), dim=0)
    values = torch.cat((v_cache[1], v_cache[0, :1]), dim=0)
    expected = reference_port.attention_single(q[0], keys, values)
    torch.testing.assert_close(out[0], expected)
    lib = sdpa_reference(q[0, 0], keys, values, 64 ** -0.5)
    torch.testing.assert_close(out[0, 0].double(), lib, atol=1e-5, rtol=1e-5)


def test_paged_append_writes_slot_and_advances_lengths():
    torch.manual_seed(1)
    q = torch.randn(1, 1, 2, 64)
    k_new = torch.randn(1, 1, 1, 64)
    v_new = torch.randn(1, 1, 1, 64)
    k_cache = torch.zeros(2, 2, 1, 64)
    v_cache = torch.zeros_like(k_cache)
    k_cache[0] = torch.randn_like(k_cache[0])
    v_cache[0] = torch.randn_like(v_cache[0])
    seqlens = torch.tensor([2], dtype=torch.int32)
    out = reference_port.attention_kvcache(q, k_cache, v_cache, cache_seqlens=seqlens,
                                           block_table=torch.tensor([[0, 1]], dtype=torch.int32),
                                           k=k_new, v=v_new)
    assert out.shape == q.shape
    assert seqlens.tolist() == [3]
    assert torch.equal(k_cache[1, 0], k_new[0, 0])
    assert torch.equal(v_cache[1, 0], v_new[0, 0])
    assert torch.equal(k_cache[1, 1], torch.zeros(1, 64))


def test_dense_append_writes_row_and_advances_lengths():
    torch.manual_seed(2)
    q = torch.randn(1, 1, 2, 64)
    k_new, v_new = torch.randn(1, 1, 1, 64), torch.randn(1, 1, 1, 64)
    k_cache = torch.zeros(1, 4, 1, 64)
    v_cache = torch.zeros_like(k_cache)
    seqlens = torch.tensor([2], dtype=torch.int32)
    reference_port.attention_kvcache(q, k_cache, v_cache, cache_seqlens=seqlens, block_table=None,
                                     k=k_new, v=v_new)
    assert seqlens.tolist() == [3]
    assert torch.equal(k_cache[0, 2], k_new[0, 0]) and torch.equal(v_cache[0, 2], v_new[0, 0])


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
def test_single_key_returns_v_row_exactly(dtype):
    b = make_paged_batch(3, 8, 2, 128, dtype, 1, seed=3)
    out = reference_port.attention_kvcache(b.q, b.k_cache, b.v_cache,
                                           cache_seqlens=b.cache_seqlens.clone(),
                                           block_table=b.block_table)
    for i in range(3):
        page = int(b.block_table[i, 0])
        for h in range(8):
            assert torch.equal(out[i, 0, h], b.v_cache[page, 0, h // 4])
    f64 = c_oracle.paged_decode_f64(b.q, b.k_cache, b.v_cache, b.block_table, b.cache_seqlens,
                                    b.scale)
    for i in range(3):
        page = int(b.block_table[i, 0])
        for h in range(8):
            assert np.array_equal(f64[i, h], b.v_cache[page, 0, h // 4].double().numpy())


def test_zero_scale_is_the_mean_of_v():
    b = make_paged_batch(2, 4, 2, 64, torch.float32, torch.tensor([5, 37]), seed=4)
    out = reference_port.attention_kvcache(b.q, b.k_cache, b.v_cache,
                                           cache_seqlens=b.cache_seqlens.clone(),
                                           block_table=b.block_table, softmax_scale=0.0)
    for i, n in enumerate([5, 37]):
        rows = gather_dense(b.v_cache, b.block_table[i].tolist(), n)
        mean = rows.double().mean(dim=0)
        for h in range(4):
            assert torch.allclose(out[i, 0, h].double(), mean[h // 2], atol=1e-6)


def test_causal_query_longer_than_key_gives_zeros_then_v():
    q = torch.randn(1, 3, 2, 64)
    k = torch.randn(1, 1, 1, 64)
    v = torch.randn_like(k)
    out = reference_port.attention_batched(q, k, v, causal=True)
    assert torch.isfinite(out).all()
    torch.testing.assert_close(out[:, :2], torch.zeros_like(out[:, :2]))
    torch.testing.assert_close(out[:, 2:], v.expand(-1, -1, 2, -1))


def test_causal_is_a_no_op_for_one_query_token():
    b = make_paged_batch(2, 8, 2, 64, torch.float32, torch.tensor([9, 40]), seed=5)
    args = dict(cache_seqlens=b.cache_seqlens, block_table=b.block_table)
    plain = reference_port.attention_kvcache(b.q, b.k_cache, b.v_cache, **args)
    causal = reference_port.attention_kvcache(b.q, b.k_cache, b.v_cache, causal=True, **args)
    torch.testing.assert_close(plain, causal)


@pytest.mark.parametrize("gq,hd", [(2, 64), (4, 128), (8, 64)])
def test_port_matches_library_attention_on_gathered_rows(gq, hd):
    lengths = torch.tensor([1, 16, 33, 200])
    b = make_paged_batch(4, 2 * gq, 2, hd, torch.float32, lengths, seed=6)
    out = reference_port.attention_kvcache(b.q, b.k_cache, b.v_cache,
                                           cache_seqlens=b.cache_seqlens.clone(),
                                           block_table=b.block_table)
    for i, n in enumerate(lengths.tolist()):
        row = b.block_table[i].tolist()
        lib = sdpa_reference(b.q[i, 0], gather_dense(b.k_cache, row, n),
                             gather_dense(b.v_cache, row, n), b.scale)
        torch.testing.assert_close(out[i, 0].double(), lib, atol=2e-5, rtol=1e-5)


def test_gqa_mapping_with_constant_v_per_kv_head():
    hq, hkv, hd = 8, 2, 64
    b = make_paged_batch(2, hq, hkv, hd, torch.float32, torch.tensor([20, 50]), seed=7)
    b.v_cache[:, :, 0] = 3.0
    b.v_cache[:, :, 1] = -5.0
    out = reference_port.attention_kvcache(b.q, b.k_cache, b.v_cache,
                                           cache_seqlens=b.cache_seqlens.clone(),
                                           block_table=b.block_table)
    for h in range(hq):
        expect = 3.0 if h < hq // hkv else -5.0
        assert torch.allclose(out[:, 0, h], torch.full_like(out[:, 0, h], expect), atol=1e-5)
    f64 = c_oracle.paged_decode_f64(b.q, b.k_cache, b.v_cache, b.block_table, b.cache_seqlens,
                                    b.scale)
    assert np.allclose(f64[:, : hq // hkv], 3.0, atol=1e-12)
    assert np.allclose(f64[:, hq // hkv:], -5.0, atol=1e-12)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_fp64_oracle_matches_fp32_port(dtype):
    lengths = torch.tensor([1, 15, 16, 17, 100, 513])
    b = make_paged_batch(6, 16, 4, 128, dtype, lengths, seed=8)
    f64 = c_oracle.paged_decode_f64(b.q, b.k_cache, b.v_cache, b.block_table, b.cache_seqlens,
                                    b.scale)
    # fp32 math on the same widened inputs, before the final cast to dtype.
    cpu32 = make_paged_batch(6, 16, 4, 128, dtype, lengths, seed=8)
    port = reference_port.attention_kvcache(
        cpu32.q.float(), cpu32.k_cache.float(), cpu32.v_cache.float(),
        cache_seqlens=cpu32.cache_seqlens.clone(), block_table=cpu32.block_table,
        softmax_scale=cpu32.scale).numpy()[:, 0]
    assert np.abs(port - f64).max() < 2e-5


def test_fp64_oracle_matches_double_library_attention():
    lengths = torch.tensor([3, 64, 250])
    b = make_paged_batch(3, 8, 2, 64, torch.float32, lengths, page_size=8, seed=9)
    f64 = c_oracle.paged_decode_f64(b.q, b.k_cache, b.v_cache, b.block_table, b.cache_seqlens,
                                    b.scale)
    for i, n in enumerate(lengths.tolist()):
        row = b.block_table[i].tolist()
        lib = sdpa_reference(b.q[i, 0], gather_dense(b.k_cache, row, n),
                             gather_dense(b.v_cache, row, n), b.scale)
        assert np.abs(f64[i] - lib.numpy()).max() < 1e-10


def test_peaked_query_selects_one_value_row():
    b = make_paged_batch(1, 4, 1, 64, torch.float32, torch.tensor([40]), seed=10)
    row = b.block_table[0].tolist()
    target = 23
    k_t = b.k_cache[row[target // 16], target % 16, 0]
    b.q[0, 0, :] = 40.0 * k_t / k_t.norm()
    f64 = c_oracle.paged_decode_f64(b.q, b.k_cache, b.v_cache, b.block_table, b.cache_seqlens,
                                    1.0)
    v_t = b.v_cache[row[target // 16], target % 16, 0].double().numpy()
    assert np.abs(f64[0, 0] - v_t).max() < 1e-6


def test_permuting_pages_with_the_table_changes_nothing():
    b = make_paged_batch(3, 8, 2, 64, torch.float32, torch.tensor([10, 47, 90]), seed=11)
    ref = c_oracle.paged_decode_f64(b.q, b.k_cache, b.v_cache, b.block_table, b.cache_seqlens,
                                    b.scale)
    perm = torch.randperm(b.k_cache.shape[0], generator=torch.Generator().manual_seed(3))
    inv = torch.empty_like(perm)
    inv[perm] = torch.arange(perm.numel())
    k2, v2 = b.k_cache[perm], b.v_cache[perm]            # new page i = old page perm[i]
    table2 = inv[b.block_table.long()].to(torch.int32)  # old page p now lives at inv[p]
    out = c_oracle.paged_decode_f64(b.q, k2, v2, table2, b.cache_seqlens, b.scale)
    assert np.array_equal(ref, out)


def test_empty_sequence_gives_zeros_in_fp64_oracle():
    b = make_paged_batch(2, 4, 2, 64, torch.float16, torch.tensor([0, 5]), seed=12)
    out = c_oracle.paged_decode_f64(b.q, b.k_cache, b.v_cache, b.block_table, b.cache_seqlens,
                                    b.scale)
    assert np.array_equal(out[0], np.zeros_like(out[0]))
    assert np.abs(out[1]).max() > 0


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_append_oracle_is_index_assignment(dtype):
    torch.manual_seed(13)
    b = make_paged_batch(3, 8, 2, 64, dtype, torch.tensor([9, 19, 33]), seed=13,
                         block_table_width=4)
    seqlens = torch.tensor([5, 16, 30], dtype=torch.int32)
    k_new = torch.randn(3, 4, 2, 64).to(dtype)
    v_new = torch.randn(3, 4, 2, 64).to(dtype)
    got_k, got_v = c_oracle.append_kv(k_new, v_new, b.k_cache, b.v_cache, b.block_table, seqlens)
    exp_k, exp_v = b.k_cache.clone(), b.v_cache.clone()
    for i in range(3):
        for t in range(4):
            pos = int(seqlens[i]) + t
            if pos // 16 >= b.block_table.shape[1]:
                continue
            page = int(b.block_table[i, pos // 16])
            exp_k[page, pos % 16] = k_new[i, t]
            exp_v[page, pos % 16] = v_new[i, t]
    assert torch.equal(got_k, exp_k) and torch.equal(got_v, exp_v)


def test_reshape_and_cache_oracle_skips_negative_slots():
    torch.manual_seed(14)
    kc = torch.randn(4, 16, 2, 64).to(torch.bfloat16)
    vc = torch.randn(4, 16, 2, 64).to(torch.bfloat16)
    key = torch.randn(5, 2, 64).to(torch.bfloat16)
    value = torch.randn(5, 2, 64).to(torch.bfloat16)
    slots = torch.tensor([0, 17, -1, 63, 40])
    got_k, got_v = c_oracle.reshape_and_cache(key, value, kc, vc, slots)
    exp_k, exp_v = kc.clone(), vc.clone()
    for t, s in enumerate(slots.tolist()):
        if s >= 0:
            exp_k[s // 16, s % 16] = key[t]
            exp_v[s // 16, s % 16] = value[t]
    assert torch.equal(got_k, exp_k) and torch.equal(got_v, exp_v)
    assert not torch.equal(got_k, kc)


@pytest.mark.parametrize("length,chunk,splits", [(1, 64, 4), (100, 16, 8), (257, 64, 5),
                                                 (1000, 512, 2), (64, 64, 1), (300, 7, 60)])
def test_split_partials_merge_to_unsplit_attention(length, chunk, splits):
    rng = np.random.default_rng(length + chunk)
    q = rng.standard_normal(64)
    k = rng.standard_normal((length, 64)) * np.where(rng.random((length, 1)) < 0.05, 8.0, 1.0)
    v = rng.standard_normal((length, 64))
    scale = 1 / math.sqrt(64)
    whole = split_model.attention_f64(q, k, v, scale)
    outs, lse = split_model.split_partials(q, k, v, scale, chunk, max(splits, -(-length // chunk)))
    merged = split_model.lse_combine(outs, lse)
    assert np.abs(merged - whole).max() < 1e-12
    # Empty splits carry -inf and weigh nothing (the sum order may move the last ulp).
    padded = split_model.lse_combine(np.vstack([outs, np.zeros((3, 64))]),
                                     np.concatenate([lse, [-np.inf] * 3]))
    assert np.abs(padded - merged).max() < 1e-14


def test_split_model_matches_fp64_oracle():
    b = make_paged_batch(1, 2, 1, 64, torch.float32, torch.tensor([333]), seed=15)
    f64 = c_oracle.paged_decode_f64(b.q, b.k_cache, b.v_cache, b.block_table, b.cache_seqlens,
                                    b.scale)
    row = b.block_table[0].tolist()
    keys = gather_dense(b.k_cache, row, 333)[:, 0].double().numpy()
    vals = gather_dense(b.v_cache, row, 333)[:, 0].double().numpy()
    outs, lse = split_model.split_partials(b.q[0, 0, 0].double().numpy(), keys, vals, b.scale,
                                           64, 6)
    assert np.abs(split_model.lse_combine(outs, lse) - f64[0, 0]).max() < 1e-12


FP8 = torch.float8_e4m3fn


def test_e4m3fn_decode_matches_torch_for_every_code():
    codes = torch.arange(256, dtype=torch.uint8)
    mine = c_oracle.e4m3fn_decode(codes)
    ref = codes.view(FP8).float()
    assert torch.equal(torch.isnan(mine), torch.isnan(ref))
    assert torch.isnan(mine).sum() == 2  # S.1111.111 only
    ok = ~torch.isnan(ref)
    assert torch.equal(mine[ok], ref[ok])
    assert mine[0x7E] == 448.0 and mine[0x01] == 2.0 ** -9 and mine[0x08] == 2.0 ** -6


def test_e4m3fn_encode_rounds_to_nearest_even_like_torch():
    g = torch.Generator().manual_seed(0)
    x = torch.cat([torch.randn(50000, generator=g) * s for s in (1e-3, 0.05, 1.0, 30.0, 150.0)])
    x = x[x.abs() < 448]
    assert torch.equal(c_oracle.e4m3fn_encode(x), x.to(FP8).view(torch.uint8))
    # Exact midpoints between neighbouring codes: ties go to the even code.
    grid = c_oracle.e4m3fn_decode(torch.arange(0, 127, dtype=torch.uint8)).double()
    mids = ((grid[1:] + grid[:-1]) / 2).float()
    mids = torch.cat([mids, -mids])
    got = c_oracle.e4m3fn_encode(mids)
    assert torch.equal(got, mids.to(FP8).view(torch.uint8))
    assert ((got & 1) == 0).all()


def test_e4m3fn_encode_is_the_nearest_code_by_brute_force():
    finite = torch.arange(256, dtype=torch.uint8)
    finite = finite[(finite & 0x7F) != 0x7F]
    values = c_oracle.e4m3fn_decode(finite).double()
    g = torch.Generator().manual_seed(1)
    x = (torch.rand(4000, generator=g, dtype=torch.float64) * 2 - 1) * 440
    x = torch.cat([x, x * 1e-3]).float()
    got = c_oracle.e4m3fn_encode(x)
    dist = (x.double()[:, None] - values[None, :]).abs()
    best = dist.min(dim=1).values
    mine = (x.double() - c_oracle.e4m3fn_decode(got).double()).abs()
    assert torch.equal(mine, best)


def test_e4m3fn_encode_saturates_and_keeps_nan():
    x = torch.tensor([448.0, 449.0, 464.0, 500.0, 1e9, float("inf"), -float("inf"), -1e9,
                      float("nan"), -0.0, 0.0, 2.0 ** -10, 2.0 ** -10 * 3])
    got = c_oracle.e4m3fn_encode(x).tolist()
    assert got[:8] == [0x7E, 0x7E, 0x7E, 0x7E, 0x7E, 0x7E, 0xFE, 0xFE]
    assert got[8] & 0x7F == 0x7F
    assert got[9:] == [0x80, 0x00, 0x00, 0x02]  # 2^-10 ties to 0; 1.5 * 2^-9 ties to 2


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_fp8_append_oracle_is_scaled_index_assignment(dtype):
    g = torch.Generator().manual_seed(2)
    key = (torch.randn(12, 2, 64, generator=g) * 3).to(dtype)
    value = (torch.randn(12, 2, 64, generator=g) * 3).to(dtype)
    k_cache = torch.randint(0, 256, (5, 4, 2, 64), generator=g, dtype=torch.uint8)
    v_cache = torch.randint(0, 256, (5, 4, 2, 64), generator=g, dtype=torch.uint8)
    slots = torch.randperm(20, generator=g)[:12]
    slots[3] = -1
    ks, vs = 0.1, 0.75
    got_k, got_v = c_oracle.reshape_and_cache_fp8(key, value, k_cache, v_cache, slots, ks, vs)
    want_k, want_v = k_cache.clone(), v_cache.clone()
    keep = slots >= 0
    pg, off = slots[keep] // 4, slots[keep] % 4
    want_k[pg, off] = (key[keep].float() / ks).clamp(-448, 448).to(FP8).view(torch.uint8)
    want_v[pg, off] = (value[keep].float() / vs).clamp(-448, 448).to(FP8).view(torch.uint8)
    assert torch.equal(got_k, want_k) and torch.equal(got_v, want_v)


def test_fp8_decode_oracle_equals_fp64_oracle_on_dequantised_caches():
    b = make_paged_batch(3, 8, 2, 64, torch.float32, torch.tensor([1, 50, 300]), seed=16)
    k8, v8 = b.k_cache.to(FP8), b.v_cache.to(FP8)
    got = c_oracle.paged_decode_fp8_f64(b.q, k8, v8, b.block_table, b.cache_seqlens, b.scale,
                                        2.0, 0.5)
    # Powers of two: the dequantised caches are exact in float32.
    kf = c_oracle.e4m3fn_decode(k8) * 2.0
    vf = c_oracle.e4m3fn_decode(v8) * 0.5
    want = c_oracle.paged_decode_f64(b.q, kf, vf, b.block_table, b.cache_seqlens, b.scale)
    assert np.abs(got - want).max() < 1e-12


# Sliding window (window_left): an extension with no reference counterpart,
# pinned by identities against the unwindowed port and by library attention.

@pytest.mark.parametrize("window", [0, 1, 15, 16, 17, 64, 299, 1000])
def test_window_equals_attention_over_the_last_keys(window):
    # One query token at position L-1 sees keys [L-1-window, L-1]: the same as
    # unwindowed attention over those keys alone, computed by slicing.
    lengths = torch.tensor([1, 5, 16, 17, 100, 300])
    b = make_paged_batch(6, 8, 2, 64, torch.float32, lengths, seed=41)
    got = reference_port.attention_kvcache(b.q, b.k_cache, b.v_cache,
                                           cache_seqlens=b.cache_seqlens.clone(),
                                           block_table=b.block_table, window_left=window)
    for i, n in enumerate(lengths.tolist()):
        row = b.block_table[i].tolist()
        keep = min(n, window + 1)
        kb = gather_dense(b.k_cache, row, n)[n - keep:]
        vb = gather_dense(b.v_cache, row, n)[n - keep:]
        want = reference_port.attention_single(b.q[i], kb, vb, softmax_scale=b.scale)
        torch.testing.assert_close(got[i], want, atol=2e-6, rtol=1e-6)


@pytest.mark.parametrize("window", [0, 3, 20])
def test_window_rows_of_several_tokens_are_single_token_windows(window):
    # Causal token t of QL sits at position L-QL+t: its output is one-token
    # windowed decode over the cache cut at that position.
    ql, lengths = 3, torch.tensor([3, 9, 40])
    b = make_paged_batch(3, 8, 4, 64, torch.float32, lengths, seed=42, q_len=ql)
    got = reference_port.attention_kvcache(b.q, b.k_cache, b.v_cache,
                                           cache_seqlens=b.cache_seqlens.clone(),
                                           block_table=b.block_table, causal=True,
                                           window_left=window)
    for i, n in enumerate(lengths.tolist()):
        for t in range(ql):
            cut = torch.tensor([n - ql + t + 1])
            one = reference_port.attention_kvcache(
                b.q[i:i + 1, t:t + 1], b.k_cache, b.v_cache, cache_seqlens=cut,
                block_table=b.block_table[i:i + 1], window_left=window)
            torch.testing.assert_close(got[i, t], one[0, 0])


@pytest.mark.parametrize("causal", [False, True])
def test_window_matches_library_attention_with_a_built_mask(causal):
    ql, window, n = 4, 6, 30
    b = make_paged_batch(1, 4, 2, 64, torch.float64, torch.tensor([n]), seed=43, q_len=ql)
    got = reference_port.attention_kvcache(b.q, b.k_cache, b.v_cache,
                                           cache_seqlens=b.cache_seqlens.clone(),
                                           block_table=b.block_table, causal=causal,
                                           window_left=window)
    row = b.block_table[0].tolist()
    keys, values = gather_dense(b.k_cache, row, n), gather_dense(b.v_cache, row, n)
    allowed = torch.zeros(ql, n, dtype=torch.bool)
    for t in range(ql):
        pos = n - ql + t
        for j in range(n):
            allowed[t, j] = j >= pos - window and (j <= pos or not causal)
    for h in range(4):
        qh = b.q[0, :, h].unsqueeze(0).unsqueeze(0)
        kh = keys[:, h // 2].unsqueeze(0).unsqueeze(0)
        vh = values[:, h // 2].unsqueeze(0).unsqueeze(0)
        want = F.scaled_dot_product_attention(qh, kh, vh, attn_mask=allowed, scale=b.scale)
        # The port computes in fp32 (as reference.py does); a wrong mask would
        # differ by O(0.1).
        torch.testing.assert_close(got[0, :, h], want[0, 0], atol=2e-6, rtol=1e-5)


def test_window_covering_the_sequence_changes_nothing():
    b = make_paged_batch(3, 8, 2, 64, torch.float32, torch.tensor([1, 50, 128]), seed=44,
                         q_len=2)
    args = dict(cache_seqlens=b.cache_seqlens, block_table=b.block_table, causal=True)
    plain = reference_port.attention_kvcache(b.q, b.k_cache, b.v_cache, **args)
    wide = reference_port.attention_kvcache(b.q, b.k_cache, b.v_cache, window_left=127, **args)
    assert torch.equal(plain, wide)


# Attention sinks (vLLM's s_aux): an extension with no reference counterpart.

def test_sinks_of_minus_infinity_change_nothing():
    b = make_paged_batch(3, 8, 2, 64, torch.float32, torch.tensor([1, 50, 300]), seed=51,
                         q_len=2)
    args = dict(cache_seqlens=b.cache_seqlens, block_table=b.block_table, causal=True)
    plain = reference_port.attention_kvcache(b.q, b.k_cache, b.v_cache, **args)
    sunk = reference_port.attention_kvcache(b.q, b.k_cache, b.v_cache,
                                            sinks=torch.full((8,), float("-inf")), **args)
    torch.testing.assert_close(plain, sunk, atol=1e-7, rtol=1e-6)


def test_sinks_match_library_attention_over_one_appended_key():
    # For one query token, a key k* with q.k* * scale = sink and a zero value
    # row makes library attention equal to attention with that sink.
    hq, hkv, hd, n = 8, 2, 64, 77
    b = make_paged_batch(1, hq, hkv, hd, torch.float64, torch.tensor([n]), seed=52)
    sinks = torch.linspace(-3.0, 4.0, hq, dtype=torch.float64)
    got = reference_port.attention_kvcache(b.q, b.k_cache, b.v_cache,
                                           cache_seqlens=b.cache_seqlens.clone(),
                                           block_table=b.block_table, sinks=sinks)
    row = b.block_table[0].tolist()
    keys, values = gather_dense(b.k_cache, row, n), gather_dense(b.v_cache, row, n)
    for h in range(hq):
        qh = b.q[0, 0, h]
        kstar = qh * sinks[h] / (b.scale * qh.dot(qh))
        kh = torch.cat([keys[:, h // (hq // hkv)], kstar[None]])[None, None]
        vh = torch.cat([values[:, h // (hq // hkv)], torch.zeros(1, hd, dtype=torch.float64)])
        want = F.scaled_dot_product_attention(qh.view(1, 1, 1, -1), kh, vh[None, None],
                                              scale=b.scale).view(-1)
        torch.testing.assert_close(got[0, 0, h], want, atol=2e-6, rtol=1e-5)


def test_a_dominant_sink_silences_the_output():
    b = make_paged_batch(2, 4, 2, 64, torch.float32, torch.tensor([5, 40]), seed=53)
    out = reference_port.attention_kvcache(b.q, b.k_cache, b.v_cache,
                                           cache_seqlens=b.cache_seqlens.clone(),
                                           block_table=b.block_table,
                                           sinks=torch.full((4,), 1.0e4))
    assert torch.equal(out, torch.zeros_like(out))


# Logit soft-capping: an extension with no reference counterpart.

def test_a_tiny_softcap_gives_uniform_weights():
    lengths = torch.tensor([3, 40])
    b = make_paged_batch(2, 4, 2, 64, torch.float32, lengths, seed=61)
    out = reference_port.attention_kvcache(b.q, b.k_cache, b.v_cache,
                                           cache_seqlens=b.cache_seqlens.clone(),
                                           block_table=b.block_table, softcap=1e-6)
    for i, n in enumerate(lengths.tolist()):
        mean = gather_dense(b.v_cache, b.block_table[i].tolist(), n).mean(0)  # [HKV, D]
        torch.testing.assert_close(out[i, 0], mean.repeat_interleave(2, 0), atol=1e-5,
                                   rtol=1e-5)


def test_a_huge_softcap_changes_nothing():
    b = make_paged_batch(2, 8, 2, 64, torch.float32, torch.tensor([30, 500]), seed=62)
    args = dict(cache_seqlens=b.cache_seqlens, block_table=b.block_table)
    plain = reference_port.attention_kvcache(b.q, b.k_cache, b.v_cache, **args)
    capped = reference_port.attention_kvcache(b.q, b.k_cache, b.v_cache, softcap=1e7, **args)
    torch.testing.assert_close(plain, capped, atol=1e-6, rtol=1e-5)


def test_softcap_on_two_keys_by_hand():
    # q = e0, k_j = a_j e0: scaled scores s_j = a_j * scale; capped weights
    # exp(cap * tanh(s_j / cap)) computed here by hand.
    cap, scale, a = 2.0, 0.5, (3.0, -1.0)
    q = torch.zeros(1, 1, 8)
    q[0, 0, 0] = 1.0
    k = torch.zeros(2, 1, 8)
    v = torch.zeros(2, 1, 8)
    for j, aj in enumerate(a):
        k[j, 0, 0] = aj
        v[j, 0, j + 1] = 1.0
    w = [math.exp(cap * math.tanh(aj * scale / cap)) for aj in a]
    out = reference_port.attention_single(q, k, v, softmax_scale=scale, softcap=cap)
    assert out[0, 0, 1].item() == pytest.approx(w[0] / sum(w), abs=1e-6)
    assert out[0, 0, 2].item() == pytest.approx(w[1] / sum(w), abs=1e-6)


# ALiBi slopes: an extension with no reference counterpart.

def test_zero_alibi_slopes_change_nothing():
    b = make_paged_batch(2, 8, 2, 64, torch.float32, torch.tensor([30, 200]), seed=71, q_len=2)
    args = dict(cache_seqlens=b.cache_seqlens, block_table=b.block_table, causal=True)
    plain = reference_port.attention_kvcache(b.q, b.k_cache, b.v_cache, **args)
    zero = reference_port.attention_kvcache(b.q, b.k_cache, b.v_cache,
                                            alibi_slopes=torch.zeros(8), **args)
    torch.testing.assert_close(plain, zero)


@pytest.mark.parametrize("causal", [True, False])
def test_alibi_weights_of_a_zero_query_by_hand(causal):
    # All raw scores 0: key j of the query at position p weighs e^(-s|p-j|);
    # with one-hot V rows the output is those weights, normalised.
    n, ql, hd = 6, 2, 8
    slopes = torch.tensor([0.5, 1.25])
    q = torch.zeros(ql, 2, hd)
    k = torch.randn(n, 1, hd)
    v = torch.zeros(n, 1, hd)
    for j in range(n):
        v[j, 0, j] = 1.0
    out = reference_port.attention_single(q, k, v, causal=causal, alibi_slopes=slopes)
    for t in range(ql):
        p = n - ql + t
        for h in range(2):
            keys = [j for j in range(n) if j <= p or not causal]
            w = {j: math.exp(-float(slopes[h]) * abs(p - j)) for j in keys}
            total = sum(w.values())
            for j in range(n):
                assert out[t, h, j].item() == pytest.approx(w.get(j, 0.0) / total, abs=1e-6)


@pytest.mark.parametrize("extras", [False, True])
def test_token_chunks_of_a_causal_query_equal_the_whole_query(extras):
    # The identity behind running a causal query past the kernel's 16 columns
    # as several launches: rows [a, e) of the whole query equal a query of
    # those tokens on sequences shortened by QL - e keys (lengths below the
    # chunk's tokens leave rows without keys, zeros in both).
    from mxflashattn_amd import native

    ql, gq = 7, 4
    b = make_paged_batch(4, 2 * gq, 2, 64, torch.float32, torch.tensor([3, 9, 40, 130]),
                         seed=151, q_len=ql)
    kw = dict(block_table=b.block_table, softmax_scale=b.scale, causal=True)
    if extras:
        kw.update(window_left=5, softcap=2.0, sinks=torch.linspace(-1.0, 1.0, 2 * gq),
                  alibi_slopes=torch.pow(2.0, -torch.arange(1, 2 * gq + 1, dtype=torch.float32)))
    rows = []
    for i in range(b.batch):
        lens = b.cache_seqlens[i:i + 1]
        one = dict(kw, block_table=b.block_table[i:i + 1])
        whole = reference_port.attention_kvcache(b.q[i:i + 1], b.k_cache, b.v_cache,
                                                 cache_seqlens=lens.clone(), **one)
        for first, end, add in native.token_chunks(ql, 16 // gq, 0):
            short = (lens + add).clamp_min(0)
            if int(short) == 0:  # no key for any of these tokens
                assert torch.all(whole[:, first:end] == 0), (i, first)
                continue
            part = reference_port.attention_kvcache(b.q[i:i + 1, first:end], b.k_cache,
                                                    b.v_cache, cache_seqlens=short.clone(), **one)
            torch.testing.assert_close(part, whole[:, first:end], rtol=1e-5, atol=1e-6)
            rows.append((i, first))
    assert len(rows) >= 6


def varlen_library(q, k, v, cu_q, cu_k, scale, causal):
    """Per segment: float64 library attention with a mask built from positions
    (query i of a segment sits at key position i + Lk - Lq); rows that see no
    key are zeros."""
    rows = []
    for i in range(len(cu_q) - 1):
        qs, ks = q[cu_q[i]:cu_q[i + 1]], k[cu_k[i]:cu_k[i + 1]]
        vs = v[cu_k[i]:cu_k[i + 1]]
        lq, lk = qs.shape[0], ks.shape[0]
        if lq == 0:
            continue
        group = qs.shape[1] // ks.shape[1]
        qh = qs.double().permute(1, 0, 2).unsqueeze(0)
        kh = ks.double().repeat_interleave(group, dim=1).permute(1, 0, 2).unsqueeze(0)
        vh = vs.double().repeat_interleave(group, dim=1).permute(1, 0, 2).unsqueeze(0)
        allowed = torch.ones(lq, lk, dtype=torch.bool)
        if causal:
            pos = torch.arange(lq).unsqueeze(1) + (lk - lq)
            allowed = torch.arange(lk).unsqueeze(0) <= pos
        o = F.scaled_dot_product_attention(qh, kh, vh, attn_mask=allowed, scale=scale)
        o = torch.nan_to_num(o, nan=0.0)[0].permute(1, 0, 2)
        o[~allowed.any(dim=1)] = 0.0
        rows.append(o)
    return torch.cat(rows, dim=0)


@pytest.mark.parametrize("causal", [False, True])
def test_varlen_port_matches_library_attention_per_segment(causal):
    torch.manual_seed(17)
    cu_q = [0, 2, 2, 3, 7]     # segment 1 has no query row
    cu_k = [0, 3, 7, 8, 10]    # segment 3: four queries over two keys
    q = torch.randn(7, 4, 64)
    k = torch.randn(10, 2, 64)
    v = torch.randn(10, 2, 64)
    out = reference_port.attention_varlen(q, k, v, cu_q, cu_k, softmax_scale=0.3, causal=causal)
    assert out.shape == q.shape
    expected = varlen_library(q, k, v, cu_q, cu_k, 0.3, causal)
    torch.testing.assert_close(out.double(), expected, atol=1e-5, rtol=1e-5)
    if causal:  # the first two queries of segment 3 see no key
        assert torch.equal(out[3:5], torch.zeros_like(out[3:5]))


def test_varlen_port_segment_boundaries_matter():
    torch.manual_seed(18)
    cu_q, cu_k = [0, 1, 2], [0, 5, 9]
    q, k, v = torch.randn(2, 2, 64), torch.randn(9, 1, 64), torch.randn(9, 1, 64)
    out = reference_port.attention_varlen(q, k, v, cu_q, cu_k)
    shifted = reference_port.attention_varlen(q, k, v, cu_q, [0, 4, 9])
    assert not torch.allclose(out[0], shifted[0]) and not torch.allclose(out[1], shifted[1])
    torch.testing.assert_close(out.double(), varlen_library(q, k, v, cu_q, cu_k, 64 ** -0.5,
                                                            False), atol=1e-5, rtol=1e-5)
