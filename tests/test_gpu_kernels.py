"""GPU parity of the HIP kernels against the CPU oracle (through the C ABI).

Tolerances: max-abs error <= 2e-3 for fp16 and <= 1.6e-2
for bf16 against the fp32-softmax oracle (oracle.reference_port); the block-table
gather and both appends are bit-exact.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from mxflashattn_amd import native
from mxflashattn_amd.workloads import PagedBatch, make_paged_batch
from oracle import c_oracle, reference_port

pytestmark = pytest.mark.gpu

TOL = {torch.float16: 2e-3, torch.bfloat16: 1.6e-2}


def oracle_out(b) -> torch.Tensor:
    """fp32 reference output [B, 1, HQ, HD] (float32) for a PagedBatch on any device."""
    cpu = b.to("cpu")
    out = reference_port.attention_kvcache(
        cpu.q, cpu.k_cache, cpu.v_cache, cache_seqlens=cpu.cache_seqlens.clone(),
        block_table=cpu.block_table, softmax_scale=cpu.scale,
    )
    return out.float()


def max_err(actual: torch.Tensor, expected: torch.Tensor) -> float:
    return (actual.float().cpu() - expected.float().cpu()).abs().max().item()


def nan_like(t: torch.Tensor) -> torch.Tensor:
    """An output buffer whose every element the kernels must overwrite."""
    return torch.full_like(t, float("nan"))


def run_native(b, **kw) -> torch.Tensor:
    kw.setdefault("out", nan_like(b.q))
    out = native.paged_decode_split(b.q, b.k_cache, b.v_cache, b.block_table, b.cache_seqlens,
                                    b.scale, **kw)
    torch.cuda.synchronize()
    assert not torch.isnan(out.float()).any(), "an output row was left unwritten"
    return out


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=["f16", "bf16"])
@pytest.mark.parametrize("head_dim", [64, 128])
@pytest.mark.parametrize("gq", [2, 4, 8])
def test_cells_ragged_match_oracle(device, dtype, head_dim, gq):
    lengths = torch.tensor([1, 15, 16, 17, 300, 1000])
    b = make_paged_batch(6, 2 * gq, 2, head_dim, dtype, lengths, seed=11 + gq).to(device)
    expected = oracle_out(b)
    # num_splits: one range per kv head, a few, more ranges than tiles, and
    # the per-sequence kernel.
    for ns in (None, 1, 3, 16, 200, native.SPLITS_PER_SEQUENCE):
        kw = {} if ns is None else dict(num_splits=ns)
        got = run_native(b, **kw)
        assert torch.isfinite(got.float()).all()
        assert max_err(got, expected) <= TOL[dtype], ns


@pytest.mark.parametrize("page_size", [1, 2, 4, 8, 32, 64, 256])
@pytest.mark.parametrize("head_dim", [64, 128])
def test_page_sizes(device, page_size, head_dim):
    lengths = torch.tensor([3, 129, 517])
    b = make_paged_batch(3, 8, 2, head_dim, torch.float16, lengths, page_size=page_size,
                         seed=5).to(device)
    expected = oracle_out(b)
    assert max_err(run_native(b), expected) <= TOL[torch.float16]
    assert max_err(run_native(b, num_splits=12), expected) <= TOL[torch.float16]
    assert max_err(run_native(b, num_splits=native.SPLITS_PER_SEQUENCE),
                   expected) <= TOL[torch.float16]


def test_single_token_returns_v_row_exactly(device):
    # One key: softmax weight is exactly 1, so the output is the V row bit for bit.
    for dtype in (torch.float16, torch.bfloat16):
        b = make_paged_batch(4, 16, 4, 128, dtype, 1, seed=3).to(device)
        got = run_native(b).cpu()
        cpu = b.to("cpu")
        for i in range(4):
            page = int(cpu.block_table[i, 0])
            for h in range(16):
                assert torch.equal(got[i, 0, h], cpu.v_cache[page, 0, h // 4])


def test_uniform_scores_average_v(device):
    # scale = 0 makes every score equal: the output is the mean of the V rows.
    b = make_paged_batch(2, 8, 2, 64, torch.float16, torch.tensor([5, 70]), seed=9).to(device)
    got = native.paged_decode_split(b.q, b.k_cache, b.v_cache, b.block_table, b.cache_seqlens,
                                    0.0)
    torch.cuda.synchronize()
    cpu = b.to("cpu")
    for i, n in enumerate([5, 70]):
        v = reference_port.gather_pages(cpu.v_cache, cpu.block_table[i].tolist(), n).float()
        mean = v.mean(dim=0)  # [HKV, D]
        for h in range(8):
            assert (got[i, 0, h].float().cpu() - mean[h // 4]).abs().max() <= 2e-3


def test_zero_length_sequence_gives_zeros(device):
    b = make_paged_batch(3, 8, 2, 128, torch.bfloat16, torch.tensor([0, 40, 0]), seed=2).to(device)
    for kw in ({}, dict(num_splits=4), dict(num_splits=1), dict(num_splits=7)):
        got = run_native(b, **kw).cpu()
        assert torch.equal(got[0], torch.zeros_like(got[0]))
        assert torch.equal(got[2], torch.zeros_like(got[2]))
        assert torch.isfinite(got.float()).all()


def test_peaky_keys_long_context(device):
    b = make_paged_batch(2, 32, 4, 128, torch.bfloat16, 16384, peaky_fraction=0.01,
                         seed=4).to(device)
    expected = oracle_out(b)
    assert max_err(run_native(b), expected) <= TOL[torch.bfloat16]


def test_large_scores_do_not_overflow(device):
    # q x 400 (csrc_native/test_m1.py:148 "ovf" case): base-2 scores reach hundreds.
    b = make_paged_batch(2, 8, 2, 128, torch.float16, torch.tensor([512, 300]), seed=6)
    b.q = (b.q.float() * 400).clamp(-60000, 60000).to(torch.float16)
    b = b.to(device)
    got = run_native(b, num_splits=8)
    assert torch.isfinite(got.float()).all()
    expected = torch.from_numpy(c_oracle.paged_decode_f64(
        b.q.cpu(), b.k_cache.cpu(), b.v_cache.cpu(), b.block_table.cpu(), b.cache_seqlens.cpu(),
        b.scale)).reshape(got.shape)
    assert max_err(got, expected) <= 2e-3


@pytest.mark.parametrize("scale", [-0.125, -1.5, 1e-4, 3.0])
@pytest.mark.parametrize("dtype,head_dim,gq", [(torch.bfloat16, 128, 4), (torch.float16, 64, 8)])
def test_negative_tiny_and_large_scales(device, scale, dtype, head_dim, gq):
    # Any finite scale is valid: a negative one turns the largest dot products
    # into the smallest scores, a large one makes the softmax nearly one-hot
    # (base-2 scores in the hundreds, the running maximum moving often).
    b = make_paged_batch(4, 2 * gq, 2, head_dim, dtype, torch.tensor([1, 37, 600, 2000]),
                         seed=70 + head_dim).to(device)
    expected = torch.from_numpy(c_oracle.paged_decode_f64(
        b.q.cpu(), b.k_cache.cpu(), b.v_cache.cpu(), b.block_table.cpu(), b.cache_seqlens.cpu(),
        scale)).reshape(b.q.shape)
    for ns in (None, 1, 7, native.SPLITS_PER_SEQUENCE):
        out = torch.full_like(b.q, float("nan"))
        native.paged_decode_split(b.q, b.k_cache, b.v_cache, b.block_table, b.cache_seqlens,
                                  scale, out=out, num_splits=ns)
        torch.cuda.synchronize()
        assert max_err(out, expected) <= TOL[dtype], (ns, max_err(out, expected))


@pytest.mark.parametrize("page_size", [4, 16])
def test_table_slots_past_each_length_are_never_read(device, page_size):
    # Serving frameworks pad block-table rows past a sequence's pages with -1
    # or leave stale ids there: the result must not depend on them.
    lengths = torch.tensor([1, 16, 17, 250, 0, 700])
    b = make_paged_batch(6, 8, 2, 128, torch.bfloat16, lengths, page_size=page_size, seed=31,
                         block_table_width=700 // page_size + 8).to(device)
    used = (b.cache_seqlens.long() + page_size - 1) // page_size
    past = torch.arange(b.block_table.shape[1], device=device)[None, :] >= used[:, None]
    for ns in (None, 1, 3, 64, native.SPLITS_PER_SEQUENCE):
        want = run_native(b, num_splits=ns)
        for pad in (-1, 2**31 - 1):
            padded = PagedBatch(b.q, b.k_cache, b.v_cache,
                                b.block_table.masked_fill(past, pad), b.cache_seqlens, b.scale)
            assert torch.equal(run_native(padded, num_splits=ns).cpu(), want.cpu()), (ns, pad)


def test_pages_past_4_gib(device):
    # K and V caches of about 4.4 GB each, every used page past the 4 GiB byte
    # offset: tile addresses and append destinations need 64-bit arithmetic.
    # The same pages in a small pool give the same result bit for bit.
    hkv, hd, ps = 2, 128, 16
    small = make_paged_batch(3, 8, hkv, hd, torch.bfloat16, torch.tensor([40, 700, 5]), seed=41,
                             block_table_width=48).to(device)
    pool = small.k_cache.shape[0]
    num_pages = (4 << 30) // (ps * hkv * hd * 2) + 16000
    k = torch.empty(num_pages, ps, hkv, hd, dtype=torch.bfloat16, device=device)
    v = torch.empty_like(k)
    k[num_pages - pool:] = small.k_cache.flip(0)  # page p -> num_pages - 1 - p
    v[num_pages - pool:] = small.v_cache.flip(0)
    big = PagedBatch(small.q, k, v, (num_pages - 1 - small.block_table).to(torch.int32),
                     small.cache_seqlens, small.scale)
    assert int(big.block_table.min()) * ps * hkv * hd * 2 >= 4 << 30
    for ns in (None, 1, 5, native.SPLITS_PER_SEQUENCE):
        assert torch.equal(run_native(big, num_splits=ns).cpu(),
                           run_native(small, num_splits=ns).cpu()), ns
    # Appends land in the same rows of the far pages.
    k_new = torch.randn(3, 2, hkv, hd, device=device).to(torch.bfloat16)
    v_new = torch.randn(3, 2, hkv, hd, device=device).to(torch.bfloat16)
    kc, vc = small.k_cache.clone(), small.v_cache.clone()
    native.append_kv(k_new, v_new, kc, vc, small.block_table, small.cache_seqlens)
    native.append_kv(k_new, v_new, k, v, big.block_table, big.cache_seqlens)
    torch.cuda.synchronize()
    assert torch.equal(k[num_pages - pool:].flip(0).cpu(), kc.cpu())
    assert torch.equal(v[num_pages - pool:].flip(0).cpu(), vc.cpu())
    # The slot form (vLLM's slot_mapping), one more token per sequence.
    pos = small.cache_seqlens.long() + 2
    page_col = (pos // ps).view(-1, 1)
    key, value = k_new[:, 0].contiguous(), v_new[:, 0].contiguous()
    for table, kd, vd in ((small.block_table, kc, vc), (big.block_table, k, v)):
        slots = table.long().gather(1, page_col).view(-1) * ps + pos % ps
        native.reshape_and_cache(key, value, kd, vd, slots)
    torch.cuda.synchronize()
    assert torch.equal(k[num_pages - pool:].flip(0).cpu(), kc.cpu())
    assert torch.equal(v[num_pages - pool:].flip(0).cpu(), vc.cpu())
    del k, v, big
    torch.cuda.empty_cache()


def test_noncontiguous_q_and_out(device):
    b = make_paged_batch(4, 16, 4, 128, torch.float16, torch.tensor([33, 64, 1, 200]),
                         seed=8).to(device)
    fused = torch.randn(4, 1, 48, 128, device=device, dtype=torch.float16)
    fused[:, :, 16:32] = b.q
    q_view = fused[:, :, 16:32]
    assert not q_view.is_contiguous()
    out_buf = torch.zeros(4, 1, 40, 128, device=device, dtype=torch.float16)
    out_view = out_buf[:, :, 8:24]
    native.paged_decode_split(q_view, b.k_cache, b.v_cache, b.block_table, b.cache_seqlens,
                              b.scale, out=out_view)
    torch.cuda.synchronize()
    assert max_err(out_view, oracle_out(b)) <= TOL[torch.float16]
    assert torch.equal(out_buf[:, :, :8].cpu(), torch.zeros(4, 1, 8, 128, dtype=torch.float16))


def test_config2_full_size_matches_oracle(device):
    from mxflashattn_amd.workloads import CONFIGS

    b = make_paged_batch(**CONFIGS["config2_qwen3_4b"], device=device)
    got = run_native(b)
    assert max_err(got, oracle_out(b)) <= TOL[torch.bfloat16]
    # Split-count independence at full size: one range per kv head (every
    # sequence whole inside it) gives the same answer as the balanced split.
    one = run_native(b, num_splits=1)
    assert max_err(got, one) <= TOL[torch.bfloat16]


def test_append_kv_bit_exact(device):
    for dtype in (torch.float16, torch.bfloat16):
        # Allocate pages for the appended rows too, so every destination is distinct.
        b = make_paged_batch(3, 8, 2, 128, dtype, torch.tensor([8, 19, 33]), seed=12,
                             block_table_width=4).to(device)
        b.cache_seqlens = torch.tensor([5, 16, 30], dtype=torch.int32, device=device)
        k_new = torch.randn(3, 3, 2, 128, device=device).to(dtype)
        v_new = torch.randn(3, 3, 2, 128, device=device).to(dtype)
        exp_k, exp_v = c_oracle.append_kv(k_new.cpu(), v_new.cpu(), b.k_cache.cpu(),
                                          b.v_cache.cpu(), b.block_table.cpu(),
                                          b.cache_seqlens.cpu())
        kc, vc = b.k_cache.clone(), b.v_cache.clone()
        native.append_kv(k_new, v_new, kc, vc, b.block_table, b.cache_seqlens)
        torch.cuda.synchronize()
        assert torch.equal(kc.cpu(), exp_k) and torch.equal(vc.cpu(), exp_v)


def test_reshape_and_cache_bit_exact(device):
    for dtype in (torch.float16, torch.bfloat16):
        kc = torch.randn(6, 16, 4, 64, device=device).to(dtype)
        vc = torch.randn(6, 16, 4, 64, device=device).to(dtype)
        key = torch.randn(5, 4, 64, device=device).to(dtype)
        value = torch.randn(5, 4, 64, device=device).to(dtype)
        slots = torch.tensor([0, 17, -1, 95, 40], device=device, dtype=torch.int64)
        exp_k, exp_v = c_oracle.reshape_and_cache(key.cpu(), value.cpu(), kc.cpu(), vc.cpu(),
                                                  slots.cpu())
        native.reshape_and_cache(key, value, kc, vc, slots)
        torch.cuda.synchronize()
        assert torch.equal(kc.cpu(), exp_k) and torch.equal(vc.cpu(), exp_v)


def test_fp64_oracle_agrees_with_fp32_port_on_gpu_inputs(device):
    # Cross-check of the two oracles on the data the kernels see.
    b = make_paged_batch(3, 8, 2, 64, torch.float16, torch.tensor([7, 100, 333]), seed=13)
    ref64 = c_oracle.paged_decode_f64(b.q, b.k_cache, b.v_cache, b.block_table, b.cache_seqlens,
                                      b.scale)
    port = oracle_out(b).reshape(ref64.shape).numpy()
    assert np.abs(port - ref64).max() <= 2e-3


@pytest.mark.parametrize("hq,hkv,head_dim", [
    (2, 1, 128), (8, 1, 64), (6, 3, 128), (24, 12, 64), (32, 16, 128), (64, 16, 64),
    (20, 20, 64), (40, 20, 128), (40, 40, 64), (80, 40, 128),
])
def test_kv_head_counts(device, hq, hkv, head_dim):
    # Workgroups hold min(HKV, waves) kv heads x waves // that sub-ranges: one
    # kv head with four sub-ranges, three heads with one, and past 8 (128-byte
    # rows) or 4 (256-byte rows) kv heads several head groups, the last one
    # partly used at 20 and 40.
    lengths = torch.tensor([1, 40, 700, 16, 33])
    b = make_paged_batch(5, hq, hkv, head_dim, torch.bfloat16, lengths, seed=21).to(device)
    expected = oracle_out(b)
    for ns in (None, 1, 2, 5, 64, native.SPLITS_PER_SEQUENCE):
        kw = {} if ns is None else dict(num_splits=ns)
        assert max_err(run_native(b, **kw), expected) <= TOL[torch.bfloat16], ns


@pytest.mark.parametrize("hkv", [5, 6, 7])
@pytest.mark.parametrize("head_dim,fp8", [(64, False), (128, False), (64, True), (128, True)],
                         ids=["hd64", "hd128", "fp8_hd64", "fp8_hd128"])
def test_five_to_seven_kv_heads(device, hkv, head_dim, fp8):
    # Rows of up to 128 bytes (16-bit HD 64, fp8 HD 64 and 128) put 5-7 kv
    # heads in one eight-wave workgroup whose other waves leave at once;
    # 256-byte rows split them over two four-wave head groups. The output
    # starts as NaN, so a head no wave computes cannot pass.
    lengths = torch.tensor([1, 40, 700, 16, 2100])
    b = make_paged_batch(5, 2 * hkv, hkv, head_dim, torch.bfloat16, lengths,
                         seed=60 + hkv).to(device)
    k_cache, v_cache = b.k_cache, b.v_cache
    if fp8:
        k_cache = b.k_cache.cpu().to(torch.float8_e4m3fn).to(device)
        v_cache = b.v_cache.cpu().to(torch.float8_e4m3fn).to(device)
        expected = torch.from_numpy(c_oracle.paged_decode_fp8_f64(
            b.q.cpu(), k_cache.cpu(), v_cache.cpu(), b.block_table.cpu(),
            b.cache_seqlens.cpu(), b.scale, 1.0, 1.0)).reshape(b.q.shape)
    else:
        expected = oracle_out(b)
    for ns in (None, 1, 5, 64, native.SPLITS_PER_SEQUENCE):
        out = torch.full_like(b.q, float("nan"))
        native.paged_decode_split(b.q, k_cache, v_cache, b.block_table, b.cache_seqlens,
                                  b.scale, out=out, num_splits=ns)
        torch.cuda.synchronize()
        err = max_err(out, expected)
        assert err <= TOL[torch.bfloat16], (ns, err)


def test_back_to_back_calls_of_changing_shapes_share_the_workspace(device):
    # Every call on a stream reuses one workspace; calls of other shapes in
    # between must not leave anything a later call reads.
    shapes = [
        (6, 32, 8, 128, torch.bfloat16, torch.tensor([900, 17, 2048, 1, 300, 64]), 40),
        (3, 16, 4, 64, torch.float16, torch.tensor([4000, 5, 129]), 200),
        (6, 32, 8, 128, torch.bfloat16, torch.tensor([900, 17, 2048, 1, 300, 64]), 7),
        (3, 16, 4, 64, torch.float16, torch.tensor([4000, 5, 129]), native.SPLITS_PER_SEQUENCE),
    ]
    batches = [make_paged_batch(*s[:6], seed=30 + i).to(device) for i, s in enumerate(shapes)]
    expected = [oracle_out(b) for b in batches]
    for _ in range(3):
        for b, exp, s in zip(batches, expected, shapes):
            got = run_native(b, num_splits=s[6])
            assert max_err(got, exp) <= TOL[b.q.dtype]


def test_head_major_cache_layout(device):
    # Cache stored [pages, HKV, PS, HD] and viewed as [pages, PS, HKV, HD]: the
    # head stride exceeds the token stride.
    b = make_paged_batch(3, 16, 4, 128, torch.float16, torch.tensor([50, 300, 17]), seed=41)
    expected = oracle_out(b)
    kc = b.k_cache.permute(0, 2, 1, 3).contiguous().permute(0, 2, 1, 3)
    vc = b.v_cache.permute(0, 2, 1, 3).contiguous().permute(0, 2, 1, 3)
    assert kc.stride(2) > kc.stride(1)
    b = b.to(device)
    out = native.paged_decode_split(b.q, kc.to(device), vc.to(device), b.block_table,
                                    b.cache_seqlens, b.scale, num_splits=9)
    torch.cuda.synchronize()
    assert max_err(out, expected) <= TOL[torch.float16]


@pytest.mark.parametrize("dtype,head_dim,gq", [(torch.bfloat16, 128, 4), (torch.float16, 64, 8)])
def test_repeated_calls_are_bitwise_reproducible(device, dtype, head_dim, gq):
    # Every piece is computed the same way on every call and the combine walks
    # the pieces in range order, so the output must not change by a single bit
    # from call to call. A combine that read a stale piece would break this.
    lengths = torch.tensor([3000, 1, 4500, 700, 2048, 17, 6000, 333])
    b = make_paged_batch(8, 8 * gq, 8, head_dim, dtype, lengths, seed=55).to(device)
    first = run_native(b).clone()
    assert max_err(first, oracle_out(b)) <= TOL[dtype]
    for _ in range(40):
        assert torch.equal(run_native(b), first)


def test_partial_then_combine_equals_one_launch(device):
    # The two stages launched separately through the C ABI give the same bits
    # as mxfa_split_decode_launch, including sequences inside one range, pieces
    # of longer ones and an empty sequence.
    lengths = torch.tensor([5000, 0, 33, 1200, 16, 7000])
    b = make_paged_batch(6, 32, 8, 128, torch.bfloat16, lengths, seed=61).to(device)
    ns = 40
    one = run_native(b, num_splits=ns).clone()
    ws = torch.empty(native.workspace_size(6, 32, 128, ns), dtype=torch.uint8, device=device)
    out = torch.full_like(b.q, float("nan"))
    native.split_decode_partial(b.q, b.k_cache, b.v_cache, b.block_table, b.cache_seqlens,
                                b.scale, out, ws, ns)
    native.split_decode_combine(ws, out, 8, ns)
    torch.cuda.synchronize()
    assert torch.equal(out, one)
    assert torch.equal(one[1], torch.zeros_like(one[1]))  # the empty sequence
    keep = torch.tensor([0, 2, 3, 4, 5], device=device)
    sub = PagedBatch(b.q[keep], b.k_cache, b.v_cache, b.block_table[keep], b.cache_seqlens[keep],
                     b.scale)
    assert max_err(one[keep], oracle_out(sub)) <= TOL[torch.bfloat16]


@pytest.mark.parametrize("head_dim", [64, 128, 256])
@pytest.mark.parametrize("lengths", [[40000], [20000, 7, 3000]], ids=["one", "three"])
def test_few_sequences_many_ranges(device, head_dim, lengths):
    # Few sequences over many ranges: hundreds to thousands of pieces per
    # (sequence, head), so the combine splits each head's chunks over 1 to 8
    # blocks to fold them in one step (or several, past that). Every split
    # count against the oracle, and the two stages against one launch.
    dtype = torch.float16 if head_dim == 128 else torch.bfloat16
    batch = len(lengths)
    b = make_paged_batch(batch, 8, 2, head_dim, dtype, torch.tensor(lengths),
                         seed=70 + head_dim + batch).to(device)
    expected = oracle_out(b)
    for ns in (60, 100, 300, 700, 2000):
        one = run_native(b, num_splits=ns)
        assert max_err(one, expected) <= TOL[dtype], ns
        ws = torch.empty(native.workspace_size(batch, 8, head_dim, ns), dtype=torch.uint8,
                         device=device)
        out = torch.full_like(b.q, float("nan"))
        native.split_decode_partial(b.q, b.k_cache, b.v_cache, b.block_table, b.cache_seqlens,
                                    b.scale, out, ws, ns)
        native.split_decode_combine(ws, out, 2, ns)
        torch.cuda.synchronize()
        assert torch.equal(out, one), ns


@pytest.mark.parametrize("ns", [None, native.SPLITS_PER_SEQUENCE], ids=["split", "per_seq"])
def test_graph_replays_match_eager(device, ns):
    # One decode call captured in a HIP graph (the workspace allocated by an
    # eager call on the capture stream first) and replayed several times with
    # unrelated eager work between replays: every replay equals the eager call.
    b = make_paged_batch(5, 16, 4, 64, torch.float16, torch.tensor([700, 3, 1500, 64, 0]),
                         seed=71).to(device)
    stream = torch.cuda.Stream(device)
    out = torch.empty_like(b.q)
    with torch.cuda.stream(stream):
        native.paged_decode_split(b.q, b.k_cache, b.v_cache, b.block_table, b.cache_seqlens,
                                  b.scale, out=out, num_splits=ns)
        eager = out.clone()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        native.paged_decode_split(b.q, b.k_cache, b.v_cache, b.block_table, b.cache_seqlens,
                                  b.scale, out=out, num_splits=ns)
    for i in range(4):
        out.fill_(float("nan"))
        with torch.cuda.stream(stream):
            graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), i
        _ = (torch.randn(4096, device=device) * i).sum().item()


def test_concurrent_streams_use_separate_workspaces(device):
    # Two streams (default priority) launch decode calls of different shapes
    # with no synchronisation between them, so their kernels may overlap on
    # the GPU; each stream has its own workspace, so every output equals the
    # single-stream result bitwise.
    g = torch.Generator().manual_seed(83)
    a = make_paged_batch(12, 32, 8, 128, torch.bfloat16,
                         torch.randint(1000, 4000, (12,), generator=g), seed=83).to(device)
    c = make_paged_batch(20, 16, 4, 64, torch.float16,
                         torch.randint(500, 3000, (20,), generator=g), seed=84).to(device)
    ref_a, ref_c = run_native(a), run_native(c)
    sa, sc = torch.cuda.Stream(device), torch.cuda.Stream(device)
    outs_a = [torch.full_like(a.q, float("nan")) for _ in range(6)]
    outs_c = [torch.full_like(c.q, float("nan")) for _ in range(6)]
    torch.cuda.synchronize()
    for oa, oc in zip(outs_a, outs_c):
        with torch.cuda.stream(sa):
            native.paged_decode_split(a.q, a.k_cache, a.v_cache, a.block_table, a.cache_seqlens,
                                      a.scale, out=oa)
        with torch.cuda.stream(sc):
            native.paged_decode_split(c.q, c.k_cache, c.v_cache, c.block_table, c.cache_seqlens,
                                      c.scale, out=oc)
    torch.cuda.synchronize()
    for i, (oa, oc) in enumerate(zip(outs_a, outs_c)):
        assert torch.equal(oa, ref_a), i
        assert torch.equal(oc, ref_c), i
    assert max_err(ref_a, oracle_out(a)) <= TOL[torch.bfloat16]


def test_maximum_batch(device):
    # 16000 sequences (the contract's maximum; the tile prefix sums fill 64 KB
    # of LDS), short ragged lengths, empty ones included.
    g = torch.Generator().manual_seed(17)
    lengths = torch.randint(0, 40, (16000,), generator=g)
    b = make_paged_batch(16000, 4, 2, 64, torch.float16, lengths, seed=17).to(device)
    expected = torch.from_numpy(c_oracle.paged_decode_f64(
        b.q.cpu(), b.k_cache.cpu(), b.v_cache.cpu(), b.block_table.cpu(), b.cache_seqlens.cpu(),
        b.scale)).reshape(b.q.shape)
    for ns in (None, 4096, native.SPLITS_PER_SEQUENCE):
        kw = {} if ns is None else dict(num_splits=ns)
        assert max_err(run_native(b, **kw), expected) <= TOL[torch.float16]


@pytest.mark.parametrize("batch", [63, 64, 65, 127, 128, 129, 255, 256, 257, 513, 1024, 4032,
                                   4033, 4353])
@pytest.mark.parametrize("kv_heads,head_dim,dtype", [(2, 128, torch.bfloat16),
                                                     (8, 64, torch.float16)],
                         ids=["4wave", "8wave"])
@pytest.mark.parametrize("window", [-1, 20])
def test_batches_past_one_length_per_thread(device, batch, kv_heads, head_dim, dtype, window):
    # The tile scan reads one length per thread up to the workgroup's
    # threads (256 for four-wave, 512 for eight-wave workgroups) and batches
    # of eight loads past that: 257 and 513 sit one past each size, 4353
    # needs two rounds of eight per thread in the four-wave kernel. The
    # search for a range's first sequence settles up to 63 candidates in one
    # round: 63, 64 and 65 sequences sit around that, 4032 and 4033 around
    # the step of 63 that still leaves two rounds. Up to 256 sequences the
    # split kernel scans inside each wave instead, four sequences per lane:
    # 127-129 fill lanes 31-32 partly and wholly, 255-257 sit around its end.
    # A window takes the extended instantiation's tile count.
    g = torch.Generator().manual_seed(batch + head_dim)
    lengths = torch.randint(0, 48, (batch,), generator=g)
    lengths[batch // 3] = 0
    b = make_paged_batch(batch, 2 * kv_heads, kv_heads, head_dim, dtype, lengths,
                         seed=batch).to(device)
    cpu = b.to("cpu")
    # Empty sequences (one in ten) give zero rows; the oracle, like the
    # reference, rejects them, so it runs them at length 1 and those rows
    # are cleared.
    empty = cpu.cache_seqlens == 0
    expected = reference_port.attention_kvcache(
        cpu.q, cpu.k_cache, cpu.v_cache, cache_seqlens=cpu.cache_seqlens.clamp(min=1),
        block_table=cpu.block_table, softmax_scale=cpu.scale, window_left=window)
    expected[empty] = 0
    assert empty.any()
    for ns in (None, 1000):
        kw = {} if ns is None else dict(num_splits=ns)
        out = run_native(b, window_left=window, **kw)
        assert max_err(out, expected) <= TOL[dtype], ns


def test_most_splits_and_largest_page(device):
    # 65535 ranges (the maximum; more than there are tiles, so R = NT) and
    # 4096-token pages.
    b = make_paged_batch(3, 8, 2, 128, torch.bfloat16, torch.tensor([5000, 1, 9000]),
                         page_size=4096, seed=18).to(device)
    expected = oracle_out(b)
    assert max_err(run_native(b, num_splits=65535), expected) <= TOL[torch.bfloat16]
    assert max_err(run_native(b), expected) <= TOL[torch.bfloat16]
    assert max_err(run_native(b, num_splits=native.SPLITS_PER_SEQUENCE),
                   expected) <= TOL[torch.bfloat16]


def test_long_context(device):
    # One 131072-token sequence next to short ones.
    b = make_paged_batch(3, 16, 2, 128, torch.bfloat16, torch.tensor([131072, 3, 700]),
                         seed=19).to(device)
    expected = torch.from_numpy(c_oracle.paged_decode_f64(
        b.q.cpu(), b.k_cache.cpu(), b.v_cache.cpu(), b.block_table.cpu(), b.cache_seqlens.cpu(),
        b.scale)).reshape(b.q.shape)
    assert max_err(run_native(b), expected) <= TOL[torch.bfloat16]
