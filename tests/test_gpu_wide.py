"""GPU parity of the kernel contract beyond the reference's: 1..16 query heads
per kv head, head dim 256, and fp8 (OCP e4m3fn) KV caches with per-tensor
scales, through the C ABI.

Oracles: the fp64 C oracle (oracle/decode_ref.c) on the same inputs; for fp8
caches, on the exactly decoded e4m3fn values with scale*k_scale and the output
times v_scale in fp64 (c_oracle.paged_decode_fp8_f64). Tolerances as for the
16-bit path: max-abs <= 2e-3 (fp16), <= 1.6e-2 (bf16), with v_scale <= 1 so
the outputs keep the magnitude of N(0, 1) rows. The fp8 append is bit-exact
against oracle_reshape_and_cache_fp8.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from mxflashattn_amd import native
from mxflashattn_amd.workloads import make_paged_batch
from oracle import c_oracle

pytestmark = pytest.mark.gpu

TOL = {torch.float16: 2e-3, torch.bfloat16: 1.6e-2}
FP8 = torch.float8_e4m3fn


def f64_expected(b) -> torch.Tensor:
    out = c_oracle.paged_decode_f64(b.q.cpu(), b.k_cache.cpu(), b.v_cache.cpu(),
                                    b.block_table.cpu(), b.cache_seqlens.cpu(), b.scale)
    return torch.from_numpy(out).reshape(b.q.shape)


def max_err(actual: torch.Tensor, expected: torch.Tensor) -> float:
    return (actual.double().cpu() - expected.double().cpu()).abs().max().item()


def per_sequence(head_dim: int, gq: int, ql: int = 1) -> tuple:
    """(SPLITS_PER_SEQUENCE,) when one launch's pieces fit the per-sequence
    kernel's 64 KB of LDS (4 waves x columns x (HD + 1) floats), else ()."""
    cols = min(ql, 16 // gq) * gq
    return (native.SPLITS_PER_SEQUENCE,) if 16 * cols * (head_dim + 1) <= 64 << 10 else ()


def decode(b, k_cache=None, v_cache=None, **kw) -> torch.Tensor:
    out = native.paged_decode_split(b.q, b.k_cache if k_cache is None else k_cache,
                                    b.v_cache if v_cache is None else v_cache, b.block_table,
                                    b.cache_seqlens, b.scale, **kw)
    torch.cuda.synchronize()
    return out


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=["f16", "bf16"])
@pytest.mark.parametrize("head_dim", [64, 128, 256])
@pytest.mark.parametrize("gq", [1, 3, 5, 6, 7, 12, 16])
def test_group_sizes_and_head_dims(device, dtype, head_dim, gq):
    lengths = torch.tensor([1, 17, 300, 0, 1000])
    b = make_paged_batch(5, 2 * gq, 2, head_dim, dtype, lengths, seed=30 + gq).to(device)
    expected = f64_expected(b)
    for ns in (None, 1, 7, 64) + per_sequence(head_dim, gq):
        kw = {} if ns is None else dict(num_splits=ns)
        got = decode(b, **kw)
        assert torch.isfinite(got.float()).all()
        assert max_err(got, expected) <= TOL[dtype], (ns, max_err(got, expected))
        assert torch.equal(got[3].cpu(), torch.zeros_like(got[3].cpu()))  # empty sequence


@pytest.mark.parametrize("page_size", [1, 4, 64])
@pytest.mark.parametrize("gq", [2, 8, 16])
def test_head_dim_256_page_sizes(device, page_size, gq):
    lengths = torch.tensor([3, 129, 517])
    b = make_paged_batch(3, 2 * gq, 2, 256, torch.bfloat16, lengths, page_size=page_size,
                         seed=7).to(device)
    expected = f64_expected(b)
    assert max_err(decode(b), expected) <= TOL[torch.bfloat16]
    assert max_err(decode(b, num_splits=12), expected) <= TOL[torch.bfloat16]


def test_many_kv_heads_one_query_head_each(device):
    # GQ 1 with 32 kv heads: 8 workgroups of 4 kv heads per range.
    b = make_paged_batch(4, 32, 32, 128, torch.float16, torch.tensor([40, 700, 1, 2500]),
                         seed=12).to(device)
    assert max_err(decode(b), f64_expected(b)) <= TOL[torch.float16]


def test_head_dim_256_config2_lengths(device):
    # A Gemma-like decode layer: B = 32, 16 q / 8 kv heads of 256, L ~ U[1024, 8192].
    b = make_paged_batch(32, 16, 8, 256, torch.bfloat16, (1024, 8192), seed=20261007).to(device)
    assert max_err(decode(b), f64_expected(b)) <= TOL[torch.bfloat16]


# ---------------------------------------------------------------------------
# fp8 caches


def fp8_caches(b, device):
    return (b.k_cache.cpu().to(FP8).to(device), b.v_cache.cpu().to(FP8).to(device))


def fp8_expected(b, k8, v8, k_scale, v_scale) -> torch.Tensor:
    out = c_oracle.paged_decode_fp8_f64(b.q.cpu(), k8.cpu(), v8.cpu(), b.block_table.cpu(),
                                        b.cache_seqlens.cpu(), b.scale, k_scale, v_scale)
    return torch.from_numpy(out).reshape(b.q.shape)


def scalar(x: float, device) -> torch.Tensor:
    return torch.tensor([x], dtype=torch.float32, device=device)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=["f16", "bf16"])
@pytest.mark.parametrize("head_dim", [64, 128, 256])
@pytest.mark.parametrize("gq", [1, 2, 4, 8, 16])
def test_fp8_cache_matches_oracle(device, dtype, head_dim, gq):
    lengths = torch.tensor([1, 16, 33, 0, 700, 2000])
    b = make_paged_batch(6, 2 * gq, 2, head_dim, dtype, lengths, seed=50 + gq).to(device)
    k8, v8 = fp8_caches(b, device)
    expected = fp8_expected(b, k8, v8, 2.0, 0.5)
    ks, vs = scalar(2.0, device), scalar(0.5, device)
    for ns in (None, 1, 5, 40) + per_sequence(head_dim, gq):
        kw = {} if ns is None else dict(num_splits=ns)
        got = decode(b, k8, v8, k_scale=ks, v_scale=vs, **kw)
        assert torch.isfinite(got.float()).all()
        assert max_err(got, expected) <= TOL[dtype], (ns, max_err(got, expected))
        assert torch.equal(got[3].cpu(), torch.zeros_like(got[3].cpu()))


@pytest.mark.parametrize("gq", [15, 16])
def test_fp8_head_dim_256_short_table_takes_the_kernel_that_fits(device, gq):
    # A table of 16 pages of 16 (256 tokens) puts fp8 HD 256 (256-byte rows) in
    # the per-sequence kernel's range, whose LDS holds 15 columns at this head
    # dim but not 16: the default count must pick a kernel that runs.
    lengths = torch.tensor([3, 256, 100, 17, 0])
    b = make_paged_batch(5, 2 * gq, 2, 256, torch.bfloat16, lengths, block_table_width=16,
                         seed=56 + gq).to(device)
    k8, v8 = fp8_caches(b, device)
    ns = native.default_num_splits(b.q, k8, b.block_table)
    assert (ns == native.SPLITS_PER_SEQUENCE) == (gq == 15)
    got = decode(b, k8, v8, k_scale=scalar(2.0, device), v_scale=scalar(0.5, device))
    assert max_err(got, fp8_expected(b, k8, v8, 2.0, 0.5)) <= TOL[torch.bfloat16]


@pytest.mark.parametrize("page_size", [1, 8, 32])
def test_fp8_small_and_large_pages(device, page_size):
    b = make_paged_batch(3, 8, 2, 128, torch.bfloat16, torch.tensor([5, 200, 999]),
                         page_size=page_size, seed=8).to(device)
    k8, v8 = fp8_caches(b, device)
    got = decode(b, k8, v8)  # no scales: 1.0
    assert max_err(got, fp8_expected(b, k8, v8, 1.0, 1.0)) <= TOL[torch.bfloat16]


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=["f16", "bf16"])
def test_fp8_single_token_returns_every_code_exactly(device, dtype):
    """One key: the output is v_scale * V row, and every finite e4m3fn value is
    exact in fp16 and bf16, so the widening of V is checked code by code."""
    codes = torch.arange(256, dtype=torch.uint8)
    finite = codes[(codes & 0x7F) != 0x7F]  # 254 codes
    hd = 128
    rows = -(-finite.numel() // hd)
    b = make_paged_batch(rows, 4, 2, hd, dtype, 1, seed=1)
    v = torch.zeros(b.v_cache.shape, dtype=torch.uint8)
    pattern = torch.cat([finite, finite[: rows * hd - finite.numel()]]).view(rows, hd)
    for i in range(rows):
        page = int(b.block_table[i, 0])
        v[page, 0, :, :] = pattern[i]
    b = b.to(device)
    k8 = b.k_cache.cpu().to(FP8).to(device)
    v8 = v.view(FP8).to(device)
    got = decode(b, k8, v8).cpu()
    want = c_oracle.e4m3fn_decode(pattern).to(dtype)
    for i in range(rows):
        for h in range(4):
            assert torch.equal(got[i, 0, h], want[i]), (i, h)


def test_fp8_scales_are_read_at_run_time_in_a_graph(device):
    b = make_paged_batch(4, 16, 4, 128, torch.bfloat16, torch.tensor([10, 300, 77, 1200]),
                         seed=21).to(device)
    k8, v8 = fp8_caches(b, device)
    ks, vs = scalar(1.0, device), scalar(1.0, device)
    out = torch.empty_like(b.q)
    stream = torch.cuda.Stream(device)
    with torch.cuda.stream(stream):
        decode(b, k8, v8, k_scale=ks, v_scale=vs, out=out)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        native.paged_decode_split(b.q, k8, v8, b.block_table, b.cache_seqlens, b.scale, out=out,
                                  k_scale=ks, v_scale=vs)
    for kx, vx in ((1.0, 1.0), (0.5, 0.25), (3.0, 1.0)):
        ks.fill_(kx)
        vs.fill_(vx)
        with torch.cuda.stream(stream):
            graph.replay()
        torch.cuda.synchronize()
        assert max_err(out, fp8_expected(b, k8, v8, kx, vx)) <= TOL[torch.bfloat16], (kx, vx)
        eager = decode(b, k8, v8, k_scale=ks, v_scale=vs)
        assert torch.equal(out.cpu(), eager.cpu())


def fp8_append_inputs(dtype, scale: float, seed: int):
    """Rows mixing every regime of the conversion: N(0, 1), values beyond the
    saturation point, e4m3fn subnormals, exact rounding ties and zeros."""
    g = torch.Generator().manual_seed(seed)
    t, hkv, hd = 40, 2, 128
    x = torch.randn(t, hkv, hd, generator=g)
    x[0] *= 1000.0                        # saturates to +-448
    x[1] *= 1e-3                          # subnormal codes
    grid = c_oracle.e4m3fn_decode(torch.arange(0, 126, dtype=torch.uint8)).double()
    mids = ((grid[1:] + grid[:-1]) / 2).float()  # exact ties in fp32
    x[2].view(-1)[: mids.numel()] = mids
    x[3] = 0.0
    x[4].view(-1)[::2] = -x[4].view(-1)[::2]
    # Pre-scale so that x / scale hits the intended values (scale a power of two).
    x = (x * scale).to(dtype)
    return x


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=["f16", "bf16"])
@pytest.mark.parametrize("k_scale,v_scale", [(1.0, 1.0), (0.25, 4.0), (0.1, 3.0)])
def test_fp8_reshape_and_cache_bit_exact(device, dtype, k_scale, v_scale):
    key = fp8_append_inputs(dtype, k_scale, 3)
    value = fp8_append_inputs(dtype, v_scale, 4)
    pages, ps = 8, 16
    k_cache = torch.randint(0, 256, (pages, ps, 2, 128), dtype=torch.uint8)
    v_cache = torch.randint(0, 256, (pages, ps, 2, 128), dtype=torch.uint8)
    slots = torch.randperm(pages * ps)[: key.shape[0]]
    slots[5] = -1  # skipped
    want_k, want_v = c_oracle.reshape_and_cache_fp8(key, value, k_cache, v_cache, slots,
                                                    k_scale, v_scale)
    kc, vc = k_cache.view(FP8).to(device), v_cache.view(FP8).to(device)
    native.reshape_and_cache(key.to(device), value.to(device), kc, vc, slots.to(device),
                             k_scale=scalar(k_scale, device), v_scale=scalar(v_scale, device))
    torch.cuda.synchronize()
    assert torch.equal(kc.cpu().view(torch.uint8), want_k)
    assert torch.equal(vc.cpu().view(torch.uint8), want_v)


def test_fp8_reshape_and_cache_keeps_nan_and_saturates_inf(device):
    key = torch.zeros(2, 1, 16, dtype=torch.bfloat16)
    key[0, 0, :4] = torch.tensor([float("nan"), float("inf"), -float("inf"), -0.0])
    cache = torch.zeros(1, 16, 1, 16, dtype=torch.uint8).view(FP8).to(device)
    vcache = cache.clone()
    native.reshape_and_cache(key.to(device), key.to(device), cache, vcache,
                             torch.tensor([0, 1], device=device))
    torch.cuda.synchronize()
    row = cache.cpu().view(torch.uint8)[0, 0, 0]
    assert int(row[0]) & 0x7F == 0x7F  # NaN stays NaN
    assert int(row[1]) == 0x7E and int(row[2]) == 0xFE  # +-448
    assert int(row[3]) == 0x80  # -0


# ---------------------------------------------------------------------------
# Several query tokens per sequence (decode with draft tokens)


def port_expected(b, causal: bool, window_left: int = -1, sinks=None,
                  softcap: float = 0.0, alibi=None) -> torch.Tensor:
    """fp32 restatement of reference.attention_kvcache (bottom-right causal mask;
    window_left >= 0 adds the sliding window of the port, pinned in test_oracle)."""
    from oracle import reference_port

    cpu = b.to("cpu")
    out = torch.zeros(cpu.q.shape, dtype=torch.float32)
    for i in range(cpu.batch):  # the reference raises on an empty sequence; zeros here
        if int(cpu.cache_seqlens[i]) == 0:
            continue
        out[i:i + 1] = reference_port.attention_kvcache(
            cpu.q[i:i + 1].float(), cpu.k_cache.float(), cpu.v_cache.float(),
            cache_seqlens=cpu.cache_seqlens[i:i + 1].clone(), block_table=cpu.block_table[i:i + 1],
            softmax_scale=cpu.scale, causal=causal, window_left=window_left,
            sinks=None if sinks is None else sinks.cpu(), softcap=softcap,
            alibi_slopes=None if alibi is None else alibi.cpu()).float()
    return out


def with_query_tokens(b, ql: int, seed: int):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(b.batch, ql, b.q_heads, b.head_dim, generator=g).to(b.q.dtype)
    b.q = q.to(b.q.device)
    return b


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=["f16", "bf16"])
@pytest.mark.parametrize("head_dim", [64, 128])
@pytest.mark.parametrize("ql,gq", [(2, 1), (2, 4), (3, 4), (4, 4), (2, 8), (8, 2), (16, 1)])
@pytest.mark.parametrize("causal", [True, False], ids=["causal", "full"])
def test_query_tokens_match_reference(device, dtype, head_dim, ql, gq, causal):
    # Lengths shorter than QL leave the first tokens without keys (zeros).
    lengths = torch.tensor([1, 2, 17, 300, 0, 1000])
    b = make_paged_batch(6, 2 * gq, 2, head_dim, dtype, lengths, seed=60 + ql).to(device)
    b = with_query_tokens(b, ql, 61)
    expected = port_expected(b, causal)
    for ns in (None, 1, 9, 64, native.SPLITS_PER_SEQUENCE):
        kw = {} if ns is None else dict(num_splits=ns)
        got = native.paged_decode_split(b.q, b.k_cache, b.v_cache, b.block_table,
                                        b.cache_seqlens, b.scale, causal=causal, **kw)
        torch.cuda.synchronize()
        assert got.shape == b.q.shape
        assert torch.isfinite(got.float()).all()
        assert max_err(got, expected) <= TOL[dtype], (ns, max_err(got, expected))
        assert torch.equal(got[4].cpu(), torch.zeros_like(got[4].cpu()))


def test_query_tokens_fp8_and_head_dim_256(device):
    b = make_paged_batch(4, 8, 2, 256, torch.bfloat16, torch.tensor([3, 64, 500, 1200]),
                         seed=70).to(device)
    b = with_query_tokens(b, 3, 71)
    assert max_err(native.paged_decode_split(b.q, b.k_cache, b.v_cache, b.block_table,
                                             b.cache_seqlens, b.scale, causal=True),
                   port_expected(b, True)) <= TOL[torch.bfloat16]
    k8, v8 = fp8_caches(b, device)
    b8 = type(b)(b.q, k8.cpu().float().to(torch.bfloat16).to(device),
                 v8.cpu().float().to(torch.bfloat16).to(device), b.block_table, b.cache_seqlens,
                 b.scale)  # the exactly dequantised caches, scales 1
    got = native.paged_decode_split(b.q, k8, v8, b.block_table, b.cache_seqlens, b.scale,
                                    causal=True)
    torch.cuda.synchronize()
    assert max_err(got, port_expected(b8, True)) <= TOL[torch.bfloat16]


def test_query_tokens_through_the_api_with_append(device):
    """flash_attn_with_kvcache with two new tokens per sequence: append, then
    causal decode of both, then lengths advanced; against the reference port."""
    import mxflashattn_amd as mx
    from oracle import reference_port

    b = make_paged_batch(3, 16, 4, 128, torch.bfloat16, torch.tensor([5, 90, 400]),
                         block_table_width=40, seed=80)
    g = torch.Generator().manual_seed(81)
    q = torch.randn(3, 2, 16, 128, generator=g).to(torch.bfloat16)
    k_new = torch.randn(3, 2, 4, 128, generator=g).to(torch.bfloat16)
    v_new = torch.randn(3, 2, 4, 128, generator=g).to(torch.bfloat16)
    kc, vc, sl = b.k_cache.clone(), b.v_cache.clone(), b.cache_seqlens.clone()
    expected = reference_port.attention_kvcache(
        q.float(), kc.float(), vc.float(), cache_seqlens=sl, block_table=b.block_table,
        k=k_new.float(), v=v_new.float(), softmax_scale=b.scale, causal=True).float()
    gpu = b.to(device)
    lens = gpu.cache_seqlens.clone()
    out = mx.flash_attn_with_kvcache(q.to(device), gpu.k_cache, gpu.v_cache, k=k_new.to(device),
                                     v=v_new.to(device), cache_seqlens=lens,
                                     block_table=gpu.block_table, softmax_scale=b.scale,
                                     causal=True)
    torch.cuda.synchronize()
    assert mx.get_last_dispatch_info().backend == mx.BACKEND_MI355X
    assert max_err(out, expected) <= TOL[torch.bfloat16]
    assert lens.cpu().tolist() == (b.cache_seqlens + 2).tolist()


@pytest.mark.parametrize("sq,sk", [(1, 70), (3, 70), (4, 4), (4, 2)])
@pytest.mark.parametrize("causal", [True, False], ids=["causal", "full"])
def test_dense_query_tokens_through_flash_attn_func(device, sq, sk, causal):
    """flash_attn_func with a few query tokens runs on the HIP kernels (dense
    k/v viewed as pages) and matches the reference's batched attention,
    bottom-right causal mask included (sq > sk leaves the first rows empty)."""
    import mxflashattn_amd as mx
    from oracle import reference_port

    g = torch.Generator().manual_seed(90 + sq)
    q = torch.randn(3, sq, 8, 64, generator=g).to(torch.float16)
    k = torch.randn(3, sk, 2, 64, generator=g).to(torch.float16)
    v = torch.randn(3, sk, 2, 64, generator=g).to(torch.float16)
    expected = reference_port.attention_batched(q.float(), k.float(), v.float(),
                                                softmax_scale=0.125, causal=causal).float()
    out = mx.flash_attn_func(q.to(device), k.to(device), v.to(device), softmax_scale=0.125,
                             causal=causal)
    torch.cuda.synchronize()
    assert mx.get_last_dispatch_info().backend == mx.BACKEND_MI355X
    assert max_err(out, expected) <= TOL[torch.float16]


@pytest.mark.parametrize("sq,sk", [(5, 70), (9, 70), (16, 70), (9, 7)])
def test_dense_causal_query_past_sixteen_columns_through_flash_attn_func(device, sq, sk):
    """flash_attn_func, GQ 4, causal, 20 to 64 columns: token chunks on the HIP
    kernels, bottom-right mask kept (sq > sk leaves the first rows empty)."""
    import mxflashattn_amd as mx
    from oracle import reference_port

    g = torch.Generator().manual_seed(140 + sq)
    q = torch.randn(3, sq, 8, 64, generator=g).to(torch.float16)
    k = torch.randn(3, sk, 2, 64, generator=g).to(torch.float16)
    v = torch.randn(3, sk, 2, 64, generator=g).to(torch.float16)
    expected = reference_port.attention_batched(q.float(), k.float(), v.float(),
                                                softmax_scale=0.125, causal=True).float()
    out = mx.flash_attn_func(q.to(device), k.to(device), v.to(device), softmax_scale=0.125,
                             causal=True)
    torch.cuda.synchronize()
    assert mx.get_last_dispatch_info().backend == mx.BACKEND_MI355X
    assert max_err(out, expected) <= TOL[torch.float16]


# ---------------------------------------------------------------------------
# Sliding window (window_left): keys before position - window_left are dropped;
# each sequence's tiles start at the first tile the window reaches.


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=["f16", "bf16"])
@pytest.mark.parametrize("head_dim", [64, 128])
@pytest.mark.parametrize("window", [0, 16, 17, 100, 5000])
@pytest.mark.parametrize("ql,gq,causal", [(1, 4, False), (2, 4, True), (3, 4, True),
                                          (4, 4, False), (2, 8, True)])
def test_window_matches_reference(device, dtype, head_dim, window, ql, gq, causal):
    lengths = torch.tensor([1, 2, 17, 300, 0, 1000, 33])
    b = make_paged_batch(7, 2 * gq, 2, head_dim, dtype, lengths, seed=80 + window).to(device)
    b = with_query_tokens(b, ql, 81)
    if ql == 1:
        b.q = b.q[:, 0]  # [B, HQ, HD]: the one-token form takes the window too
    expected = port_expected(b if ql > 1 else with_query_tokens_view(b), causal, window)
    for ns in (None, 1, 9, 64, native.SPLITS_PER_SEQUENCE):
        kw = {} if ns is None else dict(num_splits=ns)
        got = native.paged_decode_split(b.q, b.k_cache, b.v_cache, b.block_table,
                                        b.cache_seqlens, b.scale, causal=causal,
                                        window_left=window, **kw)
        torch.cuda.synchronize()
        got = got if ql > 1 else got.unsqueeze(1)
        assert torch.isfinite(got.float()).all()
        assert max_err(got, expected) <= TOL[dtype], (ns, max_err(got, expected))
        assert torch.equal(got[4].cpu(), torch.zeros_like(got[4].cpu()))


def with_query_tokens_view(b):
    """The same batch with q as [B, 1, HQ, HD] (for the reference port)."""
    return type(b)(b.q.unsqueeze(1), b.k_cache, b.v_cache, b.block_table, b.cache_seqlens,
                   b.scale)


@pytest.mark.parametrize("page_size", [1, 4, 64])
@pytest.mark.parametrize("window", [0, 5, 40])
def test_window_with_small_and_large_pages(device, page_size, window):
    b = make_paged_batch(5, 8, 2, 128, torch.bfloat16, torch.tensor([1, 9, 64, 130, 700]),
                         seed=85, page_size=page_size).to(device)
    b = with_query_tokens(b, 2, 86)
    got = native.paged_decode_split(b.q, b.k_cache, b.v_cache, b.block_table, b.cache_seqlens,
                                    b.scale, causal=True, window_left=window)
    torch.cuda.synchronize()
    assert max_err(got, port_expected(b, True, window)) <= TOL[torch.bfloat16]


@pytest.mark.parametrize("window", [0, 31, 200])
def test_window_fp8_and_head_dim_256(device, window):
    b = make_paged_batch(4, 8, 2, 256, torch.bfloat16, torch.tensor([3, 64, 500, 1200]),
                         seed=87).to(device)
    b = with_query_tokens(b, 2, 88)
    got = native.paged_decode_split(b.q, b.k_cache, b.v_cache, b.block_table, b.cache_seqlens,
                                    b.scale, causal=True, window_left=window)
    torch.cuda.synchronize()
    assert max_err(got, port_expected(b, True, window)) <= TOL[torch.bfloat16]
    k8, v8 = fp8_caches(b, device)
    b8 = type(b)(b.q, k8.cpu().float().to(torch.bfloat16).to(device),
                 v8.cpu().float().to(torch.bfloat16).to(device), b.block_table, b.cache_seqlens,
                 b.scale)  # the exactly dequantised caches, scales 1
    got = native.paged_decode_split(b.q, k8, v8, b.block_table, b.cache_seqlens, b.scale,
                                    causal=True, window_left=window)
    torch.cuda.synchronize()
    assert max_err(got, port_expected(b8, True, window)) <= TOL[torch.bfloat16]


def test_window_on_a_long_sequence(device):
    # 120,000 keys with a 128-key window: only the last tiles are read, and
    # the result matches the port's masked attention over all the keys.
    n, window = 120_000, 128
    b = make_paged_batch(2, 16, 2, 128, torch.bfloat16, torch.tensor([n, 5000]),
                         seed=89).to(device)
    got = native.paged_decode_split(b.q, b.k_cache, b.v_cache, b.block_table, b.cache_seqlens,
                                    b.scale, window_left=window)
    torch.cuda.synchronize()
    assert max_err(got, port_expected(b, False, window)) <= TOL[torch.bfloat16]


# ---------------------------------------------------------------------------
# Attention sinks (vLLM's s_aux): one logit per query head in every softmax
# denominator, added in the partial kernel for sequences whole in a range and
# in the combine for split ones.


def sink_values(hq: int, device) -> torch.Tensor:
    vals = torch.linspace(-2.0, 3.0, hq)
    vals[0] = float("-inf")     # a head without a sink
    vals[-1] = 20.0             # a sink that outweighs every key
    return vals.to(torch.float32).to(device)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=["f16", "bf16"])
@pytest.mark.parametrize("head_dim", [64, 128])
@pytest.mark.parametrize("ql,gq,causal,window", [(1, 4, False, -1), (1, 8, False, 31),
                                                 (2, 4, True, -1), (3, 4, True, 50),
                                                 (4, 2, False, -1)])
def test_sinks_match_reference(device, dtype, head_dim, ql, gq, causal, window):
    lengths = torch.tensor([1, 2, 17, 300, 0, 1000, 33])
    b = make_paged_batch(7, 2 * gq, 2, head_dim, dtype, lengths, seed=90 + ql).to(device)
    b = with_query_tokens(b, ql, 91)
    sinks = sink_values(2 * gq, device)
    expected = port_expected(b, causal, window, sinks)
    for ns in (None, 1, 9, 64, native.SPLITS_PER_SEQUENCE):
        kw = {} if ns is None else dict(num_splits=ns)
        got = native.paged_decode_split(b.q, b.k_cache, b.v_cache, b.block_table,
                                        b.cache_seqlens, b.scale, causal=causal,
                                        window_left=window, sinks=sinks, **kw)
        torch.cuda.synchronize()
        assert torch.isfinite(got.float()).all()
        assert max_err(got, expected) <= TOL[dtype], (ns, max_err(got, expected))
        assert torch.equal(got[4].cpu(), torch.zeros_like(got[4].cpu()))


def test_sinks_with_fp8_caches_and_head_dim_256(device):
    b = make_paged_batch(4, 8, 2, 256, torch.bfloat16, torch.tensor([3, 64, 500, 1200]),
                         seed=92).to(device)
    sinks = sink_values(8, device)
    got = native.paged_decode_split(b.q, b.k_cache, b.v_cache, b.block_table, b.cache_seqlens,
                                    b.scale, sinks=sinks)
    torch.cuda.synchronize()
    assert max_err(got, port_expected(b, False, -1, sinks)) <= TOL[torch.bfloat16]
    k8, v8 = fp8_caches(b, device)
    b8 = type(b)(b.q, k8.cpu().float().to(torch.bfloat16).to(device),
                 v8.cpu().float().to(torch.bfloat16).to(device), b.block_table, b.cache_seqlens,
                 b.scale)
    got = native.paged_decode_split(b.q, k8, v8, b.block_table, b.cache_seqlens, b.scale,
                                    sinks=sinks)
    torch.cuda.synchronize()
    assert max_err(got, port_expected(b8, False, -1, sinks)) <= TOL[torch.bfloat16]


def test_sinks_are_checked_on_the_host(device):
    b = make_paged_batch(2, 8, 2, 64, torch.bfloat16, torch.tensor([5, 9]), seed=93).to(device)
    for bad in (torch.zeros(7, device=device), torch.zeros(8, device=device).half(),
                torch.zeros(8), torch.zeros(16, device=device)[::2]):
        with pytest.raises(ValueError, match="sinks"):
            native.paged_decode_split(b.q, b.k_cache, b.v_cache, b.block_table,
                                      b.cache_seqlens, b.scale, sinks=bad)


def test_graph_replays_of_the_general_entry_point_match_eager(device):
    # Several query tokens, a sliding window, sinks and an fp8 cache: the
    # general entry point captured in a HIP graph (workspace from an eager call
    # on the capture stream first), replayed with eager work in between.
    b = make_paged_batch(5, 16, 4, 128, torch.bfloat16, torch.tensor([700, 3, 1500, 64, 0]),
                         seed=95).to(device)
    b = with_query_tokens(b, 2, 96)
    k8, v8 = fp8_caches(b, device)
    sinks = sink_values(16, device)
    one = torch.ones(1, dtype=torch.float32, device=device)
    stream = torch.cuda.Stream(device)
    out = torch.empty_like(b.q)

    def call():
        native.paged_decode_split(b.q, k8, v8, b.block_table, b.cache_seqlens, b.scale,
                                  out=out, causal=True, window_left=300, sinks=sinks,
                                  k_scale=one, v_scale=one)

    with torch.cuda.stream(stream):
        call()
        eager = out.clone()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        call()
    for i in range(4):
        out.fill_(float("nan"))
        with torch.cuda.stream(stream):
            graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), i
        _ = (torch.randn(4096, device=device) * i).sum().item()


# ---------------------------------------------------------------------------
# Logit soft-capping: s -> cap * tanh(s / cap) on the scaled scores.


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=["f16", "bf16"])
@pytest.mark.parametrize("head_dim", [64, 128])
@pytest.mark.parametrize("cap", [0.5, 5.0, 30.0])
@pytest.mark.parametrize("ql,gq,causal,window,with_sinks", [(1, 4, False, -1, False),
                                                            (2, 4, True, 40, True),
                                                            (2, 8, False, -1, False)])
def test_softcap_matches_reference(device, dtype, head_dim, cap, ql, gq, causal, window,
                                   with_sinks):
    lengths = torch.tensor([1, 17, 300, 0, 1000])
    b = make_paged_batch(5, 2 * gq, 2, head_dim, dtype, lengths, seed=97).to(device)
    b = with_query_tokens(b, ql, 98)
    b.q = (b.q.float() * 3).to(dtype)  # scores of a few units, where the cap bites
    sinks = sink_values(2 * gq, device) if with_sinks else None
    expected = port_expected(b, causal, window, sinks, cap)
    for ns in (None, 1, 9) + per_sequence(head_dim, gq, ql):
        kw = {} if ns is None else dict(num_splits=ns)
        got = native.paged_decode_split(b.q, b.k_cache, b.v_cache, b.block_table,
                                        b.cache_seqlens, b.scale, causal=causal,
                                        window_left=window, sinks=sinks, softcap=cap, **kw)
        torch.cuda.synchronize()
        assert torch.isfinite(got.float()).all()
        assert max_err(got, expected) <= TOL[dtype], (ns, max_err(got, expected))


def test_softcap_with_fp8_caches(device):
    b = make_paged_batch(4, 8, 2, 128, torch.bfloat16, torch.tensor([3, 64, 500, 1200]),
                         seed=99).to(device)
    k8, v8 = fp8_caches(b, device)
    b8 = type(b)(b.q, k8.cpu().float().to(torch.bfloat16).to(device),
                 v8.cpu().float().to(torch.bfloat16).to(device), b.block_table, b.cache_seqlens,
                 b.scale)
    two = torch.full((1,), 2.0, dtype=torch.float32, device=device)
    got = native.paged_decode_split(b.q, k8, v8, b.block_table, b.cache_seqlens, b.scale,
                                    softcap=4.0, k_scale=two)
    torch.cuda.synchronize()
    # k_scale 2 doubles every score before the cap: the port on 2 * K.
    b8.k_cache = (b8.k_cache.float() * 2).to(torch.bfloat16)
    assert max_err(got, port_expected(b8, False, -1, None, 4.0)) <= TOL[torch.bfloat16]


# ---------------------------------------------------------------------------
# ALiBi: s -= slope[h] * |query position - key position|, after the cap.


def alibi_slopes(hq: int, device, sign: float = 1.0) -> torch.Tensor:
    # The geometric slopes of the ALiBi paper, 2^(-8 (h + 1) / HQ), optionally negated
    # (a bias that grows with distance drives the running maximum up tile after tile).
    h = torch.arange(1, hq + 1, dtype=torch.float32)
    return (sign * torch.pow(2.0, -8.0 * h / hq)).to(device)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=["f16", "bf16"])
@pytest.mark.parametrize("head_dim", [64, 128, 256])
@pytest.mark.parametrize("ql,gq,causal,window,with_sinks,cap",
                         [(1, 4, False, -1, False, 0.0), (1, 8, True, -1, False, 0.0),
                          (3, 4, True, -1, False, 0.0), (2, 8, False, -1, False, 0.0),
                          (2, 4, True, 40, True, 0.0), (2, 4, True, -1, False, 5.0),
                          (1, 1, False, 200, True, 30.0)])
def test_alibi_matches_reference(device, dtype, head_dim, ql, gq, causal, window, with_sinks,
                                 cap):
    lengths = torch.tensor([1, 17, 300, 0, 1000, 2100])
    b = make_paged_batch(6, 2 * gq, 2, head_dim, dtype, lengths, seed=111).to(device)
    b = with_query_tokens(b, ql, 112)
    slopes = alibi_slopes(2 * gq, device)
    sinks = sink_values(2 * gq, device) if with_sinks else None
    expected = port_expected(b, causal, window, sinks, cap, slopes)
    for ns in (None, 1, 9) + per_sequence(head_dim, gq, ql):
        kw = {} if ns is None else dict(num_splits=ns)
        got = native.paged_decode_split(b.q, b.k_cache, b.v_cache, b.block_table,
                                        b.cache_seqlens, b.scale, causal=causal,
                                        window_left=window, sinks=sinks, softcap=cap,
                                        alibi_slopes=slopes, **kw)
        torch.cuda.synchronize()
        assert torch.isfinite(got.float()).all()
        assert max_err(got, expected) <= TOL[dtype], (ns, max_err(got, expected))


def test_alibi_with_negative_slopes_and_zero_slopes(device):
    lengths = torch.tensor([5, 700, 3000])
    b = make_paged_batch(3, 8, 2, 128, torch.bfloat16, lengths, seed=113).to(device)
    for slopes in (alibi_slopes(8, device, -0.05), torch.zeros(8, device=device)):
        expected = port_expected(b, False, -1, None, 0.0, slopes)
        for ns in (None, 1, 7, native.SPLITS_PER_SEQUENCE):
            kw = {} if ns is None else dict(num_splits=ns)
            got = native.paged_decode_split(b.q, b.k_cache, b.v_cache, b.block_table,
                                            b.cache_seqlens, b.scale, alibi_slopes=slopes,
                                            **kw)
            torch.cuda.synchronize()
            assert max_err(got, expected) <= TOL[torch.bfloat16], (ns, slopes[0].item())
    # Zero slopes take the extended instantiation and still match the plain one.
    plain = native.paged_decode_split(b.q, b.k_cache, b.v_cache, b.block_table,
                                      b.cache_seqlens, b.scale)
    torch.cuda.synchronize()
    assert max_err(got, plain.float()) <= TOL[torch.bfloat16]


def test_alibi_with_fp8_caches(device):
    b = make_paged_batch(4, 8, 2, 128, torch.bfloat16, torch.tensor([3, 64, 500, 1200]),
                         seed=114).to(device)
    k8, v8 = fp8_caches(b, device)
    b8 = type(b)(b.q, k8.cpu().float().to(torch.bfloat16).to(device),
                 v8.cpu().float().to(torch.bfloat16).to(device), b.block_table, b.cache_seqlens,
                 b.scale)
    slopes = alibi_slopes(8, device)
    got = native.paged_decode_split(b.q, k8, v8, b.block_table, b.cache_seqlens, b.scale,
                                    alibi_slopes=slopes)
    torch.cuda.synchronize()
    assert max_err(got, port_expected(b8, False, -1, None, 0.0, slopes)) <= TOL[torch.bfloat16]


def test_alibi_slopes_are_checked_on_the_host(device):
    b = make_paged_batch(2, 8, 2, 64, torch.bfloat16, torch.tensor([10, 20]), seed=115).to(device)
    for bad in (torch.zeros(7, device=device), torch.zeros(8, device=device, dtype=torch.float16),
                torch.zeros(8), torch.zeros(16, device=device)[::2]):
        with pytest.raises(ValueError, match="alibi_slopes"):
            native.paged_decode_split(b.q, b.k_cache, b.v_cache, b.block_table,
                                      b.cache_seqlens, b.scale, alibi_slopes=bad)


# ---------------------------------------------------------------------------
# Causal queries past the 16 kernel columns: launches of token chunks.


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=["f16", "bf16"])
@pytest.mark.parametrize("head_dim", [64, 128])
@pytest.mark.parametrize("ql,gq", [(5, 4), (8, 4), (3, 8), (4, 8), (2, 16), (3, 16), (9, 2),
                                   (17, 1)])
@pytest.mark.parametrize("extras", [False, True], ids=["plain", "extras"])
def test_causal_queries_past_sixteen_columns(device, dtype, head_dim, ql, gq, extras):
    # Lengths shorter than QL: a chunk whose sequences end before position 0
    # sees no key, as the tokens of one launch would.
    lengths = torch.tensor([1, 3, 6, 17, 300, 0, 1000])
    b = make_paged_batch(7, 2 * gq, 2, head_dim, dtype, lengths, seed=130 + ql).to(device)
    b = with_query_tokens(b, ql, 131)
    window, cap, sinks, slopes = -1, 0.0, None, None
    if extras:
        window, cap = 40, 5.0
        sinks, slopes = sink_values(2 * gq, device), alibi_slopes(2 * gq, device)
    expected = port_expected(b, True, window, sinks, cap, slopes)
    for ns in (None, 1, 9) + per_sequence(head_dim, gq, ql):
        kw = {} if ns is None else dict(num_splits=ns)
        got = native.paged_decode_split(b.q, b.k_cache, b.v_cache, b.block_table,
                                        b.cache_seqlens, b.scale, causal=True, window_left=window,
                                        sinks=sinks, softcap=cap, alibi_slopes=slopes, **kw)
        torch.cuda.synchronize()
        assert torch.isfinite(got.float()).all()
        assert max_err(got, expected) <= TOL[dtype], (ns, max_err(got, expected))
        assert torch.equal(got[5].cpu(), torch.zeros_like(got[5].cpu()))


def test_chunked_causal_query_fp8_strided_and_seqlen_add(device):
    # 6 tokens x GQ 4 (two launches) on an fp8 cache, q and out as slices of
    # wider buffers, lengths given as cache_seqlens + seqlen_add.
    b = make_paged_batch(4, 8, 2, 128, torch.bfloat16, torch.tensor([3, 64, 500, 1200]),
                         seed=133).to(device)
    b = with_query_tokens(b, 6, 134)
    k8, v8 = fp8_caches(b, device)
    b8 = type(b)(b.q, k8.cpu().float().to(torch.bfloat16).to(device),
                 v8.cpu().float().to(torch.bfloat16).to(device), b.block_table, b.cache_seqlens,
                 b.scale)
    expected = port_expected(b8, True)
    wide = torch.randn(4, 6, 11, 128, device=device).to(torch.bfloat16)
    wide[:, :, 2:10] = b.q
    obuf = torch.zeros(4, 6, 13, 128, device=device, dtype=torch.bfloat16)
    shorter = (b.cache_seqlens - 2).clamp_min(0).to(torch.int32)
    got = native.paged_decode_split(wide[:, :, 2:10], k8, v8, b.block_table, shorter, b.scale,
                                    out=obuf[:, :, 1:9], causal=True, seqlen_add=2)
    torch.cuda.synchronize()
    assert max_err(got, expected) <= TOL[torch.bfloat16]
    assert torch.equal(obuf[:, :, :1].cpu(), torch.zeros_like(obuf[:, :, :1].cpu()))
    assert torch.equal(obuf[:, :, 9:].cpu(), torch.zeros_like(obuf[:, :, 9:].cpu()))


def test_chunked_causal_query_through_the_api(device):
    """flash_attn_with_kvcache with five new tokens per sequence at GQ 4
    (20 columns, two launches): append, causal decode, lengths advanced."""
    import mxflashattn_amd as mx
    from oracle import reference_port

    b = make_paged_batch(3, 16, 4, 128, torch.bfloat16, torch.tensor([2, 90, 400]),
                         block_table_width=40, seed=135)
    g = torch.Generator().manual_seed(136)
    q = torch.randn(3, 5, 16, 128, generator=g).to(torch.bfloat16)
    k_new = torch.randn(3, 5, 4, 128, generator=g).to(torch.bfloat16)
    v_new = torch.randn(3, 5, 4, 128, generator=g).to(torch.bfloat16)
    kc, vc, sl = b.k_cache.clone(), b.v_cache.clone(), b.cache_seqlens.clone()
    expected = reference_port.attention_kvcache(
        q.float(), kc.float(), vc.float(), cache_seqlens=sl, block_table=b.block_table,
        k=k_new.float(), v=v_new.float(), softmax_scale=b.scale, causal=True).float()
    gpu = b.to(device)
    lens = gpu.cache_seqlens.clone()
    out = mx.flash_attn_with_kvcache(q.to(device), gpu.k_cache, gpu.v_cache, k=k_new.to(device),
                                     v=v_new.to(device), cache_seqlens=lens,
                                     block_table=gpu.block_table, softmax_scale=b.scale,
                                     causal=True)
    torch.cuda.synchronize()
    assert mx.get_last_dispatch_info().backend == mx.BACKEND_MI355X
    assert max_err(out, expected) <= TOL[torch.bfloat16]
    assert lens.cpu().tolist() == (b.cache_seqlens + 5).tolist()


def test_graph_replays_of_a_chunked_causal_query_follow_the_lengths(device):
    # 6 tokens x GQ 4 (two launches) with ALiBi, captured once; between replays
    # the lengths change in place, and every replay must match an eager call
    # on the same lengths (each chunk reads them on the device).
    # The table is as wide as the longest length here (1600); unused entries
    # name page 0, which the port reads the same way.
    b = make_paged_batch(4, 16, 4, 128, torch.bfloat16, torch.tensor([900, 5, 1600, 64]),
                         seed=137).to(device)
    b = with_query_tokens(b, 6, 138)
    slopes = alibi_slopes(16, device)
    lens = b.cache_seqlens.clone()
    stream = torch.cuda.Stream(device)
    out = torch.empty_like(b.q)

    def call(target):
        native.paged_decode_split(b.q, b.k_cache, b.v_cache, b.block_table, lens, b.scale,
                                  out=target, causal=True, alibi_slopes=slopes)

    with torch.cuda.stream(stream):
        call(out)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        call(out)
    for i, new in enumerate(([900, 5, 1600, 64], [3, 700, 1200, 17], [0, 6, 1, 1600])):
        lens.copy_(torch.tensor(new, dtype=torch.int32))
        torch.cuda.synchronize()
        eager = torch.empty_like(out)
        with torch.cuda.stream(stream):
            call(eager)
        out.fill_(float("nan"))
        with torch.cuda.stream(stream):
            graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), (i, new)
        b.cache_seqlens = lens.clone()
        assert max_err(out, port_expected(b, True, -1, None, 0.0, slopes)) \
            <= TOL[torch.bfloat16], (i, new)


# Batches of 65 to 256 sequences take the wave-local tile scan with four
# sequences per lane on plain calls (and the LDS scan with a window, cap,
# sinks or ALiBi): every head dim, several GQ, both 16-bit types and fp8,
# with empty sequences at lane edges and inside a lane, against the fp64
# oracle, at the heuristic's split count and a few others.
@pytest.mark.parametrize("batch", [65, 130, 256])
@pytest.mark.parametrize("head_dim", [64, 128, 256])
@pytest.mark.parametrize("gq,dtype,fp8", [(1, torch.bfloat16, False), (4, torch.float16, False),
                                          (8, torch.bfloat16, False), (4, torch.bfloat16, True)],
                         ids=["gq1-bf16", "gq4-f16", "gq8-bf16", "gq4-fp8"])
def test_four_sequences_per_lane_scan(device, batch, head_dim, gq, dtype, fp8):
    g = torch.Generator().manual_seed(batch * 7 + head_dim + gq)
    lengths = torch.randint(1, 90, (batch,), generator=g)
    lengths[[0, 3, 4, batch // 2, batch - 1]] = 0  # lane 0's first and 1's first, mid, last
    lengths[5] = 16  # a sequence ending on a tile edge
    b = make_paged_batch(batch, 2 * gq, 2, head_dim, dtype, lengths, seed=batch + gq).to(device)
    if fp8:
        k8, v8 = fp8_caches(b, device)
        expected = fp8_expected(b, k8, v8, 1.0, 1.0)
    else:
        k8, v8 = b.k_cache, b.v_cache
        expected = f64_expected(b)
    empty = b.cache_seqlens.cpu() == 0
    for ns in (None, 3, 100, 1000):
        kw = {} if ns is None else dict(num_splits=ns)
        got = decode(b, k8, v8, **kw)
        assert torch.isfinite(got.float()).all()
        assert max_err(got, expected) <= TOL[dtype], (ns, max_err(got, expected))
        assert not got.cpu()[empty].any(), ns
