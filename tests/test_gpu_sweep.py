"""A seeded random sweep over the whole kernel contract against the oracles.

Each case draws a shape (batch, kv heads, GQ, head dim, page size, lengths
including 0 and lengths shorter than the query tokens), a query token count
with QL x GQ <= 16, causal or not, fp16/bf16, an fp8 cache or not, strided q
and out, a head-major or token-major cache, and a split count, then compares
the HIP result with the reference port (fp32; exactly dequantised caches for
fp8) at the north-star tolerances. A second sweep adds a sliding window,
attention sinks and/or soft-capping to every case (the extended kernel
instantiation), and ALiBi slopes to about half of them (drawn from a stream of
their own). A third sweep redraws each case as a causal query of more than 16
columns (QL x GQ up to 64: launches of token chunks), with the extras of the
second sweep on half of them. A fourth runs cases of all three kinds through
the per-sequence kernel (num_splits = SPLITS_PER_SEQUENCE), whose pieces live
in LDS: a launch of 16 columns at head dim 256 does not fit and must be
refused. A fifth draws its kv heads from 5, 6, 7, 9, 10 and 12 (workgroups
with idle waves, two or more head groups) and mixes the other four kinds. Seeds
are fixed: every run checks the same cases.
"""

from __future__ import annotations

import random

import pytest
import torch

from mxflashattn_amd import native
from mxflashattn_amd.workloads import make_paged_batch
from oracle import reference_port

pytestmark = pytest.mark.gpu

TOL = {torch.float16: 2e-3, torch.bfloat16: 1.6e-2}
FP8 = torch.float8_e4m3fn
SENTINEL = 7.0  # fills an output buffer outside the slice the call writes


def draw(seed: int, hkv_choices: tuple = (1, 2, 3, 4, 8)) -> dict:
    r = random.Random(seed)
    hkv = r.choice(hkv_choices)
    gq = r.choice([1, 2, 3, 4, 5, 8, 16])
    ql = r.choice([q for q in (1, 1, 1, 2, 3, 4, 8) if q * gq <= 16])
    batch = r.randint(1, 9)
    ps = r.choice([1, 2, 8, 16, 16, 16, 64, 256])
    lengths = [r.choice([0, 1, 2, r.randint(3, 40), r.randint(40, 700), r.randint(700, 3000)])
               for _ in range(batch)]
    return dict(hkv=hkv, gq=gq, ql=ql, batch=batch, ps=ps, lengths=lengths,
                hd=r.choice([64, 128, 256]), dtype=r.choice([torch.float16, torch.bfloat16]),
                fp8=r.random() < 0.3, causal=r.random() < 0.6, strided=r.random() < 0.4,
                head_major=r.random() < 0.25, ns=r.choice([None, None, 1, 3, 17, 300]))


def draw_extras(seed: int, hq: int) -> dict:
    """Window, sinks and soft-cap for the extended sweep (at least one is on),
    and ALiBi slopes or None."""
    r = random.Random(10_000 + seed)
    while True:
        window = r.choice([-1, -1, 0, 1, 15, 16, 100, 2000])
        sinks = None
        if r.random() < 0.5:
            vals = [r.uniform(-3.0, 4.0) for _ in range(hq)]
            if r.random() < 0.3:
                vals[r.randrange(hq)] = float("-inf")
            if r.random() < 0.2:
                vals[r.randrange(hq)] = 25.0
            sinks = torch.tensor(vals, dtype=torch.float32)
        softcap = r.choice([0.0, 0.0, 1.0, 10.0, 50.0])
        if window >= 0 or sinks is not None or softcap > 0:
            break
    a = random.Random(20_000 + seed)
    alibi = None
    if a.random() < 0.5:  # geometric slopes, or arbitrary ones of either sign
        if a.random() < 0.5:
            alibi = torch.pow(2.0, -8.0 * torch.arange(1, hq + 1, dtype=torch.float32) / hq)
        else:
            alibi = torch.tensor([a.uniform(-0.02, 0.5) for _ in range(hq)],
                                 dtype=torch.float32)
    return dict(window=window, sinks=sinks, softcap=softcap, alibi=alibi)


def expected(q, kc, vc, bt, sl, scale, causal, window=-1, sinks=None,
             softcap=0.0, alibi=None) -> torch.Tensor:
    out = torch.zeros(q.shape, dtype=torch.float32)
    for i in range(q.shape[0]):
        if int(sl[i]) == 0:  # the reference raises on an empty sequence; the kernel gives 0
            continue
        out[i:i + 1] = reference_port.attention_kvcache(
            q[i:i + 1].float(), kc.float(), vc.float(), cache_seqlens=sl[i:i + 1].clone(),
            block_table=bt[i:i + 1], softmax_scale=scale, causal=causal, window_left=window,
            sinks=sinks, softcap=softcap, alibi_slopes=alibi).float()
    return out


@pytest.mark.parametrize("seed", range(150))
def test_random_contract_sweep(device, seed):
    run_case(device, seed, extended=False)


@pytest.mark.parametrize("seed", range(150, 300))
def test_random_extended_sweep(device, seed):
    run_case(device, seed, extended=True)


@pytest.mark.parametrize("seed", range(300, 360))
def test_random_chunked_sweep(device, seed):
    run_case(device, seed, extended=seed % 2 == 0, chunked_query=True)


@pytest.mark.parametrize("seed", range(360, 480))
def test_random_per_sequence_sweep(device, seed):
    run_case(device, seed, extended=seed % 3 == 1, chunked_query=seed % 3 == 2,
             per_sequence=True)


# Every per-sequence case at head dim 256 in the seeds above. Built for two
# waves per SIMD (a 256-register budget), the per-sequence kernel spilled
# 65-201 VGPRs and returned wrong outputs on all of them (max error 0.6-3.6)
# until a change that left its arithmetic alone but gave the compiler less to
# keep live; the library ships one wave per SIMD there (no spills, and the
# build now fails on any spill). They run again here by name.
HD256_PER_SEQUENCE_SEEDS = (364, 377, 378, 379, 380, 381, 390, 396, 397, 400, 403, 406, 409, 418,
                            421, 422, 437, 444, 448, 451, 453, 454, 457, 473)


@pytest.mark.parametrize("seed", HD256_PER_SEQUENCE_SEEDS)
def test_hd256_per_sequence_regression(device, seed):
    c = draw(seed)
    assert c["hd"] == 256
    run_case(device, seed, extended=seed % 3 == 1, chunked_query=seed % 3 == 2,
             per_sequence=True)


@pytest.mark.parametrize("seed", range(480, 600))
def test_random_odd_kv_heads_sweep(device, seed):
    run_case(device, seed, extended=seed % 4 == 1, chunked_query=seed % 4 == 2,
             per_sequence=seed % 4 == 3, hkv_choices=(5, 6, 7, 9, 10, 12))


# Batches of 65 to 256 sequences: the tile scan runs inside each wave with
# four sequences per lane on plain calls with pages of at least 16 tokens, and
# through LDS otherwise (a window, cap, sinks or ALiBi, or smaller pages).
@pytest.mark.parametrize("seed", range(600, 630))
def test_random_large_batch_sweep(device, seed):
    run_case(device, seed, extended=seed % 3 == 1, large_batch=True)


def redraw_large_batch(c: dict, seed: int) -> dict:
    """The case redrawn with 65 to 256 mostly short sequences (empty ones among them)."""
    r = random.Random(40_000 + seed)
    batch = r.randint(65, 256)
    lengths = [r.choice([0, 1, r.randint(2, 40), r.randint(40, 200)]) for _ in range(batch)]
    return dict(c, batch=batch, lengths=lengths)


def chunked(c: dict, seed: int) -> dict:
    """The case as a causal query past the kernel's 16 columns (GQ >= 2)."""
    r = random.Random(30_000 + seed)
    gq = c["gq"] if c["gq"] >= 2 else r.choice([2, 4, 8])
    ql = r.choice([q for q in range(16 // gq + 1, 64 // gq + 1)])
    return dict(c, gq=gq, ql=ql, causal=True)


def run_case(device, seed: int, extended: bool, chunked_query: bool = False,
             per_sequence: bool = False, hkv_choices: tuple = (1, 2, 3, 4, 8),
             large_batch: bool = False):
    c = draw(seed, hkv_choices)
    if large_batch:
        c = redraw_large_batch(c, seed)
    if chunked_query:
        c = chunked(c, seed)
    if per_sequence:
        c = dict(c, ns=native.SPLITS_PER_SEQUENCE)
    hq = c["hkv"] * c["gq"]
    b = make_paged_batch(c["batch"], hq, c["hkv"], c["hd"], c["dtype"],
                         torch.tensor(c["lengths"]), page_size=c["ps"], seed=1000 + seed,
                         q_len=c["ql"])
    kc, vc = b.k_cache, b.v_cache
    if c["fp8"]:
        kc, vc = kc.to(FP8), vc.to(FP8)
    extras = (draw_extras(seed, hq) if extended
              else dict(window=-1, sinks=None, softcap=0.0, alibi=None))
    ref = expected(b.q, kc, vc, b.block_table, b.cache_seqlens, b.scale, c["causal"], **extras)
    kd, vd = kc.to(device), vc.to(device)
    if c["head_major"]:  # [pages, HKV, PS, HD] storage viewed as [pages, PS, HKV, HD]
        kd = kd.permute(0, 2, 1, 3).contiguous().permute(0, 2, 1, 3)
        vd = vd.permute(0, 2, 1, 3).contiguous().permute(0, 2, 1, 3)
    q = b.q.to(device)
    # The output starts as NaN, so a row the kernels never write fails the
    # finiteness check (an empty sequence's expected zeros included).
    out = torch.full(q.shape, float("nan"), device=device, dtype=c["dtype"])
    if c["strided"]:  # q and out as slices of wider buffers
        wide = torch.randn(c["batch"], c["ql"], hq + 3, c["hd"], device=device).to(c["dtype"])
        wide[:, :, 2:2 + hq] = q
        q = wide[:, :, 2:2 + hq]
        # A distinct sentinel outside the slice, NaN inside it.
        obuf = torch.full((c["batch"], c["ql"], hq + 5, c["hd"]), SENTINEL, device=device,
                          dtype=c["dtype"])
        out = obuf[:, :, 1:1 + hq]
        out.fill_(float("nan"))
    kw = {} if c["ns"] is None else dict(num_splits=c["ns"])
    if chunked_query:
        assert c["ql"] * c["gq"] > 16 and c["causal"]
    sinks, alibi = extras["sinks"], extras["alibi"]
    cols = min(c["ql"], 16 // c["gq"]) * c["gq"]  # query columns of one launch
    if per_sequence and 4 * cols * (c["hd"] + 1) * 4 > 64 << 10:
        with pytest.raises(native.UnsupportedConfig, match="mxfa_split_decode"):
            native.paged_decode_split(q, kd, vd, b.block_table.to(device),
                                      b.cache_seqlens.to(device), b.scale, out=out,
                                      causal=c["causal"], window_left=extras["window"], **kw)
        return
    got = native.paged_decode_split(q, kd, vd, b.block_table.to(device),
                                    b.cache_seqlens.to(device), b.scale, out=out,
                                    causal=c["causal"], window_left=extras["window"],
                                    sinks=None if sinks is None else sinks.to(device),
                                    softcap=extras["softcap"],
                                    alibi_slopes=None if alibi is None else alibi.to(device), **kw)
    torch.cuda.synchronize()
    assert got.data_ptr() == out.data_ptr()
    assert torch.isfinite(got.float()).all(), (c, extras, "unwritten output rows")
    err = (got.float().cpu() - ref).abs().max().item()
    assert err <= TOL[c["dtype"]], (c, extras, err)
    if c["strided"]:  # nothing written outside the slice
        assert (obuf[:, :, :1] == SENTINEL).all()
        assert (obuf[:, :, 1 + hq:] == SENTINEL).all()
