"""Writes tests/golden/reference_vectors.npz: inputs and outputs of the
reference's own ATen build (oracle/_ref, compiled by oracle/build_ref.py from
the reference's csrc/mxmac sources) on small seeded decode cases.

Run in a checkout where oracle/_ref is built (it needs the reference's
sources):  python tests/golden/make_golden.py

The fixture is data only: every array is stored as its raw bits (bf16 as
uint16) with numpy's non-pickled format, so tests load it with
``numpy.load(allow_pickle=False)`` and need neither the reference nor its
build. The cases follow the decode calls the reference's tests make:

- ``table_order``: one sequence of 3 keys over a table [1, 0] of two-token
  pages (tests/test_api.py:136-155), fp16;
- ``paged_*``: flash_attn_with_kvcache over a paged cache, ragged lengths,
  a scrambled table (paged_kv.cpp:53-126), at GQ 1, 2, 4, 8, head dims 64 and
  128, page sizes 1, 16 and 32, fp16 and bf16, and a softmax scale of 0;
- ``append_*``: the same call with new k/v appended at cache_seqlens, with
  the lengths after the call and every cache row it rewrote, as (page,
  slot) indices and rows (tests/test_api.py:158-181, paged_kv.cpp:80-123):
  one token (decode step) and three query tokens with the causal mask;
- ``dense_kvcache``: a dense [B, S, HKV, D] cache (no block table);
- ``varlen``: flash_attn_varlen_func with one query row per segment and a
  segment with none (attention_forward.cpp);
- ``dense_func``: flash_attn_func with one query token per sequence.
"""

from __future__ import annotations

import pathlib
import sys

import numpy as np
import torch

ROOT = pathlib.Path(__file__).resolve().parents[2]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

from mxflashattn_amd.workloads import make_paged_batch  # noqa: E402
from oracle import ref_aten  # noqa: E402

OUT = pathlib.Path(__file__).with_name("reference_vectors.npz")


def to_array(t: torch.Tensor) -> np.ndarray:
    t = t.detach().cpu().contiguous()
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).numpy().view(np.uint16)
    return t.numpy()


def paged_case(ref, name, batch, hq, hkv, hd, dtype, lengths, page_size, seed, scale=None):
    b = make_paged_batch(batch, hq, hkv, hd, dtype, torch.tensor(lengths),
                         page_size=page_size, pool_factor=1.0, seed=seed)
    sc = b.scale if scale is None else scale
    out = ref.flash_attn_with_kvcache(b.q, b.k_cache, b.v_cache, None, None,
                                      b.cache_seqlens.clone(), b.block_table, sc, False)
    return name, dict(kind="kvcache", q=b.q, k_cache=b.k_cache, v_cache=b.v_cache,
                      block_table=b.block_table, cache_seqlens=b.cache_seqlens, scale=sc,
                      causal=False, out=out)


def changed_rows(before: torch.Tensor, after: torch.Tensor):
    """(page, slot) of every cache row the call rewrote, and the rows after it."""
    diff = (before.view(torch.int16) != after.view(torch.int16)).flatten(2).any(-1)
    index = diff.nonzero()
    return index.to(torch.int64), after[index[:, 0], index[:, 1]]


def append_case(ref, name, dtype, new_tokens, causal, seed):
    # Pages for the lengths after the append, so no two sequences share one;
    # rows past the old lengths hold random values the append overwrites.
    old = torch.tensor([0, 15, 16, 40])
    b = make_paged_batch(4, 8, 2, 64, dtype, old + new_tokens, page_size=16, pool_factor=1.0,
                         seed=seed)
    seqlens = (b.cache_seqlens - new_tokens).to(torch.int32)
    g = torch.Generator().manual_seed(seed + 1)
    k_new = torch.randn(4, new_tokens, 2, 64, generator=g).to(dtype)
    v_new = torch.randn(4, new_tokens, 2, 64, generator=g).to(dtype)
    q = torch.randn(4, new_tokens, 8, 64, generator=g).to(dtype)
    kc, vc, sl = b.k_cache.clone(), b.v_cache.clone(), seqlens.clone()
    out = ref.flash_attn_with_kvcache(q, kc, vc, k_new, v_new, sl, b.block_table, b.scale,
                                      causal)
    k_index, k_rows = changed_rows(b.k_cache, kc)
    v_index, v_rows = changed_rows(b.v_cache, vc)
    return name, dict(kind="kvcache", q=q, k_cache=b.k_cache, v_cache=b.v_cache, k=k_new,
                      v=v_new, block_table=b.block_table, cache_seqlens=seqlens,
                      scale=b.scale, causal=causal, out=out, k_cache_after_index=k_index,
                      k_cache_after_rows=k_rows, v_cache_after_index=v_index,
                      v_cache_after_rows=v_rows, cache_seqlens_after=sl)


def cases(ref):
    g = torch.Generator().manual_seed(20261007)
    # table_order: pages [2, 2, 1, 64], table [[1, 0]], three keys.
    q = torch.randn(1, 1, 2, 64, generator=g).half()
    kc = torch.randn(2, 2, 1, 64, generator=g).half()
    vc = torch.randn(2, 2, 1, 64, generator=g).half()
    bt = torch.tensor([[1, 0]], dtype=torch.int32)
    sl = torch.tensor([3], dtype=torch.int32)
    yield "table_order", dict(kind="kvcache", q=q, k_cache=kc, v_cache=vc, block_table=bt,
                              cache_seqlens=sl, scale=0.125, causal=False,
                              out=ref.flash_attn_with_kvcache(q, kc, vc, None, None, sl.clone(),
                                                              bt, 0.125, False))
    yield paged_case(ref, "paged_gq4_d64_f16", 4, 8, 2, 64, torch.float16, [1, 17, 40, 33], 16, 31)
    yield paged_case(ref, "paged_gq8_d128_bf16", 3, 8, 1, 128, torch.bfloat16, [1, 40, 50], 16, 32)
    yield paged_case(ref, "paged_gq2_d64_ps1_f16", 4, 4, 2, 64, torch.float16, [1, 5, 33, 17], 1, 33)
    yield paged_case(ref, "paged_gq1_d128_ps32_f16", 2, 1, 1, 128, torch.float16, [20, 40], 32, 34)
    yield paged_case(ref, "paged_gq8_d64_bf16_scale0", 2, 16, 2, 64, torch.bfloat16, [9, 50], 16, 35,
                     scale=0.0)
    yield append_case(ref, "append_decode_bf16", torch.bfloat16, 1, False, 36)
    yield append_case(ref, "append_causal3_f16", torch.float16, 3, True, 37)
    # dense_kvcache: [3, 24, 2, 64] caches, lengths 1, 23 and 12.
    kc = torch.randn(3, 24, 2, 64, generator=g).half()
    vc = torch.randn(3, 24, 2, 64, generator=g).half()
    q = torch.randn(3, 1, 8, 64, generator=g).half()
    sl = torch.tensor([1, 23, 12], dtype=torch.int32)
    yield "dense_kvcache", dict(kind="kvcache", q=q, k_cache=kc, v_cache=vc, cache_seqlens=sl,
                                scale=0.125, causal=False,
                                out=ref.flash_attn_with_kvcache(q, kc, vc, None, None, sl.clone(),
                                                                None, 0.125, False))
    # varlen: four segments of 7, 2, 21 and 1 keys; the second has no query row.
    cu_q = torch.tensor([0, 1, 1, 2, 3], dtype=torch.int32)
    cu_k = torch.tensor([0, 7, 9, 30, 31], dtype=torch.int32)
    q = torch.randn(3, 8, 64, generator=g).half()
    k = torch.randn(31, 2, 64, generator=g).half()
    v = torch.randn(31, 2, 64, generator=g).half()
    yield "varlen", dict(kind="varlen", q=q, k=k, v=v, cu_seqlens_q=cu_q, cu_seqlens_k=cu_k,
                         max_seqlen_q=1, max_seqlen_k=21, scale=0.2, causal=False,
                         out=ref.flash_attn_varlen_func(q, k, v, cu_q, cu_k, 1, 21, False, 0.2))
    # dense_func: [2, 1, 8, 64] queries against [2, 11, 4, 64] keys.
    q = torch.randn(2, 1, 8, 64, generator=g).to(torch.bfloat16)
    k = torch.randn(2, 11, 4, 64, generator=g).to(torch.bfloat16)
    v = torch.randn(2, 11, 4, 64, generator=g).to(torch.bfloat16)
    yield "dense_func", dict(kind="func", q=q, k=k, v=v, scale=0.3, causal=False,
                             out=ref.flash_attn_func(q, k, v, False, 0.3))


def flatten(all_cases) -> dict[str, np.ndarray]:
    arrays: dict[str, np.ndarray] = {}
    names = []
    for name, case in all_cases:
        names.append(name)
        dtype = str(case["q"].dtype).removeprefix("torch.")
        arrays[f"{name}__dtype"] = np.array(dtype)
        for key, value in case.items():
            if isinstance(value, torch.Tensor):
                arrays[f"{name}__{key}"] = to_array(value)
            else:
                arrays[f"{name}__{key}"] = np.array(value)
    arrays["cases"] = np.array(names)
    return arrays


def main() -> None:
    ref = ref_aten.load()
    if ref is None:
        raise SystemExit("oracle/_ref is not built: run oracle/build_ref.py where the "
                         "reference's sources are present")
    arrays = flatten(cases(ref))
    np.savez_compressed(OUT, **arrays)
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes, {len(arrays['cases'])} cases)")


if __name__ == "__main__":
    main()
