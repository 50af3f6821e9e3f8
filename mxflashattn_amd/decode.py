"""Routes from the public API to the HIP split-KV decode (``mi355x_split_decode``).

Each ``route_*`` function inspects a validated call and returns a
``DecodeRoute``: ``reason`` names why the HIP path cannot take the call (then
the dispatch chain continues), otherwise ``run`` launches it. Checks here read
only shapes, dtypes and devices, never device data, so a qualifying call does
not synchronise the stream.

  flash_attn_with_kvcache  paged or dense cache, q_len QL with QL * GQ <= 16
                           (one token, or a few draft tokens at the end of
                           each sequence with the reference's bottom-right
                           causal mask), optional k/v append (append kernel,
                           then decode over seqlens + S_new, then
                           cache_seqlens += S_new on the device).
  flash_attn_func          q_len QL with QL * GQ <= 16: k/v [B, S, HKV, D] is a
                           dense cache of S tokens per sequence.
  flash_attn_varlen_func   every sequence has at most one query token: packed
                           k/v are a cache of one-token pages whose block table
                           row b is cu_seqlens_k[b] + arange(max_seqlen_k).

A dense cache [B, S, HKV, D] is viewed as pages of P tokens, P the largest
power of two dividing S (capped at 256), with block table row b =
b * S/P + arange(S/P): the same bytes, no copy.
"""

from __future__ import annotations

import torch

from . import native
from .dispatch import DecodeRoute

_ACCEL = {"cuda"}


def _query_length_reason(q: torch.Tensor, kv_heads: int, causal: bool) -> str | None:
    """q is [B, QL, HQ, D]: QL query tokens x GQ heads fill the kernel's columns,
    or, for a causal query, up to four launches of them (token chunks)."""
    ql, gq = q.shape[1], q.shape[-2] // kv_heads
    limit = native.CHUNKED_COLUMNS if causal else native.KERNEL_COLUMNS
    if ql < 1 or ql * gq > limit:
        return f"query_length_{ql}_times_gqa_{gq}_exceeds_{limit}"
    return None


def _common_reason(q: torch.Tensor, kv_heads: int, head_dim: int) -> str | None:
    if q.device.type not in _ACCEL:
        return "requires_accelerator_tensor"
    if q.dtype not in native.DTYPE_CODES:
        return "supports_only_float16_and_bfloat16"
    if head_dim not in native.SUPPORTED_HEAD_DIMS:
        return f"head_dim_{head_dim}_not_in_{native.SUPPORTED_HEAD_DIMS}"
    hq = q.shape[-2]
    # Any group of 1..16 query heads per kv head runs here (the reference's
    # kernel stops at {2, 4, 8}; the API hands such calls down its chain).
    if kv_heads <= 0 or hq % kv_heads or hq // kv_heads not in native.KERNEL_GQA:
        return f"gqa_ratio_{hq}/{kv_heads}_not_in_1..16"
    return None


def _dense_page_size(seq: int) -> int:
    page = 1
    while page < 256 and seq % (page * 2) == 0:
        page *= 2
    return page


def _dense_as_pages(cache: torch.Tensor) -> torch.Tensor | None:
    """[B, S, HKV, D] -> [B*S/P, P, HKV, D] view, or None when not viewable."""
    b, s = cache.shape[0], cache.shape[1]
    page = _dense_page_size(s)
    try:
        return cache.view(b * (s // page), page, cache.shape[2], cache.shape[3])
    except RuntimeError:
        return None


def _dense_table(batch: int, pages_per_seq: int, device: torch.device) -> torch.Tensor:
    base = torch.arange(batch, device=device, dtype=torch.int32).unsqueeze(1) * pages_per_seq
    return base + torch.arange(pages_per_seq, device=device, dtype=torch.int32).unsqueeze(0)


def route_kvcache(q, k_cache, v_cache, k, v, cache_seqlens, block_table, scale,
                  causal, out: torch.Tensor | None = None) -> DecodeRoute:
    """``out`` (q's shape and dtype, last dim contiguous) receives the result
    in place; otherwise the run allocates it."""
    reason = _common_reason(q, k_cache.shape[2], q.shape[-1]) or _query_length_reason(
        q, k_cache.shape[2], bool(causal))
    if reason is not None:
        return DecodeRoute(reason)
    if k_cache.stride(-1) != 1 or v_cache.stride() != k_cache.stride():
        return DecodeRoute("cache_layout_not_supported")
    if block_table is None:
        kc, vc = _dense_as_pages(k_cache), _dense_as_pages(v_cache)
        if kc is None or vc is None:
            return DecodeRoute("dense_cache_not_viewable_as_pages")
        width = kc.shape[0] // q.shape[0]
    else:
        ps = k_cache.shape[1]
        if ps & (ps - 1) or ps > 4096:
            return DecodeRoute(f"page_size_{ps}_not_a_power_of_two_up_to_4096")
        kc, vc = k_cache, v_cache
        width = block_table.shape[1]
    reason = native.layout_reason(q, kc, vc, width)
    if reason is not None:
        return DecodeRoute(reason)
    if k is not None and (k.stride(-1) != 1 or v.stride(-1) != 1):
        k, v = k.contiguous(), v.contiguous()

    def run() -> torch.Tensor:
        if block_table is None:
            table = _dense_table(q.shape[0], kc.shape[0] // q.shape[0], q.device)
        else:
            table = block_table
        new = 0 if k is None else k.shape[1]
        if new:
            native.append_kv(k, v, kc, vc, table, cache_seqlens)
        result = native.paged_decode_split(q, kc, vc, table, cache_seqlens, scale,
                                           seqlen_add=new, causal=causal, out=out)
        if new:
            cache_seqlens.add_(new)
        return result

    return DecodeRoute(None, run)


def route_dense(q, k, v, scale, causal) -> DecodeRoute:
    reason = _common_reason(q, k.shape[2], q.shape[-1]) or _query_length_reason(
        q, k.shape[2], bool(causal))
    if reason is not None:
        return DecodeRoute(reason)
    kc, vc = _dense_as_pages(k), _dense_as_pages(v)
    if kc is None or vc is None or kc.stride(-1) != 1 or vc.stride() != kc.stride():
        return DecodeRoute("dense_kv_not_viewable_as_pages")
    reason = native.layout_reason(q, kc, vc, kc.shape[0] // q.shape[0])
    if reason is not None:
        return DecodeRoute(reason)

    def run() -> torch.Tensor:
        batch = q.shape[0]
        table = _dense_table(batch, kc.shape[0] // batch, q.device)
        lengths = torch.full((batch,), k.shape[1], dtype=torch.int32, device=q.device)
        return native.paged_decode_split(q, kc, vc, table, lengths, scale, causal=causal)

    return DecodeRoute(None, run)


def route_varlen(q, k, v, cu_seqlens_k: torch.Tensor, q_offsets: list[int], k_offsets: list[int],
                 max_seqlen_k: int, scale, causal) -> DecodeRoute:
    """Packed decode: sequence b's keys are rows [cu_k[b], cu_k[b+1]) of k/v,
    read in place as one-token pages. The block table and lengths are built
    on the device from ``cu_seqlens_k`` (no host-to-device copy) when every
    sequence has its query row, the usual decode batch."""
    reason = _common_reason(q, k.shape[1], q.shape[-1])
    if reason is not None:
        return DecodeRoute(reason)
    q_lens = [b - a for a, b in zip(q_offsets, q_offsets[1:])]
    if any(n > 1 for n in q_lens):
        return DecodeRoute("varlen_query_length_above_one")
    if k.stride(-1) != 1 or v.stride() != k.stride():
        return DecodeRoute("kv_layout_not_supported")
    # Sequences with a query row, in row order.
    rows = [i for i, n in enumerate(q_lens) if n == 1]
    if not rows:
        return DecodeRoute("varlen_without_query_rows")
    kc = k.unsqueeze(1)  # [T, 1, HKV, D]: one token per page
    vc = v.unsqueeze(1)
    # Table width from the offsets themselves: a max_seqlen_k smaller than a
    # sequence would otherwise cut that sequence short.
    width = max(1, max(k_offsets[i + 1] - k_offsets[i] for i in rows))
    reason = native.layout_reason(q.unsqueeze(1), kc, vc, width)
    if reason is not None:
        return DecodeRoute(reason)

    def run() -> torch.Tensor:
        device = q.device
        cu = cu_seqlens_k.to(torch.int32)
        starts, lengths = cu[:-1], cu[1:] - cu[:-1]
        if len(rows) != len(q_lens):
            pick = torch.as_tensor(rows, dtype=torch.int64).pin_memory().to(device,
                                                                          non_blocking=True)
            starts, lengths = starts.index_select(0, pick), lengths.index_select(0, pick)
        table = starts.unsqueeze(1) + torch.arange(width, dtype=torch.int32,
                                                   device=device).unsqueeze(0)
        out = native.paged_decode_split(q.unsqueeze(1), kc, vc, table, lengths.contiguous(),
                                        scale)
        return out.squeeze(1)

    return DecodeRoute(None, run)
