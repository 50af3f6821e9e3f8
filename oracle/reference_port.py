"""fp32 torch-CPU restatement of ``mxflashattn/reference.py`` (test infrastructure only).

This is the parity oracle for the fp16/bf16 tolerances (output compared with an
fp32-softmax reference) and the timed CPU baseline of bench.py ("port").
Semantics follow the reference function by function:

  attention_single   reference.py:8-40   [seq, heads, dim]; fp32 q.K^T * scale,
                                         optional causal mask aligned to the key
                                         end, softmax, NaN->0, P.V, cast to q dtype.
  attention_batched  reference.py:43-57  per batch item.
  attention_varlen   reference.py:60-85  per cumulative-length segment.
  attention_kvcache  reference.py:88-139 optional append of k/v at positions
                                         cache_seqlens[b] + t (paged: page
                                         block_table[b, pos // PS], row pos % PS),
                                         gather, attention, then cache_seqlens += S_new.

window_left (attention_single, attention_kvcache) has no reference
counterpart: the reference rejects sliding windows (validation.py:56-76). With
window_left >= 0 the query at key position p also drops keys before
p - window_left, on top of the causal mask. It is pinned by identities against
the unwindowed port (tests/test_oracle.py), not by the reference.

sinks (float32 [HQ], same scale as the scaled scores) is vLLM's s_aux: one
extra softmax column per head with a zero value row; the reference drops it
(integrations/vllm/vllm_plugin.py:335-339). Pinned against library attention
over one appended key whose score is the sink (tests/test_oracle.py).

softcap > 0 caps every scaled score s to softcap * tanh(s / softcap) before the
masks (FlashAttention's softcap); the reference rejects it
(validation.py:56-76). Pinned by its limits: a tiny cap gives uniform weights
(the mean of the visible V rows), a huge one no change.

alibi_slopes (float32 [HQ]) adds -slope * |p - j| to the score of the query
at position p and key j, after the cap and before the masks (FlashAttention's
alibi_slopes); the reference rejects them (validation.py:56-76). Pinned by
zero slopes and by a zero query, whose weights are exactly e^(-slope*|p-j|).
"""

from __future__ import annotations

import math

import torch


def attention_single(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, *,
                     softmax_scale: float | None = None, causal: bool = False,
                     window_left: int = -1, sinks: torch.Tensor | None = None,
                     softcap: float = 0.0,
                     alibi_slopes: torch.Tensor | None = None) -> torch.Tensor:
    """q [Lq, HQ, D], k/v [Lk, HKV, D] -> [Lq, HQ, D] in q.dtype (reference.py:8-40)."""
    if q.shape[0] == 0:
        return q.clone()
    lq, hq, d = q.shape
    lk, hkv, _ = k.shape
    if lk == 0:
        raise ValueError("attention requires at least one key/value token")
    scale = softmax_scale if softmax_scale is not None else 1.0 / math.sqrt(d)
    group = hq // hkv
    # [HQ, Lq, D] x [HQ, D, Lk]; head h reads kv head h // group.
    qf = q.float().permute(1, 0, 2)
    kf = k.float().permute(1, 0, 2).repeat_interleave(group, dim=0)
    vf = v.float().permute(1, 0, 2).repeat_interleave(group, dim=0)
    scores = torch.bmm(qf, kf.transpose(1, 2).contiguous()) * scale
    if softcap > 0:
        scores = softcap * torch.tanh(scores / softcap)
    # query i sits at key position i + (Lk - Lq).
    qpos = torch.arange(lq).unsqueeze(1) + (lk - lq)
    kpos = torch.arange(lk).unsqueeze(0)
    if alibi_slopes is not None:
        dist = (qpos - kpos).abs().float().unsqueeze(0)  # [1, Lq, Lk]
        scores = scores - alibi_slopes.float().view(hq, 1, 1) * dist
    if causal:  # it may not see later keys
        scores = scores.masked_fill((kpos > qpos).unsqueeze(0), float("-inf"))
    if window_left >= 0:  # nor keys more than window_left before it
        scores = scores.masked_fill((kpos < qpos - window_left).unsqueeze(0), float("-inf"))
    if sinks is not None:  # one more column per head, dropped after the softmax
        sink = sinks.float().view(hq, 1, 1).expand(hq, lq, 1)
        probs = torch.softmax(torch.cat([scores, sink], dim=-1), dim=-1)[..., :lk]
    else:
        probs = torch.softmax(scores, dim=-1)
    probs = torch.nan_to_num(probs, nan=0.0, posinf=0.0, neginf=0.0)
    return torch.bmm(probs, vf).permute(1, 0, 2).to(q.dtype)


def attention_batched(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, *,
                      softmax_scale: float | None = None, causal: bool = False) -> torch.Tensor:
    """[B, L, H, D] per batch item (reference.py:43-57)."""
    if q.shape[0] == 0:
        return q.clone()
    return torch.stack([
        attention_single(q[i], k[i], v[i], softmax_scale=softmax_scale, causal=causal)
        for i in range(q.shape[0])
    ])


def attention_varlen(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                     cu_q: list[int], cu_k: list[int], *, softmax_scale: float | None = None,
                     causal: bool = False) -> torch.Tensor:
    """Packed [T, H, D] segments (reference.py:60-85)."""
    parts = [
        attention_single(q[cu_q[i]:cu_q[i + 1]], k[cu_k[i]:cu_k[i + 1]], v[cu_k[i]:cu_k[i + 1]],
                         softmax_scale=softmax_scale, causal=causal)
        for i in range(len(cu_q) - 1)
    ]
    return torch.cat(parts, dim=0) if parts else q[:0].clone()


def gather_pages(cache: torch.Tensor, pages: list[int], length: int) -> torch.Tensor:
    """Rows 0..length-1 of a paged sequence: [length, HKV, D] (reference.py:123-126)."""
    ps = cache.shape[1]
    need = (length + ps - 1) // ps
    idx = torch.tensor(pages[:need], dtype=torch.long)
    return cache.index_select(0, idx).reshape(need * ps, *cache.shape[2:])[:length]


def attention_kvcache(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor, *,
                      cache_seqlens: torch.Tensor, block_table: torch.Tensor | None,
                      k: torch.Tensor | None = None, v: torch.Tensor | None = None,
                      softmax_scale: float | None = None, causal: bool = False,
                      window_left: int = -1, sinks: torch.Tensor | None = None,
                      softcap: float = 0.0,
                      alibi_slopes: torch.Tensor | None = None) -> torch.Tensor:
    """Decode/append against a dense or paged cache (reference.py:88-139).

    Mutates the caches (append) and cache_seqlens (+= S_new) like the reference.
    """
    lengths = [int(x) for x in cache_seqlens.tolist()]
    s_new = 0 if k is None else k.shape[1]
    outs = []
    for b in range(q.shape[0]):
        old = lengths[b]
        total = old + s_new
        if block_table is None:
            if s_new:
                k_cache[b, old:total] = k[b]
                v_cache[b, old:total] = v[b]
            kb, vb = k_cache[b, :total], v_cache[b, :total]
        else:
            ps = k_cache.shape[1]
            row = [int(x) for x in block_table[b].tolist()]
            for t in range(s_new):
                page, off = divmod(old + t, ps)
                k_cache[row[page], off] = k[b, t]
                v_cache[row[page], off] = v[b, t]
            kb = gather_pages(k_cache, row, total)
            vb = gather_pages(v_cache, row, total)
        outs.append(attention_single(q[b], kb, vb, softmax_scale=softmax_scale, causal=causal,
                                     window_left=window_left, sinks=sinks,
                                     softcap=softcap, alibi_slopes=alibi_slopes))
    if k is not None:
        cache_seqlens.add_(s_new)
    return torch.stack(outs) if outs else q.clone()
