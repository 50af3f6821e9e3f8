"""PyTorch path behind MXFLASHATTN_ALLOW_FALLBACK=1 (the ``reference`` backend).

The public API keeps the reference's opt-in fallback contract
(mxflashattn/dispatch.py:153-170): calls the HIP backend cannot take (CPU
tensors, float32, unsupported head counts) may run here when the caller asks
for it explicitly. It is never used for a call the HIP backend qualifies for.
Semantics follow mxflashattn/reference.py: fp32 scores, optional causal mask
aligned to the key end, softmax with NaN -> 0, output cast to q's dtype; paged
caches are gathered through the block table and appended k/v advance
cache_seqlens in place.
"""

from __future__ import annotations

import math

import torch


def _attend(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, scale: float | None,
            causal: bool) -> torch.Tensor:
    """q [Lq, HQ, D], k/v [Lk, HKV, D] -> [Lq, HQ, D] (mxflashattn/reference.py:8-40)."""
    lq, hq, d = q.shape
    if lq == 0:
        return q.clone()
    lk, hkv = k.shape[0], k.shape[1]
    if lk == 0:
        raise ValueError("attention requires at least one key/value token")
    s = (1.0 / math.sqrt(d)) if scale is None else scale
    g = hq // hkv
    # Query head h reads kv head h // g: group the query heads per kv head.
    qf = q.float().reshape(lq, hkv, g, d).permute(1, 2, 0, 3)      # [HKV, G, Lq, D]
    kf = k.float().permute(1, 2, 0).unsqueeze(1)                    # [HKV, 1, D, Lk]
    vf = v.float().permute(1, 0, 2).unsqueeze(1)                    # [HKV, 1, Lk, D]
    scores = torch.matmul(qf, kf) * s                               # [HKV, G, Lq, Lk]
    if causal:
        row = torch.arange(lq, device=q.device).unsqueeze(1) + (lk - lq)
        col = torch.arange(lk, device=q.device).unsqueeze(0)
        scores = scores.masked_fill(col > row, float("-inf"))
    probs = torch.nan_to_num(torch.softmax(scores, dim=-1), nan=0.0, posinf=0.0, neginf=0.0)
    out = torch.matmul(probs, vf)                                   # [HKV, G, Lq, D]
    return out.permute(2, 0, 1, 3).reshape(lq, hq, d).to(q.dtype)


def attention_batched(q, k, v, *, softmax_scale=None, causal=False) -> torch.Tensor:
    if q.shape[0] == 0:
        return q.clone()
    return torch.stack([_attend(q[i], k[i], v[i], softmax_scale, causal)
                        for i in range(q.shape[0])])


def attention_varlen(q, k, v, q_offsets: list[int], k_offsets: list[int], *,
                     softmax_scale=None, causal=False) -> torch.Tensor:
    parts = [
        _attend(q[q_offsets[i]:q_offsets[i + 1]], k[k_offsets[i]:k_offsets[i + 1]],
                v[k_offsets[i]:k_offsets[i + 1]], softmax_scale, causal)
        for i in range(len(q_offsets) - 1)
    ]
    return torch.cat(parts, dim=0) if parts else q[:0].clone()


def attention_kvcache(q, k_cache, v_cache, *, cache_seqlens, block_table, k=None, v=None,
                      softmax_scale=None, causal=False) -> torch.Tensor:
    """Dense or paged cache, optional append (mxflashattn/reference.py:88-139)."""
    lengths = cache_seqlens.detach().cpu().tolist()
    new = 0 if k is None else k.shape[1]
    outputs = []
    for i in range(q.shape[0]):
        start = int(lengths[i])
        end = start + new
        if block_table is None:
            if new:
                k_cache[i, start:end] = k[i]
                v_cache[i, start:end] = v[i]
            keys, values = k_cache[i, :end], v_cache[i, :end]
        else:
            ps = k_cache.shape[1]
            pages = block_table[i].detach().cpu().tolist()
            for t in range(new):
                page, offset = divmod(start + t, ps)
                k_cache[int(pages[page]), offset] = k[i, t]
                v_cache[int(pages[page]), offset] = v[i, t]
            used = torch.tensor([int(x) for x in pages[:(end + ps - 1) // ps]], dtype=torch.long,
                                device=k_cache.device)
            keys = k_cache.index_select(0, used).flatten(0, 1)[:end]
            values = v_cache.index_select(0, used).flatten(0, 1)[:end]
        outputs.append(_attend(q[i], keys, values, softmax_scale, causal))
    if k is not None:
        cache_seqlens.add_(new)
    return torch.stack(outputs) if outputs else q.clone()
