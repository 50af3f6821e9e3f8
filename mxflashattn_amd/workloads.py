"""Seeded synthetic paged-KV decode batches (the shapes of the benchmark configs).

Inputs follow the reference kernel test's recipe (csrc_native/test_m1.py:40-47):
q/k/v ~ N(0, 1), a random permutation of physical pages as the block table,
scale 1/sqrt(head_dim). Generation runs on a torch.Generator of the target
device (or the CPU), so the same seed gives the same batch on every box.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch

DEFAULT_SEED = 20261007  # csrc_native/test_m1.py:40


@dataclass
class PagedBatch:
    q: torch.Tensor             # [B, 1, HQ, HD]
    k_cache: torch.Tensor       # [P, PS, HKV, HD]
    v_cache: torch.Tensor       # [P, PS, HKV, HD]
    block_table: torch.Tensor   # int32 [B, W]
    cache_seqlens: torch.Tensor  # int32 [B]
    scale: float
    window_left: int = -1       # sliding window of the decode call (-1: none)

    @property
    def batch(self) -> int:
        return self.q.shape[0]

    @property
    def q_heads(self) -> int:
        return self.q.shape[2]

    @property
    def kv_heads(self) -> int:
        return self.k_cache.shape[2]

    @property
    def head_dim(self) -> int:
        return self.q.shape[3]

    @property
    def page_size(self) -> int:
        return self.k_cache.shape[1]

    def total_tokens(self) -> int:
        return int(self.cache_seqlens.sum().item())

    def attended_tokens(self) -> torch.Tensor:
        """Keys per sequence that some query token sees: L_b, or with a
        sliding window min(L_b, window_left + QL) (the QL tokens' windows
        together)."""
        lens = self.cache_seqlens.to(torch.int64).cpu()
        if self.window_left < 0:
            return lens
        return torch.clamp(lens, max=self.window_left + self.q.shape[1])

    def kv_bytes(self) -> int:
        """K and V bytes the call must read: sum_b 2 * A_b * HKV * HD * elem,
        A_b the attended keys (L_b without a window), elem the cache's
        element (2 bytes, or 1 for an fp8 cache)."""
        return (2 * int(self.attended_tokens().sum()) * self.kv_heads * self.head_dim
                * self.k_cache.element_size())

    def algorithmic_bytes(self) -> int:
        """KV + q + out + used block-table entries + lengths."""
        ps = self.page_size
        lens = self.cache_seqlens.to(torch.int64).cpu()
        first = ((lens - self.attended_tokens()) // ps)
        pages = int(((lens + ps - 1) // ps - first).sum().item())
        qo = 2 * self.q.numel() * self.q.element_size()
        return self.kv_bytes() + qo + 4 * pages + 4 * self.batch

    def to(self, device: torch.device | str) -> "PagedBatch":
        return PagedBatch(self.q.to(device), self.k_cache.to(device), self.v_cache.to(device),
                          self.block_table.to(device), self.cache_seqlens.to(device), self.scale,
                          self.window_left)


def make_paged_batch(
    batch: int,
    q_heads: int,
    kv_heads: int,
    head_dim: int,
    dtype: torch.dtype,
    lengths: torch.Tensor | tuple[int, int] | int,
    *,
    page_size: int = 16,
    pool_factor: float = 1.25,
    num_pages: int | None = None,
    block_table_width: int | None = None,
    peaky_fraction: float = 0.0,
    peaky_scale: float = 8.0,
    seed: int = DEFAULT_SEED,
    device: torch.device | str = "cpu",
    kv_dtype: torch.dtype | None = None,
    q_len: int = 1,
    window_left: int = -1,
    packed: bool = False,
) -> PagedBatch:
    """Build one synthetic decode batch.

    lengths: a tensor of per-sequence lengths, an inclusive (lo, hi) range for
    uniform integers, or one length for every sequence. The page pool holds
    ceil(pool_factor * pages needed) pages unless num_pages is given; every
    sequence gets distinct pages from a random permutation of the pool.
    peaky_fraction of the K rows are multiplied by peaky_scale. kv_dtype
    float8_e4m3fn stores the caches as fp8 (the same N(0, 1) draws, rounded to
    nearest even; their dequantisation scales are 1). q_len > 1 gives every
    sequence that many query tokens (the last q_len positions of its length).
    window_left is recorded for the decode call (a sliding window) and changes
    the bytes the call must read, not the data. packed (page_size 1): the keys
    of all sequences are packed end to end, as flash_attn_varlen_func hands
    them over ([total_tokens, HKV, HD] viewed as one-token pages), and table
    row b is offset_b + arange(width) (past the sequence end it repeats the
    last token, which the length never reaches).
    """
    device = torch.device(device)
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    if isinstance(lengths, torch.Tensor):
        lens = lengths.to(torch.int64).cpu()
    elif isinstance(lengths, tuple):
        lo, hi = lengths
        cpu_gen = torch.Generator().manual_seed(seed)
        lens = torch.randint(lo, hi + 1, (batch,), generator=cpu_gen, dtype=torch.int64)
    else:
        lens = torch.full((batch,), int(lengths), dtype=torch.int64)
    need = [(int(x) + page_size - 1) // page_size for x in lens]
    total_need = sum(need)
    if packed:
        if page_size != 1:
            raise ValueError("packed keys are one-token pages (page_size 1)")
        num_pages = max(1, total_need)
        width = block_table_width or max(1, max(need) if need else 1)
        starts = torch.cumsum(torch.tensor([0] + need[:-1], dtype=torch.int64), 0)
        pos = torch.arange(width, dtype=torch.int64)[None, :]
        last = (starts + torch.tensor(need, dtype=torch.int64) - 1).clamp(min=0)[:, None]
        table = torch.minimum(starts[:, None] + pos, last).clamp(max=num_pages - 1)
        table = table.to(torch.int32)
    else:
        if num_pages is None:
            num_pages = max(1, math.ceil(pool_factor * total_need))
        if num_pages < total_need:
            raise ValueError(f"pool of {num_pages} pages cannot hold {total_need} pages")
        width = block_table_width or max(1, max(need) if need else 1)
        perm = torch.randperm(num_pages, generator=torch.Generator().manual_seed(seed + 1))
        table = torch.zeros((batch, width), dtype=torch.int32)
        cursor = 0
        for b, n in enumerate(need):
            table[b, :n] = perm[cursor:cursor + n].to(torch.int32)
            cursor += n

    def randn(*shape: int) -> torch.Tensor:
        return torch.randn(*shape, generator=gen, device=device, dtype=torch.float32).to(dtype)

    q = randn(batch, q_len, q_heads, head_dim)
    k_cache = randn(num_pages, page_size, kv_heads, head_dim)
    v_cache = randn(num_pages, page_size, kv_heads, head_dim)
    if peaky_fraction > 0:
        rows = k_cache.view(-1, head_dim)
        pick = torch.rand(rows.shape[0], generator=gen, device=device) < peaky_fraction
        rows[pick] = (rows[pick].float() * peaky_scale).to(dtype)
    if kv_dtype is not None and kv_dtype != dtype:
        k_cache, v_cache = k_cache.to(kv_dtype), v_cache.to(kv_dtype)
    return PagedBatch(
        q=q,
        k_cache=k_cache,
        v_cache=v_cache,
        block_table=table.to(device),
        cache_seqlens=lens.to(torch.int32).to(device),
        scale=head_dim ** -0.5,
        window_left=window_left,
    )


# The benchmark configurations of BASELINE.json (configs 1-4) and the six
# GQ x HD cells of config 2, as keyword arguments of make_paged_batch.
CONFIGS = {
    "config1_cpu_ref": dict(batch=4, q_heads=8, kv_heads=2, head_dim=64, dtype=torch.float16,
                            lengths=(1, 512), num_pages=128, block_table_width=32),
    "config2_qwen3_4b": dict(batch=32, q_heads=32, kv_heads=8, head_dim=128,
                             dtype=torch.bfloat16, lengths=(1024, 8192)),
    "config3_highbatch_gq2_d64": dict(batch=128, q_heads=16, kv_heads=8, head_dim=64,
                                      dtype=torch.float16, lengths=(1, 512)),
    "config4_long_gq8_d128": dict(batch=16, q_heads=32, kv_heads=4, head_dim=128,
                                  dtype=torch.bfloat16, lengths=16384, peaky_fraction=0.01),
    "config4_long_gq8_d64": dict(batch=16, q_heads=32, kv_heads=4, head_dim=64,
                                 dtype=torch.bfloat16, lengths=16384, peaky_fraction=0.01),
}

CELLS = {
    f"cell_gq{32 // hkv}_d{hd}": dict(batch=32, q_heads=32, kv_heads=hkv, head_dim=hd,
                                      dtype=torch.bfloat16, lengths=(1024, 8192))
    for hkv in (16, 8, 4) for hd in (128, 64)
}


# Shapes beyond the reference's contract (head dim 256, 1 or 16 query heads per
# kv head, fp8 caches), at config 2's batch and lengths.
WIDE = {
    "wide_fp8_config2": dict(batch=32, q_heads=32, kv_heads=8, head_dim=128,
                             dtype=torch.bfloat16, lengths=(1024, 8192),
                             kv_dtype=torch.float8_e4m3fn),
    "wide_fp8_gq8_d128": dict(batch=32, q_heads=32, kv_heads=4, head_dim=128,
                              dtype=torch.bfloat16, lengths=(1024, 8192),
                              kv_dtype=torch.float8_e4m3fn),
    "wide_hd256_gq2": dict(batch=32, q_heads=16, kv_heads=8, head_dim=256,
                           dtype=torch.bfloat16, lengths=(1024, 8192)),
    "wide_gq1_d128": dict(batch=32, q_heads=32, kv_heads=32, head_dim=128,
                          dtype=torch.bfloat16, lengths=(1024, 8192)),
    "wide_gq16_d128": dict(batch=32, q_heads=64, kv_heads=4, head_dim=128,
                           dtype=torch.bfloat16, lengths=(1024, 8192)),
    # Config 2 verifying 4 tokens per sequence (3 draft tokens), causal: the
    # same KV bytes as one token.
    "wide_q4_config2": dict(batch=32, q_heads=32, kv_heads=8, head_dim=128,
                            dtype=torch.bfloat16, lengths=(1024, 8192), q_len=4, causal=True),
    # Eight draft tokens at GQ 4: 32 columns, two launches of four tokens.
    "wide_q8_config2": dict(batch=32, q_heads=32, kv_heads=8, head_dim=128,
                            dtype=torch.bfloat16, lengths=(1024, 8192), q_len=8, causal=True),
    # Config 2 with a 1024-key sliding window (the local layers of models that
    # alternate local and global attention): each sequence reads its last
    # 1024 keys, 1/4.5 of the full call's bytes.
    "wide_window1024_config2": dict(batch=32, q_heads=32, kv_heads=8, head_dim=128,
                                    dtype=torch.bfloat16, lengths=(1024, 8192),
                                    window_left=1023),
    # One long sequence (a single long-context request): every range holds a
    # piece of it, so the combine folds hundreds of pieces per head.
    "wide_one_seq_128k_d128": dict(batch=1, q_heads=32, kv_heads=8, head_dim=128,
                                   dtype=torch.bfloat16, lengths=131072),
    "wide_one_seq_64k_d256": dict(batch=1, q_heads=16, kv_heads=2, head_dim=256,
                                  dtype=torch.bfloat16, lengths=65536),
    # Config 2 as flash_attn_varlen_func decode lays it out: the keys packed
    # end to end and read as one-token pages (the per-lane page-id kernels).
    "wide_varlen_config2": dict(batch=32, q_heads=32, kv_heads=8, head_dim=128,
                                dtype=torch.bfloat16, lengths=(1024, 8192), page_size=1,
                                packed=True),
}
