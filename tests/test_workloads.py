"""Synthetic batches and the bench.py contract that needs no GPU."""

import subprocess
import sys
from pathlib import Path

import pytest
import torch

from mxflashattn_amd.workloads import CELLS, CONFIGS, DEFAULT_SEED, make_paged_batch

REPO = Path(__file__).resolve().parents[1]


def test_block_tables_use_distinct_pages():
    b = make_paged_batch(8, 8, 2, 64, torch.float16, (1, 300), seed=3)
    used = []
    for i, n in enumerate(b.cache_seqlens.tolist()):
        used += b.block_table[i, : (n + 15) // 16].tolist()
    assert len(used) == len(set(used))
    assert all(0 <= p < b.k_cache.shape[0] for p in used)


def test_batches_are_reproducible_from_the_seed():
    a = make_paged_batch(4, 8, 2, 64, torch.bfloat16, (1, 100), seed=DEFAULT_SEED)
    b = make_paged_batch(4, 8, 2, 64, torch.bfloat16, (1, 100), seed=DEFAULT_SEED)
    assert torch.equal(a.k_cache, b.k_cache) and torch.equal(a.block_table, b.block_table)
    assert torch.equal(a.cache_seqlens, b.cache_seqlens)


def test_byte_counts():
    b = make_paged_batch(2, 8, 2, 64, torch.float16, torch.tensor([17, 32]))
    assert b.kv_bytes() == 2 * 49 * 2 * 64 * 2
    qo = 2 * 2 * 8 * 64 * 2
    assert b.algorithmic_bytes() == b.kv_bytes() + qo + 4 * (2 + 2) + 4 * 2


def test_pool_too_small_is_rejected():
    with pytest.raises(ValueError, match="cannot hold"):
        make_paged_batch(2, 8, 2, 64, torch.float16, 100, num_pages=3)


def test_peaky_rows_are_scaled():
    plain = make_paged_batch(1, 8, 1, 64, torch.float32, 4096)
    peaky = make_paged_batch(1, 8, 1, 64, torch.float32, 4096, peaky_fraction=0.01)
    ratio = (peaky.k_cache.abs().amax(dim=-1) / plain.k_cache.abs().amax(dim=-1)).flatten()
    scaled = torch.isclose(ratio, torch.tensor(8.0)).float().mean().item()
    assert 0.003 < scaled < 0.03
    assert torch.equal(peaky.v_cache, plain.v_cache)


def test_configs_match_the_benchmark_shapes():
    c2 = CONFIGS["config2_qwen3_4b"]
    assert (c2["batch"], c2["q_heads"], c2["kv_heads"], c2["head_dim"]) == (32, 32, 8, 128)
    assert c2["lengths"] == (1024, 8192) and c2["dtype"] == torch.bfloat16
    assert sorted(CELLS) == sorted(f"cell_gq{g}_d{d}" for g in (2, 4, 8) for d in (64, 128))
    for spec in CELLS.values():
        assert spec["q_heads"] // spec["kv_heads"] in (2, 4, 8)


def test_bench_refuses_more_than_one_gpu():
    proc = subprocess.run([sys.executable, str(REPO / "bench.py"), "--gpus", "2"],
                          capture_output=True, text=True, timeout=300)
    assert proc.returncode == 2
    assert "measures one GPU" in proc.stderr
    assert proc.stdout == ""


def test_window_changes_the_bytes_a_call_reads():
    lengths = torch.tensor([5, 100, 2000])
    plain = make_paged_batch(3, 8, 2, 64, torch.float16, lengths, seed=3)
    win = make_paged_batch(3, 8, 2, 64, torch.float16, lengths, seed=3, window_left=99)
    assert torch.equal(plain.k_cache, win.k_cache)  # same data
    assert plain.kv_bytes() == 2 * 2105 * 2 * 64 * 2
    assert win.attended_tokens().tolist() == [5, 100, 100]
    assert win.kv_bytes() == 2 * 205 * 2 * 64 * 2
    # Pages overlapping the window: 1 + 7 + pages 118..124 (keys 1900..1999).
    assert win.algorithmic_bytes() - win.kv_bytes() == 2 * win.q.numel() * 2 + 4 * (1 + 7 + 7) + 12
    two = make_paged_batch(3, 8, 2, 64, torch.float16, lengths, seed=3, window_left=99, q_len=2)
    assert two.attended_tokens().tolist() == [5, 100, 101]
    assert win.to("cpu").window_left == 99
