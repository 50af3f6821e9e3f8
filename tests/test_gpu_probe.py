"""The streaming probe (mxfa_stream_probe_launch) reads exactly the bytes the
decode kernel reads (GPU).

Per kv head, the XOR of every word the probe's waves wrote must equal the XOR
of every 32-bit word of the valid K and V rows of that kv head (each valid
token once; rows past a sequence end read as zero) and of the group's q rows
once per piece (a sequence cut into pieces by the balanced ranges loads its q
once per piece), computed here on the CPU from the same inputs. A probe that
skipped, repeated (an even number of times) or misaddressed a tile would
change the XOR.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from mxflashattn_amd import native
from mxflashattn_amd.workloads import make_paged_batch

pytestmark = pytest.mark.gpu


def xor_words(a: np.ndarray, axis) -> np.ndarray:
    return np.bitwise_xor.reduce(a, axis=axis)


def expected_per_kv_head(b, num_splits: int) -> np.ndarray:
    cpu = b.to("cpu")
    ps, hkv, hd = cpu.page_size, cpu.kv_heads, cpu.head_dim
    gq = cpu.q_heads // hkv
    width = cpu.block_table.shape[1]
    lens = np.minimum(cpu.cache_seqlens.numpy().astype(np.int64), width * ps)
    tiles = (lens + 15) // 16
    starts = np.concatenate([[0], np.cumsum(tiles)])
    nt = int(starts[-1])
    r = min(num_splits, nt)
    lo = np.array([(i * nt) // r for i in range(r + 1)], dtype=np.int64)
    k = cpu.k_cache.view(torch.int16).numpy().view(np.uint32)  # [P, PS, HKV, HD/2]
    v = cpu.v_cache.view(torch.int16).numpy().view(np.uint32)
    q = cpu.q.view(torch.int16).numpy().view(np.uint32)  # [B, 1, HQ, HD/2]
    bt = cpu.block_table.numpy()
    acc = np.zeros(hkv, dtype=np.uint32)
    for s in range(cpu.batch):
        n = int(lens[s])
        if n == 0:
            continue
        pos = np.arange(n)
        pages = bt[s, pos // ps]
        for cache in (k, v):
            rows = cache[pages, pos % ps]  # [n, HKV, HD/2]
            acc ^= xor_words(xor_words(rows, 0), 1)
        pieces = int(np.count_nonzero((lo[:-1] < starts[s + 1]) & (lo[1:] > starts[s])))
        if pieces % 2:
            acc ^= xor_words(q[s, 0].reshape(hkv, gq * hd // 2), 1)
    return acc


CASES = [
    # (batch, q_heads, kv_heads, head_dim, page_size, max_len): 4-wave 256-byte
    # rows, 4-wave and 8-wave 128-byte rows, two sub-ranges per workgroup; the
    # wave-local scan with four sequences per lane (130) and the LDS scan past
    # its 256 (300).
    (7, 32, 8, 128, 16, 3000),
    (9, 32, 4, 64, 16, 4000),
    (6, 16, 8, 64, 64, 2500),
    (5, 8, 2, 128, 32, 1500),
    (130, 16, 8, 64, 16, 600),
    (300, 8, 2, 128, 16, 400),
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: "x".join(map(str, c)))
def test_probe_reads_every_valid_byte_once(device, case):
    batch, hq, hkv, hd, ps, max_len = case
    g = torch.Generator().manual_seed(hd + hkv)
    lengths = torch.randint(1, max_len, (batch,), generator=g)
    lengths[1] = 0  # an empty sequence
    lengths[2] = 1
    lengths[3] = 17
    b = make_paged_batch(batch, hq, hkv, hd, torch.bfloat16, lengths, page_size=ps,
                         seed=hd * 3 + hkv).to(device)
    heuristic = native.default_num_splits(b.q, b.k_cache, b.block_table)
    for ns in (1, 7, 100, max(1, heuristic)):
        want = expected_per_kv_head(b, ns)
        for depth in (0, 2, 3, 4):
            sink = torch.zeros(hkv, ns, 64, dtype=torch.int32, device=device)
            native.stream_probe(b.q, b.k_cache, b.v_cache, b.block_table, b.cache_seqlens, ns,
                                sink=sink, tiles_in_flight=depth)
            torch.cuda.synchronize()
            got = xor_words(sink.cpu().numpy().view(np.uint32).reshape(hkv, -1), 1)
            assert np.array_equal(got, want), (case, ns, depth)


def test_probe_refuses_shapes_it_does_not_walk(device):
    b = make_paged_batch(2, 8, 2, 256, torch.bfloat16, torch.tensor([5, 9]), seed=3).to(device)
    with pytest.raises(native.UnsupportedConfig, match="mxfa_stream_probe_launch"):
        native.stream_probe(b.q, b.k_cache, b.v_cache, b.block_table, b.cache_seqlens, 4)


@pytest.mark.parametrize("layout", [0, 1])
@pytest.mark.parametrize("depth", [4, 8, 16])
@pytest.mark.parametrize("workgroups", [1, 7, 512])
def test_stream_read_reads_every_word_once(device, layout, depth, workgroups):
    # mxfa_stream_read_launch: the XOR of the sink equals the XOR of every
    # 32-bit word of the bytes read, for byte counts that leave a partial last
    # chunk, more waves than chunks, and one word past a slice boundary.
    g = torch.Generator().manual_seed(depth * 10 + layout)
    data = torch.randint(-2**31, 2**31 - 1, (3 * 2**20 // 4 + 100,), dtype=torch.int32,
                         generator=g)
    buf = data.to(device)
    for nbytes in (16, 1040, 3 * 2**20 + 400, buf.numel() * 4):
        sink = native.stream_read(buf, nbytes, layout=layout, depth=depth, workgroups=workgroups)
        torch.cuda.synchronize()
        got = int(np.bitwise_xor.reduce(sink.cpu().numpy().view(np.uint32)))
        want = int(np.bitwise_xor.reduce(data[:nbytes // 4].numpy().view(np.uint32)))
        assert got == want, (nbytes, got, want)


def test_stream_read_refuses_bad_arguments(device):
    buf = torch.zeros(1024, dtype=torch.int32, device=device)
    with pytest.raises(native.UnsupportedConfig, match="mxfa_stream_read_launch"):
        native.stream_read(buf, depth=2)
    with pytest.raises(ValueError):
        native.stream_read(buf, 4097)
