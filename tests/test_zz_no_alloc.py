"""mxfa_split_decode_noalloc_launch against mxfa_split_decode_launch (GPU).

The no-allocation entry point runs the same kernels with the library's own
device array as workspace, so its output must equal the workspace entry
point's bit for bit. Two calls in a row, the second with a smaller input (the
array keeps the first call's contents), then a size beyond the array, which
must be refused before any launch. Then the use it is for: the call captured
in a HIP graph in a fresh process, as the process's first call of the entry
point and after an eager one, each replay equal to the workspace entry point.
"""

from __future__ import annotations

import os
import subprocess
import sys
from pathlib import Path

import pytest
import torch

from mxflashattn_amd import native
from mxflashattn_amd.workloads import CONFIGS, make_paged_batch

pytestmark = pytest.mark.gpu


def decode_both(b, num_splits=None):
    with_ws = native.paged_decode_split(b.q, b.k_cache, b.v_cache, b.block_table,
                                        b.cache_seqlens, b.scale, num_splits=num_splits)
    no_alloc = torch.full_like(b.q, float("nan"))
    native.paged_decode_split_noalloc(b.q, b.k_cache, b.v_cache, b.block_table,
                                      b.cache_seqlens, b.scale, out=no_alloc,
                                      num_splits=num_splits)
    torch.cuda.synchronize()
    return with_ws, no_alloc


def test_no_alloc_matches_workspace_entry_point_on_two_calls(device):
    first = make_paged_batch(**CONFIGS["config2_qwen3_4b"], device=device)
    second = make_paged_batch(3, 16, 4, 64, torch.float16, torch.tensor([5, 700, 33]),
                              seed=61).to(device)
    for b in (first, second):  # the second call is the smaller one
        ws_bytes = native.workspace_size(b.batch, b.q_heads, b.head_dim,
                                         native.default_num_splits(b.q, b.k_cache,
                                                                   b.block_table))
        assert ws_bytes <= native.SCRATCH_BYTES
        with_ws, no_alloc = decode_both(b)
        assert torch.equal(with_ws, no_alloc)
    # A split count that crosses every sequence, on the smaller input.
    with_ws, no_alloc = decode_both(second, num_splits=40)
    assert torch.equal(with_ws, no_alloc)
    # The per-sequence kernel uses no workspace at all.
    with_ws, no_alloc = decode_both(second, num_splits=native.SPLITS_PER_SEQUENCE)
    assert torch.equal(with_ws, no_alloc)


def test_no_alloc_refuses_inputs_beyond_its_array(device):
    b = make_paged_batch(2, 32, 8, 128, torch.bfloat16, torch.tensor([100, 200]),
                         seed=62).to(device)
    splits = 300  # 32 heads x 300 ranges x 2 x 128 floats: 9.8 MB > 8 MiB
    assert native.workspace_size(b.batch, 32, 128, splits) > native.SCRATCH_BYTES
    out = torch.zeros_like(b.q)
    with pytest.raises(RuntimeError, match="8 MiB"):
        native.paged_decode_split_noalloc(b.q, b.k_cache, b.v_cache, b.block_table,
                                          b.cache_seqlens, b.scale, out=out, num_splits=splits)
    torch.cuda.synchronize()
    assert torch.equal(out, torch.zeros_like(out))  # nothing was launched


# Run in a fresh process (the library's per-device lookup of its array's
# address happens on the first call there): capture the no-allocation call on
# a side stream, replay it three times, each into a NaN-filled output, and
# compare every replay bitwise with the workspace entry point's eager result.
_CAPTURE_CHILD = r"""
import sys
import torch
sys.path.insert(0, sys.argv[2])
from mxflashattn_amd import native
from mxflashattn_amd.workloads import make_paged_batch

mode = sys.argv[1]
device = torch.device("cuda", 0)
b = make_paged_batch(5, 32, 8, 128, torch.bfloat16, torch.tensor([700, 1, 3000, 64, 2048]),
                     seed=71).to(device)
native.library()
ns = native.default_num_splits(b.q, b.k_cache, b.block_table)
assert ns > 0, ns  # the split path, whose workspace is the library's array
out = torch.full_like(b.q, float("nan"))
side = torch.cuda.Stream(device)
print(f"[child] mode={mode} num_splits={ns}", flush=True)
if mode == "after_eager":
    with torch.cuda.stream(side):
        native.paged_decode_split_noalloc(b.q, b.k_cache, b.v_cache, b.block_table,
                                          b.cache_seqlens, b.scale, out=out, num_splits=ns)
    torch.cuda.synchronize()
graph = torch.cuda.CUDAGraph()
with torch.cuda.graph(graph, stream=side):
    native.paged_decode_split_noalloc(b.q, b.k_cache, b.v_cache, b.block_table,
                                      b.cache_seqlens, b.scale, out=out, num_splits=ns)
want = native.paged_decode_split(b.q, b.k_cache, b.v_cache, b.block_table, b.cache_seqlens,
                                 b.scale, num_splits=ns)
torch.cuda.synchronize()
assert torch.isfinite(want.float()).all()
for i in range(3):
    out.fill_(float("nan"))
    torch.cuda.synchronize()
    graph.replay()
    torch.cuda.synchronize()
    assert torch.equal(out, want), f"replay {i} differs"
print(f"[child] {mode}: three replays equal the workspace entry point", flush=True)
"""


@pytest.mark.parametrize("mode", ["first_call_captured", "after_eager"])
def test_no_alloc_captured_in_a_graph(device, mode):
    repo = str(Path(__file__).resolve().parents[1])
    proc = subprocess.run([sys.executable, "-c", _CAPTURE_CHILD, mode, repo],
                          capture_output=True, text=True, timeout=300, env=dict(os.environ))
    print(proc.stdout, proc.stderr[-3000:], flush=True)
    assert proc.returncode == 0, proc.stderr[-3000:]
    assert "three replays equal" in proc.stdout
