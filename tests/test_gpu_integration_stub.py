"""The reference-side ctypes stub printed in the integration guide, run as written.

The stub is what a maintainer would put in the reference's plugin in place of
its mxmmain.so load (integrations/vllm/vllm_plugin.py:171-182,286-289). This
test executes the code block from the document against this build's library
and checks it against the package's own path, so the document cannot drift
from the ABI."""

from __future__ import annotations

import re
from pathlib import Path

import pytest
import torch

from mxflashattn_amd import native
from mxflashattn_amd.workloads import make_paged_batch

pytestmark = pytest.mark.gpu

DOC = Path(__file__).resolve().parents[1] / "INTEGRATION.md"


def _stub_source() -> str:
    text = DOC.read_text(encoding="utf-8")
    section = text[text.index("## 3."):]
    block = re.search(r"```python\n(.*?)```", section, re.S)
    assert block, f"{DOC.name} section 3 has no python block"
    return block.group(1)


def test_integration_stub_runs_as_documented(device, monkeypatch):
    monkeypatch.setenv("MXFLASHATTN_AMD_LIB", str(native.LIB_PATH))
    ns: dict = {}
    exec(compile(_stub_source(), str(DOC), "exec"), ns)
    g = torch.Generator().manual_seed(91)
    for dtype, hkv, hd in ((torch.bfloat16, 8, 128), (torch.float16, 4, 64)):
        b = make_paged_batch(7, 4 * hkv, hkv, hd, dtype,
                             torch.randint(1, 3000, (7,), generator=g), seed=92).to(device)
        # q as vLLM hands it over: a strided slice of a wider buffer.
        wide = torch.zeros(b.q.shape[0], 1, b.q.shape[2] + 3, hd, dtype=dtype, device=device)
        wide[:, :, 1:1 + b.q.shape[2]] = b.q
        q = wide[:, :, 1:1 + b.q.shape[2]]
        stream = torch.cuda.current_stream(device).cuda_stream
        got = ns["paged_decode_split"](q, b.k_cache, b.v_cache, b.block_table, b.cache_seqlens,
                                       b.scale, stream, 8, 1024)
        want = native.paged_decode_split(b.q, b.k_cache, b.v_cache, b.block_table,
                                         b.cache_seqlens, b.scale)
        torch.cuda.synchronize()
        assert torch.equal(got, want), (dtype, hkv, hd)
