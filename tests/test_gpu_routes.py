"""GPU runs of the routes that sit in front of the kernels, against the oracle.

- flash_attn_varlen_func decode (one query row per sequence): packed k/v
  read in place as one-token pages, against reference_port.attention_varlen
  (reference.py:60-85), with a sequence that has no query row;
- the vLLM compat wrapper's native route (MXFA_NATIVE_DECODE=1): q a strided
  [T, HQ, D] slice of a fused QKV buffer, with and without ``out=``, and its
  dispatch event (vllm_plugin.py:266-300);
- decode_forward in its graph-padded (MXFLASHATTN_GRAPH_DECODE=1) and
  transparent (MXFLASHATTN_TRANSPARENT=1) modes (decoder_adapter.py:132-157,
  236-286), and forward_decode writing into vLLM's output buffer;
- the per-stream workspace growing after a graph was captured on that stream.

Tolerances: fp16 2e-3, bf16 1.6e-2 max-abs against the fp32 port.
"""

from __future__ import annotations

from types import SimpleNamespace

import pytest
import torch

import mxflashattn_amd as mx
from mxflashattn_amd import native
from mxflashattn_amd.integrations.vllm import backend, decoder_adapter, native_decode
from mxflashattn_amd.workloads import make_paged_batch
from oracle import reference_port

pytestmark = pytest.mark.gpu

TOL = {torch.float16: 2e-3, torch.bfloat16: 1.6e-2}


def max_err(a: torch.Tensor, b: torch.Tensor) -> float:
    return (a.float().cpu() - b.float().cpu()).abs().max().item()


def port_kvcache(b, q=None) -> torch.Tensor:
    cpu = b.to("cpu")
    return reference_port.attention_kvcache(
        cpu.q if q is None else q.cpu(), cpu.k_cache, cpu.v_cache,
        cache_seqlens=cpu.cache_seqlens.clone(), block_table=cpu.block_table,
        softmax_scale=cpu.scale).float()


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=["f16", "bf16"])
@pytest.mark.parametrize("head_dim", [64, 128])
@pytest.mark.parametrize("gq", [2, 4, 8])
def test_varlen_decode_matches_port(device, dtype, head_dim, gq):
    hkv = 2
    lens = [1, 37, 300, 16, 1029]
    g = torch.Generator().manual_seed(100 * gq + head_dim)
    cu_k = torch.tensor([0] + torch.tensor(lens).cumsum(0).tolist(), dtype=torch.int32)
    k = torch.randn(int(cu_k[-1]), hkv, head_dim, generator=g).to(dtype)
    v = torch.randn(int(cu_k[-1]), hkv, head_dim, generator=g).to(dtype)
    q = torch.randn(len(lens), gq * hkv, head_dim, generator=g).to(dtype)
    cu_q = torch.arange(len(lens) + 1, dtype=torch.int32)
    expected = reference_port.attention_varlen(q, k, v, cu_q.tolist(), cu_k.tolist()).float()
    got = mx.flash_attn_varlen_func(q.to(device), k.to(device), v.to(device), cu_q.to(device),
                                    cu_k.to(device), max_seqlen_q=1, max_seqlen_k=max(lens))
    torch.cuda.synchronize()
    assert mx.get_last_dispatch_info().backend == mx.BACKEND_MI355X
    assert got.shape == q.shape
    assert max_err(got, expected) <= TOL[dtype]


def test_varlen_decode_with_a_sequence_without_query_row(device):
    dtype, hkv, hd = torch.bfloat16, 4, 128
    lens = [20, 5, 700]
    g = torch.Generator().manual_seed(7)
    cu_k = [0, 20, 25, 725]
    k = torch.randn(725, hkv, hd, generator=g).to(dtype)
    v = torch.randn(725, hkv, hd, generator=g).to(dtype)
    q = torch.randn(2, 16, hd, generator=g).to(dtype)  # sequence 1 has no query row
    cu_q = [0, 1, 1, 2]
    expected = reference_port.attention_varlen(q, k, v, cu_q, cu_k).float()
    got = mx.flash_attn_varlen_func(
        q.to(device), k.to(device), v.to(device), torch.tensor(cu_q, dtype=torch.int32,
                                                               device=device),
        torch.tensor(cu_k, dtype=torch.int32, device=device), max_seqlen_q=1,
        max_seqlen_k=max(lens))
    torch.cuda.synchronize()
    assert mx.get_last_dispatch_info().backend == mx.BACKEND_MI355X
    assert max_err(got, expected) <= TOL[dtype]


def fused_qkv_query(b, device) -> torch.Tensor:
    """q as vLLM hands it over: a [T, HQ, D] slice of a fused [T, (HQ+2HKV)*D] buffer."""
    t, hq, hd = b.batch, b.q_heads, b.head_dim
    fused = torch.randn(t, (hq + 2 * b.kv_heads) * hd, device=device, dtype=b.q.dtype)
    fused[:, :hq * hd] = b.q.reshape(t, hq * hd)
    q = fused[:, :hq * hd].view(t, hq, hd)
    assert not q.is_contiguous()
    return q


@pytest.mark.parametrize("with_out", [False, True])
def test_vllm_compat_native_route(device, monkeypatch, with_out):
    monkeypatch.setenv("MXFA_NATIVE_DECODE", "1")
    monkeypatch.delenv("MXFA_WIDE_CONTRACT", raising=False)
    monkeypatch.setattr(native_decode, "official_kvcache", None)
    b = make_paged_batch(6, 32, 8, 128, torch.bfloat16, torch.tensor([1, 16, 17, 250, 1500, 3]),
                         seed=31).to(device)
    q = fused_qkv_query(b, device)
    backend.clear_dispatch_events(truncate_log=False)
    kwargs = dict(k_cache=b.k_cache, v_cache=b.v_cache, cache_seqlens=b.cache_seqlens,
                  block_table=b.block_table, softmax_scale=b.scale, causal=True,
                  scheduler_metadata=None, fa_version=2)
    out = torch.full((b.batch, 32, 128), float("nan"), device=device, dtype=b.q.dtype)
    if with_out:
        kwargs["out"] = out
    result = native_decode.mx_kvcache_compat(q, **kwargs)
    torch.cuda.synchronize()
    if with_out:
        assert result.data_ptr() == out.data_ptr()
    assert result.shape == (b.batch, 32, 128)
    assert max_err(result, port_kvcache(b).reshape(b.batch, 32, 128)) <= TOL[torch.bfloat16]
    events = backend.get_dispatch_events()
    assert events[-1]["path"] == "mi355x_split_decode"
    assert events[-1]["operation"] == "paged_decode_split"
    assert events[-1]["fallback"] == "false"
    assert int(events[-1]["np"]) == native.default_num_splits(q.unsqueeze(1), b.k_cache,
                                                              b.block_table)


def test_vllm_compat_hands_back_unsupported_head_dim(device, monkeypatch):
    monkeypatch.setenv("MXFA_NATIVE_DECODE", "1")
    monkeypatch.delenv("MXFA_WIDE_CONTRACT", raising=False)
    seen = []
    monkeypatch.setattr(native_decode, "official_kvcache",
                        lambda *a, **k: seen.append(k) or "handed back")
    b = make_paged_batch(2, 16, 8, 256, torch.bfloat16, 40, seed=3).to(device)
    got = native_decode.mx_kvcache_compat(b.q.squeeze(1), k_cache=b.k_cache, v_cache=b.v_cache,
                                          cache_seqlens=b.cache_seqlens,
                                          block_table=b.block_table, s_aux=None)
    assert got == "handed back" and "s_aux" in seen[0]


def vllm_metadata(b, **extra):
    fields = dict(num_actual_tokens=b.batch, max_query_len=1,
                  query_start_loc=torch.arange(b.batch + 1, dtype=torch.int32,
                                               device=b.q.device),
                  max_seq_len=int(b.cache_seqlens.max()), seq_lens=b.cache_seqlens,
                  block_table=b.block_table, scheduler_metadata=None, causal=True,
                  use_cascade=False)
    fields.update(extra)
    return SimpleNamespace(**fields)


def vllm_cache(b) -> torch.Tensor:
    return torch.stack([b.k_cache, b.v_cache])  # [2, blocks, PS, HKV, HD]


def test_decode_forward_graph_mode_with_padded_query(device, monkeypatch):
    monkeypatch.setenv("MXFLASHATTN_GRAPH_DECODE", "1")
    b = make_paged_batch(5, 16, 4, 64, torch.float16, torch.tensor([9, 128, 1, 700, 33]),
                         seed=41).to(device)
    pad = 3  # capture padding: query rows past the metadata's batch
    query = torch.randn(b.batch + pad, 16, 64, device=device, dtype=b.q.dtype)
    query[:b.batch] = b.q.squeeze(1)
    meta = vllm_metadata(b, num_actual_tokens=b.batch + pad, max_query_len=1)
    result, layout = decoder_adapter.decode_forward(query, vllm_cache(b), meta,
                                                    softmax_scale=b.scale, causal=True)
    torch.cuda.synchronize()
    assert layout is None and result.shape == (b.batch, 16 * 64)
    assert mx.get_last_dispatch_info().backend == mx.BACKEND_MI355X
    assert max_err(result, port_kvcache(b).reshape(b.batch, -1)) <= TOL[torch.float16]


def test_decode_forward_graph_mode_split_decode_metadata(device, monkeypatch):
    monkeypatch.setenv("MXFLASHATTN_GRAPH_DECODE", "1")
    b = make_paged_batch(4, 32, 8, 128, torch.bfloat16, torch.tensor([400, 2, 1000, 77]),
                         seed=43).to(device)
    query = torch.randn(b.batch + 2, 32, 128, device=device, dtype=b.q.dtype)
    query[:b.batch] = b.q.squeeze(1)
    # Mixed-batch metadata: the decode part is described by its own fields.
    meta = vllm_metadata(b, max_query_len=7, num_decode_tokens=b.batch, num_decodes=b.batch,
                         decode_seq_lens=b.cache_seqlens, decode_block_table=b.block_table,
                         seq_lens=torch.zeros(b.batch + 2, dtype=torch.int32, device=device))
    result, _ = decoder_adapter.decode_forward(query, vllm_cache(b), meta,
                                               softmax_scale=b.scale, causal=True)
    torch.cuda.synchronize()
    assert max_err(result, port_kvcache(b).reshape(b.batch, -1)) <= TOL[torch.bfloat16]


def test_decode_forward_graph_mode_replayed(device, monkeypatch):
    monkeypatch.setenv("MXFLASHATTN_GRAPH_DECODE", "1")
    b = make_paged_batch(3, 32, 8, 128, torch.bfloat16, torch.tensor([50, 1100, 6]),
                         seed=45).to(device)
    query = b.q.squeeze(1).clone()
    cache = vllm_cache(b)
    meta = vllm_metadata(b)
    out = torch.empty(b.batch, 32 * 128, device=device, dtype=b.q.dtype)
    stream = torch.cuda.Stream(device)
    with torch.cuda.stream(stream):
        eager, _ = decoder_adapter.decode_forward(query, cache, meta, softmax_scale=b.scale)
        eager = eager.clone()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        res, _ = decoder_adapter.decode_forward(query, cache, meta, softmax_scale=b.scale,
                                                out=out)
    for _ in range(3):
        out.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)
    assert max_err(eager, port_kvcache(b).reshape(b.batch, -1)) <= TOL[torch.bfloat16]
    del graph


def test_decode_forward_transparent_mode(device, monkeypatch):
    monkeypatch.setenv("MXFLASHATTN_TRANSPARENT", "1")
    monkeypatch.delenv("MXFLASHATTN_GRAPH_DECODE", raising=False)
    b = make_paged_batch(4, 16, 8, 64, torch.float16, torch.tensor([3, 300, 64, 65]),
                         seed=47).to(device)
    meta = vllm_metadata(b, seq_lens=b.cache_seqlens.view(1, -1))  # capture-shaped seq_lens
    result, layout = decoder_adapter.decode_forward(b.q.squeeze(1).contiguous(), vllm_cache(b),
                                                    meta, softmax_scale=b.scale)
    torch.cuda.synchronize()
    assert layout is None
    assert mx.get_last_dispatch_info().backend == mx.BACKEND_MI355X
    assert max_err(result, port_kvcache(b).reshape(b.batch, -1)) <= TOL[torch.float16]


def test_forward_decode_writes_into_vllm_output(device, monkeypatch):
    for name in ("MXFLASHATTN_GRAPH_DECODE", "MXFLASHATTN_TRANSPARENT"):
        monkeypatch.delenv(name, raising=False)
    b = make_paged_batch(4, 32, 8, 128, torch.bfloat16, torch.tensor([17, 2000, 1, 512]),
                         seed=49).to(device)
    output = torch.full((b.batch + 2, 32 * 128), 7.0, device=device, dtype=b.q.dtype)
    result = decoder_adapter.forward_decode(b.q.squeeze(1).contiguous(), vllm_cache(b),
                                            vllm_metadata(b), output, softmax_scale=b.scale)
    torch.cuda.synchronize()
    assert result is output
    assert max_err(output[:b.batch], port_kvcache(b).reshape(b.batch, -1)) <= TOL[torch.bfloat16]
    assert torch.equal(output[b.batch:].cpu(), torch.full((2, 32 * 128), 7.0,
                                                          dtype=b.q.dtype))


def fresh_stream() -> torch.cuda.ExternalStream:
    """A stream no earlier test used (torch's own streams come from a pool),
    so the workspace keyed by it starts empty. Default priority."""
    import ctypes

    hip = ctypes.CDLL("libamdhip64.so")
    handle = ctypes.c_void_p()
    assert hip.hipStreamCreate(ctypes.byref(handle)) == 0
    return torch.cuda.ExternalStream(handle.value)


def test_workspace_growth_after_capture_keeps_captured_buffer(device):
    """A larger eager call on a stream that holds a captured graph grows the
    workspace; the graph's replays must still use memory nobody else owns."""
    stream = fresh_stream()
    small = make_paged_batch(2, 32, 8, 128, torch.bfloat16, torch.tensor([900, 3000]),
                             seed=51).to(device)
    large = make_paged_batch(600, 32, 8, 128, torch.bfloat16, (1, 200), seed=52).to(device)
    out = torch.empty_like(small.q)

    def call(b, o=None):
        # num_splits 200 puts every sequence of `small` across range ends, so
        # the replay writes and reads the workspace.
        return native.paged_decode_split(b.q, b.k_cache, b.v_cache, b.block_table,
                                         b.cache_seqlens, b.scale, out=o, num_splits=200)

    with torch.cuda.stream(stream):
        eager = call(small).clone()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        call(small, out)
    retired = native.retired_workspace_bytes()
    with torch.cuda.stream(stream):
        big = call(large)  # needs a larger workspace on the same stream
    torch.cuda.synchronize()
    assert native.retired_workspace_bytes() > retired  # the workspace grew
    # Fresh allocations of the retired size must not alias the captured buffer.
    fillers = [torch.full((1 << 20,), 3, dtype=torch.uint8, device=device) for _ in range(8)]
    torch.cuda.synchronize()
    for _ in range(3):
        out.zero_()
        with torch.cuda.stream(stream):
            graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)
        for f in fillers:
            assert bool((f == 3).all())
    assert max_err(eager, port_kvcache(small)) <= TOL[torch.bfloat16]
    assert max_err(big, port_kvcache(large)) <= TOL[torch.bfloat16]
    del graph


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=["f16", "bf16"])
def test_torch_operator_and_ctypes_paths_agree_bitwise(device, monkeypatch, dtype):
    """The C++ operator (csrc/torch_op.cpp) takes the common one-token call;
    the ctypes binding takes it when the operator is switched off. Same C ABI,
    same kernels: the outputs are the same bits, with a strided q and out."""
    assert native.torch_op() is not None, "the torch operator is not built"
    b = make_paged_batch(7, 32, 8, 128, dtype, torch.tensor([1, 17, 300, 2, 2049, 64, 5]),
                         seed=71).to(device)
    q = fused_qkv_query(b, device).view(b.batch, 1, 32, 128)
    outs = []
    for use_op in (True, False):
        monkeypatch.setattr(native, "USE_TORCH_OP", use_op)
        buf = torch.full((b.batch, 1, 40, 128), 3.0, device=device, dtype=dtype)
        got = native.paged_decode_split(q, b.k_cache, b.v_cache, b.block_table,
                                        b.cache_seqlens, b.scale, out=buf[:, :, 4:36])
        torch.cuda.synchronize()
        assert got.data_ptr() == buf[:, :, 4:36].data_ptr()
        outs.append(buf.clone())
    assert torch.equal(outs[0], outs[1])
    assert max_err(outs[0][:, :, 4:36], port_kvcache(b)) <= TOL[dtype]
