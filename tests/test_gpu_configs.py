"""Full-size GPU parity on every benchmark configuration.

Each of configs 1-4 is built at its stated size (workloads.CONFIGS) and decoded
through the public API (backend recorded as mi355x_split_decode) and through
the binding at the heuristic split count and at one range per kv head; every
output is checked against the fp32 port of reference.attention_kvcache at the
north-star tolerances (fp16 2e-3, bf16 1.6e-2 max-abs). Config 4 adds the
fp64 C oracle, whose peaky keys stress the LSE merge.

Config 5 runs the full 36-layer, batch-128 decode step of the vLLM backend
path: the layer-0 page append is compared bit for bit with the C oracle's
reshape_and_cache, one layer's attention on the live caches with the port, and
graph-replayed steps must give finite logits.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import mxflashattn_amd as mx
from mxflashattn_amd import native
from mxflashattn_amd.workloads import CONFIGS, make_paged_batch
from oracle import c_oracle, reference_port

pytestmark = pytest.mark.gpu

TOL = {torch.float16: 2e-3, torch.bfloat16: 1.6e-2}


def port_out(b) -> torch.Tensor:
    cpu = b.to("cpu")
    return reference_port.attention_kvcache(
        cpu.q, cpu.k_cache, cpu.v_cache, cache_seqlens=cpu.cache_seqlens.clone(),
        block_table=cpu.block_table, softmax_scale=cpu.scale).float()


def max_err(a: torch.Tensor, b: torch.Tensor) -> float:
    return (a.float().cpu() - b.float().cpu()).abs().max().item()


@pytest.mark.parametrize("name", sorted(CONFIGS))
def test_config_full_size_matches_port(device, name):
    spec = CONFIGS[name]
    b = make_paged_batch(**spec, device=device)
    tol = TOL[spec["dtype"]]
    expected = port_out(b)
    api_out = mx.flash_attn_with_kvcache(b.q, b.k_cache, b.v_cache,
                                         cache_seqlens=b.cache_seqlens,
                                         block_table=b.block_table, softmax_scale=b.scale,
                                         out=torch.full_like(b.q, float("nan")))
    torch.cuda.synchronize()
    info = mx.get_last_dispatch_info()
    assert info.backend == mx.BACKEND_MI355X and info.fallback_reason is None
    assert torch.isfinite(api_out.float()).all()
    assert max_err(api_out, expected) <= tol, name
    for ns in (None, 1):
        got = native.paged_decode_split(b.q, b.k_cache, b.v_cache, b.block_table,
                                        b.cache_seqlens, b.scale, num_splits=ns,
                                        out=torch.full_like(b.q, float("nan")))
        torch.cuda.synchronize()
        assert torch.isfinite(got.float()).all()
        assert max_err(got, expected) <= tol, (name, ns)


@pytest.mark.parametrize("name", ["config4_long_gq8_d128", "config4_long_gq8_d64"])
def test_config4_matches_fp64_oracle(device, name):
    b = make_paged_batch(**CONFIGS[name], device=device)
    got = native.paged_decode_split(b.q, b.k_cache, b.v_cache, b.block_table, b.cache_seqlens,
                                    b.scale, out=torch.full_like(b.q, float("nan")))
    torch.cuda.synchronize()
    assert torch.isfinite(got.float()).all()
    ref = c_oracle.paged_decode_f64(b.q.cpu(), b.k_cache.cpu(), b.v_cache.cpu(),
                                    b.block_table.cpu(), b.cache_seqlens.cpu(), b.scale)
    assert max_err(got, torch.from_numpy(ref).reshape(got.shape)) <= TOL[torch.bfloat16]


def test_config5_full_decode_step(device):
    from mxflashattn_amd.integrations.vllm import decode_step as ds

    shape = ds.QWEN3_4B  # 36 layers, hidden 2560, 32q/8kv heads of 128
    batch, new_tokens = 128, 8
    model = ds.DecoderModel(shape, device)
    prompt = ds.lognormal_prompt_lengths(batch, 1024, 1.0, 16, 8192, 20261007)
    state = ds.build_state(model, batch, prompt, new_tokens)

    # One eager step, recording layer 0's append inputs and one layer's
    # attention inputs and output.
    watch = 17
    record = {}
    attention = model.attention

    def recording(layer, q, k, v, kv_cache, meta, out):
        if layer == 0:
            record["cache0"] = kv_cache.cpu()
            record["kv0"] = (k.cpu(), v.cpu())
            record["slots"] = meta.slot_mapping.cpu()
        attention(layer, q, k, v, kv_cache, meta, out)
        if layer == 0:
            record["cache0_after"] = kv_cache.cpu()
        if layer == watch:
            torch.cuda.synchronize()
            record["q"] = q.cpu()
            record["out"] = out.cpu()
            record["cache"] = kv_cache.cpu()
            record["seq_lens"] = meta.seq_lens.cpu()
            record["table"] = meta.block_table.cpu()

    model.attention = recording
    logits = model.step(state.tokens, state.positions, state.kv_caches, state.meta)
    torch.cuda.synchronize()
    model.attention = attention
    assert torch.isfinite(logits.float()).all()

    # Layer-0 append: bit-exact against the C oracle.
    kc, vc = record["cache0"].unbind(0)
    k0, v0 = record["kv0"]
    exp_k, exp_v = c_oracle.reshape_and_cache(k0, v0, kc, vc, record["slots"])
    got_k, got_v = record["cache0_after"].unbind(0)
    assert torch.equal(got_k, exp_k) and torch.equal(got_v, exp_v)

    # Layer `watch` attention on the live cache against the port.
    kc, vc = record["cache"].unbind(0)
    q = record["q"].reshape(batch, 1, shape.q_heads, shape.head_dim)
    expected = reference_port.attention_kvcache(
        q, kc, vc, cache_seqlens=record["seq_lens"].clone(), block_table=record["table"],
        softmax_scale=model.scale).float().reshape(batch, -1)
    assert max_err(record["out"], expected) <= TOL[torch.bfloat16]

    # Graph-replayed steps: capture once, advance the runner state between replays.
    stream = torch.cuda.Stream(device)
    ds.advance(state)
    with torch.cuda.stream(stream):
        model.step(state.tokens, state.positions, state.kv_caches, state.meta)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        glogits = model.step(state.tokens, state.positions, state.kv_caches, state.meta)
    with torch.cuda.stream(stream):
        for _ in range(3):
            graph.replay()
            state.tokens.copy_(glogits.argmax(-1))
            ds.advance(state)
    torch.cuda.synchronize()
    assert torch.isfinite(glogits.float()).all()
    lens = state.meta.seq_lens.cpu().to(torch.int64)
    assert torch.equal(lens, prompt + 5)  # one advance in build_state, one before capture, three after replays
    del graph
