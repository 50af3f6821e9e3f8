"""Config-5 decode step driver: metadata bookkeeping on the CPU, and on the GPU
the plugin path (cache update + decode through the backend functions) against
the same model with oracle attention, eager and HIP-graph replayed."""

from __future__ import annotations

import pytest
import torch

from mxflashattn_amd.integrations.vllm import decode_step
from mxflashattn_amd.integrations.vllm.decode_step import DecoderModel, DecoderShape
from oracle import reference_port

TINY = DecoderShape(layers=2, hidden=256, q_heads=8, kv_heads=2, head_dim=128, intermediate=512,
                    vocab=1000)


def test_prompt_lengths_follow_the_stated_distribution():
    lens = decode_step.lognormal_prompt_lengths(4096, 1024, 1.0, 16, 8192, seed=3)
    assert lens.min() >= 16 and lens.max() <= 8192
    assert 900 <= float(lens.float().median()) <= 1150  # median of the lognormal
    assert (lens == 8192).any()  # the upper clip is 2.1 sigma above the median
    wide = decode_step.lognormal_prompt_lengths(4096, 1024, 3.0, 16, 8192, seed=3)
    assert (wide == 16).any() and (wide == 8192).any() and wide.min() == 16


def test_state_tables_slots_and_lengths():
    model = DecoderModel(TINY, torch.device("cpu"))
    prompt = torch.tensor([5, 40, 200, 17])
    st = decode_step.build_state(model, 4, prompt, new_tokens=20, page_size=16)
    table, meta = st.meta.block_table, st.meta
    pages = ((prompt + 20 + 15) // 16).tolist()
    used = torch.cat([table[b, :n] for b, n in enumerate(pages)])
    assert sorted(used.tolist()) == list(range(sum(pages)))  # every page once
    assert meta.seq_lens.tolist() == (prompt + 1).tolist()
    assert st.positions.tolist() == prompt.tolist()
    for _ in range(3):
        pos = st.positions
        expect = table.gather(1, (pos // 16)[:, None]).squeeze(1).long() * 16 + pos % 16
        assert torch.equal(meta.slot_mapping, expect)
        decode_step.advance(st)
    assert meta.seq_lens.tolist() == (prompt + 4).tolist()


class OracleAttentionModel(DecoderModel):
    """The same decoder with the cache write and attention restated in torch."""

    def attention(self, layer, q, k, v, kv_cache, meta, out):
        ps = kv_cache.shape[2]
        slots = meta.slot_mapping
        kv_cache[0, slots // ps, slots % ps] = k
        kv_cache[1, slots // ps, slots % ps] = v
        o = reference_port.attention_kvcache(
            q.unsqueeze(1).cpu(), kv_cache[0].cpu(), kv_cache[1].cpu(),
            cache_seqlens=meta.seq_lens.cpu(), block_table=meta.block_table.cpu(),
            softmax_scale=self.scale)
        out.copy_(o.reshape(out.shape).to(out.device))


@pytest.mark.gpu
def test_plugin_path_matches_oracle_attention_eager_and_graph(device):
    torch.manual_seed(0)
    native_model = DecoderModel(TINY, device, seed=5)
    ref_model = OracleAttentionModel(TINY, device, seed=5)
    prompt = torch.tensor([5, 40, 200, 17])
    st = decode_step.build_state(native_model, 4, prompt, new_tokens=6, page_size=16)
    ref_caches = [c.clone() for c in st.kv_caches]
    # Eager: two steps, the second after advancing the metadata.
    for _ in range(2):
        logits = native_model.step(st.tokens, st.positions, st.kv_caches, st.meta)
        expected = ref_model.step(st.tokens, st.positions, ref_caches, st.meta)
        torch.cuda.synchronize()
        assert (logits.float() - expected.float()).abs().max().item() <= 5e-2
        # Layer 0's new K/V rows depend on the weights and tokens only: the page
        # append is bit-exact there. Later layers see attention outputs that
        # differ by rounding, so their rows agree to bf16 precision.
        assert torch.equal(st.kv_caches[0], ref_caches[0])
        for a, b in zip(st.kv_caches[1:], ref_caches[1:]):
            assert (a.float() - b.float()).abs().max().item() <= 5e-2
        decode_step.advance(st)
    # Graph: capture one step, replay it three times with eager work between,
    # every replay equal to the eager step on the same inputs.
    stream = torch.cuda.Stream(device)
    with torch.cuda.stream(stream):
        eager = native_model.step(st.tokens, st.positions, st.kv_caches, st.meta).clone()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        captured = native_model.step(st.tokens, st.positions, st.kv_caches, st.meta)
    for _ in range(3):
        with torch.cuda.stream(stream):
            graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(captured, eager)
        _ = torch.randn(1000, device=device).sum().item()  # unrelated eager work


class OracleFp8AttentionModel(DecoderModel):
    """The decoder with an fp8 cache: the cache write restated with torch's
    round-to-nearest-even e4m3fn conversion after saturation (the append
    kernel's semantics, pinned in tests/test_oracle.py), attention on the
    exactly dequantised cache."""

    def attention(self, layer, q, k, v, kv_cache, meta, out):
        ps = kv_cache.shape[2]
        slots = meta.slot_mapping
        kv_cache[0, slots // ps, slots % ps] = (k.float() / self.k_scale).clamp(-448, 448).to(
            torch.float8_e4m3fn)
        kv_cache[1, slots // ps, slots % ps] = (v.float() / self.v_scale).clamp(-448, 448).to(
            torch.float8_e4m3fn)
        o = reference_port.attention_kvcache(
            q.unsqueeze(1).float().cpu(), kv_cache[0].float().cpu() * self.k_scale.cpu(),
            kv_cache[1].float().cpu() * self.v_scale.cpu(),
            cache_seqlens=meta.seq_lens.cpu(), block_table=meta.block_table.cpu(),
            softmax_scale=self.scale)
        out.copy_(o.reshape(out.shape).to(out.device, out.dtype))


@pytest.mark.gpu
def test_plugin_path_with_fp8_cache_matches_oracle(device):
    native_model = DecoderModel(TINY, device, seed=5, kv_cache_dtype="fp8")
    ref_model = OracleFp8AttentionModel(TINY, device, seed=5, kv_cache_dtype="fp8")
    for m in (native_model, ref_model):  # non-trivial per-tensor scales
        m.k_scale.fill_(0.5)
        m.v_scale.fill_(0.25)
    prompt = torch.tensor([5, 40, 200, 17])
    st = decode_step.build_state(native_model, 4, prompt, new_tokens=6, page_size=16)
    assert st.kv_caches[0].dtype == torch.float8_e4m3fn
    ref_caches = [c.clone() for c in st.kv_caches]
    for _ in range(2):
        logits = native_model.step(st.tokens, st.positions, st.kv_caches, st.meta)
        expected = ref_model.step(st.tokens, st.positions, ref_caches, st.meta)
        torch.cuda.synchronize()
        assert (logits.float() - expected.float()).abs().max().item() <= 5e-2
        # Layer 0's new rows depend on weights and tokens only: the quantising
        # append is bit-exact there.
        assert torch.equal(st.kv_caches[0].view(torch.uint8), ref_caches[0].view(torch.uint8))
        decode_step.advance(st)


@pytest.mark.gpu
@pytest.mark.parametrize("with_sinks", [False, True], ids=["plain", "sinks_softcap_alibi"])
@pytest.mark.parametrize("kv_dtype", ["auto", "fp8"])
def test_adapter_window_decode_matches_oracle(device, kv_dtype, with_sinks):
    """forward_decode with a layer's sliding window and attention sinks (the
    backend under the wider contract), on a vLLM-layout cache [2, blocks, PS,
    HKV, HD], against the port's windowed attention with sinks; fp8 caches on
    their exactly decoded values. The second case adds soft-capping and ALiBi."""
    from types import SimpleNamespace

    from mxflashattn_amd.integrations.vllm import decoder_adapter

    g = torch.Generator().manual_seed(31)
    hq, hkv, hd, ps = 8, 2, 128, 16
    lengths = torch.tensor([1, 40, 300, 1000], dtype=torch.int32)
    need = [(int(n) + ps - 1) // ps for n in lengths]
    blocks = sum(need) + 3
    perm = torch.randperm(blocks, generator=g).to(torch.int32)
    table = torch.zeros(4, max(need), dtype=torch.int32)
    at = 0
    for b, n in enumerate(need):
        table[b, :n] = perm[at:at + n]
        at += n
    cache = torch.randn(2, blocks, ps, hkv, hd, generator=g).to(torch.bfloat16)
    if kv_dtype == "fp8":
        codes = cache.float().to(torch.float8_e4m3fn)
        ref_cache, dev_cache = codes.float().to(torch.bfloat16), codes.view(torch.uint8)
    else:
        ref_cache, dev_cache = cache, cache
    q = torch.randn(4, hq, hd, generator=g).to(torch.bfloat16)
    meta = SimpleNamespace(num_actual_tokens=4, max_query_len=1, use_cascade=False, causal=True,
                           seq_lens=lengths.to(device), block_table=table.to(device),
                           query_start_loc=torch.arange(5, device=device), max_seq_len=1000,
                           scheduler_metadata=None)
    one = torch.ones(1, dtype=torch.float32, device=device)
    scale = hd ** -0.5
    sinks = torch.linspace(-2.0, 2.0, hq) if with_sinks else None
    cap = 3.0 if with_sinks else 0.0
    slopes = torch.pow(2.0, -torch.arange(1, hq + 1, dtype=torch.float32)) if with_sinks else None
    for window in (-1, 0, 17, 100, 5000):
        out = torch.full((4, hq * hd), float("nan"), dtype=torch.bfloat16, device=device)
        decoder_adapter.forward_decode(q.to(device), dev_cache.to(device), meta, out,
                                       softmax_scale=scale, kv_cache_dtype=kv_dtype,
                                       k_scale=one, v_scale=one, window_left=window,
                                       sinks=None if sinks is None else sinks.to(device),
                                       softcap=cap,
                                       alibi_slopes=None if slopes is None else slopes.to(device))
        torch.cuda.synchronize()
        want = reference_port.attention_kvcache(
            q.unsqueeze(1), ref_cache[0], ref_cache[1], cache_seqlens=lengths.clone(),
            block_table=table, softmax_scale=scale, window_left=window, sinks=sinks,
            softcap=cap, alibi_slopes=slopes)
        err = (out.float().cpu() - want.reshape(4, -1).float()).abs().max().item()
        assert err <= 1.6e-2, (window, err)
