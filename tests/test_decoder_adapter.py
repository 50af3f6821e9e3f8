"""vLLM decode metadata -> flash_attn_with_kvcache (integrations/vllm/decoder_adapter.py).

A ``VllmBatch`` builds what vLLM hands the backend for a decode step: the
packed query [tokens, HQ, HD], the cache [2, blocks, PS, HKV, HD] and a
metadata object with vLLM's field names, over seeded random lengths and a
shuffled block table. The decode call is swapped for a recorder that keeps
its arguments and answers with the oracle port, so each of the adapter's
three modes (default, MXFLASHATTN_GRAPH_DECODE, MXFLASHATTN_TRANSPARENT) is
checked for what it passes on and for the rows it returns. The rejection
strings are the adapter's contract (the reference's decoder_adapter.py).
"""

from __future__ import annotations

from types import SimpleNamespace

import pytest
import torch

from mxflashattn_amd.integrations.vllm import decoder_adapter as da
from oracle import reference_port

MODES = {"default": {}, "graph": {"MXFLASHATTN_GRAPH_DECODE": "1"},
         "transparent": {"MXFLASHATTN_TRANSPARENT": "1"}}


class VllmBatch:
    def __init__(self, batch=3, hq=8, hkv=2, hd=64, ps=16, seed=0, pad=0):
        g = torch.Generator().manual_seed(seed)
        self.lengths = torch.randint(1, 3 * ps, (batch,), generator=g, dtype=torch.int32)
        pages = (self.lengths + ps - 1) // ps
        width = int(pages.max())
        blocks = int(pages.sum()) + 2
        perm = torch.randperm(blocks, generator=g).to(torch.int32)
        self.table = torch.zeros(batch, width, dtype=torch.int32)
        at = 0
        for b, n in enumerate(pages.tolist()):
            self.table[b, :n] = perm[at:at + n]
            at += n
        self.cache = torch.randn(2, blocks, ps, hkv, hd, generator=g).to(torch.float16)
        self.query = torch.randn(batch + pad, hq, hd, generator=g).to(torch.float16)
        self.batch, self.hq, self.hd = batch, hq, hd
        self.meta = SimpleNamespace(
            num_actual_tokens=batch, max_query_len=1,
            query_start_loc=torch.arange(batch + 1, dtype=torch.int32),
            max_seq_len=int(self.lengths.max()), seq_lens=self.lengths.clone(),
            block_table=self.table.clone(), scheduler_metadata=None, causal=True,
            use_cascade=False, slot_mapping=torch.zeros(batch, dtype=torch.int64))

    def expected(self, scale) -> torch.Tensor:
        q = self.query[:self.batch].view(self.batch, 1, self.hq, self.hd)
        return reference_port.attention_kvcache(
            q, self.cache[0], self.cache[1], cache_seqlens=self.lengths.clone(),
            block_table=self.table, softmax_scale=scale).reshape(self.batch, -1)


@pytest.fixture
def recorder(monkeypatch):
    calls = []

    def fake(q, key_cache, value_cache, **kwargs):
        calls.append(dict(q=q, key_cache=key_cache, value_cache=value_cache, **kwargs))
        out = reference_port.attention_kvcache(
            q, key_cache, value_cache, cache_seqlens=kwargs["cache_seqlens"].clone(),
            block_table=kwargs["block_table"], softmax_scale=kwargs["softmax_scale"])
        if kwargs.get("out") is not None:
            kwargs["out"].copy_(out)
            return kwargs["out"]
        return out

    monkeypatch.setattr(da, "flash_attn_with_kvcache", fake)
    for name in ("MXFLASHATTN_GRAPH_DECODE", "MXFLASHATTN_TRANSPARENT"):
        monkeypatch.delenv(name, raising=False)
    return calls


@pytest.mark.parametrize("mode", list(MODES))
@pytest.mark.parametrize("seed", [0, 1])
def test_every_mode_decodes_the_metadata_rows(recorder, monkeypatch, mode, seed):
    for name, value in MODES[mode].items():
        monkeypatch.setenv(name, value)
    vb = VllmBatch(seed=seed)
    out, layout = da.decode_forward(vb.query, vb.cache, vb.meta, softmax_scale=0.11)
    torch.testing.assert_close(out, vb.expected(0.11))
    (call,) = recorder
    assert call["q"].shape == (vb.batch, 1, vb.hq, vb.hd)
    assert call["cache_seqlens"].dtype == torch.int32
    assert torch.equal(call["cache_seqlens"], vb.lengths)
    assert torch.equal(call["block_table"], vb.table)
    # The key and value caches are views of vLLM's one buffer, no copies.
    assert call["key_cache"].data_ptr() == vb.cache.data_ptr()
    assert call["value_cache"].data_ptr() == vb.cache[1].data_ptr()
    assert (layout is None) == (mode != "default")
    if layout is not None:
        assert layout.batch_size == vb.batch and layout.kv_cache_shape == tuple(vb.cache.shape)


def test_default_mode_reads_no_device_data_unless_strict(recorder, monkeypatch):
    vb = VllmBatch(seed=2)
    layout = da.fast_layout(vb.query, vb.cache, vb.meta)
    assert layout.seq_lens == () and layout.query_lens == (1,) * vb.batch
    strict = da.inspect_layout(vb.query, vb.cache, vb.meta)
    assert strict.seq_lens == tuple(vb.lengths.tolist())
    assert strict.query_start_loc == tuple(range(vb.batch + 1))


def test_graph_mode_ignores_capture_padding(recorder, monkeypatch):
    monkeypatch.setenv("MXFLASHATTN_GRAPH_DECODE", "1")
    vb = VllmBatch(seed=3, pad=5)
    vb.meta.num_actual_tokens = vb.batch + 5
    vb.meta.max_query_len = 6  # the padded bucket, not a prefill
    out, _ = da.decode_forward(vb.query, vb.cache, vb.meta, softmax_scale=0.2)
    assert recorder[0]["q"].shape[0] == vb.batch
    torch.testing.assert_close(out, vb.expected(0.2))


def test_graph_mode_prefers_the_split_decode_fields(recorder, monkeypatch):
    monkeypatch.setenv("MXFLASHATTN_GRAPH_DECODE", "1")
    vb = VllmBatch(seed=4, pad=2)
    vb.meta.max_query_len = 9
    vb.meta.seq_lens = torch.full((vb.batch + 2,), 999, dtype=torch.int32)  # not used
    vb.meta.num_decode_tokens, vb.meta.num_decodes = vb.batch, vb.batch
    vb.meta.decode_seq_lens, vb.meta.decode_block_table = vb.lengths, vb.table
    out, _ = da.decode_forward(vb.query, vb.cache, vb.meta, softmax_scale=0.2)
    torch.testing.assert_close(out, vb.expected(0.2))
    vb.meta.num_decode_tokens = vb.batch + 1
    with pytest.raises(da.DecoderAdapterBlocked,
                       match="decode_tokens_not_divisible_by_num_decodes"):
        da.decode_forward(vb.query, vb.cache, vb.meta, softmax_scale=0.2)


def test_transparent_mode_flattens_capture_shaped_lengths(recorder, monkeypatch):
    monkeypatch.setenv("MXFLASHATTN_TRANSPARENT", "1")
    vb = VllmBatch(seed=5)
    vb.meta.seq_lens = vb.lengths.view(1, -1).to(torch.int64)
    out, layout = da.decode_forward(vb.query, vb.cache, vb.meta, softmax_scale=0.3)
    assert layout is None
    assert recorder[0]["cache_seqlens"].shape == (vb.batch,)
    assert recorder[0]["cache_seqlens"].dtype == torch.int32
    torch.testing.assert_close(out, vb.expected(0.3))


def test_forward_decode_fills_the_output_buffer_and_records_the_path(recorder, monkeypatch):
    from mxflashattn_amd.integrations.vllm import backend

    monkeypatch.setattr(da, "get_last_dispatch_info",
                        lambda: SimpleNamespace(backend="mi355x_split_decode",
                                                operation="flash_attn_with_kvcache",
                                                fallback_reason=None))
    backend.clear_dispatch_events(truncate_log=False)
    vb = VllmBatch(seed=6)
    output = torch.full((vb.batch + 1, vb.hq * vb.hd), -5.0, dtype=torch.float16)
    assert da.forward_decode(vb.query, vb.cache, vb.meta, output, softmax_scale=0.1) is output
    torch.testing.assert_close(output[:vb.batch], vb.expected(0.1))
    assert bool((output[vb.batch] == -5.0).all())  # rows past the batch untouched
    assert "out" in recorder[0]  # the rows were handed over, not copied afterwards
    assert backend.get_dispatch_events()[-1] == {
        "path": "mi355x_split_decode", "operation": "flash_attn_with_kvcache",
        "fallback": "false"}


def _without(meta, name):
    fields = dict(vars(meta))
    fields.pop(name)
    return SimpleNamespace(**fields)


BLOCKED = [
    ("prefill", lambda vb: setattr(vb.meta, "max_query_len", 2), "single_token_decode"),
    ("cascade", lambda vb: setattr(vb.meta, "use_cascade", True),
     "cascade_attention_not_supported_by_adapter"),
    ("causal flag", lambda vb: setattr(vb.meta, "causal", False),
     "metadata_causal_flag_is_false"),
    ("cache rank", lambda vb: setattr(vb, "cache", vb.cache[0]), "kv_cache_shape"),
    ("query rank", lambda vb: setattr(vb, "query", vb.query[None]), "query_rank"),
    ("fp32 cache", lambda vb: setattr(vb, "cache", vb.cache.float()),
     "kv_cache_dtype_not_supported"),
    ("gqa", lambda vb: setattr(vb, "query", vb.query[:, :3]),
     "query_and_kv_head_counts_are_not_gqa_compatible"),
    ("missing field", lambda vb: setattr(vb, "meta", _without(vb.meta, "scheduler_metadata")),
     "metadata_missing_fields:scheduler_metadata"),
]


@pytest.mark.parametrize("name,spoil,reason", BLOCKED, ids=[b[0] for b in BLOCKED])
def test_calls_outside_the_contract_are_blocked(recorder, name, spoil, reason):
    vb = VllmBatch(seed=7)
    spoil(vb)
    with pytest.raises(da.DecoderAdapterBlocked, match=reason):
        da.decode_forward(vb.query, vb.cache, vb.meta, softmax_scale=0.1)
    assert recorder == []


@pytest.mark.parametrize("mode", ["graph", "transparent"])
def test_cascade_is_blocked_in_every_mode(recorder, monkeypatch, mode):
    for name, value in MODES[mode].items():
        monkeypatch.setenv(name, value)
    vb = VllmBatch(seed=8)
    vb.meta.use_cascade = True
    with pytest.raises(da.DecoderAdapterBlocked, match="cascade"):
        da.decode_forward(vb.query, vb.cache, vb.meta, softmax_scale=0.1)
    with pytest.raises(da.DecoderAdapterBlocked, match="cascade"):
        da.forward_decode(vb.query, vb.cache.view(torch.uint8), vb.meta,
                          torch.empty(vb.batch, vb.hq * vb.hd, dtype=torch.float16),
                          softmax_scale=0.1, kv_cache_dtype="fp8")


def test_strict_layout_checks_the_offsets(recorder):
    vb = VllmBatch(seed=9)
    vb.meta.num_actual_tokens = vb.batch + 1
    with pytest.raises(da.DecoderAdapterBlocked,
                       match="query_start_loc_does_not_cover_num_actual_tokens"):
        da.inspect_layout(vb.query, vb.cache, vb.meta)
    vb.meta.num_actual_tokens = vb.batch
    vb.meta.block_table = vb.table[:-1]
    with pytest.raises(da.DecoderAdapterBlocked, match="block_table_rows_do_not_match_batch"):
        da.inspect_layout(vb.query, vb.cache, vb.meta)
