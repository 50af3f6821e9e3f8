"""vLLM metadata adapter (mirrors the reference's tests/test_decoder_adapter.py)."""

from dataclasses import dataclass

import pytest
import torch

from mxflashattn_amd.integrations.vllm import decoder_adapter
from mxflashattn_amd.integrations.vllm.decoder_adapter import (
    DecoderAdapterBlocked,
    decode_forward,
    inspect_layout,
)
from oracle import reference_port

pytestmark = pytest.mark.filterwarnings(
    "ignore:MXFlashAttn is using the PyTorch reference path:RuntimeWarning")


@dataclass
class Metadata:
    num_actual_tokens: int
    max_query_len: int
    query_start_loc: torch.Tensor
    max_seq_len: int
    seq_lens: torch.Tensor
    block_table: torch.Tensor
    slot_mapping: torch.Tensor
    use_cascade: bool = False
    scheduler_metadata: torch.Tensor | None = None
    causal: bool = True


def make_case(query_lens=(1, 1)):
    q = torch.randn(sum(query_lens), 4, 64, dtype=torch.float16)
    cache = torch.randn(2, 4, 16, 2, 64, dtype=torch.float16)
    starts = [0]
    for length in query_lens:
        starts.append(starts[-1] + length)
    metadata = Metadata(
        num_actual_tokens=sum(query_lens), max_query_len=max(query_lens),
        query_start_loc=torch.tensor(starts), max_seq_len=17,
        seq_lens=torch.tensor([17, 16]), block_table=torch.tensor([[0, 1], [2, 3]]),
        slot_mapping=torch.tensor([0, 1]),
    )
    return q, cache, metadata


def test_decode_adapter_exercises_paged_api_with_explicit_fallback(monkeypatch):
    monkeypatch.setenv("MXFLASHATTN_ALLOW_FALLBACK", "1")
    q, cache, metadata = make_case()
    output, layout = decode_forward(q, cache, metadata, softmax_scale=64**-0.5)
    assert output.shape == (2, 4 * 64)
    assert layout.query_lens == (1, 1)
    expected = reference_port.attention_kvcache(
        q.view(2, 1, 4, 64), cache[0], cache[1], cache_seqlens=torch.tensor([17, 16]),
        block_table=torch.tensor([[0, 1], [2, 3]]), softmax_scale=64**-0.5)
    torch.testing.assert_close(output, expected.reshape(2, -1))


def test_prefill_is_blocked_instead_of_delegated():
    q, cache, metadata = make_case((2, 1))
    with pytest.raises(DecoderAdapterBlocked, match="single_token_decode"):
        decode_forward(q, cache, metadata, softmax_scale=64**-0.5)


def test_layout_rejects_wrong_cache_rank():
    q, _, metadata = make_case()
    with pytest.raises(DecoderAdapterBlocked, match="kv_cache_shape"):
        inspect_layout(q, torch.empty(2, 4, 16, 64), metadata)


def test_inspect_layout_reads_offsets(monkeypatch):
    q, cache, metadata = make_case()
    layout = inspect_layout(q, cache, metadata)
    assert layout.seq_lens == (17, 16)
    assert layout.query_start_loc == (0, 1, 2)
    assert layout.block_table_shape == (2, 2)
    metadata.num_actual_tokens = 3
    with pytest.raises(DecoderAdapterBlocked, match="query_start_loc"):
        inspect_layout(q, cache, metadata)


def test_cascade_and_fp8_are_blocked():
    q, cache, metadata = make_case()
    metadata.use_cascade = True
    with pytest.raises(DecoderAdapterBlocked, match="cascade"):
        decode_forward(q, cache, metadata, softmax_scale=0.125)
    metadata.use_cascade = False
    with pytest.raises(DecoderAdapterBlocked, match="kv_cache_dtype"):
        decode_forward(q, cache.float(), metadata, softmax_scale=0.125)


@pytest.mark.parametrize("mode", ["MXFLASHATTN_GRAPH_DECODE", "MXFLASHATTN_TRANSPARENT"])
def test_cascade_is_blocked_on_every_path(monkeypatch, mode):
    # A cascade call's pages hold only each request's suffix: decoding them
    # alone would miss the shared prefix.
    monkeypatch.setenv(mode, "1")
    monkeypatch.setattr(decoder_adapter, "flash_attn_with_kvcache",
                        lambda *a, **k: pytest.fail("cascade must not be decoded"))
    q, cache, metadata = make_case()
    metadata.use_cascade = True
    with pytest.raises(DecoderAdapterBlocked, match="cascade"):
        decode_forward(q, cache, metadata, softmax_scale=0.125)
    with pytest.raises(DecoderAdapterBlocked, match="cascade"):
        decoder_adapter.forward_decode(q, cache.view(torch.uint8), metadata,
                                       torch.empty(2, 256, dtype=q.dtype),
                                       softmax_scale=0.125, kv_cache_dtype="fp8")


def test_transparent_path_flattens_capture_seq_lens(monkeypatch):
    monkeypatch.setenv("MXFLASHATTN_TRANSPARENT", "1")
    monkeypatch.setenv("MXFLASHATTN_ALLOW_FALLBACK", "1")
    q, cache, metadata = make_case()
    metadata.seq_lens = metadata.seq_lens.reshape(1, -1)
    seen = {}

    def fake_flash(q, key_cache, value_cache, **kwargs):
        seen["cache_seqlens"] = kwargs["cache_seqlens"]
        seen["block_table"] = kwargs["block_table"]
        return torch.zeros_like(q)

    monkeypatch.setattr(decoder_adapter, "flash_attn_with_kvcache", fake_flash)
    output, layout = decode_forward(q, cache, metadata, softmax_scale=64**-0.5)
    assert output.shape == (2, 4 * 64)
    assert layout is None
    assert seen["cache_seqlens"].shape == (2,)
    assert seen["cache_seqlens"].dtype == torch.int32
    assert seen["block_table"].shape == (2, 2)


def test_graph_path_drops_capture_padding(monkeypatch):
    """Graph capture pads the query to a bucket; only metadata rows are attended."""
    monkeypatch.setenv("MXFLASHATTN_GRAPH_DECODE", "1")
    q, cache, metadata = make_case()
    padded = torch.cat([q, torch.zeros(6, 4, 64, dtype=q.dtype)])
    metadata.max_query_len = 8
    seen = {}

    def fake_flash(q, key_cache, value_cache, **kwargs):
        seen["q"] = q.shape
        return torch.zeros_like(q)

    monkeypatch.setattr(decoder_adapter, "flash_attn_with_kvcache", fake_flash)
    output, layout = decode_forward(padded, cache, metadata, softmax_scale=0.125)
    assert seen["q"] == (2, 1, 4, 64)
    assert output.shape == (2, 256) and layout is None
