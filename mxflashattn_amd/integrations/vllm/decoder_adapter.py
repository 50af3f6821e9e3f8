"""Bridge from vLLM decoder metadata to ``flash_attn_with_kvcache``.

Single-token decode only: the packed vLLM query [tokens, heads, dim] and the
[2, blocks, block_size, kv_heads, dim] cache become the paged API call; prefill,
cascade attention and FP8 caches are rejected with DecoderAdapterBlocked.
Follows integrations/vllm/decoder_adapter.py:31-286 of the reference (same
metadata fields, environment switches and rejection reasons).
"""

from __future__ import annotations

import os
from dataclasses import dataclass
from typing import Any

import torch

from ... import api, native
from ...dispatch import get_last_dispatch_info
from .backend import record_event
from .native_decode import reshape_and_cache_flash

# inspect_layout() reads query_start_loc / seq_lens back to the host (a device
# sync per layer per step); it runs only when MXFLASHATTN_STRICT_LAYOUT=1.
STRICT_LAYOUT = os.getenv("MXFLASHATTN_STRICT_LAYOUT", "0") == "1"

_REQUIRED = (
    "num_actual_tokens", "max_query_len", "query_start_loc", "max_seq_len",
    "seq_lens", "block_table", "scheduler_metadata", "causal", "use_cascade",
)


def _transparent_enabled() -> bool:
    return os.getenv("MXFLASHATTN_TRANSPARENT", "0") == "1"


def flash_attn_with_kvcache(*args, **kwargs):
    """Indirection so tests and hosts can swap the decode call."""
    return api.flash_attn_with_kvcache(*args, **kwargs)


@dataclass(frozen=True, slots=True)
class DecoderLayout:
    num_actual_tokens: int
    batch_size: int
    query_lens: tuple[int, ...]
    max_query_len: int
    seq_lens: tuple[int, ...]
    query_start_loc: tuple[int, ...]
    block_table_shape: tuple[int, int]
    kv_cache_shape: tuple[int, int, int, int, int]
    scheduler_metadata_present: bool


class DecoderAdapterBlocked(RuntimeError):
    """Raised when vLLM metadata is outside the verified adapter contract."""


def _check_shapes(query: torch.Tensor, kv_cache: torch.Tensor, attn_metadata: Any) -> None:
    missing = [name for name in _REQUIRED if not hasattr(attn_metadata, name)]
    if missing:
        raise DecoderAdapterBlocked(f"metadata_missing_fields:{','.join(missing)}")
    if query.ndim != 3:
        raise DecoderAdapterBlocked(f"query_rank:{query.ndim},expected:3")
    if kv_cache.ndim != 5 or kv_cache.shape[0] != 2:
        raise DecoderAdapterBlocked(
            f"kv_cache_shape:{tuple(kv_cache.shape)},expected:[2,blocks,block_size,kv_heads,head_dim]"
        )


def inspect_layout(query: torch.Tensor, kv_cache: torch.Tensor, attn_metadata: Any) -> DecoderLayout:
    """Validate and record the decoder layout, reading offsets back to the host."""
    _check_shapes(query, kv_cache, attn_metadata)
    starts = tuple(int(x) for x in attn_metadata.query_start_loc.detach().cpu().tolist())
    seq_lens = tuple(int(x) for x in attn_metadata.seq_lens.detach().cpu().tolist())
    if (len(starts) != len(seq_lens) + 1 or starts[0] != 0
            or starts[-1] != int(attn_metadata.num_actual_tokens)):
        raise DecoderAdapterBlocked("query_start_loc_does_not_cover_num_actual_tokens")
    block_table = attn_metadata.block_table
    if block_table.ndim != 2 or block_table.shape[0] != len(seq_lens):
        raise DecoderAdapterBlocked("block_table_rows_do_not_match_batch")
    return DecoderLayout(
        num_actual_tokens=int(attn_metadata.num_actual_tokens),
        batch_size=len(seq_lens),
        query_lens=tuple(b - a for a, b in zip(starts, starts[1:])),
        max_query_len=int(attn_metadata.max_query_len),
        seq_lens=seq_lens,
        query_start_loc=starts,
        block_table_shape=(int(block_table.shape[0]), int(block_table.shape[1])),
        kv_cache_shape=tuple(int(x) for x in kv_cache.shape),
        scheduler_metadata_present=attn_metadata.scheduler_metadata is not None,
    )


def fast_layout(query: torch.Tensor, kv_cache: torch.Tensor, attn_metadata: Any) -> DecoderLayout:
    """Layout capture without any device-to-host synchronisation."""
    _check_shapes(query, kv_cache, attn_metadata)
    block_table = attn_metadata.block_table
    if block_table.ndim != 2:
        raise DecoderAdapterBlocked("block_table_rows_do_not_match_batch")
    batch = int(block_table.shape[0])
    max_query_len = int(attn_metadata.max_query_len)
    return DecoderLayout(
        num_actual_tokens=int(attn_metadata.num_actual_tokens),
        batch_size=batch,
        query_lens=tuple([max_query_len] * batch),
        max_query_len=max_query_len,
        seq_lens=(),
        query_start_loc=(),
        block_table_shape=(batch, int(block_table.shape[1])),
        kv_cache_shape=tuple(int(x) for x in kv_cache.shape),
        scheduler_metadata_present=attn_metadata.scheduler_metadata is not None,
    )


def _no_cascade(attn_metadata: Any) -> None:
    # Cascade attention splits a shared prefix out of every request's pages:
    # decoding the per-request pages alone would miss it.
    if bool(getattr(attn_metadata, "use_cascade", False)):
        raise DecoderAdapterBlocked("cascade_attention_not_supported_by_adapter")


def _int32_on(t: torch.Tensor, device: torch.device) -> torch.Tensor:
    # Convert only when needed: an unconditional .to() costs a dispatch per layer.
    if t.device == device and t.dtype == torch.int32:
        return t
    return t.to(device=device, dtype=torch.int32)


def _rows_out(out: torch.Tensor | None, q: torch.Tensor) -> torch.Tensor | None:
    """The first rows of vLLM's output buffer ([tokens, heads*dim] or
    [tokens, heads, dim]) viewed as q's [B, QL, HQ, D], or None when they
    cannot be viewed so (the result is then copied)."""
    if out is None or out.dtype != q.dtype or out.device != q.device:
        return None
    rows = q.shape[0] * q.shape[1]
    if out.shape[0] < rows or out[0].numel() != q.shape[2] * q.shape[3]:
        return None
    try:
        return out[:rows].view(q.shape)
    except RuntimeError:
        return None


def decode_forward(query: torch.Tensor, kv_cache: torch.Tensor, attn_metadata: Any, *,
                   softmax_scale: float, causal: bool = True,
                   out: torch.Tensor | None = None) -> tuple[torch.Tensor, Any]:
    """Run one-token paged decode; returns ([tokens, heads*dim], layout or None).

    vLLM writes the new token into the cache before attention, so k/v are
    omitted and seq_lens describes the populated cache. ``out`` (vLLM's output
    buffer) receives the result in place when its rows can be viewed as the
    query; the returned tensor is then a view of it.
    """
    if os.getenv("MXFLASHATTN_GRAPH_DECODE", "0") == "1":
        _no_cascade(attn_metadata)
        has_padded_decode = (
            attn_metadata.seq_lens.ndim == 1
            and attn_metadata.block_table.ndim == 2
            and attn_metadata.seq_lens.numel() == attn_metadata.block_table.shape[0]
            and attn_metadata.seq_lens.numel() < query.shape[0]
        )
        has_split_decode = (
            int(getattr(attn_metadata, "num_decode_tokens", 0) or 0) > 0
            and int(getattr(attn_metadata, "num_decodes", 0) or 0) > 0
            and getattr(attn_metadata, "decode_seq_lens", None) is not None
            and getattr(attn_metadata, "decode_block_table", None) is not None
        )
        mql = int(getattr(attn_metadata, "max_query_len", 0))
        if mql != 1 and not has_padded_decode and not has_split_decode:
            raise DecoderAdapterBlocked(f"only_single_token_decode_supported:max_query_len={mql}")
        return _decode_forward_graph(query, kv_cache, attn_metadata,
                                     softmax_scale=softmax_scale, causal=causal, out=out)
    if _transparent_enabled():
        _no_cascade(attn_metadata)
        if int(attn_metadata.max_query_len) != 1:
            raise DecoderAdapterBlocked(
                f"only_single_token_decode_supported:max_query_len={int(attn_metadata.max_query_len)}"
            )
        key_cache, value_cache = kv_cache.unbind(0)
        n = int(attn_metadata.num_actual_tokens)
        q = query[:n].reshape(n, 1, query.shape[1], query.shape[2])
        # Capture metadata may expose seq_lens as [1, batch]; flatten it on the device.
        cache_seqlens = _int32_on(attn_metadata.seq_lens.reshape(-1), query.device)
        block_table = _int32_on(attn_metadata.block_table, query.device)
        result = flash_attn_with_kvcache(q, key_cache, value_cache, cache_seqlens=cache_seqlens,
                                         block_table=block_table, softmax_scale=softmax_scale,
                                         causal=causal, **_out_kw(out, q))
        return result.reshape(n, -1), None
    layout = (inspect_layout(query, kv_cache, attn_metadata) if STRICT_LAYOUT
              else fast_layout(query, kv_cache, attn_metadata))
    result = _paged_decode(query, kv_cache, attn_metadata, layout.batch_size,
                           layout.num_actual_tokens, layout.max_query_len,
                           softmax_scale=softmax_scale, causal=causal, out=out)
    return result, layout


def _paged_decode(query: torch.Tensor, kv_cache: torch.Tensor, attn_metadata: Any, batch: int,
                  num_actual_tokens: int, max_query_len: int, *, softmax_scale: float,
                  causal: bool, out: torch.Tensor | None) -> torch.Tensor:
    """The checks and the call of decode_forward's default mode, once the
    layout's batch, token count and query length are known; returns
    [tokens, heads*dim]."""
    if not bool(attn_metadata.causal) and causal:
        raise DecoderAdapterBlocked("metadata_causal_flag_is_false")
    _no_cascade(attn_metadata)
    if max_query_len != 1:
        raise DecoderAdapterBlocked(
            f"only_single_token_decode_supported:max_query_len={max_query_len}"
        )
    if kv_cache.dtype not in (torch.float16, torch.bfloat16):
        raise DecoderAdapterBlocked(f"kv_cache_dtype_not_supported:{kv_cache.dtype}")
    if query.shape[1] % kv_cache.shape[3]:
        raise DecoderAdapterBlocked("query_and_kv_head_counts_are_not_gqa_compatible")
    q = query[:num_actual_tokens].reshape(batch, 1, query.shape[1], query.shape[2])
    result = flash_attn_with_kvcache(
        q, kv_cache[0], kv_cache[1],
        cache_seqlens=_int32_on(attn_metadata.seq_lens, query.device),
        block_table=_int32_on(attn_metadata.block_table, query.device),
        softmax_scale=softmax_scale, causal=causal, **_out_kw(out, q),
    )
    return result.reshape(num_actual_tokens, -1)


def _out_kw(out: torch.Tensor | None, q: torch.Tensor) -> dict:
    view = _rows_out(out, q)
    return {} if view is None else {"out": view}


def _decode_forward_graph(query: torch.Tensor, kv_cache: torch.Tensor, attn_metadata: Any, *,
                          softmax_scale: float, causal: bool = True,
                          out: torch.Tensor | None = None):
    """Static-shape (graph) decode: prefer the split decode metadata when present,
    else one query row per metadata row (capture padding stays out of the call)."""
    key_cache, value_cache = kv_cache.unbind(0)
    decode_n = int(getattr(attn_metadata, "num_decode_tokens", 0) or 0)
    decode_batch = int(getattr(attn_metadata, "num_decodes", 0) or 0)
    decode_seq = getattr(attn_metadata, "decode_seq_lens", None)
    decode_bt = getattr(attn_metadata, "decode_block_table", None)
    if decode_n > 0 and decode_batch > 0 and decode_seq is not None and decode_bt is not None:
        if decode_n % decode_batch:
            raise DecoderAdapterBlocked("decode_tokens_not_divisible_by_num_decodes")
        q = query[:decode_n].reshape(decode_batch, decode_n // decode_batch, query.shape[1],
                                     query.shape[2])
        cache_seqlens = decode_seq.reshape(-1)
        block_table = decode_bt
        batch = decode_batch
    else:
        raw_seq = attn_metadata.seq_lens.reshape(-1)
        batch = int(raw_seq.numel()) if raw_seq.numel() < query.shape[0] else query.shape[0]
        q = query[:batch].reshape(batch, 1, query.shape[1], query.shape[2])
        cache_seqlens = raw_seq
        block_table = attn_metadata.block_table
    cache_seqlens = _int32_on(cache_seqlens, query.device)
    block_table = _int32_on(block_table, query.device)
    if cache_seqlens.numel() != batch or block_table.shape[0] != batch:
        raise DecoderAdapterBlocked("decode_metadata_batch_mismatch")
    result = flash_attn_with_kvcache(
        q, key_cache, value_cache, cache_seqlens=cache_seqlens.contiguous(),
        block_table=block_table.contiguous(), softmax_scale=softmax_scale, causal=causal,
        **_out_kw(out, q),
    )
    return result.reshape(q.shape[0] * q.shape[1], -1), None


def _native_decode(query: torch.Tensor, kv_cache: torch.Tensor, attn_metadata: Any,
                   output: torch.Tensor, softmax_scale: float, k_scale: Any, v_scale: Any,
                   fp8: bool, window_left: int, sinks: Any = None,
                   softcap: float = 0.0, alibi_slopes: Any = None) -> torch.Tensor:
    """One-token decode straight on the HIP kernels, for what the public API
    (like the reference's) does not take: an fp8 (e4m3fn) cache, a sliding
    window, attention sinks, logit soft-capping, ALiBi."""
    _no_cascade(attn_metadata)
    if int(attn_metadata.max_query_len) != 1:
        raise DecoderAdapterBlocked(
            f"only_single_token_decode_supported:max_query_len={int(attn_metadata.max_query_len)}")
    if not output.is_contiguous():
        raise DecoderAdapterBlocked("native_decode_needs_a_contiguous_output")
    caches = kv_cache.view(native.FP8_DTYPE) if fp8 else kv_cache
    key_cache, value_cache = caches.unbind(0)
    n = int(attn_metadata.num_actual_tokens)
    q = query[:n].reshape(n, 1, query.shape[1], query.shape[2])
    target = output[:n].view(n, 1, query.shape[1], query.shape[2])
    scales = dict(k_scale=k_scale, v_scale=v_scale) if fp8 else {}
    native.paged_decode_split(q, key_cache, value_cache,
                              _int32_on(attn_metadata.block_table, query.device),
                              _int32_on(attn_metadata.seq_lens.reshape(-1), query.device),
                              softmax_scale, out=target, window_left=window_left,
                              sinks=sinks, softcap=softcap, alibi_slopes=alibi_slopes,
                              **scales)
    event = {"path": "mi355x_split_decode", "operation": "paged_decode_split",
             "fallback": "false"}
    if fp8:
        event["kv_cache_dtype"] = "fp8_e4m3"
    if window_left >= 0:
        event["window_left"] = str(window_left)
    if sinks is not None:
        event["sinks"] = "true"
    if softcap > 0:
        event["softcap"] = str(softcap)
    if alibi_slopes is not None:
        event["alibi"] = "true"
    record_event(event)
    return output


def forward_decode(query: torch.Tensor, kv_cache: torch.Tensor, attn_metadata: Any,
                   output: torch.Tensor, *, softmax_scale: float, kv_cache_dtype: str = "auto",
                   k_scale: Any = None, v_scale: Any = None,
                   window_left: int = -1, sinks: Any = None,
                   softcap: float = 0.0, alibi_slopes: Any = None) -> torch.Tensor:
    """The decode body of the backend's ``forward``: one-token paged decode into
    vLLM's output buffer, with the dispatch event the reference plugin records
    (integrations/vllm/vllm_plugin.py:297-299,399-431). Raises
    DecoderAdapterBlocked for calls outside the adapter contract (prefill,
    cascade), which the backend hands to vLLM. kv_cache_dtype "fp8"/"fp8_e4m3"
    (cache stored as e4m3fn or its uint8 codes) decodes with the layer's
    per-tensor k_scale / v_scale, window_left >= 0 with the layer's sliding
    window (the query at position i sees keys >= i - window_left), and sinks
    (float32 [HQ]) with the layer's attention sinks, softcap > 0 with its logit
    soft-capping, alibi_slopes (float32 [HQ]) with its ALiBi slopes; the
    reference has none of these."""
    fp8 = kv_cache_dtype in ("fp8", "fp8_e4m3")
    if (fp8 or window_left >= 0 or sinks is not None or softcap > 0
            or alibi_slopes is not None):
        return _native_decode(query, kv_cache, attn_metadata, output, softmax_scale, k_scale,
                              v_scale, fp8, window_left, sinks, softcap, alibi_slopes)
    causal = bool(attn_metadata.causal)
    if (STRICT_LAYOUT or os.getenv("MXFLASHATTN_GRAPH_DECODE", "0") == "1"
            or _transparent_enabled()):
        result, _ = decode_forward(query, kv_cache, attn_metadata, softmax_scale=softmax_scale,
                                   causal=causal, out=output)
    else:
        # decode_forward's default mode with fast_layout's checks but without
        # building the layout record, which this caller does not use.
        _check_shapes(query, kv_cache, attn_metadata)
        block_table = attn_metadata.block_table
        if block_table.ndim != 2:
            raise DecoderAdapterBlocked("block_table_rows_do_not_match_batch")
        result = _paged_decode(query, kv_cache, attn_metadata, int(block_table.shape[0]),
                               int(attn_metadata.num_actual_tokens),
                               int(attn_metadata.max_query_len), softmax_scale=softmax_scale,
                               causal=causal, out=output)
    info = get_last_dispatch_info()
    if info is None:
        raise RuntimeError("MXFlashAttn decoder returned without dispatch evidence")
    record_event({"path": info.backend, "operation": info.operation,
                  "fallback": "false" if info.fallback_reason is None else "true"})
    target = output[: result.shape[0]]
    if target.numel() != result.numel():
        raise RuntimeError(
            f"MXFlashAttn decoder output size mismatch: target={tuple(target.shape)} "
            f"result={tuple(result.shape)}")
    if result.data_ptr() != target.data_ptr():  # not written in place
        target.copy_(result.reshape_as(target))
    return output


def kv_cache_update(key: torch.Tensor, value: torch.Tensor, kv_cache: torch.Tensor,
                    slot_mapping: torch.Tensor, kv_cache_dtype: str = "auto",
                    k_scale: Any = None, v_scale: Any = None) -> None:
    """The backend's ``do_kv_cache_update``: new K/V rows of [tokens, HKV, HD]
    into the [2, blocks, PS, HKV, HD] cache at slot_mapping (vllm_plugin.py:507-511);
    an fp8 cache stores them quantised with the layer's k_scale / v_scale."""
    key_cache, value_cache = kv_cache.unbind(0)
    reshape_and_cache_flash(key, value, key_cache, value_cache, slot_mapping, kv_cache_dtype,
                            k_scale, v_scale)
