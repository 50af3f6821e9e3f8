"""vLLM attention backend classes (needs vLLM; import fails cleanly without it).

Structure of integrations/vllm/vllm_plugin.py:351-511 of the reference:
``MXFlashAttnImpl`` keeps vLLM's own FlashAttention metadata split and output
write-back and swaps only the attention calls. With
MXFLASHATTN_GRAPH_OFFICIAL_SPLIT=1 the implementation's module-level
``flash_attn_with_kvcache`` is replaced by ``native_decode.mx_kvcache_compat``
for the duration of the forward call (restored in ``finally``); an "invalid
argument" failure is retried once with the untouched functions. The reference
also swaps ``flash_attn_varlen_func`` there; prefill is not on this path, so it
stays vLLM's. Encoder layers (``attn_type`` "encoder" / "encoder_only", which
the reference sends to its dense API and on to the vendor kernel) run vLLM's
own forward, and so do sliding-window, attention-sink, soft-capped and ALiBi
layers unless the wider contract is on (then the kernel applies the window, the
sinks, the cap and the slopes); the reference's forward
sends all of them to its decoder regardless. Otherwise the forward runs ``decode_forward`` (public
API) and falls back to vLLM for prefill. The KV-cache update uses the HIP append kernel
(``reshape_and_cache_flash``).
Classes live at module scope because vLLM resolves the backend by import path
in its worker processes.
"""

from __future__ import annotations

import os

import torch
from vllm.v1.attention.backends.flash_attn import (  # noqa: F401  (requires vLLM)
    FlashAttentionBackend,
    FlashAttentionImpl,
)

from . import native_decode
from .backend import record_event
from .decoder_adapter import DecoderAdapterBlocked, forward_decode, kv_cache_update


def _forward_official_split(impl, layer, query, key, value, kv_cache, metadata, output,
                            output_scale, output_block_scale):
    fn = FlashAttentionImpl.forward
    glb = fn.__globals__
    had_kv = "flash_attn_with_kvcache" in glb
    old_kv = glb.get("flash_attn_with_kvcache")
    native_decode.official_kvcache = old_kv
    glb["flash_attn_with_kvcache"] = native_decode.mx_kvcache_compat
    event = {"path": "vendor_direct", "operation": "official_split_mx", "fallback": "false"}
    try:
        try:
            result = super(MXFlashAttnImpl, impl).forward(
                layer, query, key, value, kv_cache, metadata, output, output_scale,
                output_block_scale)
        except Exception as exc:
            if "invalid argument" not in str(exc).lower():
                raise
            glb["flash_attn_with_kvcache"] = old_kv
            result = super(MXFlashAttnImpl, impl).forward(
                layer, query, key, value, kv_cache, metadata, output, output_scale,
                output_block_scale)
            event = {"path": "vendor_direct",
                     "operation": "official_split_invalid_argument_fallback",
                     "fallback": "true", "fallback_reason": "official_split_invalid_argument"}
    finally:
        if had_kv:
            glb["flash_attn_with_kvcache"] = old_kv
        else:
            glb.pop("flash_attn_with_kvcache", None)
        native_decode.official_kvcache = None
    record_event(event)
    return result


def _layer_window(impl) -> int:
    """The layer's sliding window as the kernel's window_left (-1: none);
    vLLM stores it as FlashAttention's (window - 1, 0)."""
    mapped = native_decode.window_for_kernel(getattr(impl, "sliding_window", None), True, 1)
    return -1 if mapped is None else mapped[0]


def _layer_vector(impl, name: str, query):
    """A per-query-head vector of the layer (vLLM's attention sinks, ALiBi
    slopes) as the kernel's float32 [HQ] on the query's GPU: (vector, usable).
    The slopes are fixed at construction and may live on the host, so a device
    copy of them is kept on the layer; sinks are a weight, taken where they are."""
    value = getattr(impl, name, None)
    if value is None:
        return None, True
    if (name == "alibi_slopes" and isinstance(value, torch.Tensor)
            and isinstance(query, torch.Tensor) and value.device != query.device):
        cached = getattr(impl, "_mxfa_alibi_slopes", None)
        if cached is None or cached[0] is not value or cached[1].device != query.device:
            cached = (value, value.to(device=query.device, dtype=torch.float32).contiguous())
            impl._mxfa_alibi_slopes = cached
        value = cached[1]
    vector = native_decode._sinks_for_kernel(value, query)
    return vector, vector is not None


def _layer_option(impl) -> str | None:
    """An option of the layer that the decode kernel does not compute (vLLM's
    FlashAttentionImpl applies them in its own forward), or None. Sliding
    windows, attention sinks, soft-capping and ALiBi are computed under the
    wider contract."""
    if getattr(impl, "alibi_slopes", None) is not None and not native_decode.wide_contract():
        return "alibi"
    window = getattr(impl, "sliding_window", None)
    if (window is not None and not native_decode._no_window(window, True, 1)
            and not native_decode.wide_contract()):
        return "window"
    if getattr(impl, "logits_soft_cap", None) and not native_decode.wide_contract():
        return "softcap"
    if getattr(impl, "sinks", None) is not None and not native_decode.wide_contract():
        return "attention_sinks"
    return None


def _decodes_here(kv_dtype: str) -> bool:
    """Whether decode over this cache format runs on the HIP kernels: 16-bit
    caches always, e4m3fn caches under the wider contract."""
    if kv_dtype in native_decode.SIXTEEN_BIT_KV_DTYPES:
        return True
    return kv_dtype in native_decode.FP8_KV_DTYPES and native_decode.wide_contract()


class MXFlashAttnImpl(FlashAttentionImpl):
    def forward(self, layer, query, key, value, kv_cache, attn_metadata, output=None,
                output_scale=None, output_block_scale=None):
        if attn_metadata is None:
            if output is None:
                raise ValueError("vLLM must provide an output buffer for profiling")
            return output.fill_(0)
        if os.getenv("MXFLASHATTN_SPLIT_PURE", "0") == "1":
            return super().forward(layer, query, key, value, kv_cache, attn_metadata, output,
                                   output_scale, output_block_scale)
        if os.getenv("MXFLASHATTN_GRAPH_OFFICIAL_SPLIT", "0") == "1":
            return _forward_official_split(self, layer, query, key, value, kv_cache,
                                           attn_metadata, output, output_scale,
                                           output_block_scale)
        if output is None:
            raise ValueError("vLLM must provide an output buffer")
        # vLLM's AttentionType values compare equal to these strings.
        if getattr(self, "attn_type", "decoder") in ("encoder", "encoder_only"):
            result = super().forward(layer, query, key, value, kv_cache, attn_metadata, output,
                                     output_scale, output_block_scale)
            record_event({"path": "vendor_direct", "operation": "encoder", "fallback": "false"})
            return result
        option = _layer_option(self)
        sinks, alibi = (None, True), (None, True)
        if option is None:
            sinks = _layer_vector(self, "sinks", query)
            alibi = _layer_vector(self, "alibi_slopes", query)
            if not sinks[1]:
                option = "attention_sinks"  # not one float per query head on this GPU
            elif not alibi[1]:
                option = "alibi"
        if option is None and (output_scale is not None or output_block_scale is not None):
            option = "output_quantization"  # vLLM's forward decides (it raises for it)
        if option is not None:
            # Sliding windows, ALiBi, soft-capping, sinks, a quantised output:
            # vLLM's forward.
            result = super().forward(layer, query, key, value, kv_cache, attn_metadata, output,
                                     output_scale, output_block_scale)
            record_event({"path": "vendor_direct", "operation": "layer_option",
                          "fallback": "true", "fallback_reason": option})
            return result
        kv_dtype = getattr(self, "kv_cache_dtype", "auto") or "auto"
        if not _decodes_here(kv_dtype):
            # fp8 caches are vLLM's unless the wider contract is on; e5m2 and
            # other formats always are.
            return super().forward(layer, query, key, value, kv_cache, attn_metadata, output,
                                   output_scale, output_block_scale)
        try:
            return forward_decode(query, kv_cache, attn_metadata, output,
                                  softmax_scale=self.scale, kv_cache_dtype=kv_dtype,
                                  k_scale=getattr(layer, "_k_scale", None),
                                  v_scale=getattr(layer, "_v_scale", None),
                                  window_left=_layer_window(self),
                                  sinks=sinks[0], alibi_slopes=alibi[0],
                                  softcap=float(getattr(self, "logits_soft_cap", 0.0) or 0.0))
        except DecoderAdapterBlocked as exc:
            record_event({"path": "vendor_prefill_or_blocked", "reason": str(exc)})
            if "single_token_decode" in str(exc):
                return super().forward(layer, query, key, value, kv_cache, attn_metadata,
                                       output, output_scale, output_block_scale)
            raise

    def do_kv_cache_update(self, layer, key, value, kv_cache, slot_mapping):
        kv_dtype = getattr(self, "kv_cache_dtype", "auto") or "auto"
        if kv_dtype not in native_decode.SIXTEEN_BIT_KV_DTYPES + native_decode.FP8_KV_DTYPES:
            return super().do_kv_cache_update(layer, key, value, kv_cache, slot_mapping)
        kv_cache_update(key, value, kv_cache, slot_mapping, kv_dtype,
                        getattr(layer, "_k_scale", None), getattr(layer, "_v_scale", None))


class MXFlashAttnBackend(FlashAttentionBackend):
    @staticmethod
    def get_name() -> str:
        # vLLM indexes its backend enum by this name.
        return "FLASH_ATTN"

    @staticmethod
    def get_impl_cls():
        return MXFlashAttnImpl
