"""Decode routing inside vLLM's attention call, independent of vLLM itself.

``try_native_decode`` replaces the reference's ``_try_native_decode``
(integrations/vllm/vllm_plugin.py:199-317): behind MXFA_NATIVE_DECODE=1 it
sends single-token paged decode straight to the HIP split-KV kernels.
Unsupported calls are handed back (return None) by explicit guards, with no
exception on the hot path: no block table or lengths, alibi, a positive
window, a dtype other than fp16/bf16 or different from the cache's, q_len > 1,
head dim outside {64, 128}, GQA ratio outside {2, 4, 8}, or a page size that is
not a power of two. The caller then runs the original implementation.

MXFA_WIDE_CONTRACT=1 widens the guards to what the kernels take: head dim 256,
1..16 query heads per kv head, fp8 (e4m3fn) caches with per-tensor
k_descale / v_descale (a scalar, or a tensor expanded from one), and q of
[B, QL, HQ, D] (draft-token verification, with the call's causal flag; QL x
GQ <= 16, or <= 64 for a causal query, which runs as up to four token chunks). It also takes a sliding window, soft-capping and ALiBi slopes of
one per query head ([HQ]; a per-sequence [B, HQ] table is handed back).

``mx_kvcache_compat`` replaces ``_mx_kvcache_compat`` (:319-349): it drops
vLLM-only keyword arguments, tries the native route, else the original vendor
function, else the public API. ``reshape_and_cache_flash`` is the cache write
with vLLM's signature, on the HIP append kernel.
"""

from __future__ import annotations

import os
from typing import Any, Callable

import torch

from ... import api, native
from .backend import record_event

# Set by the vLLM plugin around a forward call: the vendor function the
# compat wrapper hands unsupported calls back to.
official_kvcache: Callable[..., Any] | None = None

# vLLM kv_cache_dtype values whose caches the HIP kernels hold: the model's
# own 16-bit type ("auto" or named), and OCP e4m3fn with per-tensor scales.
SIXTEEN_BIT_KV_DTYPES = ("auto", None, "bfloat16", "float16", "half")
FP8_KV_DTYPES = ("fp8", "fp8_e4m3")

_VLLM_ONLY_KWARGS = ("s_aux", "return_softmax_lse", "scheduler_metadata", "fa_version",
                     "q_descale", "k_descale", "v_descale")


def wide_contract() -> bool:
    return os.getenv("MXFA_WIDE_CONTRACT", "0") == "1"


def _per_tensor(scale: Any) -> bool:
    """None, a float, or a float32 tensor holding one value (numel 1 or all
    strides 0, as vLLM's layer scale expanded to [B, HKV])."""
    if scale is None or isinstance(scale, (int, float)):
        return True
    return (isinstance(scale, torch.Tensor) and scale.dtype == torch.float32
            and (scale.numel() == 1 or all(st == 0 for st in scale.stride())))


def _no_window(window: Any, causal: bool, ql: int) -> bool:
    """True when window_size masks nothing for this call. FlashAttention's
    (left, right): -1 is unbounded. Any left bound >= 0 hides keys (0 keeps
    only the query's own position); a right bound matters only when a query
    token could see keys after it (several tokens, not causal). The
    reference's guard rejects positive sizes only (vllm_plugin.py:236-247)."""
    if window is None:
        return True
    try:
        left, right = (window, -1) if not isinstance(window, (tuple, list)) else window
        left, right = int(left), int(right)
    except (TypeError, ValueError):
        return False
    return left < 0 and (right < 0 or causal or ql == 1)


def window_for_kernel(window: Any, causal: bool, ql: int) -> tuple[int, bool] | None:
    """FlashAttention's window_size as the kernel's (window_left, causal), or
    None when the kernel cannot express it. -1 is unbounded on either side; a
    right bound of 0 is the causal mask; a positive right bound matters only
    for several non-causal query tokens, which the kernel has no bound for."""
    if window is None:
        return -1, causal
    try:
        left, right = (window, -1) if not isinstance(window, (tuple, list)) else window
        left, right = int(left), int(right)
    except (TypeError, ValueError):
        return None
    if right > 0 and not causal and ql > 1:
        return None
    return (left if left >= 0 else -1), causal or (right == 0 and ql > 1)


def _guard(args: tuple, kwargs: dict, wide: bool = False,
           descales: tuple = (None, None)) -> tuple[str | None, tuple]:
    """(reason, (q, k_cache, v_cache, block_table, seqlens, window_left, causal,
    softcap, alibi_slopes)); reason None = take it. Sliding windows, soft-capping
    and per-head ALiBi slopes are taken under the wider contract."""
    q = args[0] if args else kwargs.get("q")
    if q is None or q.dim() not in (3, 4):
        return "query_rank", ()
    bt = kwargs.get("block_table")
    sl = kwargs.get("cache_seqlens")
    if bt is None or sl is None or sl.shape[0] != q.shape[0]:
        return "block_table_or_seqlens", ()
    alibi = kwargs.get("alibi_slopes")
    if alibi is not None:
        alibi = _sinks_for_kernel(alibi, q) if wide else None
        if alibi is None:
            return "alibi", ()
    ql = q.shape[1] if q.dim() == 4 else 1
    causal = bool(kwargs.get("causal", False))
    window = kwargs.get("window_size")
    if wide:
        mapped = window_for_kernel(window, causal, ql)
        if mapped is None:
            return "window", ()
        window_left, causal = mapped
    elif not _no_window(window, causal, ql):
        return "window", ()
    else:
        window_left = -1
    try:
        softcap = float(kwargs.get("softcap") or 0.0)
    except (TypeError, ValueError):
        return "softcap", ()
    if softcap != 0.0 and not (wide and 0.0 < softcap < float("inf")):
        return "softcap", ()
    k_cache = kwargs.get("k_cache", args[1] if len(args) > 1 else None)
    v_cache = kwargs.get("v_cache", args[2] if len(args) > 2 else None)
    if k_cache is None or v_cache is None:
        return "caches", ()
    fp8 = wide and k_cache.dtype == native.FP8_DTYPE and v_cache.dtype == k_cache.dtype
    if q.dtype not in native.DTYPE_CODES or (k_cache.dtype != q.dtype and not fp8):
        return "dtype", ()
    if fp8 and not all(_per_tensor(d) for d in descales):
        return "descale_not_per_tensor", ()
    if q.dim() == 4 and q.shape[1] != 1 and not wide:
        return "query_length", ()
    if k_cache.dim() != 4 or v_cache.shape != k_cache.shape:
        return "cache_rank", ()
    hd, hq, hkv = q.shape[-1], q.shape[-2], k_cache.shape[2]
    head_dims = native.KERNEL_HEAD_DIMS if wide else native.SUPPORTED_HEAD_DIMS
    gqa = native.KERNEL_GQA if wide else native.SUPPORTED_GQA
    if hd not in head_dims or k_cache.shape[3] != hd:
        return "head_dim", ()
    if hkv <= 0 or hq % hkv or hq // hkv not in gqa:
        return "gqa_ratio", ()
    columns = native.CHUNKED_COLUMNS if causal else native.KERNEL_COLUMNS
    if q.dim() == 4 and q.shape[1] * (hq // hkv) > columns:
        return "query_length", ()  # causal queries run as up to four token chunks
    ps = k_cache.shape[1]
    if ps <= 0 or ps & (ps - 1) or ps > 4096:
        return "page_size", ()
    if q.device.type != "cuda":
        return "device", ()
    return None, (q, k_cache, v_cache, bt, sl, window_left, causal, softcap, alibi)


def try_native_decode(args: tuple, kwargs: dict, k_descale: Any = None,
                      v_descale: Any = None, sinks: Any = None) -> torch.Tensor | None:
    """HIP decode of a vLLM flash_attn_with_kvcache call, or None to hand it back."""
    if os.getenv("MXFA_NATIVE_DECODE", "0") != "1":
        return None
    reason, picked = _guard(args, kwargs, wide_contract(), (k_descale, v_descale))
    if reason is not None:
        record_event({"path": "native_decode", "fallback": "true",
                      "fallback_reason": f"guard:{reason}"})
        return None
    try:
        return _native_decode(picked, kwargs, k_descale, v_descale, sinks)
    except native.NativeLibraryError:
        raise  # a missing or stale build is a deployment error, not a shape to hand back
    except Exception as exc:  # as vllm_plugin.py:314-317: never take the model down
        record_event({"path": "native_decode", "fallback": "true",
                      "fallback_reason": repr(exc)})
        return None


def _native_decode(picked: tuple, kwargs: dict, k_descale: Any, v_descale: Any,
                   sinks: Any = None) -> torch.Tensor:
    q, k_cache, v_cache, bt, sl, window_left, causal, softcap, alibi = picked
    hq, hd = q.shape[-2], q.shape[-1]
    # An explicit 0.0 is a scale (uniform weights), not "use the default".
    scale = kwargs.get("softmax_scale")
    scale = hd ** -0.5 if scale is None else float(scale)
    # vLLM passes q as [T, HQ, D] or [B, 1, HQ, D], possibly a strided slice of
    # the fused QKV buffer: the kernel takes the strides as they are.
    q4 = q.reshape(q.shape[0], 1, hq, hd) if q.dim() == 3 else q
    provided = kwargs.get("out")
    out = None
    if provided is not None and provided.numel() == q4.numel() and provided.dtype == q.dtype:
        view = provided.view(q4.shape) if provided.is_contiguous() else None
        if view is not None:
            out = view
    ns = native.default_num_splits(q4, k_cache, bt)
    scales = {}
    if k_cache.dtype == native.FP8_DTYPE:
        scales = {"k_scale": k_descale, "v_scale": v_descale}
    result = native.paged_decode_split(q4, k_cache, v_cache, bt, sl, scale, out=out,
                                       num_splits=ns, causal=causal, window_left=window_left,
                                       sinks=sinks, softcap=softcap, alibi_slopes=alibi,
                                       **scales)
    if provided is not None and out is None:
        provided.copy_(result.reshape_as(provided))
        result = provided
    elif provided is not None:
        result = provided
    else:
        result = result.reshape(q.shape)
    record_event({"path": "mi355x_split_decode", "operation": "paged_decode_split",
                  "fallback": "false", "np": str(ns)})
    return result


def _sinks_for_kernel(s_aux: Any, q: Any) -> torch.Tensor | None:
    """A per-query-head vector (vLLM's s_aux, FlashAttention's alibi_slopes)
    as the kernel takes it (float32 [HQ] on q's GPU), or None when it is not one."""
    if not (isinstance(s_aux, torch.Tensor) and isinstance(q, torch.Tensor)):
        return None
    if s_aux.dim() != 1 or s_aux.shape[0] != q.shape[-2] or s_aux.device != q.device:
        return None
    return s_aux.to(torch.float32).contiguous()


def mx_kvcache_compat(*args, **kwargs):
    """Stand-in for vLLM's flash_attn_with_kvcache inside its attention forward.

    A call that asks for the log-sum-exp is never taken, nor one with attention
    sinks (``s_aux``) unless the wider contract is on (then they are the
    kernel's per-head sinks). A call
    that is not taken goes back to vLLM's own function with every keyword vLLM
    passed. The reference (vllm_plugin.py:335-339) strips the vLLM-only
    keywords for every call, because its vendor wheel does not accept them;
    vLLM's function on ROCm does, and stripping ``s_aux`` there would drop the
    sinks silently. Only the fallback to this package's public API, which has
    no such parameters, goes without them."""
    given = {name: kwargs[name] for name in _VLLM_ONLY_KWARGS if name in kwargs}
    popped = {name: kwargs.pop(name, None) for name in _VLLM_ONLY_KWARGS}
    declined, sinks = None, None
    if popped["return_softmax_lse"]:
        declined = "softmax_lse"
    elif popped["s_aux"] is not None:
        q = args[0] if args else kwargs.get("q")
        sinks = _sinks_for_kernel(popped["s_aux"], q) if wide_contract() else None
        if sinks is None:
            declined = "attention_sinks"
    if declined is None:
        result = try_native_decode(args, kwargs, popped["k_descale"], popped["v_descale"],
                                   sinks=sinks)
        if result is not None:
            return result
    elif os.getenv("MXFA_NATIVE_DECODE", "0") == "1":
        record_event({"path": "native_decode", "fallback": "true",
                      "fallback_reason": f"guard:{declined}"})
    # Shapes the public API rejects must reach the original implementation
    # instead of raising inside vLLM.
    if official_kvcache is not None:
        return official_kvcache(*args, **kwargs, **given)
    if popped["s_aux"] is not None:
        raise NotImplementedError("attention sinks (s_aux) are not supported by the "
                                  "MXFlashAttn API; call vLLM's flash_attn_with_kvcache")
    if popped["return_softmax_lse"]:
        kwargs["return_softmax_lse"] = True  # the API raises its own error for it
    k_cache = kwargs.get("k_cache", args[1] if len(args) > 1 else None)
    if isinstance(k_cache, torch.Tensor) and k_cache.dtype == native.FP8_DTYPE:
        # An fp8 cache is meaningless without its scales: give them back.
        for name in ("q_descale", "k_descale", "v_descale"):
            if popped[name] is not None:
                kwargs[name] = popped[name]
    return api.flash_attn_with_kvcache(*args, **kwargs)


def reshape_and_cache_flash(key: torch.Tensor, value: torch.Tensor, key_cache: torch.Tensor,
                            value_cache: torch.Tensor, slot_mapping: torch.Tensor,
                            kv_cache_dtype: str = "auto", k_scale: Any = None,
                            v_scale: Any = None) -> None:
    """vLLM cache write (slot t -> page slot // PS, row slot % PS; slot < 0 skipped).

    kv_cache_dtype "fp8" / "fp8_e4m3": the caches hold e4m3fn (vLLM allocates
    them as uint8) and each row is stored as e4m3fn(x / scale) with the layer's
    per-tensor k_scale / v_scale."""
    n = slot_mapping.shape[0]
    if kv_cache_dtype in ("fp8", "fp8_e4m3"):
        if key_cache.dtype == torch.uint8:
            key_cache, value_cache = (key_cache.view(native.FP8_DTYPE),
                                      value_cache.view(native.FP8_DTYPE))
        if key_cache.dtype != native.FP8_DTYPE:
            raise ValueError(f"kv_cache_dtype {kv_cache_dtype!r} needs uint8/e4m3fn caches")
        native.reshape_and_cache(key[:n], value[:n], key_cache, value_cache, slot_mapping,
                                 k_scale=k_scale, v_scale=v_scale)
        return
    if kv_cache_dtype not in SIXTEEN_BIT_KV_DTYPES:
        raise NotImplementedError(f"kv_cache_dtype {kv_cache_dtype!r} is not supported")
    native.reshape_and_cache(key[:n], value[:n], key_cache, value_cache, slot_mapping)
