"""Backend chain with recorded dispatch evidence.

Order for every public operation:

  1. ``mi355x_split_decode``  the HIP split-KV paged decode of this package, for
     single-token decode on an accelerator tensor of a supported shape
     (HD in {64,128}, GQA in {2,4,8}, fp16/bf16, power-of-two page size).
     When the shape qualifies but the HIP library is missing or a launch fails,
     the error propagates: there is no silent fallback from a qualifying call.
  2. ``vendor_direct``        a MetaX ``flash_attn`` wheel (never present on ROCm;
     kept so the chain behaves like mxflashattn/dispatch.py:40-62,114-125).
  3. ``mxmac_aten_correctness`` an ``mxflashattn_amd._C`` ATen extension when one
     is importable (none is built here; the slot tolerates its absence,
     mxflashattn/dispatch.py:127-151).
  4. ``reference``            the PyTorch path, only with
     MXFLASHATTN_ALLOW_FALLBACK=1, with a RuntimeWarning
     (mxflashattn/dispatch.py:153-170).

``DispatchInfo`` of the last call is kept per thread (mxflashattn/dispatch.py:19-30).
"""

from __future__ import annotations

import importlib
import importlib.metadata
import os
import threading
import warnings
from dataclasses import dataclass
from functools import lru_cache
from typing import Any, Callable

import torch

BACKEND_MI355X = "mi355x_split_decode"
BACKEND_VENDOR = "vendor_direct"
BACKEND_ATEN = "mxmac_aten_correctness"
BACKEND_REFERENCE = "reference"


class BackendUnavailableError(RuntimeError):
    """Raised when native execution is unavailable and fallback was not enabled."""


@dataclass(frozen=True)
class DispatchInfo:
    backend: str
    operation: str
    fallback_reason: str | None = None


_state = threading.local()


def get_last_dispatch_info() -> DispatchInfo | None:
    return getattr(_state, "dispatch_info", None)


def _record(info: DispatchInfo) -> None:
    _state.dispatch_info = info


# The public API's fast path records its (shared, immutable) DispatchInfo here.
record_dispatch = _record


def _native_extension() -> Any | None:
    try:
        return importlib.import_module("mxflashattn_amd._C")
    except (ImportError, OSError):
        return None


@lru_cache(maxsize=1)
def _metax_flash_attn_module() -> Any | None:
    try:
        module = importlib.import_module("flash_attn")
    except (ImportError, OSError):
        return None
    try:
        version = importlib.metadata.version("flash-attn")
    except importlib.metadata.PackageNotFoundError:
        version = str(getattr(module, "__version__", ""))
    if "metax" not in version.casefold():
        return None
    return module


def _flash_attn_function(operation: str) -> Callable[..., torch.Tensor] | None:
    if os.getenv("MXFLASHATTN_BACKEND", "auto").strip().casefold() == "aten":
        return None
    module = _metax_flash_attn_module()
    if module is None:
        return None
    function = getattr(module, operation, None)
    return function if callable(function) else None


def native_unavailable_reason(
    tensor: torch.Tensor,
    operation: str,
    *,
    require_aten: bool = False,
) -> str | None:
    """Why vendor/ATen execution cannot serve the call (mxflashattn/dispatch.py:65-86)."""
    if tensor.device.type not in {"cuda", "maca", "musa"}:
        return "native_backend_requires_accelerator_tensor"
    if tensor.dtype not in (torch.float16, torch.bfloat16):
        return "native_backend_supports_only_float16_and_bfloat16"
    if _flash_attn_function(operation) is not None and not require_aten:
        return None
    extension = _native_extension()
    if extension is None:
        if require_aten:
            return "zero_softmax_scale_requires_aten_extension"
        return "native_extension_not_built_or_not_importable"
    if not bool(extension.is_available()):
        return "native_extension_reports_unavailable_runtime"
    if not hasattr(extension, operation):
        return f"native_extension_does_not_implement_{operation}"
    return None


class DecodeRoute:
    """A call the MI355X backend can take: ``reason`` is None when it qualifies.

    ``run`` performs the call on the current stream and returns the output.
    """

    __slots__ = ("reason", "run")

    def __init__(self, reason: str | None, run: Callable[[], torch.Tensor] | None = None):
        self.reason = reason
        self.run = run


def dispatch(
    operation: str,
    tensor: torch.Tensor,
    extension_args: tuple[Any, ...],
    reference: Callable[[], torch.Tensor],
    *,
    native_args: tuple[Any, ...],
    native_kwargs: dict[str, Any],
    decode_route: DecodeRoute | None = None,
) -> torch.Tensor:
    """Run ``operation`` on the first backend of the chain that serves it."""
    _state.dispatch_info = None
    decode_reason: str | None = None
    if decode_route is not None:
        if decode_route.reason is None:
            result = decode_route.run()
            _record(DispatchInfo(backend=BACKEND_MI355X, operation=operation))
            return result
        decode_reason = f"{BACKEND_MI355X}:{decode_route.reason}"

    # Scale 0.0 goes to the ATen path when the vendor would treat it as
    # "default scale" (mxflashattn/dispatch.py:105).
    require_aten = native_kwargs.get("softmax_scale") == 0.0
    vendor = None if require_aten else _flash_attn_function(operation)
    failure_reason: str | None = native_unavailable_reason(tensor, operation,
                                                           require_aten=require_aten)
    if vendor is not None:
        try:
            result = vendor(*native_args, **native_kwargs)
            if operation == "flash_attn_with_kvcache" and native_kwargs.get("k") is not None:
                native_kwargs["cache_seqlens"].add_(native_kwargs["k"].shape[1])
            _record(DispatchInfo(backend=BACKEND_VENDOR, operation=operation))
            return result
        except Exception as exc:  # recorded, then the chain continues
            failure_reason = f"vendor_call_failed:{type(exc).__name__}:{exc}"

    extension = _native_extension()
    extension_reason = ""
    if extension is not None:
        try:
            available = bool(extension.is_available())
        except Exception as exc:
            available = False
            extension_reason = f"aten_availability_check_failed:{type(exc).__name__}:{exc}"
        if available and hasattr(extension, operation):
            try:
                result = getattr(extension, operation)(*extension_args)
                _record(DispatchInfo(backend=BACKEND_ATEN, operation=operation,
                                     fallback_reason=failure_reason))
                return result
            except Exception as exc:
                extension_reason = f"aten_call_failed:{type(exc).__name__}:{exc}"
        elif not hasattr(extension, operation):
            extension_reason = f"aten_extension_does_not_implement_{operation}"
        elif not extension_reason:
            extension_reason = "aten_extension_reports_unavailable_runtime"

    reason = ";".join(part for part in (failure_reason, decode_reason, extension_reason) if part)
    if not reason:
        reason = "vendor_unavailable_or_parameter_incompatible"
    if os.getenv("MXFLASHATTN_ALLOW_FALLBACK", "").strip() != "1":
        raise BackendUnavailableError(
            f"MXFlashAttn dispatch failed ({reason}); set MXFLASHATTN_ALLOW_FALLBACK=1 "
            "to explicitly allow the PyTorch reference path"
        )
    _record(DispatchInfo(backend=BACKEND_REFERENCE, operation=operation, fallback_reason=reason))
    warnings.warn(
        f"MXFlashAttn is using the PyTorch reference path: {reason}",
        RuntimeWarning,
        stacklevel=3,
    )
    return reference()
