"""MI355X-native split-KV paged decode behind the MXFlashAttn operator API.

Drop-in for the reference package ``mxflashattn`` on the decode path:
``flash_attn_with_kvcache`` / ``flash_attn_func`` / ``flash_attn_varlen_func``
with the same arguments and errors, the dispatch chain with
``get_last_dispatch_info``, plus the HIP ops (``paged_decode_split``,
``reshape_and_cache``) that the vLLM integration calls directly. The kernels
live in ``_lib/libmxfa_mi355x.so`` (C ABI: include/mxfa_mi355x.h).
"""

from .accuracy import ErrorSummary, summarize_error
from .api import flash_attn_func, flash_attn_varlen_func, flash_attn_with_kvcache
from .dispatch import (
    BACKEND_MI355X,
    BackendUnavailableError,
    DispatchInfo,
    get_last_dispatch_info,
)
from .native import append_kv, paged_decode_split, reshape_and_cache
from .policy import AdaptiveDispatchPolicy, DispatchDecision, DispatchPolicyConfig, WorkloadShape

__all__ = [
    "AdaptiveDispatchPolicy",
    "BACKEND_MI355X",
    "BackendUnavailableError",
    "DispatchDecision",
    "DispatchInfo",
    "DispatchPolicyConfig",
    "ErrorSummary",
    "append_kv",
    "flash_attn_func",
    "flash_attn_varlen_func",
    "flash_attn_with_kvcache",
    "get_last_dispatch_info",
    "paged_decode_split",
    "reshape_and_cache",
    "summarize_error",
    "WorkloadShape",
]

__version__ = "0.1.0"
