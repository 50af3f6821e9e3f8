"""Dispatch evidence and vLLM registration (integrations/vllm/backend.py:1-158 of the reference).

Every attention call through the plugin can record a small JSON event naming
the path that served it. Events are kept in memory and, when
MXFLASHATTN_DISPATCH_LOG (or a sibling of MXFLASHATTN_PLUGIN_IMPORT_LOG) names
a file, appended to it as JSON lines; MXFLASHATTN_DISPATCH_SAMPLE=N keeps only
every N-th line so the write cost stays off the hot path. The in-memory buffer
keeps the most recent MXFLASHATTN_DISPATCH_EVENTS_MAX events (65,536 by
default): a server records one per layer per step, which an unbounded list
(the reference's) turns into a leak over a long run; the log file, when set,
keeps every line.
"""

from __future__ import annotations

import collections
import json
import os
import threading

import torch

from ... import api

DISPATCH_EVENTS_MAX = int(os.getenv("MXFLASHATTN_DISPATCH_EVENTS_MAX", "65536") or 65536)
DISPATCH_EVENTS: collections.deque[dict[str, str]] = collections.deque(maxlen=DISPATCH_EVENTS_MAX)
_LOCK = threading.Lock()
_JSON_CACHE: dict[tuple[tuple[str, str], ...], str] = {}
_counter = 0

BACKEND_CLASS_PATH = "mxflashattn_amd.integrations.vllm.vllm_plugin.MXFlashAttnBackend"


def get_dispatch_events() -> list[dict[str, str]]:
    with _LOCK:
        return list(DISPATCH_EVENTS)


def clear_dispatch_events(truncate_log: bool = True) -> None:
    """Drop buffered events; truncate_log=False keeps lines already written."""
    with _LOCK:
        DISPATCH_EVENTS.clear()
    if truncate_log:
        path = os.getenv("MXFLASHATTN_DISPATCH_LOG")
        if path:
            try:
                open(path, "w", encoding="utf-8").close()
            except OSError:
                pass


def _log_path() -> str | None:
    path = os.getenv("MXFLASHATTN_DISPATCH_LOG")
    if not path:
        plugin_log = os.getenv("MXFLASHATTN_PLUGIN_IMPORT_LOG")
        if plugin_log:
            path = plugin_log.removesuffix(".plugin.log") + ".dispatch.jsonl"
    return path or None


def record_event(event: dict[str, str]) -> None:
    global _counter
    with _LOCK:
        DISPATCH_EVENTS.append(event)
        _counter += 1
        count = _counter
    path = _log_path()
    if not path:
        return
    sample = int(os.getenv("MXFLASHATTN_DISPATCH_SAMPLE", "0") or 0)
    if sample > 1 and count % sample != 1:
        return
    key = tuple(sorted((str(k), str(v)) for k, v in event.items()))
    line = _JSON_CACHE.get(key)
    if line is None:
        line = json.dumps(event, sort_keys=True) + "\n"
        _JSON_CACHE[key] = line
    try:
        with open(path, "a", encoding="utf-8") as stream:
            stream.write(line)
    except OSError:
        pass


# Name used by the reference plugin.
_record_event = record_event


def attention_forward(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor, *,
                      causal: bool, scale: float) -> torch.Tensor:
    """Dense [tokens, heads, dim] vLLM tensors through the public API."""
    if query.ndim != 3 or key.ndim != 3 or value.shape != key.shape:
        raise ValueError("vLLM Q/K/V must use [tokens, heads, head_dim] layout")
    out = api.flash_attn_func(query.unsqueeze(0), key.unsqueeze(0), value.unsqueeze(0),
                              causal=causal, softmax_scale=scale)
    return out.squeeze(0)


def register_vllm_v1_backend() -> dict[str, str]:
    """Point vLLM's FLASH_ATTN backend at this package's classes (needs vLLM)."""
    try:
        from vllm.v1.attention.backends.registry import AttentionBackendEnum, register_backend
    except Exception as exc:
        return {"registered": "false",
                "reason": f"vllm_v1_api_unavailable: {type(exc).__name__}: {exc}"}
    register_backend(AttentionBackendEnum.FLASH_ATTN, class_path=BACKEND_CLASS_PATH)
    return {
        "registered": "true",
        "backend_name": "MXFLASHATTN_MI355X",
        "backend_path": BACKEND_CLASS_PATH,
        "decoder_path": "mi355x_split_decode",
        "encoder_path": "mxflashattn_public_api",
    }
