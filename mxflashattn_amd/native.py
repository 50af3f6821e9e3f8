"""ctypes binding of ``libmxfa_mi355x.so`` (C ABI: ``include/mxfa_mi355x.h``).

This module is the thin host layer between torch tensors and the C entry
points: it checks shapes, passes raw device pointers and element strides, keeps
a per-(device, stream) workspace so steady-state calls allocate nothing, and
launches on the caller's current HIP stream without synchronising.

Reference counterpart: the pybind module ``mxmmain`` (``csrc_native/m1_binding.cpp``),
``paged_decode_split`` at ``csrc_native/m1_binding.cpp:78-115``.
"""

from __future__ import annotations

import ctypes
import functools
import os
import threading
from pathlib import Path

import torch

# MXFLASHATTN_AMD_LIB points the binding at another build of the same C ABI.
LIB_PATH = Path(
    os.environ.get("MXFLASHATTN_AMD_LIB")
    or Path(__file__).resolve().parent / "_lib" / "libmxfa_mi355x.so"
)
ABI_VERSION = 12

MXFA_OK = 0
MXFA_EUNSUPPORTED = -1
MXFA_EINVAL = -2
MXFA_EWORKSPACE = -3
MXFA_ELAUNCH = -4
MXFA_ESCRATCH = -5
# num_splits value of the one-launch per-sequence kernel (MXFA_SPLITS_PER_SEQUENCE):
# every (sequence, kv head) is one workgroup whose four waves merge in LDS.
SPLITS_PER_SEQUENCE = -1
# Workspace of mxfa_split_decode_noalloc_launch (the library's own device array).
SCRATCH_BYTES = 8 << 20

# MXFA_POISON_OUTPUTS=1, a debugging aid (the GPU parity tests set it): before
# every launch outside graph capture the output is filled with NaN and the
# workspace with 0xff bytes (NaN pieces, prefix sums of -1), so a row or a
# piece the kernels fail to write shows up as NaN instead of a stale value,
# such as the previous call's correct answer in a block the caching allocator
# handed back. The torch operator reads the same variable.
POISON_OUTPUTS = os.environ.get("MXFA_POISON_OUTPUTS", "") == "1"

DTYPE_CODES = {torch.float16: 0, torch.bfloat16: 1}
DTYPE_FP8_E4M3 = 2
# OCP e4m3fn, the fp8 format of gfx950 (MI300's e4m3fnuz is a different code).
FP8_DTYPE = torch.float8_e4m3fn

# The reference's decode contract (vllm_plugin.py:220-261 hands other shapes
# back); the guards that mirror the reference use these.
SUPPORTED_HEAD_DIMS = (64, 128)
SUPPORTED_GQA = (2, 4, 8)
# What the kernels take: head dims 64/128/256, 1..16 query heads per kv head,
# 16-bit or fp8 caches; query tokens per sequence x query heads per kv head
# <= 16 (the MFMA columns).
KERNEL_HEAD_DIMS = (64, 128, 256)
KERNEL_GQA = tuple(range(1, 17))
KERNEL_COLUMNS = 16
# Query tokens x GQ that the routing layers send here for a causal query: at
# most four launches of token chunks, each reading its sequences' keys again.
CHUNKED_COLUMNS = 4 * KERNEL_COLUMNS

# Every entry point declared in include/mxfa_mi355x.h.
EXPORTED_SYMBOLS = (
    "mxfa_abi_version",
    "mxfa_strerror",
    "mxfa_split_heuristic",
    "mxfa_split_heuristic_fp8",
    "mxfa_split_decode_workspace_size",
    "mxfa_split_decode_launch",
    "mxfa_split_decode_noalloc_launch",
    "mxfa_split_decode_partial_launch",
    "mxfa_split_decode_combine_launch",
    "mxfa_split_decode_fp8_launch",
    "mxfa_split_decode_fp8_partial_launch",
    "mxfa_split_decode_multi_launch",
    "mxfa_stream_probe_launch",
    "mxfa_stream_read_launch",
    "mxfa_reshape_and_cache_launch",
    "mxfa_reshape_and_cache_fp8_launch",
    "mxfa_append_kv_launch",
)


class NativeLibraryError(RuntimeError):
    """The HIP library is missing, failed to load or has the wrong ABI."""


class UnsupportedConfig(RuntimeError):
    """The kernel contract does not cover this shape/dtype (MXFA_EUNSUPPORTED)."""


_i = ctypes.c_int
_i64 = ctypes.c_int64
_p = ctypes.c_void_p
_f = ctypes.c_float
_sz = ctypes.c_size_t

_SPLIT_ARGS = [_p, _i64, _i64, _p, _p, _i64, _i64, _i64, _p, _i64, _p, _i, _p, _i64, _i64, _p,
               _sz, _f, _i, _i, _i, _i, _i, _i, _i, _i, _i]

_SIGNATURES = {
    "mxfa_abi_version": (_i, []),
    "mxfa_strerror": (ctypes.c_char_p, [_i]),
    "mxfa_split_heuristic": (_i, [_i, _i, _i, _i, _i, _i, _i, ctypes.POINTER(_i)]),
    "mxfa_split_heuristic_fp8": (_i, [_i, _i, _i, _i, _i, _i, _i, ctypes.POINTER(_i)]),
    "mxfa_split_decode_workspace_size": (_i, [_i, _i, _i, _i, ctypes.POINTER(_sz)]),
    "mxfa_split_decode_launch": (_i, _SPLIT_ARGS + [_p]),
    "mxfa_split_decode_noalloc_launch": (_i, _SPLIT_ARGS[:15] + _SPLIT_ARGS[17:] + [_p]),
    "mxfa_split_decode_partial_launch": (_i, _SPLIT_ARGS + [_p]),
    "mxfa_split_decode_fp8_launch": (_i, _SPLIT_ARGS + [_p, _p, _p]),
    "mxfa_split_decode_fp8_partial_launch": (_i, _SPLIT_ARGS + [_p, _p, _p]),
    "mxfa_split_decode_multi_launch": (
        _i,
        [_p, _i64, _i64, _i64, _i, _i, _i, _p, _f, _p, _p, _p, _i64, _i64, _i64, _p, _i64, _p,
         _i, _p, _i64,
         _i64, _i64, _p, _sz, _f, _i, _i, _i, _i, _i, _i, _i, _i, _i, _p, _p, _i, _p],
    ),
    "mxfa_stream_probe_launch": (
        _i,
        [_p, _i64, _i64, _p, _p, _i64, _i64, _i64, _p, _i64, _p, _i, _p, _sz, _i, _i, _i, _i, _i,
         _i, _i, _i, _i, _i, _p],
    ),
    "mxfa_stream_read_launch": (_i, [_p, ctypes.c_uint64, _i, _i, _i, _p, _sz, _p]),
    "mxfa_split_decode_combine_launch": (
        _i,
        [_p, _sz, _p, _i64, _i64, _i, _i, _i, _i, _i, _i, _p],
    ),
    "mxfa_reshape_and_cache_launch": (
        _i,
        [_p, _p, _i64, _i64, _p, _p, _i64, _i64, _i64, _p, _i, _i, _i, _i, _i, _i, _p],
    ),
    "mxfa_reshape_and_cache_fp8_launch": (
        _i,
        [_p, _p, _i64, _i64, _p, _p, _i64, _i64, _i64, _p, _i, _i, _i, _i, _i, _i, _p, _p, _p],
    ),
    "mxfa_append_kv_launch": (
        _i,
        [_p, _p, _i64, _i64, _i64, _p, _p, _i64, _i64, _i64, _p, _i64, _p, _i, _i, _i, _i,
         _i, _i, _i, _i, _p],
    ),
}

_load_lock = threading.Lock()
_lib: ctypes.CDLL | None = None
_load_error: str | None = None


def library() -> ctypes.CDLL:
    """Load the library once; raise NativeLibraryError with the reason otherwise."""
    global _lib, _load_error
    if _lib is not None:
        return _lib
    with _load_lock:
        if _lib is not None:
            return _lib
        if not LIB_PATH.exists():
            _load_error = (
                f"native library not built: {LIB_PATH} is missing "
                "(run python -m mxflashattn_amd._build)"
            )
            raise NativeLibraryError(_load_error)
        try:
            lib = ctypes.CDLL(str(LIB_PATH))
        except OSError as exc:
            _load_error = f"native library failed to load: {exc}"
            raise NativeLibraryError(_load_error) from exc
        for name, (restype, argtypes) in _SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = restype
            fn.argtypes = argtypes
        version = lib.mxfa_abi_version()
        if version != ABI_VERSION:
            _load_error = f"native library ABI {version} does not match {ABI_VERSION}"
            raise NativeLibraryError(_load_error)
        _lib = lib
        return lib


_op_lock = threading.Lock()
_op: object | None = None
# False forces the ctypes path (for comparisons); the operator is used when built.
USE_TORCH_OP = True


def torch_op():
    """The torch operator in front of the C ABI (``csrc/torch_op.cpp``), or
    None when it is not built. It takes the common one-token decode in C++
    and hands every other call back (returns None) to the ctypes path."""
    global _op
    if _op is None:
        with _op_lock:
            if _op is None:
                import importlib.util
                import sysconfig

                library()  # the operator links this library: load and check it first
                path = LIB_PATH.parent / ("_mxfa_torch" + sysconfig.get_config_var("EXT_SUFFIX"))
                module = False
                if path.exists():
                    spec = importlib.util.spec_from_file_location("_mxfa_torch", path)
                    module = importlib.util.module_from_spec(spec)
                    spec.loader.exec_module(module)
                    if module.abi_version() != ABI_VERSION:
                        raise NativeLibraryError(
                            f"torch operator ABI {module.abi_version()} does not match "
                            f"{ABI_VERSION}")
                _op = module
    return _op or None


def unavailable_reason() -> str | None:
    """None when the library loads, else the reason it does not."""
    try:
        library()
    except NativeLibraryError as exc:
        return str(exc)
    return None


def _check(rc: int, what: str) -> None:
    if rc == MXFA_OK:
        return
    text = library().mxfa_strerror(rc).decode()
    if rc == MXFA_EUNSUPPORTED:
        raise UnsupportedConfig(f"{what}: {text}")
    raise RuntimeError(f"{what} failed ({rc}): {text}")


@functools.lru_cache(maxsize=256)
def split_heuristic(batch: int, q_heads: int, kv_heads: int, head_dim: int, page_size: int,
                    block_table_width: int, num_cus: int, fp8: bool = False) -> int:
    """Balanced ranges per kv head for a launch; integer-only, no device access."""
    ns = _i()
    name = "mxfa_split_heuristic_fp8" if fp8 else "mxfa_split_heuristic"
    _check(
        getattr(library(), name)(batch, q_heads, kv_heads, head_dim, page_size,
                                 block_table_width, num_cus, ctypes.byref(ns)),
        name,
    )
    return ns.value


@functools.lru_cache(maxsize=256)
def workspace_size(batch: int, q_heads: int, head_dim: int, num_splits: int) -> int:
    out = _sz()
    _check(library().mxfa_split_decode_workspace_size(batch, q_heads, head_dim, num_splits,
                                                       ctypes.byref(out)),
           "mxfa_split_decode_workspace_size")
    return out.value


@functools.lru_cache(maxsize=16)
def num_cus(device_index: int) -> int:
    return int(torch.cuda.get_device_properties(device_index).multi_processor_count)


class _Workspace:
    """Grow-only scratch per (device, stream), reused across calls.

    A launch on one stream never shares its workspace with another stream's
    launches, so calls on different streams cannot race on it.

    A HIP graph captured on a stream keeps the workspace address of the
    capture in its kernel arguments. When a later call needs a larger buffer,
    the smaller one is therefore never released: it moves to a keep-alive list
    for the life of the process, so replays of earlier captures still write
    into memory that nothing else owns. Growth doubles, so the retired buffers
    together stay smaller than the live one.
    """

    def __init__(self) -> None:
        self._buffers: dict[tuple[int, int], torch.Tensor] = {}
        self._retired: list[torch.Tensor] = []
        self._lock = threading.Lock()

    def get(self, device: torch.device, stream: int, nbytes: int) -> torch.Tensor:
        key = (device.index if device.index is not None else _current_device(), stream)
        with self._lock:
            buf = self._buffers.get(key)
            if buf is None or buf.numel() < nbytes:
                size = max(nbytes, 1 << 20)
                if buf is not None:
                    size = max(size, buf.numel() * 2)
                    self._retired.append(buf)
                buf = torch.empty(size, dtype=torch.uint8, device=device)
                self._buffers[key] = buf
            return buf

    def retired_bytes(self) -> int:
        with self._lock:
            return sum(t.numel() for t in self._retired)


WORKSPACE = _Workspace()


def retired_workspace_bytes() -> int:
    """Bytes of workspaces replaced by larger ones and kept alive, over the
    ctypes path's cache and the torch operator's."""
    op = torch_op()
    return WORKSPACE.retired_bytes() + (op.workspace_bytes()[1] if op is not None else 0)


def _poison(out: torch.Tensor | None, ws: torch.Tensor | None = None) -> None:
    """NaN-fill ``out`` and 0xff-fill ``ws`` when MXFA_POISON_OUTPUTS is set,
    on the current stream, except under graph capture."""
    if not POISON_OUTPUTS or torch.cuda.is_current_stream_capturing():
        return
    if out is not None:
        out.fill_(float("nan"))
    if ws is not None:
        ws.fill_(0xFF)


def _dtype_code(t: torch.Tensor) -> int:
    code = DTYPE_CODES.get(t.dtype)
    if code is None:
        raise UnsupportedConfig(f"dtype {t.dtype} is not float16/bfloat16")
    return code


def _int32_contig(t: torch.Tensor, name: str) -> torch.Tensor:
    if t.dtype != torch.int32:
        t = t.to(torch.int32)
    if t.dim() == 2:
        if t.stride(1) != 1:
            t = t.contiguous()
    elif not t.is_contiguous():
        t = t.contiguous()
    return t


# The raw current-stream accessor skips the Stream object torch would build
# (a few microseconds per call on the host).
_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)
_current_device = getattr(torch._C, "_cuda_getDevice", None) or torch.cuda.current_device


def _stream_handle(device: torch.device) -> int:
    if _raw_stream is not None:
        return _raw_stream(device.index if device.index is not None else _current_device())
    return torch.cuda.current_stream(device).cuda_stream


def _require_device(*tensors: torch.Tensor) -> torch.device:
    """All tensors on one GPU, which must be the current HIP device.

    The kernels dereference raw pointers: a host tensor or a tensor of another
    GPU would fault instead of raising, so this is checked before every launch.
    """
    device = tensors[0].device
    if device.type != "cuda":
        raise ValueError(f"MI355X kernels need GPU tensors, got a tensor on {device}")
    for t in tensors[1:]:
        if t.device != device:
            raise ValueError(f"all tensors must be on {device}, got one on {t.device}")
    current = _current_device()
    if (device.index or 0) != current:
        raise ValueError(f"tensors are on {device} but the current device is "
                         f"cuda:{current}; call under torch.cuda.device")
    return device


def check_decode_shapes(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                        causal: bool = False) -> None:
    """Raise UnsupportedConfig when the kernel contract does not cover the call."""
    if q.dim() not in (3, 4) or (q.dim() == 4 and q.shape[1] < 1):
        raise UnsupportedConfig(f"q must be [B,QL,HQ,HD] or [B,HQ,HD], got {tuple(q.shape)}")
    if k_cache.dim() != 4 or v_cache.shape != k_cache.shape:
        raise UnsupportedConfig("caches must be [pages, page_size, kv_heads, head_dim]")
    hq, hd = q.shape[-2], q.shape[-1]
    hkv = k_cache.shape[2]
    if hd not in KERNEL_HEAD_DIMS or k_cache.shape[3] != hd:
        raise UnsupportedConfig(f"head_dim {hd} not in {KERNEL_HEAD_DIMS}")
    if hkv <= 0 or hq % hkv or hq // hkv not in KERNEL_GQA:
        raise UnsupportedConfig(f"GQA ratio {hq}/{hkv} not in 1..16")
    ql = q.shape[1] if q.dim() == 4 else 1
    if ql * (hq // hkv) > KERNEL_COLUMNS and not causal:
        raise UnsupportedConfig(f"{ql} query tokens x GQA {hq // hkv} exceeds {KERNEL_COLUMNS} "
                                "(causal calls run in token chunks)")
    if q.dtype not in DTYPE_CODES:
        raise UnsupportedConfig("q must be float16 or bfloat16")
    if v_cache.dtype != k_cache.dtype or k_cache.dtype not in (q.dtype, FP8_DTYPE):
        raise UnsupportedConfig("caches must share q's dtype or both be float8_e4m3fn")
    ps = k_cache.shape[1]
    if ps <= 0 or ps & (ps - 1) or ps > 4096:
        raise UnsupportedConfig(f"page size {ps} is not a power of two <= 4096")


# Limits of the C ABI (csrc/split_decode.hip check_split_args): sequences per
# launch (the tile prefix sums live in LDS), keys per table row, and the
# 16-byte alignment of the cache fragments.
MAX_BATCH = 16000
MAX_KV_HEADS = 65535
MAX_TABLE_KEYS = 1 << 30


def layout_reason(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                  block_table_width: int) -> str | None:
    """Why the kernels cannot take these tensors as laid out, or None.

    Reads shapes, strides and addresses only (never device data). q itself is
    copied when its layout does not suit the kernel, so only the caches and
    the sizes matter here."""
    batch, hd = q.shape[0], q.shape[-1]
    ps, hkv = k_cache.shape[1], k_cache.shape[2]
    esz = k_cache.element_size()
    if batch > MAX_BATCH:
        return f"batch_{batch}_exceeds_{MAX_BATCH}"
    if hkv > MAX_KV_HEADS:
        return f"kv_heads_{hkv}_exceeds_{MAX_KV_HEADS}"
    max_len = block_table_width * ps
    if max_len > MAX_TABLE_KEYS or batch * ((max_len + 15) // 16) >= 1 << 31:
        return "block_table_capacity_exceeds_kernel_limit"
    if k_cache.stride(-1) != 1 or v_cache.stride() != k_cache.stride():
        return "cache_layout_not_supported"
    if k_cache.data_ptr() % 16 or v_cache.data_ptr() % 16:
        return "cache_not_16_byte_aligned"
    sp, st, sh = k_cache.stride(0), k_cache.stride(1), k_cache.stride(2)
    if min(sp, st, sh) < 0 or any((s * esz) % 16 for s in (sp, st, sh)):
        return "cache_strides_not_multiples_of_16_bytes"
    if ps > 1 and st < hd:
        return "cache_token_rows_overlap"
    if (15 * st + hd) * esz >= 1 << 30 or (ps - 1) * st * esz >= 1 << 32 or sh * esz >= 1 << 32:
        return "cache_strides_exceed_kernel_limit"
    return None


def _launch_args(q, k_cache, v_cache, block_table, cache_seqlens, out, workspace, ws_bytes,
                 softmax_scale, num_splits, seqlen_add, stream=None):
    batch, hq, hd = q.shape[0], q.shape[-2], q.shape[-1]
    pages, ps, hkv = k_cache.shape[0], k_cache.shape[1], k_cache.shape[2]
    qs, os_, cs = q.stride(), out.stride(), k_cache.stride()
    return (
        q.data_ptr(), qs[0], qs[-2], k_cache.data_ptr(), v_cache.data_ptr(), cs[0], cs[1], cs[2],
        block_table.data_ptr(), block_table.stride(0), cache_seqlens.data_ptr(), seqlen_add,
        out.data_ptr(), os_[0], os_[-2], workspace, ws_bytes,
        float(softmax_scale), batch, hq, hkv, hd, ps, block_table.shape[1], pages,
        DTYPE_CODES[q.dtype], num_splits, _stream_handle(q.device) if stream is None else stream,
    )


class _ScalarCache:
    """Device float32 scalars for scales passed as Python floats.

    Each is made by a fill kernel on the current stream (no host-to-device
    copy and no synchronisation) and kept for the life of the process, since
    a captured graph holds its address. A value first seen while the stream is
    capturing is refused: a fill recorded into a graph runs only at replay,
    so eager calls would read the scalar before it exists. At most ``limit``
    distinct values are kept per device; past that, float scales are refused
    with a clear error (pass a float32 device tensor instead).
    """

    def __init__(self, limit: int = 64) -> None:
        self.limit = limit
        self._values: dict[tuple[int, float], torch.Tensor] = {}
        self._lock = threading.Lock()

    def ptr(self, value: float, device: torch.device, name: str) -> int:
        key = (device.index or 0, value)
        with self._lock:
            t = self._values.get(key)
            if t is None:
                if torch.cuda.is_current_stream_capturing():
                    raise ValueError(f"{name}={value} is first used inside graph capture; pass "
                                     "a float32 device tensor, or make one eager call first")
                if sum(1 for k in self._values if k[0] == key[0]) >= self.limit:
                    raise ValueError(f"{name}: more than {self.limit} distinct float scales on "
                                     f"{device}; pass a float32 device tensor")
                t = self._values[key] = torch.full((1,), value, dtype=torch.float32,
                                                   device=device)
            return t.data_ptr()


_SCALARS = _ScalarCache()


def _scale_ptr(scale, device: torch.device, name: str) -> int:
    """Device address of an fp32 dequantisation scale: a one-element (or
    broadcast, all strides 0) float32 GPU tensor, a Python float (kept in a
    cached device scalar) or None (1.0)."""
    if scale is None:
        return 0
    if isinstance(scale, torch.Tensor):
        if scale.dtype != torch.float32 or scale.device != device:
            raise ValueError(f"{name} must be a float32 tensor on {device}")
        if scale.numel() != 1 and any(st != 0 for st in scale.stride()):
            raise UnsupportedConfig(f"{name} must be one per-tensor scale")
        return scale.data_ptr()
    return _SCALARS.ptr(float(scale), device, name)


def token_chunks(q_len: int, per_launch: int, seqlen_add: int) -> list[tuple[int, int, int]]:
    """(first, end, seqlen_add) of each launch of a causal query of q_len tokens
    when one launch holds per_launch tokens. Tokens [first, end) run as the
    last end - first tokens of sequences shortened by q_len - end keys, which
    keeps each token's position, causal mask, window and ALiBi distances."""
    out = []
    for first in range(0, q_len, per_launch):
        end = min(first + per_launch, q_len)
        out.append((first, end, seqlen_add - (q_len - end)))
    return out


def _prepare(q, k_cache, v_cache, block_table, cache_seqlens, out, causal: bool = False):
    q, block_table, cache_seqlens = _prepare_inputs(q, k_cache, v_cache, block_table,
                                                    cache_seqlens, causal)
    if out is None:
        out = torch.empty(q.shape, dtype=q.dtype, device=q.device)
    if out.shape != q.shape or out.dtype != q.dtype or out.stride(-1) != 1:
        raise ValueError("out must match q's shape and dtype with a contiguous last dim")
    if torch._debug_has_internal_overlap(out) == 1:
        # Different workgroups write different rows; rows sharing memory would race.
        raise ValueError("out must not have internally overlapping memory")
    _require_device(q, out)
    return q, block_table, cache_seqlens, out


def _prepare_inputs(q, k_cache, v_cache, block_table, cache_seqlens, causal: bool = False):
    check_decode_shapes(q, k_cache, v_cache, causal)
    batch = q.shape[0]
    hd = q.shape[-1]
    if q.stride(-1) != 1 or (q.shape[-2] > 1 and q.stride(-2) < hd) or (
            q.dim() == 4 and q.shape[1] > 1 and q.stride(1) % 8) or q.data_ptr() % 16 or (
            any(s % 8 for s in q.stride()[:-1])):
        # The kernel reads q in 16-byte fragments: 16-byte aligned, strides
        # in multiples of 8 elements. A packed copy always is.
        q = q.clone(memory_format=torch.contiguous_format)
    if k_cache.stride(-1) != 1 or v_cache.stride() != k_cache.stride():
        raise UnsupportedConfig("k_cache and v_cache must share strides with a contiguous last dim")
    if k_cache.shape[1] > 1 and k_cache.stride(1) < hd:
        raise UnsupportedConfig("cache token rows overlap (token stride < head_dim)")
    _require_device(q, k_cache, v_cache, block_table, cache_seqlens)
    block_table = _int32_contig(block_table, "block_table")
    cache_seqlens = _int32_contig(cache_seqlens, "cache_seqlens")
    if block_table.dim() != 2 or block_table.shape[0] != batch or block_table.shape[1] < 1:
        raise ValueError("block_table must be [batch, width >= 1]")
    if cache_seqlens.numel() != batch:
        raise ValueError("cache_seqlens must have one entry per sequence")
    return q, block_table, cache_seqlens


def _launch_multi(q, k_cache, v_cache, block_table, cache_seqlens, out, workspace, ws_bytes,
                  softmax_scale, num_splits, seqlen_add, stream, causal, k_scale, v_scale,
                  window_left, sinks, softcap, alibi_slopes):
    if q.dim() == 3:
        q, out = q.unsqueeze(1), out.unsqueeze(1)
    batch, ql, hq, hd = q.shape
    pages, ps, hkv = k_cache.shape[0], k_cache.shape[1], k_cache.shape[2]
    qs, os_, cs = q.stride(), out.stride(), k_cache.stride()
    fp8 = k_cache.dtype == FP8_DTYPE
    rc = library().mxfa_split_decode_multi_launch(
        q.data_ptr(), qs[0], qs[1], qs[2], ql, int(bool(causal)), int(window_left),
        _sinks_ptr(sinks, q), float(softcap), _sinks_ptr(alibi_slopes, q, "alibi_slopes"),
        k_cache.data_ptr(),
        v_cache.data_ptr(), cs[0], cs[1], cs[2], block_table.data_ptr(), block_table.stride(0),
        cache_seqlens.data_ptr(), seqlen_add, out.data_ptr(), os_[0], os_[1], os_[2], workspace,
        ws_bytes, float(softmax_scale), batch, hq, hkv, hd, ps, block_table.shape[1], pages,
        DTYPE_CODES[q.dtype], DTYPE_FP8_E4M3 if fp8 else DTYPE_CODES[q.dtype],
        _scale_ptr(k_scale, q.device, "k_scale") if fp8 else 0,
        _scale_ptr(v_scale, q.device, "v_scale") if fp8 else 0, num_splits, stream)
    _check(rc, "mxfa_split_decode_multi_launch")


def _sinks_ptr(values, q: torch.Tensor, name: str = "sinks") -> int:
    """Device address of a per-query-head float32 vector (sinks, ALiBi
    slopes): [HQ], contiguous, on q's GPU; None gives 0 (none)."""
    if values is None:
        return 0
    if (not isinstance(values, torch.Tensor) or values.dtype != torch.float32
            or values.device != q.device or values.dim() != 1 or values.shape[0] != q.shape[-2]
            or not values.is_contiguous()):
        raise ValueError(f"{name} must be a contiguous float32 [{q.shape[-2]}] tensor on "
                         f"{q.device}")
    return values.data_ptr()


def default_num_splits(q: torch.Tensor, k_cache: torch.Tensor, block_table: torch.Tensor) -> int:
    """The heuristic's count for q ([B, HQ, HD] or [B, QL, HQ, HD]). It is
    asked for the columns of one launch, HQ times the query tokens a launch
    takes (QL, or 16 / GQ of them for longer causal queries), which decide
    whether the per-sequence kernel's LDS holds them."""
    hq, hkv = q.shape[-2], k_cache.shape[2]
    ql = q.shape[1] if q.dim() == 4 else 1
    tokens = min(ql, max(1, KERNEL_COLUMNS // max(1, hq // hkv)))
    return split_heuristic(q.shape[0], hq * tokens, hkv, q.shape[-1], k_cache.shape[1],
                           block_table.shape[1], num_cus(q.device.index or 0),
                           k_cache.dtype == FP8_DTYPE)


def paged_decode_split(
    q: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    block_table: torch.Tensor,
    cache_seqlens: torch.Tensor,
    softmax_scale: float,
    *,
    out: torch.Tensor | None = None,
    num_splits: int | None = None,
    seqlen_add: int = 0,
    k_scale: torch.Tensor | float | None = None,
    v_scale: torch.Tensor | float | None = None,
    causal: bool = False,
    window_left: int = -1,
    sinks: torch.Tensor | None = None,
    softcap: float = 0.0,
    alibi_slopes: torch.Tensor | None = None,
) -> torch.Tensor:
    """Split-KV paged decode on the current stream; returns ``out`` shaped like q.

    q: [B, QL, HQ, HD] or [B, HQ, HD] (any strides with a contiguous last dim);
    QL > 1 query tokens sit at the last QL positions of each sequence, and
    ``causal`` masks the keys after each one (QL * HQ/HKV <= 16 per launch; a
    causal call with more runs as launches of 16 // (HQ/HKV) tokens, each
    reading its sequences' keys again);
    caches: [pages, PS, HKV, HD] of q's dtype, or float8_e4m3fn with the
    per-tensor dequantisation scales k_scale / v_scale (float32 device scalars
    for graph capture); block_table: int32 [B, W]; cache_seqlens: int32 [B].
    The attended length of sequence b is cache_seqlens[b] + seqlen_add.
    window_left >= 0: sliding window, the token at position i sees keys
    >= i - window_left (FlashAttention's window_size (window_left, 0) with
    causal, (window_left, -1) without).
    sinks: float32 [HQ] per-head logits on the scale of the scaled scores,
    each added once to its row's softmax denominator (vLLM's s_aux).
    softcap > 0: every scaled score s becomes softcap * tanh(s / softcap).
    alibi_slopes: float32 [HQ]; -slope * |p - j| is added to the score of the
    query at position p and key j, after the cap.
    num_splits: balanced work ranges per kv head, or SPLITS_PER_SEQUENCE for
    the one-launch per-sequence kernel (default: split_heuristic, which picks
    the latter for batches of short sequences by the block table's capacity).
    """
    if (USE_TORCH_OP and k_scale is None and v_scale is None and window_left < 0
            and sinks is None and softcap == 0 and alibi_slopes is None
            and (q.dim() == 3 or q.shape[1] == 1)):
        op = torch_op()
        if op is not None:
            result = op.decode(q, k_cache, v_cache, block_table, cache_seqlens,
                               float(softmax_scale), out,
                               None if num_splits is None else int(num_splits),
                               int(seqlen_add))
            if result is not None:
                return result
    if out is not None and (out.data_ptr() % 8 or any(st % 4 for st in out.stride()[:-1])):
        # The kernels store 8-byte pieces of each output row; a view that is
        # not laid out for that gets the result through a packed copy.
        final = out
        result = paged_decode_split(
            q, k_cache, v_cache, block_table, cache_seqlens, softmax_scale,
            num_splits=num_splits, seqlen_add=seqlen_add, k_scale=k_scale, v_scale=v_scale,
            causal=causal, window_left=window_left, sinks=sinks, softcap=softcap,
            alibi_slopes=alibi_slopes)
        return final.copy_(result)
    if int(window_left) < -1:
        raise ValueError(f"window_left must be >= -1, got {window_left}")
    if not (0.0 <= float(softcap) < float("inf")):
        raise ValueError(f"softcap must be finite and >= 0, got {softcap}")
    q, block_table, cache_seqlens, out = _prepare(q, k_cache, v_cache, block_table,
                                                  cache_seqlens, out, bool(causal))
    lib = library()
    if num_splits is None:
        num_splits = default_num_splits(q, k_cache, block_table)
    stream = _stream_handle(q.device)
    ql = q.shape[1] if q.dim() == 4 else 1
    per_launch = KERNEL_COLUMNS // (q.shape[-2] // k_cache.shape[2])
    ws_bytes = workspace_size(q.shape[0], q.shape[-2] * min(ql, per_launch), q.shape[-1],
                              num_splits)
    ws = WORKSPACE.get(q.device, stream, ws_bytes)
    _poison(out)
    if ql > 1 or window_left >= 0 or sinks is not None or softcap > 0 or (
            alibi_slopes is not None):
        for first, end, add in token_chunks(ql, per_launch, int(seqlen_add)):
            whole = first == 0 and end == ql
            _poison(None, ws)
            _launch_multi(q if whole else q[:, first:end], k_cache, v_cache, block_table,
                          cache_seqlens, out if whole else out[:, first:end], ws.data_ptr(),
                          ws_bytes, softmax_scale, num_splits, add, stream, causal, k_scale,
                          v_scale, window_left, sinks, softcap, alibi_slopes)
        return out
    _poison(None, ws)
    args = _launch_args(q, k_cache, v_cache, block_table, cache_seqlens, out, ws.data_ptr(),
                        ws_bytes, softmax_scale, num_splits, seqlen_add, stream)
    if k_cache.dtype == FP8_DTYPE:
        rc = lib.mxfa_split_decode_fp8_launch(*args[:-1], _scale_ptr(k_scale, q.device, "k_scale"),
                                              _scale_ptr(v_scale, q.device, "v_scale"), args[-1])
        _check(rc, "mxfa_split_decode_fp8_launch")
    else:
        rc = lib.mxfa_split_decode_launch(*args)
        _check(rc, "mxfa_split_decode_launch")
    return out


def paged_decode_split_noalloc(
    q: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    block_table: torch.Tensor,
    cache_seqlens: torch.Tensor,
    softmax_scale: float,
    *,
    out: torch.Tensor,
    num_splits: int | None = None,
    seqlen_add: int = 0,
) -> torch.Tensor:
    """One-token decode of 16-bit caches through mxfa_split_decode_noalloc_launch:
    the workspace is the library's own device array (SCRATCH_BYTES per GPU), so
    the launch allocates nothing; ``out`` is required. Calls that overlap in
    time on one GPU share that array and must not run concurrently."""
    if k_cache.dtype == FP8_DTYPE or (q.dim() == 4 and q.shape[1] != 1):
        raise UnsupportedConfig("the no-allocation entry point takes one-token 16-bit decode")
    q, block_table, cache_seqlens, out = _prepare(q, k_cache, v_cache, block_table,
                                                  cache_seqlens, out)
    if num_splits is None:
        num_splits = default_num_splits(q, k_cache, block_table)
    args = _launch_args(q, k_cache, v_cache, block_table, cache_seqlens, out, 0, 0,
                        softmax_scale, num_splits, seqlen_add)
    rc = library().mxfa_split_decode_noalloc_launch(*args[:15], *args[17:])
    _check(rc, "mxfa_split_decode_noalloc_launch")
    return out


def split_decode_partial(
    q: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    block_table: torch.Tensor,
    cache_seqlens: torch.Tensor,
    softmax_scale: float,
    out: torch.Tensor,
    workspace: torch.Tensor,
    num_splits: int,
    seqlen_add: int = 0,
    k_scale: torch.Tensor | float | None = None,
    v_scale: torch.Tensor | float | None = None,
) -> None:
    """Partial stage only: sequences inside one work range land in ``out``, the
    pieces of the others in ``workspace``; ``split_decode_combine`` finishes.
    With num_splits = SPLITS_PER_SEQUENCE this is the whole call (one kernel)."""
    q, block_table, cache_seqlens, out = _prepare(q, k_cache, v_cache, block_table,
                                                  cache_seqlens, out)
    _require_device(q, workspace)
    if not workspace.is_contiguous():
        raise ValueError("workspace must be contiguous")
    nbytes = workspace.numel() * workspace.element_size()
    args = _launch_args(q, k_cache, v_cache, block_table, cache_seqlens, out,
                        workspace.data_ptr(), nbytes, softmax_scale, num_splits, seqlen_add)
    if k_cache.dtype == FP8_DTYPE:
        rc = library().mxfa_split_decode_fp8_partial_launch(
            *args[:-1], _scale_ptr(k_scale, q.device, "k_scale"),
            _scale_ptr(v_scale, q.device, "v_scale"), args[-1])
        _check(rc, "mxfa_split_decode_fp8_partial_launch")
    else:
        rc = library().mxfa_split_decode_partial_launch(*args)
        _check(rc, "mxfa_split_decode_partial_launch")


def stream_probe(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                 block_table: torch.Tensor, cache_seqlens: torch.Tensor, num_splits: int,
                 sink: torch.Tensor | None = None, tiles_in_flight: int = 0) -> torch.Tensor:
    """The streaming probe (mxfa_stream_probe_launch): the split partial
    kernel's gather at ``num_splits`` ranges with no attention math, on the
    current stream. Returns the sink, int32 [HKV, num_splits, 64], each lane's
    XOR of the words its wave loaded (only what the launch's ranges cover is
    written). ``tiles_in_flight`` 0 is the decode kernel's own pipeline depth."""
    q, block_table, cache_seqlens = _prepare_inputs(q, k_cache, v_cache, block_table,
                                                    cache_seqlens)
    hkv = k_cache.shape[2]
    if sink is None:
        sink = torch.empty(hkv, num_splits, 64, dtype=torch.int32, device=q.device)
    if sink.dtype != torch.int32 or not sink.is_contiguous() or sink.device != q.device:
        raise ValueError("sink must be a contiguous int32 tensor on q's device")
    qs, cs = q.stride(), k_cache.stride()
    rc = library().mxfa_stream_probe_launch(
        q.data_ptr(), qs[0], qs[-2], k_cache.data_ptr(), v_cache.data_ptr(), cs[0], cs[1], cs[2],
        block_table.data_ptr(), block_table.stride(0), cache_seqlens.data_ptr(), 0,
        sink.data_ptr(), sink.numel() * 4, q.shape[0], q.shape[-2], hkv, q.shape[-1],
        k_cache.shape[1], block_table.shape[1], k_cache.shape[0], _dtype_code(q), int(num_splits),
        int(tiles_in_flight), _stream_handle(q.device))
    _check(rc, "mxfa_stream_probe_launch")
    return sink


def stream_read(buf: torch.Tensor, nbytes: int | None = None, *, layout: int = 0,
                depth: int = 8, workgroups: int | None = None,
                sink: torch.Tensor | None = None) -> torch.Tensor:
    """The plain streaming read (mxfa_stream_read_launch): one pass over the
    first ``nbytes`` bytes of ``buf`` (a contiguous GPU tensor; all of it by
    default) with no other work, on the current stream. ``workgroups``
    defaults to one per CU. Returns the sink, int32 [workgroups * 256], each
    lane's XOR of the words it read."""
    if buf.device.type != "cuda" or not buf.is_contiguous():
        raise ValueError("buf must be a contiguous tensor on a GPU")
    total = buf.numel() * buf.element_size()
    nbytes = total if nbytes is None else int(nbytes)
    if nbytes > total:
        raise ValueError(f"nbytes {nbytes} exceeds the buffer's {total} bytes")
    if workgroups is None:
        workgroups = num_cus(buf.device.index or 0)
    if sink is None:
        sink = torch.empty(workgroups * 256, dtype=torch.int32, device=buf.device)
    if sink.dtype != torch.int32 or not sink.is_contiguous() or sink.device != buf.device:
        raise ValueError("sink must be a contiguous int32 tensor on buf's device")
    rc = library().mxfa_stream_read_launch(buf.data_ptr(), nbytes, int(layout), int(depth),
                                           int(workgroups), sink.data_ptr(), sink.numel() * 4,
                                           _stream_handle(buf.device))
    _check(rc, "mxfa_stream_read_launch")
    return sink


def split_decode_combine(workspace: torch.Tensor, out: torch.Tensor, kv_heads: int,
                         num_splits: int) -> torch.Tensor:
    """LSE merge of the pieces in ``workspace`` into ``out`` ([B,1,HQ,HD] or [B,HQ,HD])."""
    _require_device(out, workspace)
    if not workspace.is_contiguous() or out.stride(-1) != 1:
        raise ValueError("workspace must be contiguous and out's last dim contiguous")
    if out.dim() not in (3, 4) or (out.dim() == 4 and out.shape[1] != 1):
        raise ValueError(f"out must be [B,1,HQ,HD] or [B,HQ,HD], got {tuple(out.shape)}")
    batch, hq, hd = out.shape[0], out.shape[-2], out.shape[-1]
    os_ = out.stride()
    rc = library().mxfa_split_decode_combine_launch(
        workspace.data_ptr(), workspace.numel() * workspace.element_size(), out.data_ptr(),
        os_[0], os_[-2], batch, hq, kv_heads, hd, _dtype_code(out), num_splits,
        _stream_handle(out.device),
    )
    _check(rc, "mxfa_split_decode_combine_launch")
    return out


def reshape_and_cache(
    key: torch.Tensor,
    value: torch.Tensor,
    key_cache: torch.Tensor,
    value_cache: torch.Tensor,
    slot_mapping: torch.Tensor,
    *,
    k_scale: torch.Tensor | float | None = None,
    v_scale: torch.Tensor | float | None = None,
) -> None:
    """vLLM-format paged append: row t -> slot_mapping[t] (skipped when < 0).

    float8_e4m3fn caches store e4m3fn_rne(saturate(x / scale)) with the
    per-tensor k_scale / v_scale; 16-bit caches are a bit-exact copy."""
    if USE_TORCH_OP and k_scale is None and v_scale is None:
        op = torch_op()
        # The common 16-bit call goes through the C++ operator; it launches
        # nothing and returns False for any other call, taken below.
        if op is not None and op.reshape_and_cache(key, value, key_cache, value_cache,
                                                   slot_mapping):
            return
    if key.dim() != 3 or value.shape != key.shape:
        raise ValueError("key/value must be [num_tokens, kv_heads, head_dim]")
    if key_cache.dim() != 4 or value_cache.shape != key_cache.shape:
        raise ValueError("caches must be [pages, page_size, kv_heads, head_dim]")
    if key.shape[1:] != key_cache.shape[2:]:
        raise ValueError("key/value heads and head_dim must match the cache")
    fp8 = key_cache.dtype == FP8_DTYPE
    if value.dtype != key.dtype or value_cache.dtype != key_cache.dtype or (
            not fp8 and key.dtype != key_cache.dtype):
        raise ValueError("key/value and caches must share a dtype (or the caches be fp8)")
    if key.stride() != value.stride() or key.stride(-1) != 1:
        key, value = key.contiguous(), value.contiguous()
    if value_cache.stride() != key_cache.stride() or key_cache.stride(-1) != 1:
        raise UnsupportedConfig("caches must share strides with a contiguous last dim")
    _require_device(key, value, key_cache, value_cache, slot_mapping)
    slots = slot_mapping
    if slots.dtype != torch.int64:
        slots = slots.to(torch.int64)
    slots = slots.contiguous()
    n = key.shape[0]
    if slots.numel() < n:
        raise ValueError("slot_mapping must have one entry per token")
    cs = key_cache.stride()
    common = (key.data_ptr(), value.data_ptr(), key.stride(0), key.stride(1),
              key_cache.data_ptr(), value_cache.data_ptr(), cs[0], cs[1], cs[2], slots.data_ptr(),
              n, key.shape[1], key.shape[2], key_cache.shape[1], key_cache.shape[0],
              _dtype_code(key))
    if fp8:
        rc = library().mxfa_reshape_and_cache_fp8_launch(
            *common, _scale_ptr(k_scale, key.device, "k_scale"),
            _scale_ptr(v_scale, key.device, "v_scale"), _stream_handle(key.device))
        _check(rc, "mxfa_reshape_and_cache_fp8_launch")
    else:
        rc = library().mxfa_reshape_and_cache_launch(*common, _stream_handle(key.device))
        _check(rc, "mxfa_reshape_and_cache_launch")


def append_kv(
    k: torch.Tensor,
    v: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    block_table: torch.Tensor,
    cache_seqlens: torch.Tensor,
) -> None:
    """Block-table append: k[b, t] -> position cache_seqlens[b] + t (seqlens unchanged)."""
    if k.dim() != 4 or v.shape != k.shape:
        raise ValueError("k/v must be [batch, new_tokens, kv_heads, head_dim]")
    if k_cache.dim() != 4 or v_cache.shape != k_cache.shape:
        raise ValueError("caches must be [pages, page_size, kv_heads, head_dim]")
    if k.shape[2:] != k_cache.shape[2:]:
        raise ValueError("k/v heads and head_dim must match the cache")
    if k.dtype != k_cache.dtype or v.dtype != k.dtype or v_cache.dtype != k.dtype:
        raise ValueError("k/v and caches must share a dtype")
    _require_device(k, v, k_cache, v_cache, block_table, cache_seqlens)
    if k.stride() != v.stride() or k.stride(-1) != 1:
        k, v = k.contiguous(), v.contiguous()
    if v_cache.stride() != k_cache.stride() or k_cache.stride(-1) != 1:
        raise UnsupportedConfig("caches must share strides with a contiguous last dim")
    block_table = _int32_contig(block_table, "block_table")
    cache_seqlens = _int32_contig(cache_seqlens, "cache_seqlens")
    if block_table.dim() != 2 or block_table.shape[0] != k.shape[0] or block_table.shape[1] < 1:
        raise ValueError("block_table must be [batch, width >= 1]")
    if cache_seqlens.numel() != k.shape[0]:
        raise ValueError("cache_seqlens must have one entry per sequence")
    cs = k_cache.stride()
    rc = library().mxfa_append_kv_launch(
        k.data_ptr(), v.data_ptr(), k.stride(0), k.stride(1), k.stride(2), k_cache.data_ptr(),
        v_cache.data_ptr(), cs[0], cs[1], cs[2], block_table.data_ptr(), block_table.stride(0),
        cache_seqlens.data_ptr(), k.shape[0], k.shape[1], k.shape[2], k.shape[3],
        k_cache.shape[1], block_table.shape[1], k_cache.shape[0], _dtype_code(k),
        _stream_handle(k.device),
    )
    _check(rc, "mxfa_append_kv_launch")
