"""ctypes wrapper of ``oracle/libdecode_ref.so`` (test infrastructure only).

Builds the library with ``make -C oracle`` on first use when it is missing.
Inputs are CPU torch tensors; fp16/bf16 values are widened to float32 exactly
before the fp64 computation.
"""

from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np
import torch

ORACLE_DIR = Path(__file__).resolve().parent
LIB_PATH = ORACLE_DIR / "libdecode_ref.so"

_lib: ctypes.CDLL | None = None


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(ORACLE_DIR)], check=True)
    return LIB_PATH


def library() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        lib = ctypes.CDLL(str(LIB_PATH))
        p = ctypes.c_void_p
        i = ctypes.c_int
        lib.oracle_paged_decode_f64.argtypes = [p, p, p, p, i, p, i, i, i, i, i, i,
                                                ctypes.c_double, p]
        lib.oracle_paged_decode_f64.restype = i
        lib.oracle_append_kv_u16.argtypes = [p, p, p, p, p, i, p, i, i, i, i, i, i]
        lib.oracle_append_kv_u16.restype = i
        lib.oracle_reshape_and_cache_u16.argtypes = [p, p, p, p, p, i, i, i, i, i]
        lib.oracle_reshape_and_cache_u16.restype = i
        sz = ctypes.c_size_t
        lib.oracle_e4m3fn_decode.argtypes = [p, p, sz]
        lib.oracle_e4m3fn_decode.restype = i
        lib.oracle_e4m3fn_encode.argtypes = [p, p, sz]
        lib.oracle_e4m3fn_encode.restype = i
        f = ctypes.c_float
        lib.oracle_reshape_and_cache_fp8.argtypes = [p, p, i, f, f, p, p, p, i, i, i, i, i]
        lib.oracle_reshape_and_cache_fp8.restype = i
        _lib = lib
    return _lib


def _f32(t: torch.Tensor) -> np.ndarray:
    return np.ascontiguousarray(t.detach().cpu().float().numpy())


def _i32(t: torch.Tensor) -> np.ndarray:
    return np.ascontiguousarray(t.detach().cpu().to(torch.int32).numpy())


def _u16(t: torch.Tensor) -> np.ndarray:
    return np.ascontiguousarray(t.detach().cpu().contiguous().view(torch.int16).numpy()).view(np.uint16)


def _ptr(a: np.ndarray) -> int:
    return a.ctypes.data


def paged_decode_f64(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                     block_table: torch.Tensor, seqlens: torch.Tensor,
                     scale: float) -> np.ndarray:
    """q [B,HQ,D] (or [B,1,HQ,D]) -> fp64 [B,HQ,D]; zeros for empty sequences."""
    qb = _f32(q.reshape(q.shape[0], q.shape[-2], q.shape[-1]))
    kc, vc = _f32(k_cache), _f32(v_cache)
    bt, sl = _i32(block_table), _i32(seqlens)
    b, hq, d = qb.shape
    p, ps, hkv, _ = kc.shape
    out = np.zeros((b, hq, d), dtype=np.float64)
    rc = library().oracle_paged_decode_f64(_ptr(qb), _ptr(kc), _ptr(vc), _ptr(bt), bt.shape[1],
                                           _ptr(sl), b, hq, hkv, d, ps, p, float(scale),
                                           _ptr(out))
    if rc != 0:
        raise ValueError(f"oracle_paged_decode_f64 rejected the inputs ({rc})")
    return out


def append_kv(k: torch.Tensor, v: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
              block_table: torch.Tensor, seqlens: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Bitwise block-table append on copies of the caches; returns the new caches."""
    kk, vv = _u16(k), _u16(v)
    kc, vc = _u16(k_cache).copy(), _u16(v_cache).copy()
    bt, sl = _i32(block_table), _i32(seqlens)
    b, s, hkv, d = kk.shape
    library().oracle_append_kv_u16(_ptr(kk), _ptr(vv), _ptr(kc), _ptr(vc), _ptr(bt), bt.shape[1],
                                   _ptr(sl), b, s, hkv, d, kc.shape[1], kc.shape[0])
    as_t = lambda a: torch.from_numpy(a.view(np.int16)).view(k_cache.dtype)
    return as_t(kc), as_t(vc)


def reshape_and_cache(key: torch.Tensor, value: torch.Tensor, k_cache: torch.Tensor,
                      v_cache: torch.Tensor, slots: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Bitwise slot-mapping append on copies of the caches; returns the new caches."""
    kk, vv = _u16(key), _u16(value)
    kc, vc = _u16(k_cache).copy(), _u16(v_cache).copy()
    sm = np.ascontiguousarray(slots.detach().cpu().to(torch.int64).numpy())
    t, hkv, d = kk.shape
    library().oracle_reshape_and_cache_u16(_ptr(kk), _ptr(vv), _ptr(kc), _ptr(vc), _ptr(sm), t,
                                           hkv, d, kc.shape[1], kc.shape[0])
    as_t = lambda a: torch.from_numpy(a.view(np.int16)).view(k_cache.dtype)
    return as_t(kc), as_t(vc)


def _u8(t: torch.Tensor) -> np.ndarray:
    return np.ascontiguousarray(t.detach().cpu().contiguous().view(torch.uint8).numpy())


def e4m3fn_decode(codes: torch.Tensor) -> torch.Tensor:
    """fp8 e4m3fn tensor (or its uint8 codes) -> float32, exact; NaN codes -> NaN."""
    raw = _u8(codes)
    out = np.empty(raw.shape, dtype=np.float32)
    library().oracle_e4m3fn_decode(_ptr(raw), _ptr(out), raw.size)
    return torch.from_numpy(out)


def e4m3fn_encode(x: torch.Tensor) -> torch.Tensor:
    """float32 -> e4m3fn codes (uint8): saturating, round to nearest even."""
    xs = np.ascontiguousarray(x.detach().cpu().float().numpy())
    out = np.empty(xs.shape, dtype=np.uint8)
    library().oracle_e4m3fn_encode(_ptr(xs), _ptr(out), xs.size)
    return torch.from_numpy(out)


def paged_decode_fp8_f64(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                         block_table: torch.Tensor, seqlens: torch.Tensor, scale: float,
                         k_scale: float, v_scale: float) -> np.ndarray:
    """fp64 attention over an fp8 cache dequantised as k_scale*K, v_scale*V:
    the exact fp8 values go to the fp64 oracle with scale*k_scale, and the
    output is multiplied by v_scale (both in fp64)."""
    kf = e4m3fn_decode(k_cache)
    vf = e4m3fn_decode(v_cache)
    out = paged_decode_f64(q, kf, vf, block_table, seqlens, float(scale) * float(k_scale))
    return out * float(v_scale)


def reshape_and_cache_fp8(key: torch.Tensor, value: torch.Tensor, k_cache: torch.Tensor,
                          v_cache: torch.Tensor, slots: torch.Tensor, k_scale: float,
                          v_scale: float) -> tuple[torch.Tensor, torch.Tensor]:
    """Slot-mapping append into copies of fp8 caches; returns the new caches (uint8 codes)."""
    kk, vv = _u16(key), _u16(value)
    kc, vc = _u8(k_cache).copy(), _u8(v_cache).copy()
    sm = np.ascontiguousarray(slots.detach().cpu().to(torch.int64).numpy())
    t, hkv, d = kk.shape
    library().oracle_reshape_and_cache_fp8(_ptr(kk), _ptr(vv), int(key.dtype == torch.bfloat16),
                                           float(k_scale), float(v_scale), _ptr(kc), _ptr(vc),
                                           _ptr(sm), t, hkv, d, kc.shape[1], kc.shape[0])
    return torch.from_numpy(kc), torch.from_numpy(vc)
