"""The C ABI without a GPU: the library loads, exports what the header declares,
and its integer-only entry points and argument checks behave as documented.

No kernel is launched here: every launch entry below is given arguments that
its host-side checks reject before any HIP call (the checks run first in each
entry point of csrc/split_decode.hip and csrc/kv_append.hip).
"""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest
import torch

from mxflashattn_amd import native

HEADER = Path(__file__).resolve().parents[1] / "include" / "mxfa_mi355x.h"


def header_functions() -> list[str]:
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return re.findall(r"^[A-Za-z_][\w \*]*?\b(mxfa_\w+)\s*\(", text, flags=re.M)


def header_defines() -> dict[str, int]:
    out = {}
    for name, value in re.findall(r"#define (MXFA_\w+)\s+\(?(-?\d+)\)?", HEADER.read_text()):
        out[name] = int(value)
    return out


@pytest.fixture(scope="module")
def lib():
    return native.library()


def test_library_loads_and_reports_header_abi(lib):
    assert native.unavailable_reason() is None
    assert lib.mxfa_abi_version() == header_defines()["MXFA_ABI_VERSION"]


def test_every_header_function_is_exported_and_bound(lib):
    declared = header_functions()
    assert len(declared) == len(set(declared)) == 17
    for name in declared:
        assert hasattr(lib, name), name
    assert set(declared) == set(native.EXPORTED_SYMBOLS) == set(native._SIGNATURES)


def test_return_codes_match_header():
    d = header_defines()
    assert (d["MXFA_OK"], d["MXFA_EUNSUPPORTED"], d["MXFA_EINVAL"], d["MXFA_EWORKSPACE"],
            d["MXFA_ELAUNCH"], d["MXFA_ESCRATCH"]) == (
                native.MXFA_OK, native.MXFA_EUNSUPPORTED, native.MXFA_EINVAL,
                native.MXFA_EWORKSPACE, native.MXFA_ELAUNCH, native.MXFA_ESCRATCH)
    assert native.SCRATCH_BYTES == 8 << 20
    assert native.DTYPE_CODES == {torch.float16: d["MXFA_DTYPE_F16"],
                                  torch.bfloat16: d["MXFA_DTYPE_BF16"]}


def test_strerror_is_distinct_per_code(lib):
    texts = {code: lib.mxfa_strerror(code).decode() for code in (0, -1, -2, -3, -4, -5)}
    assert len(set(texts.values())) == 6
    assert "8 MiB" in texts[-5]
    assert "unsupported" in texts[-1]
    assert lib.mxfa_strerror(-99).decode()


def heuristic_closed_form(b, hq, hkv, hd, ps, btw, cus, elem_bytes=2):
    # Short sequences by the table's capacity C = btw * ps: page size >= 16,
    # W = B * HKV * ceil(C / 16) <= 16384, and head rows of <= 128 bytes with
    # C <= 768, or 256-byte rows with C <= 384 (C <= 512 from B * HKV = 64 on)
    # and W <= 8192 at head dim 256: the per-sequence kernel.
    # Its LDS (4 waves x columns x (HD + 1) floats, columns = HQ / HKV) must
    # stay within 64 KB.
    cap, row = btw * ps, hd * elem_bytes
    units = b * hkv
    work = units * -(-cap // 16)
    mid = (row <= 256 and (cap <= 384 or (cap <= 512 and units >= 64))
           and (hd < 256 or work <= 8192))
    fits = 16 * -(-hq // hkv) * (hd + 1) <= 64 << 10
    if ps >= 16 and work <= 16384 and fits and ((row <= 128 and cap <= 768) or mid):
        return native.SPLITS_PER_SEQUENCE
    # Otherwise one wave per (kv head, range): a workgroup has 4 waves for
    # HKV <= 4, else 8 for head rows of <= 128 bytes and 4 for longer ones;
    # min(HKV, waves) kv heads x waves // that sub-ranges, one workgroup per CU.
    waves = 4 if hkv <= 4 else (8 if row <= 128 else 4)
    kh = min(hkv, waves)
    subs = waves // kh
    gx = -(-hkv // kh)
    n = cus * subs // gx
    n = min(n, b * -(-(btw * ps) // 16))
    return max(1, min(n, 65535))


@pytest.mark.parametrize("args", [
    (32, 32, 8, 128, 16, 512, 256),    # config 2: 256 CUs x 8 waves / 8 kv heads
    (32, 32, 16, 128, 16, 512, 256),   # GQ2: 16 kv heads, two workgroups per range
    (32, 32, 4, 64, 16, 512, 256),     # GQ8 HD64: four kv heads, one range per workgroup
    (32, 24, 6, 64, 16, 512, 256),     # 6 kv heads of 8 waves: one range per workgroup
    (32, 24, 6, 128, 16, 512, 256),    # 6 kv heads, 256-byte rows: two head groups
    (1, 2, 1, 64, 16, 1, 256),         # one tile in total: per sequence
    (1, 2, 1, 64, 8, 2, 256),          # one tile, pages of 8: split
    (4, 8, 2, 64, 16, 32, 256),        # config 1's table: per sequence
    (128, 16, 8, 64, 16, 32, 256),     # config 3: B * HKV * 32 tiles past the bound
    (64, 32, 8, 64, 16, 32, 256),      # on the work bound
    (64, 32, 8, 64, 16, 48, 256),      # C 768: past the work bound
    (32, 32, 8, 64, 16, 48, 256),      # C 768 inside it
    (32, 32, 8, 64, 16, 49, 256),      # C 784
    (8, 32, 8, 128, 16, 24, 256),      # 256-byte rows, C 384
    (8, 32, 8, 128, 16, 25, 256),      # C 400
    (8, 32, 8, 128, 16, 32, 256),      # C 512, B * HKV 64
    (4, 32, 8, 128, 16, 32, 256),      # C 512, B * HKV 32
    (128, 16, 8, 128, 16, 32, 256),    # C 512 past the work bound
    (32, 16, 8, 256, 16, 16, 256),     # HD 256 (fp8: 256-byte rows), W 4096
    (128, 16, 8, 256, 16, 16, 256),    # W 16384: past the HD 256 bound
    (8, 120, 8, 256, 16, 16, 256),     # HD 256, 15 columns: the LDS holds them
    (8, 128, 8, 256, 16, 16, 256),     # HD 256, 16 columns: it does not
    (8, 128, 8, 128, 16, 16, 256),     # HD 128, 16 columns: it does
    (8, 32, 8, 128, 64, 6, 256),       # C 384 in pages of 64
    (8, 16, 4, 256, 16, 4, 256),       # 512-byte rows: always split
    (256, 16, 8, 64, 16, 64, 256),
    (4, 32, 4, 128, 256, 128, 304),    # other CU count
    (16384, 64, 8, 128, 16, 4096, 256),
    (8, 24, 3, 128, 16, 64, 256),      # kv heads not a power of two
    (4, 8, 2, 64, 16, 128, 256),       # config 1: two sub-ranges of two kv heads
    (32, 32, 8, 64, 16, 512, 256),     # GQ4 HD64: eight waves
    (8, 96, 12, 128, 16, 64, 256),
    (32, 64, 4, 256, 16, 512, 256),    # HD256 GQ16
    (16, 48, 16, 256, 16, 128, 256),   # HD256 GQ3
    (32, 32, 32, 128, 16, 512, 256),   # GQ1: 32 kv heads, 8 workgroups per range
])
def test_split_heuristic_closed_form(args):
    assert native.split_heuristic(*args) == heuristic_closed_form(*args)
    # fp8 caches: one-byte rows.
    assert native.split_heuristic(*args, True) == heuristic_closed_form(*args, 1)


@pytest.mark.parametrize("hd", [64, 128, 256])
def test_split_heuristic_over_every_kv_head_count(hd):
    # Every kv head count 1..40 with GQ 1, 2 and 4, a long table (split
    # path) and a short one (per-sequence where it applies), 16-bit and fp8
    # rows: the C rule and its closed form agree everywhere.
    for hkv in range(1, 41):
        for gq in (1, 2, 4):
            for b, btw in ((32, 512), (8, 24)):
                args = (b, gq * hkv, hkv, hd, 16, btw, 256)
                assert native.split_heuristic(*args) == heuristic_closed_form(*args), args
                assert native.split_heuristic(*args, True) == heuristic_closed_form(*args, 1), args


def test_split_heuristic_known_values():
    assert native.split_heuristic(32, 32, 8, 128, 16, 512, 256) == 128
    assert native.split_heuristic(32, 32, 4, 64, 16, 512, 256) == 256
    assert native.split_heuristic(32, 32, 8, 64, 16, 512, 256) == 256
    assert native.split_heuristic(32, 32, 16, 128, 16, 512, 256) == 64
    assert native.split_heuristic(4, 8, 2, 64, 16, 128, 256) == 512
    assert native.split_heuristic(1, 2, 1, 64, 16, 1, 256) == native.SPLITS_PER_SEQUENCE
    assert native.SPLITS_PER_SEQUENCE == -1
    # config 1 (table of 32 pages of 16) and config 3 (B128, 8 kv heads, same table).
    assert native.split_heuristic(4, 8, 2, 64, 16, 32, 256) == -1
    assert native.split_heuristic(128, 16, 8, 64, 16, 32, 256) == 256
    # fp8 HD 128 has 128-byte rows: the 16-bit HD 64 bounds.
    assert native.split_heuristic(32, 32, 8, 128, 16, 48, 256, True) == -1
    assert native.split_heuristic(32, 32, 8, 128, 16, 48, 256) == 128
    # fp8 HD 256 (256-byte rows): 15 columns fit the per-sequence kernel's LDS, 16 do not.
    assert native.split_heuristic(8, 120, 8, 256, 16, 16, 256, True) == -1
    assert native.split_heuristic(8, 128, 8, 256, 16, 16, 256, True) > 0
    # fp8 config 2: eight waves hold all 8 kv heads, one workgroup per range.
    assert native.split_heuristic(32, 32, 8, 128, 16, 512, 256, True) == 256
    assert native.split_heuristic(32, 32, 4, 128, 16, 512, 256, True) == 256
    assert native.split_heuristic(32, 16, 8, 256, 16, 512, 256, True) == 128


def test_split_heuristic_rejects_bad_sizes(lib):
    ns = ctypes.c_int(-7)
    for bad in [(0, 32, 8, 128, 16, 512, 256), (32, 32, 0, 128, 16, 512, 256),
                (32, 32, 8, 128, 16, 0, 256), (32, 32, 8, 128, 16, 512, 0)]:
        assert lib.mxfa_split_heuristic(*bad, ctypes.byref(ns)) == native.MXFA_EINVAL
        assert lib.mxfa_split_heuristic_fp8(*bad, ctypes.byref(ns)) == native.MXFA_EINVAL
    assert lib.mxfa_split_heuristic(32, 32, 8, 128, 16, 512, 256, None) == native.MXFA_EINVAL
    assert lib.mxfa_split_heuristic_fp8(32, 32, 8, 128, 16, 512, 256, None) == native.MXFA_EINVAL
    assert ns.value == -7


@pytest.mark.parametrize("b,hq,hd,ns", [(32, 32, 128, 32), (1, 2, 64, 1), (700, 64, 64, 999)])
def test_workspace_size_formula(b, hq, hd, ns):
    expect = (hq * ns * 2 * hd + hq * ns * 2 + b + 1) * 4
    assert native.workspace_size(b, hq, hd, ns) == expect


def test_workspace_size_rejects_bad_sizes(lib):
    out = ctypes.c_size_t(0)
    assert lib.mxfa_split_decode_workspace_size(0, 32, 128, 4, ctypes.byref(out)) == -2
    assert lib.mxfa_split_decode_workspace_size(1, 32, 128, 0, ctypes.byref(out)) == -2
    assert lib.mxfa_split_decode_workspace_size(1, 32, 128, 4, None) == -2
    assert lib.mxfa_split_decode_workspace_size(1, 32, 128, -2, ctypes.byref(out)) == -2


def test_per_sequence_kernel_needs_no_workspace(lib):
    assert native.workspace_size(32, 32, 128, native.SPLITS_PER_SEQUENCE) == 0
    # Nothing to merge: the combine stage returns at once, launching nothing.
    assert lib.mxfa_split_decode_combine_launch(None, 0, None, 0, 0, 32, 32, 8, 128, 1, -1,
                                                None) == native.MXFA_OK


FAKE = 0x100000  # 16-byte aligned, never dereferenced: every case below fails a host check


def decode_args(**over):
    """A well-formed argument tuple for mxfa_split_decode_launch, with overrides."""
    a = dict(q=FAKE, q_sb=32 * 128, q_sh=128, k=FAKE, v=FAKE, c_sp=16 * 8 * 128, c_st=8 * 128,
             c_sh=128, bt=FAKE, bt_stride=64, seqlens=FAKE, seqlen_add=0, out=FAKE,
             o_sb=32 * 128, o_sh=128, ws=FAKE, ws_bytes=1 << 30, scale=0.088, batch=32, hq=32,
             hkv=8, hd=128, ps=16, btw=64, pages=4096, dtype=1, ns=32, stream=None)
    a.update(over)
    return tuple(a.values())


@pytest.mark.parametrize("over,code", [
    (dict(q=None), -2), (dict(k=None), -2), (dict(bt=None), -2), (dict(seqlens=None), -2),
    (dict(out=None), -2), (dict(batch=0), -2), (dict(ns=0), -2), (dict(seqlen_add=-1), -2),
    (dict(scale=float("nan")), -2), (dict(scale=float("inf")), -2),
    (dict(hd=96), -1), (dict(hd=192), -1), (dict(hd=512), -1), (dict(hq=136), -1),
    (dict(hq=36), -1), (dict(dtype=2), -1), (dict(ps=12), -1), (dict(ps=8192), -1),
    (dict(ns=70000), -1), (dict(batch=16001), -1), (dict(btw=1 << 27, ps=16), -1),
    (dict(q=FAKE + 2), -2), (dict(k=FAKE + 8), -2), (dict(q_sh=100), -2), (dict(c_st=1028), -2),
    (dict(o_sh=130), -2), (dict(out=FAKE + 2), -2),
    (dict(c_st=64), -2), (dict(q_sh=64), -2),  # overlapping rows
    # Output rows that share memory (an expand()ed view, strides below the
    # extent of the dims inside them) would be written by different workgroups.
    (dict(o_sh=0), -2), (dict(o_sb=0), -2), (dict(o_sh=64), -2), (dict(o_sb=31 * 128), -2),
    # A head-major output (batch innermost) is disjoint: it passes the output
    # checks and stops at the workspace size.
    (dict(o_sb=128, o_sh=32 * 128, ws_bytes=1000), -3),
    (dict(ws=None), -3), (dict(ws=FAKE + 8), -3), (dict(ws_bytes=1000), -3),
    # num_splits: ranges >= 1 or the per-sequence kernel (-1), which needs no
    # workspace but keeps every other check; its pieces live in LDS (64 KB at
    # most: HD 256 with 16 columns does not fit).
    (dict(ns=-2), -2), (dict(ns=-1, batch=0), -2), (dict(ns=-1, hd=96), -1),
    (dict(ns=-1, q=FAKE + 2), -2), (dict(ns=-1, ws=None, ws_bytes=0, out=None), -2),
    (dict(ns=-1, hd=256, hq=128, q_sb=128 * 256, q_sh=256, o_sb=128 * 256, o_sh=256,
          c_sp=16 * 8 * 256, c_st=8 * 256, c_sh=256), -1),
])
def test_decode_launch_rejects_before_launching(lib, over, code):
    assert lib.mxfa_split_decode_launch(*decode_args(**over)) == code
    assert lib.mxfa_split_decode_partial_launch(*decode_args(**over)) == code
    fp8 = decode_args(**over)
    assert lib.mxfa_split_decode_fp8_launch(*fp8[:-1], FAKE, FAKE, None) == code
    assert lib.mxfa_split_decode_fp8_partial_launch(*fp8[:-1], None, None, None) == code


@pytest.mark.parametrize("over,code", [
    # fp8 caches: byte strides must stay multiples of 16 (16 e4m3fn elements).
    (dict(c_st=8 * 128 + 8), -2), (dict(c_sh=136), -2), (dict(c_sp=16 * 8 * 128 + 8), -2),
    (dict(c_st=64), -2), (dict(hd=192), -1), (dict(ws_bytes=1000), -3),
])
def test_fp8_decode_launch_rejects_before_launching(lib, over, code):
    args = decode_args(**over)[:-1]
    assert lib.mxfa_split_decode_fp8_launch(*args, FAKE, FAKE, None) == code
    assert lib.mxfa_split_decode_fp8_partial_launch(*args, FAKE, FAKE, None) == code


def test_fp8_decode_rejects_misaligned_scale_pointers(lib):
    args = decode_args()[:-1]
    assert lib.mxfa_split_decode_fp8_launch(*args, FAKE + 2, FAKE, None) == -2
    assert lib.mxfa_split_decode_fp8_launch(*args, FAKE, FAKE + 1, None) == -2
    # 16-bit strides that are fine for 16-bit caches (8 elements) are not for
    # fp8 caches (8 bytes).
    odd = decode_args(c_st=8 * 128 + 8, ws_bytes=1000)
    assert lib.mxfa_split_decode_launch(*odd) == -3  # strides pass, workspace fails
    assert lib.mxfa_split_decode_fp8_launch(*odd[:-1], FAKE, FAKE, None) == -2


def multi_args(**over):
    """A well-formed argument tuple for mxfa_split_decode_multi_launch (QL = 2)."""
    a = dict(q=FAKE, q_sb=2 * 32 * 128, q_st=32 * 128, q_sh=128, ql=2, causal=1, window=-1,
             sinks=None, softcap=0.0, alibi=None, k=FAKE, v=FAKE,
             c_sp=16 * 8 * 128, c_st=8 * 128, c_sh=128, bt=FAKE, bt_stride=64, seqlens=FAKE,
             seqlen_add=0, out=FAKE, o_sb=2 * 32 * 128, o_st=32 * 128, o_sh=128, ws=FAKE,
             ws_bytes=1 << 30, scale=0.088, batch=32, hq=32, hkv=8, hd=128, ps=16, btw=64,
             pages=4096, dtype=1, kv_dtype=1, ks=None, vs=None, ns=32, stream=None)
    a.update(over)
    return tuple(a.values())


@pytest.mark.parametrize("over,code", [
    (dict(ql=0), -2), (dict(ql=5), -1), (dict(ql=2, hkv=2), -1),   # QL x GQ > 16
    (dict(q_st=100), -2), (dict(o_st=130), -2),
    (dict(o_st=128, o_sh=128), -2),                                 # token rows overlap heads
    (dict(kv_dtype=0), -1), (dict(kv_dtype=2, ks=FAKE + 1), -2),
    (dict(ws_bytes=native.workspace_size(32, 32, 128, 32)), -3),     # sized for QL = 1
    (dict(hd=96), -1), (dict(q=None), -2),
    (dict(window=-2), -2), (dict(window=(1 << 30) + 1), -1),        # sliding window range
    (dict(window=0, ws_bytes=1000), -3), (dict(window=1 << 30, ws_bytes=1000), -3),
    (dict(sinks=FAKE + 2), -2), (dict(sinks=FAKE, ws_bytes=1000), -3),   # sink pointer
    (dict(softcap=-1.0), -2), (dict(softcap=float("nan")), -2), (dict(softcap=float("inf")), -2),
    (dict(softcap=30.0, ws_bytes=1000), -3),
    (dict(alibi=FAKE + 1), -2), (dict(alibi=FAKE, ws_bytes=1000), -3),
    (dict(seqlen_add=-(1 << 30) - 1), -2),                          # below the negative floor
    (dict(seqlen_add=-(1 << 30), ws_bytes=1000), -3),               # a negative add is taken
])
def test_multi_launch_rejects_before_launching(lib, over, code):
    assert lib.mxfa_split_decode_multi_launch(*multi_args(**over)) == code


def test_multi_launch_workspace_is_per_query_token(lib):
    need = native.workspace_size(32, 64, 128, 32)  # q_heads x q_len rows
    assert lib.mxfa_split_decode_multi_launch(*multi_args(ws_bytes=need - 1)) == -3


def test_combine_rejects_before_launching(lib):
    ws = native.workspace_size(4, 8, 64, 3)
    f = lib.mxfa_split_decode_combine_launch
    assert f(None, ws, FAKE, 512, 64, 4, 8, 2, 64, 0, 3, None) == -2
    assert f(FAKE, ws - 4, FAKE, 512, 64, 4, 8, 2, 64, 0, 3, None) == -3
    assert f(FAKE, ws, FAKE, 512, 64, 4, 8, 2, 96, 0, 3, None) == -1
    assert f(FAKE, ws, FAKE, 512, 64, 4, 8, 3, 64, 0, 3, None) == -1  # GQ not an integer
    assert f(FAKE, ws, FAKE, 512, 64, 4, 8, 2, 64, 5, 3, None) == -1
    assert f(FAKE, ws, FAKE, 512, 64, 0, 8, 2, 64, 0, 3, None) == -2
    assert f(FAKE, ws, FAKE + 2, 512, 64, 4, 8, 2, 64, 0, 3, None) == -2
    assert f(FAKE, ws, FAKE, 0, 64, 4, 8, 2, 64, 0, 3, None) == -2  # rows of all sequences alias
    assert f(FAKE, ws, FAKE, 512, 0, 4, 8, 2, 64, 0, 3, None) == -2  # rows of all heads alias


def probe_args(**over):
    """A well-formed argument tuple for mxfa_stream_probe_launch, with overrides."""
    a = dict(q=FAKE, q_sb=32 * 128, q_sh=128, k=FAKE, v=FAKE, c_sp=16 * 8 * 128, c_st=8 * 128,
             c_sh=128, bt=FAKE, bt_stride=64, seqlens=FAKE, seqlen_add=0, sink=FAKE,
             sink_bytes=1 << 30, batch=32, hq=32, hkv=8, hd=128, ps=16, btw=64, pages=4096,
             dtype=1, ns=32, nbuf=0, stream=None)
    a.update(over)
    return tuple(a.values())


@pytest.mark.parametrize("over,code", [
    (dict(q=None), -2), (dict(k=None), -2), (dict(batch=0), -2), (dict(hq=36), -1),
    (dict(hd=256, q_sb=32 * 256, q_sh=256, c_sp=16 * 8 * 256, c_st=8 * 256, c_sh=256), -1),
    (dict(ps=8, c_sp=8 * 8 * 128), -1), (dict(ns=-1), -1), (dict(nbuf=1), -1), (dict(nbuf=5), -1),
    (dict(dtype=2), -1), (dict(sink=None), -3), (dict(sink=FAKE + 2), -3),
    (dict(sink_bytes=8 * 32 * 256 - 4), -3),
])
def test_stream_probe_rejects_before_launching(lib, over, code):
    assert lib.mxfa_stream_probe_launch(*probe_args(**over)) == code


@pytest.mark.parametrize("over,code", [
    (dict(buf=None), -2), (dict(buf=FAKE + 8), -2), (dict(nbytes=0), -2), (dict(nbytes=1000), -2),
    (dict(layout=2), -2), (dict(layout=-1), -2), (dict(workgroups=0), -2), (dict(depth=2), -1),
    (dict(depth=32), -1), (dict(sink=None), -3), (dict(sink=FAKE + 2), -3),
    (dict(sink_bytes=4 * 1024 - 4), -3),
])
def test_stream_read_rejects_before_launching(lib, over, code):
    a = dict(buf=FAKE, nbytes=1 << 20, layout=0, depth=8, workgroups=4, sink=FAKE,
             sink_bytes=4 * 1024, stream=None)
    a.update(over)
    assert lib.mxfa_stream_read_launch(*a.values()) == code


def test_decode_workspace_boundary_is_exact(lib):
    need = native.workspace_size(32, 32, 128, 32)
    assert lib.mxfa_split_decode_launch(*decode_args(ws_bytes=need - 1)) == -3


def test_append_entry_points_reject_before_launching(lib):
    rc = lib.mxfa_reshape_and_cache_launch(FAKE, FAKE, 1024, 128, FAKE, FAKE, 16384, 1024, 128,
                                           None, 4, 8, 128, 16, 100, 1, None)
    assert rc == -2  # tokens but no slot mapping
    rc = lib.mxfa_reshape_and_cache_launch(FAKE, FAKE, 1024, 128, FAKE, FAKE, 16384, 1024, 128,
                                           FAKE, 4, 8, 100, 16, 100, 1, None)
    assert rc == -1  # head dim not a multiple of 8
    rc = lib.mxfa_reshape_and_cache_launch(FAKE, FAKE, 1024, 128, FAKE, FAKE, 16384, 1024, 128,
                                           FAKE, 4, 8, 128, 16, 100, 7, None)
    assert rc == -1  # dtype
    rc = lib.mxfa_append_kv_launch(FAKE, FAKE, 4096, 1024, 128, FAKE, FAKE, 16384, 1024, 128,
                                   None, 8, None, 2, 4, 8, 128, 16, 8, 100, 1, None)
    assert rc == -2  # rows to write but no table
    rc = lib.mxfa_append_kv_launch(FAKE, FAKE, 4096, 1024, 128, FAKE + 4, FAKE, 16384, 1024, 128,
                                   FAKE, 8, FAKE, 2, 4, 8, 128, 16, 8, 100, 1, None)
    assert rc == -2  # misaligned cache


def test_fp8_append_rejects_before_launching(lib):
    f = lib.mxfa_reshape_and_cache_fp8_launch
    ok = (FAKE, FAKE, 1024, 128, FAKE, FAKE, 16384, 1024, 128, FAKE, 4, 8, 128, 16, 100, 1,
          FAKE, FAKE, None)

    def call(**over):
        names = ("key", "value", "s_t", "s_h", "kc", "vc", "c_sp", "c_st", "c_sh", "slots", "n",
                 "hkv", "hd", "ps", "pages", "dtype", "ks", "vs", "stream")
        a = dict(zip(names, ok))
        a.update(over)
        return f(*a.values())

    assert call(slots=None) == -2
    assert call(hd=120) == -1           # not a multiple of 16
    assert call(dtype=5) == -1
    assert call(c_st=1032) == -2        # byte stride not a multiple of 16
    assert call(kc=FAKE + 8) == -2
    assert call(ks=FAKE + 2) == -2
    assert call(n=0, slots=None) == 0   # nothing to write


def test_empty_appends_are_no_ops(lib):
    assert lib.mxfa_reshape_and_cache_launch(FAKE, FAKE, 1024, 128, FAKE, FAKE, 16384, 1024,
                                             128, None, 0, 8, 128, 16, 100, 1, None) == 0
    assert lib.mxfa_append_kv_launch(FAKE, FAKE, 4096, 1024, 128, FAKE, FAKE, 16384, 1024, 128,
                                     None, 8, None, 0, 4, 8, 128, 16, 8, 100, 1, None) == 0


def test_python_layer_refuses_host_tensors():
    q = torch.zeros(2, 1, 8, 64, dtype=torch.float16)
    cache = torch.zeros(4, 16, 2, 64, dtype=torch.float16)
    bt = torch.zeros(2, 2, dtype=torch.int32)
    sl = torch.ones(2, dtype=torch.int32)
    with pytest.raises(ValueError, match="GPU tensors"):
        native.paged_decode_split(q, cache, cache, bt, sl, 0.125)
    with pytest.raises(ValueError, match="GPU tensors"):
        native.reshape_and_cache(torch.zeros(3, 2, 64, dtype=torch.float16),
                                 torch.zeros(3, 2, 64, dtype=torch.float16), cache, cache,
                                 torch.arange(3))
    with pytest.raises(ValueError, match="GPU tensors"):
        native.append_kv(torch.zeros(2, 1, 2, 64, dtype=torch.float16),
                         torch.zeros(2, 1, 2, 64, dtype=torch.float16), cache, cache, bt, sl)


@pytest.mark.parametrize("hq,hkv,hd,dtype,ps,match", [
    (8, 2, 96, torch.float16, 16, "head_dim"), (6, 4, 64, torch.float16, 16, "GQA"),
    (34, 2, 64, torch.float16, 16, "GQA"), (8, 2, 64, torch.float32, 16, "float16"),
    (8, 2, 64, torch.float16, 12, "page size"),
])
def test_python_shape_contract(hq, hkv, hd, dtype, ps, match):
    q = torch.zeros(2, 1, hq, hd, dtype=dtype)
    cache = torch.zeros(4, ps, hkv, hd, dtype=dtype)
    with pytest.raises(native.UnsupportedConfig, match=match):
        native.check_decode_shapes(q, cache, cache)


def test_causal_queries_past_sixteen_columns_run_in_token_chunks():
    q = torch.zeros(2, 5, 16, 64, dtype=torch.bfloat16)   # 5 tokens x GQ 4 = 20 columns
    cache = torch.zeros(4, 16, 4, 64, dtype=torch.bfloat16)
    with pytest.raises(native.UnsupportedConfig, match="exceeds"):
        native.check_decode_shapes(q, cache, cache)
    native.check_decode_shapes(q, cache, cache, causal=True)
    # 4 tokens per launch; each chunk ends where its sequences are cut.
    assert native.token_chunks(5, 4, 0) == [(0, 4, -1), (4, 5, 0)]
    assert native.token_chunks(7, 2, 3) == [(0, 2, -2), (2, 4, 0), (4, 6, 2), (6, 7, 3)]
    assert native.token_chunks(3, 16, 0) == [(0, 3, 0)]
    assert native.token_chunks(16, 1, 0)[0] == (0, 1, -15)


@pytest.mark.parametrize("hq,hkv,hd,cache_dtype", [
    (6, 2, 64, torch.float16), (16, 1, 128, torch.bfloat16), (16, 16, 256, torch.bfloat16),
    (32, 8, 128, torch.float8_e4m3fn), (12, 4, 256, torch.float8_e4m3fn),
])
def test_python_shape_contract_wider_than_the_reference(hq, hkv, hd, cache_dtype):
    """GQ 1..16, HD 256 and fp8 caches pass the kernel contract."""
    q = torch.zeros(2, 1, hq, hd, dtype=torch.bfloat16 if cache_dtype != torch.float16
                    else torch.float16)
    cache = torch.zeros(4, 16, hkv, hd, dtype=cache_dtype)
    native.check_decode_shapes(q, cache, cache)


def test_python_shape_contract_rejects_mixed_and_fnuz_caches():
    q = torch.zeros(2, 1, 8, 64, dtype=torch.bfloat16)
    fp8 = torch.zeros(4, 16, 2, 64, dtype=torch.float8_e4m3fn)
    with pytest.raises(native.UnsupportedConfig):
        native.check_decode_shapes(q, fp8, torch.zeros(4, 16, 2, 64, dtype=torch.bfloat16))
    fnuz = torch.zeros(4, 16, 2, 64, dtype=torch.float8_e4m3fnuz)
    with pytest.raises(native.UnsupportedConfig):
        native.check_decode_shapes(q, fnuz, fnuz)


def test_no_alloc_entry_refuses_oversized_and_invalid_calls_before_launch(lib):
    # 32 heads x 300 ranges x 2 x 128 floats is more than the 8 MiB array; the
    # size check runs before any HIP call, so no GPU is needed.
    fn = lib.mxfa_split_decode_noalloc_launch
    args = [1, 0, 0, 1, 1, 0, 0, 0, 1, 0, 1, 0, 1, 0, 0, 0.1, 2, 32, 8, 128, 16, 4, 8, 1, 300,
            None]
    assert fn(*args) == native.MXFA_ESCRATCH
    args[16] = 0  # batch
    assert fn(*args) == native.MXFA_EINVAL
