"""Per-wave timeline of the split decode kernels on an MI355X (profiling aid).

The profiling build of the library (``-DMXFA_WAVE_STAMPS``, into
``_lib/stamped/``) stamps, per wave of the partial (or per-sequence) kernel,
the real-time clock (100 MHz) at kernel entry, when the lengths have arrived,
after the tile scan, when the range's first sequence is known, when the first
page id has arrived, when the first tiles' loads are issued, when the first
tile's data has arrived and at the end, with the wave's tile count; and per
block of the combine kernel its entry, when the prefix sums are read, when
the pieces are folded and its end. This module runs decode calls of the named
bench workloads on that build and prints one JSON line per workload with the
medians, over six calls, of (µs after the partial kernel's first wave entry):

  entry_last       the last wave's entry
  lengths_med      lengths arrived, median wave (waves with no sequence to
                   read pass at once)
  lengths_wg_med   the lengths' round trip: per workgroup, the last wave's
                   arrival after the first wave's entry; median workgroup
  prologue_med     tile scan done, median wave
  search_med       range's first sequence known, median wave
  page_id_med      first page id arrived, median wave
  loop_med/last    first tiles' loads issued, median / last wave
  data_med/last    first tile's data arrived, median / last wave
  end_med/last     end, median / last wave
  us_per_tile      median per-wave time per tile once streaming
  slowest_wg       slowest workgroup's time per tile over the median one
  corr_end_speed   correlation of workgroups' end times with their speed
  combine_*        the combine kernel's first block entry, median block's
                   prefix sums read / pieces folded, and last block end
                   (absent where the call has no combine launch)

Build here (hipcc, no GPU needed):  python -m mxflashattn_amd.wave_timeline --build
Run on the GPU box:                 python -m mxflashattn_amd.wave_timeline cell_gq8_d64 ...
"""

from __future__ import annotations

import argparse
import ctypes
import json
import statistics
import sys
from pathlib import Path

STAMPED_LIB = Path(__file__).resolve().parent / "_lib" / "stamped" / "libmxfa_mi355x.so"
# Buffer layout of the profiling build (split_kernels.h): WAVES_MAX waves of
# WAVE_WORDS words, then COMBINE_BLOCKS blocks of COMBINE_WORDS words.
WAVES_MAX = 65536
WAVE_WORDS = 16
COMBINE_BLOCKS = 65536
COMBINE_WORDS = 4


def build() -> Path:
    from . import _build

    # The stamps keep clock values live across the prologue: two fp8
    # instantiations then hold 20 bytes per lane in scratch, which the
    # shipped build refuses but a timing aid may carry.
    return _build.build(lib_path=STAMPED_LIB, extra=("-DMXFA_WAVE_STAMPS",), torch_op=False,
                        check_registers=False)


def _summary(stamps, combine) -> dict:
    import numpy as np

    rows = []
    for d, cb in zip(stamps, combine):
        d = d[d[:, 5] == 1].astype(np.float64)
        t0 = d[:, 0].min()

        def rel(k):  # words 8-11 stay 0 where a kernel does not stamp them
            v = d[:, k]
            return (np.where(v > 0, v, t0) - t0) * 0.01

        entry, pro, loop, end = rel(0), rel(1), rel(2), rel(3)
        tiles = np.maximum(d[:, 4], 1)
        speed = (end - loop) / tiles
        wg = d[:, 6]
        groups = np.unique(wg)
        wg_speed = np.array([speed[wg == g].mean() for g in groups])
        wg_end = np.array([end[wg == g].max() for g in groups])
        lengths = rel(8)
        lengths_wg = np.array([lengths[wg == g].max() - entry[wg == g].min() for g in groups])
        row = dict(
            waves=len(d), tiles_med=float(np.median(tiles)), entry_last=float(entry.max()),
            lengths_med=float(np.median(lengths)),
            lengths_wg_med=float(np.median(lengths_wg)) if d[:, 8].any() else 0.0,
            prologue_med=float(np.median(pro)),
            search_med=float(np.median(rel(9))), page_id_med=float(np.median(rel(10))),
            loop_med=float(np.median(loop)), loop_last=float(loop.max()),
            data_med=float(np.median(rel(11))), data_last=float(rel(11).max()),
            end_med=float(np.median(end)), end_last=float(end.max()),
            us_per_tile=float(np.median(speed)),
            slowest_wg=float(wg_speed.max() / np.median(wg_speed)),
            corr_end_speed=float(np.corrcoef(wg_end, wg_speed)[0, 1]) if len(groups) > 2 else 0.0,
        )
        cb = cb[cb[:, 0] > 0].astype(np.float64)
        if len(cb):
            c_rel = (cb - t0) * 0.01
            folded = c_rel[cb[:, 2] > 0, 2]
            row.update(
                combine_blocks=len(cb), combine_entry_first=float(c_rel[:, 0].min()),
                combine_read_med=float(np.median(c_rel[:, 1])),
                combine_fold_med=float(np.median(folded)) if len(folded) else 0.0,
                combine_end_last=float(c_rel[:, 3].max()),
            )
        rows.append(row)
    keys = [k for k in rows[0] if all(k in r for r in rows)]
    return {k: round(statistics.median(r[k] for r in rows), 3) for k in keys}


def run(names: list[str], calls: int = 6) -> list[dict]:
    import torch

    from . import native
    from .workloads import CELLS, CONFIGS, WIDE, make_paged_batch

    if not STAMPED_LIB.exists():
        raise SystemExit(f"{STAMPED_LIB} is missing: run python -m mxflashattn_amd.wave_timeline "
                         "--build first")
    native.LIB_PATH = STAMPED_LIB  # the ctypes path loads the profiling build
    native.USE_TORCH_OP = False
    lib = native.library()
    lib.mxfa_wave_stamps_set.argtypes = [ctypes.c_void_p]
    device = torch.device("cuda", 0)
    words = WAVES_MAX * WAVE_WORDS + COMBINE_BLOCKS * COMBINE_WORDS
    buf = torch.zeros(words, dtype=torch.int64, device=device)
    lib.mxfa_wave_stamps_set(buf.data_ptr())
    out = []
    try:
        for name in names:
            spec = {**CELLS, **CONFIGS, **WIDE}[name]
            b = make_paged_batch(**{k: v for k, v in spec.items() if k != "causal"},
                                 device=device)
            res = torch.empty_like(b.q)
            ns = native.default_num_splits(b.q, b.k_cache, b.block_table)
            stamps, combine = [], []
            for _ in range(calls):
                for _ in range(4):  # untimed calls first
                    native.paged_decode_split(b.q, b.k_cache, b.v_cache, b.block_table,
                                              b.cache_seqlens, b.scale, out=res, num_splits=ns)
                torch.cuda.synchronize()
                buf.zero_()
                native.paged_decode_split(b.q, b.k_cache, b.v_cache, b.block_table,
                                          b.cache_seqlens, b.scale, out=res, num_splits=ns)
                torch.cuda.synchronize()
                host = buf.cpu().numpy()
                stamps.append(host[:WAVES_MAX * WAVE_WORDS].reshape(WAVES_MAX, WAVE_WORDS))
                combine.append(host[WAVES_MAX * WAVE_WORDS:].reshape(COMBINE_BLOCKS, COMBINE_WORDS))
            line = {"workload": name, "num_splits": ns, **_summary(stamps, combine)}
            print(json.dumps(line), flush=True)
            out.append(line)
            del b
            torch.cuda.empty_cache()
    finally:
        lib.mxfa_wave_stamps_set(None)
    return out


def main(argv: list[str] | None = None) -> int:
    ap = argparse.ArgumentParser(description=__doc__,
                                 formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("workloads", nargs="*")
    ap.add_argument("--build", action="store_true", help="build the profiling library and exit")
    ap.add_argument("--calls", type=int, default=6)
    args = ap.parse_args(argv)
    if args.build:
        print(build())
        return 0
    run(args.workloads or ["config2_qwen3_4b"], args.calls)
    return 0


if __name__ == "__main__":
    sys.exit(main())
