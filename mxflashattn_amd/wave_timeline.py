"""Per-wave timeline of the split partial kernel on an MI355X (profiling aid).

The profiling build of the library (``-DMXFA_WAVE_STAMPS``, into
``_lib/stamped/``) stamps, per wave, the real-time clock (100 MHz) at kernel
entry, after the tile scan, when the first tiles' loads are issued and at the
end, with the wave's tile count. This module runs decode calls of the named
bench workloads on that build and prints one JSON line per workload with the
medians, over six calls, of:

  entry_last       the last wave's entry (µs after the first wave's)
  prologue_med     tile scan done, median wave
  loop_med/last    first tiles' loads issued, median / last wave
  end_med/last     end, median / last wave
  us_per_tile      median per-wave time per tile once streaming
  slowest_wg       slowest workgroup's time per tile over the median one
  corr_end_speed   correlation of workgroups' end times with their speed

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
WAVES_MAX = 65536


def build() -> Path:
    from . import _build

    return _build.build(lib_path=STAMPED_LIB, extra=("-DMXFA_WAVE_STAMPS",), torch_op=False)


def _summary(stamps, calls: int) -> dict:
    import numpy as np

    rows = []
    for d in stamps:
        d = d[d[:, 5] == 1].astype(np.float64)
        t0 = d[:, 0].min()
        entry, pro, loop, end = [(d[:, k] - t0) * 0.01 for k in range(4)]
        tiles = np.maximum(d[:, 4], 1)
        speed = (end - loop) / tiles
        wg = d[:, 6]
        groups = np.unique(wg)
        wg_speed = np.array([speed[wg == g].mean() for g in groups])
        wg_end = np.array([end[wg == g].max() for g in groups])
        rows.append(dict(
            waves=len(d), tiles_med=float(np.median(tiles)), entry_last=float(entry.max()),
            prologue_med=float(np.median(pro)), loop_med=float(np.median(loop)),
            loop_last=float(loop.max()), end_med=float(np.median(end)), end_last=float(end.max()),
            us_per_tile=float(np.median(speed)),
            slowest_wg=float(wg_speed.max() / np.median(wg_speed)),
            corr_end_speed=float(np.corrcoef(wg_end, wg_speed)[0, 1]) if len(groups) > 2 else 0.0,
        ))
    return {k: round(statistics.median(r[k] for r in rows), 3) for k in rows[0]}


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
    buf = torch.zeros(WAVES_MAX * 8, dtype=torch.int64, device=device)
    lib.mxfa_wave_stamps_set(buf.data_ptr())
    out = []
    try:
        for name in names:
            spec = {**CELLS, **CONFIGS, **WIDE}[name]
            b = make_paged_batch(**{k: v for k, v in spec.items() if k != "causal"},
                                 device=device)
            res = torch.empty_like(b.q)
            ns = native.default_num_splits(b.q, b.k_cache, b.block_table)
            stamps = []
            for _ in range(calls):
                for _ in range(4):  # untimed calls first
                    native.paged_decode_split(b.q, b.k_cache, b.v_cache, b.block_table,
                                              b.cache_seqlens, b.scale, out=res, num_splits=ns)
                torch.cuda.synchronize()
                buf.zero_()
                native.paged_decode_split(b.q, b.k_cache, b.v_cache, b.block_table,
                                          b.cache_seqlens, b.scale, out=res, num_splits=ns)
                torch.cuda.synchronize()
                stamps.append(buf.view(WAVES_MAX, 8).cpu().numpy())
            line = {"workload": name, "num_splits": ns, **_summary(stamps, calls)}
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
