#!/usr/bin/env python3
"""Decode-attention benchmark on one MI355X (BASELINE.json metric).

One step = one split-KV paged decode call (two kernels: the split partial
kernel, then the LSE combine of the sequences that cross a work-range end; one
per-sequence kernel where the split heuristic picks it for short sequences)
over the whole synthetic batch of the named workload, inputs already resident
in HBM. The KV pool is rotated across copies
totalling >= 1 GB so the 256 MB Infinity Cache cannot serve repeated reads.
Prints ONE JSON line:

  value        effective KV GB/s = sum_b 4*L_b*HKV*HD / (us per call); us per
               call is the median of 10 timed regions of exactly --steps
               calls, each region one replay of a HIP graph holding those
               calls (no host launch overhead), after 100 ms of untimed
               replays (clock ramp after the idle input build); timed_calls
               counts them all
  us_per_call_eager  the same calls launched one by one from Python, median of
               per-call HIP events
  us_per_call_warm   graph replays on one KV pool, never rotated (cache-warm
               where the working set fits the Infinity Cache; not `value`)
  stream_probe the partial kernel's gather alone, no math (mxfa_stream_probe_launch),
               at the kernel's pipeline depth and at 2-4 tiles in flight per
               wave: microseconds and algorithmic GB/s, the access pattern's
               ceiling on this device
  read_ceiling the plain streaming read (mxfa_stream_read_launch) of the same
               byte counts as config 2, GQ8 HD64 and config 3, best over
               layouts, bytes in flight and workgroups per CU: the device's
               read rate with no access pattern at all
  roofline     the dominant kernel, split_partial_kernel, alone: algorithmic
               bytes (KV + q + out + used block-table entries + lengths) / its
               average duration (HIP events around graph replays of
               partial-only launches, on the launch stream), against 8 TB/s
  cpu_baseline the reference's own CPU implementation of the path (its ATen
               backend csrc/mxmac, built from its sources into oracle/_ref)
               on the host cores, bounded sample of the workload, plus config 1
               (the reference's CPU-runnable case); the fp32 restatement
               (oracle.reference_port) is timed beside it
  cells        the six GQ x HD cells of config 2 and configs 1, 3, 4
  wide         shapes beyond the reference's contract at config 2's batch and
               lengths: fp8 (e4m3fn) caches, head dim 256, GQ 1 and 16,
               4 query tokens per sequence (causal draft-token verification)
               and a 1024-key sliding window
  decode_step  config 5: decode tok/s of a 36-layer random-init Qwen3-4B-shaped
               model whose attention runs through the vLLM backend path
               (HIP-graph replayed steps), and attention's share of the step;
               decode_step_eager the same steps launched from Python (vLLM's
               enforce_eager, the reference's end-to-end mode);
               decode_step_fp8 is the same step with an fp8 KV cache
  host_us_per_call  host time of one eager decode call through the public API,
               the C++ operator and the binding (and with the operator off)
"""

from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import sys
import time
from pathlib import Path

import torch

REPO = Path(__file__).resolve().parent
sys.path.insert(0, str(REPO))

HBM_PEAK_GBS = 8000.0
METRIC = "decode-attn effective KV GB/s (% of HBM peak) + µs/call, B=32 GQ4 HD128 bf16"
MAIN_WORKLOAD = "config2_qwen3_4b"
ROTATE_BYTES = 1 << 30
WARM_MS = 100.0  # untimed graph replays right before every timed region


def parse_args() -> argparse.Namespace:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawTextHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--workload", default=MAIN_WORKLOAD)
    ap.add_argument("--no-cells", action="store_true", help="skip the per-cell table")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-decode-step", action="store_true", help="skip config 5")
    ap.add_argument("--no-wide", action="store_true",
                    help="skip the shapes beyond the reference's contract")
    ap.add_argument("--no-host-overhead", action="store_true",
                    help="skip the host-time-per-call section (config 2 launches)")
    ap.add_argument("--no-read-ceiling", action="store_true",
                    help="skip the plain streaming-read ceiling")
    ap.add_argument("--read-ceiling-bytes", default=None,
                    help="only measure the plain read ceiling at these comma-separated "
                         "byte counts and print it as one JSON line")
    ap.add_argument("--cpu-reps", type=int, default=15)
    return ap.parse_args()


def build_pools(spec: dict, device: torch.device):
    """One batch plus extra copies of its caches so the rotation covers >= 1 GB."""
    from mxflashattn_amd.workloads import make_paged_batch

    base = make_paged_batch(**{k: v for k, v in spec.items() if k != "causal"}, device=device)
    cache_bytes = 2 * base.k_cache.numel() * base.k_cache.element_size()
    copies = max(2, math.ceil(ROTATE_BYTES / max(1, cache_bytes)))
    pools = [(base.k_cache, base.v_cache)]
    for _ in range(copies - 1):
        pools.append((base.k_cache.clone(), base.v_cache.clone()))
    return base, pools


def time_calls(fn, pools, steps: int, warmup: int, stream) -> tuple[float, float]:
    """(median us per call from per-call events, mean us per call over the whole run).

    Events are recorded on ``stream``, the stream the kernels are launched on.
    """
    for i in range(warmup):
        fn(*pools[i % len(pools)])
    torch.cuda.synchronize()
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(steps)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(steps)]
    first = torch.cuda.Event(enable_timing=True)
    last = torch.cuda.Event(enable_timing=True)
    first.record(stream)
    for i in range(steps):
        starts[i].record(stream)
        fn(*pools[(warmup + i) % len(pools)])
        ends[i].record(stream)
    last.record(stream)
    torch.cuda.synchronize()
    per = [s.elapsed_time(e) * 1e3 for s, e in zip(starts, ends)]
    return statistics.median(per), first.elapsed_time(last) * 1e3 / steps


def time_graph(fn, pools, calls: int, warmup: int, stream, rounds: int = 10) -> tuple[float, int]:
    """(median us per call, calls timed) of ``rounds`` timed regions on ``stream``.

    Each timed region is exactly ``calls`` calls: one replay of a HIP graph
    that holds ``calls`` calls walking the pool rotation, between two events
    on the stream the kernels run on. The regions run back to back and the
    median region is reported. ``warmup`` eager calls on the same stream
    come first (they also size the workspace there, so nothing is allocated
    inside the capture), then untimed replays for at least WARM_MS.
    """
    with torch.cuda.stream(stream):
        for i in range(warmup):
            fn(*pools[i % len(pools)])
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        for i in range(calls):
            fn(*pools[i % len(pools)])
    events = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
              for _ in range(rounds)]
    # Untimed replays for at least WARM_MS first: after the host has built
    # the inputs the GPU has idled, and the first ~15 ms of work after an
    # idle spell run 3-10 % slower while clocks ramp up.
    t_end = time.perf_counter() + WARM_MS / 1e3
    with torch.cuda.stream(stream):
        while True:
            graph.replay()
            torch.cuda.synchronize()
            if time.perf_counter() >= t_end:
                break
        for first, last in events:
            first.record(stream)
            graph.replay()
            last.record(stream)
    torch.cuda.synchronize()
    del graph
    per_call = [a.elapsed_time(b) * 1e3 / calls for a, b in events]
    return statistics.median(per_call), calls * rounds


# Plain streaming read settings: (layout, KB per wave step, workgroups per CU).
READ_SETTINGS = [(layout, depth, wgs) for layout in (0, 1) for depth in (4, 8, 16)
                 for wgs in (1, 2)]


def read_ceiling(device, sizes: dict[str, int], calls: int = 64) -> dict:
    """The device's plain read rate at each named byte count.

    mxfa_stream_read_launch reads the bytes once with no other work, at every
    READ_SETTINGS combination; each setting is timed like the decode calls
    (graph replays, median of 10 regions), rotating over disjoint slices of
    one buffer that cover >= ROTATE_BYTES, as the KV pools do. Byte counts
    are rounded up to a multiple of 16. Reported: the best setting's GB/s
    (bytes / us) and every setting's.
    """
    from mxflashattn_amd import native

    cus = native.num_cus(device.index or 0)
    plans = {}
    for name, nbytes in sizes.items():
        nbytes = (int(nbytes) + 15) // 16 * 16
        stride = (nbytes + 4095) // 4096 * 4096
        copies = max(2, math.ceil(ROTATE_BYTES / nbytes))
        plans[name] = (nbytes, stride, copies)
    buf = torch.empty(max(s * c for _, s, c in plans.values()), dtype=torch.uint8, device=device)
    sink = torch.empty(max(w for _, _, w in READ_SETTINGS) * cus * 256, dtype=torch.int32,
                       device=device)
    side = torch.cuda.Stream(device)
    out = {}
    for name, (nbytes, stride, copies) in plans.items():
        views = [(buf[i * stride:i * stride + nbytes],) for i in range(copies)]
        rates = {}
        for layout, depth, wgs in READ_SETTINGS:
            def run(view, layout=layout, depth=depth, wgs=wgs):
                native.stream_read(view, nbytes, layout=layout, depth=depth,
                                   workgroups=wgs * cus, sink=sink)

            us = time_graph(run, views, calls, 2, side)[0]
            rates[f"layout{layout}_{depth}kb_{wgs}wg"] = (round(nbytes / (us * 1e-6) / 1e9, 1),
                                                          round(us, 3))
        best = max(rates, key=lambda k: rates[k][0])
        out[name] = {"bytes": nbytes, "best_gb_s": rates[best][0], "best_us": rates[best][1],
                     "best_setting": best,
                     "gb_s_by_setting": {k: v[0] for k, v in rates.items()}}
    del buf
    torch.cuda.empty_cache()
    return out


def measure_workload(name: str, spec: dict, device, steps: int, warmup: int) -> dict:
    from mxflashattn_amd import native

    base, pools = build_pools(spec, device)
    stream = torch.cuda.current_stream(device)
    out = torch.empty_like(base.q)
    ns = native.default_num_splits(base.q, base.k_cache, base.block_table)

    causal = bool(spec.get("causal", False))
    window = base.window_left

    def call(kc, vc):
        native.paged_decode_split(base.q, kc, vc, base.block_table, base.cache_seqlens,
                                  base.scale, out=out, num_splits=ns, causal=causal,
                                  window_left=window)

    us_eager, us_eager_mean = time_calls(call, pools, steps, warmup, stream)
    side = torch.cuda.Stream(device)
    us_graph, timed_calls = time_graph(call, pools, steps, warmup, side)
    # Warm: the same graph replays on one pool that is never rotated, so a
    # working set under the 256 MB Infinity Cache is partly served from it.
    # Reported beside the rotated figure of record, never as `value`.
    us_warm, _ = time_graph(call, pools[:1], steps, 0, side)

    # The dominant kernel alone: partial-only launches, same inputs and stream.
    ws = torch.empty(native.workspace_size(base.batch, base.q_heads, base.head_dim, ns),
                     dtype=torch.uint8, device=device)

    def partial(kc, vc):
        native.split_decode_partial(base.q, kc, vc, base.block_table, base.cache_seqlens,
                                    base.scale, out, ws, ns)

    # The partial-only entry point takes one token and no window.
    single = base.q.shape[1] == 1 and window < 0
    us_partial = time_graph(partial, pools, steps, warmup, side)[0] if single else None
    kv = base.kv_bytes()
    alg = base.algorithmic_bytes()

    # The streaming probe: the partial kernel's own gather (same ranges, grid,
    # descriptors and loads) with no attention math, at the kernel's pipeline
    # depth ("kernel") and at 2-4 tiles in flight per wave: the ceiling of the
    # access pattern on this device.
    probe = None
    if (single and ns > 0 and base.k_cache.dtype in (torch.float16, torch.bfloat16)
            and base.page_size >= 16 and base.head_dim in (64, 128)):
        sink = torch.zeros(base.kv_heads, ns, 64, dtype=torch.int32, device=device)
        probe = {}
        for depth in (0, 2, 3, 4):
            def run_probe(kc, vc, depth=depth):
                native.stream_probe(base.q, kc, vc, base.block_table, base.cache_seqlens, ns,
                                    sink=sink, tiles_in_flight=depth)

            us = time_graph(run_probe, pools, steps, warmup, side)[0]
            probe["kernel" if depth == 0 else f"tiles_in_flight_{depth}"] = {
                "us": round(us, 3), "alg_gb_s": round(alg / (us * 1e-6) / 1e9, 1)}
    gbs = kv / (us_graph * 1e-6) / 1e9
    res = {
        "us_per_call": round(us_graph, 3),
        "us_per_call_eager": round(us_eager, 3),
        "us_per_call_eager_mean": round(us_eager_mean, 3),
        "kv_gb_s": round(gbs, 1),
        "pct_hbm_peak": round(100.0 * gbs / HBM_PEAK_GBS, 2),
        "kv_gb_s_eager": round(kv / (us_eager * 1e-6) / 1e9, 1),
        "us_per_call_warm": round(us_warm, 3),
        "kv_gb_s_warm": round(kv / (us_warm * 1e-6) / 1e9, 1),
        "kv_bytes": kv,
        "algorithmic_bytes": alg,
        "alg_gb_s": round(alg / (us_graph * 1e-6) / 1e9, 1),
        "partial_kernel_us": round(us_partial, 3) if us_partial else None,
        "partial_kernel_gb_s": round(alg / (us_partial * 1e-6) / 1e9, 1) if us_partial else None,
        "num_splits": ns,
        "stream_probe": probe,
        "rotation_copies": len(pools),
        "timed_calls": timed_calls,
    }
    del pools, base
    torch.cuda.empty_cache()
    return res


def _time_cpu(spec: dict, reps: int, ref) -> tuple[float, object]:
    """Median seconds per call on one batch (CPU tensors): the reference's own
    ATen build (oracle/_ref) when ``ref`` is given, else the fp32 restatement."""
    from mxflashattn_amd.workloads import make_paged_batch
    from oracle import reference_port

    b = make_paged_batch(**{k: v for k, v in spec.items() if k != "causal"}, device="cpu")
    times = []
    for i in range(reps + 1):
        t0 = time.perf_counter()
        if ref is not None:
            ref.flash_attn_with_kvcache(b.q, b.k_cache, b.v_cache, None, None,
                                        b.cache_seqlens.clone(), b.block_table, b.scale, False)
        else:
            reference_port.attention_kvcache(b.q, b.k_cache, b.v_cache,
                                             cache_seqlens=b.cache_seqlens.clone(),
                                             block_table=b.block_table, softmax_scale=b.scale)
        if i:
            times.append(time.perf_counter() - t0)
    return statistics.median(times), b


def cpu_baseline(name: str, spec: dict, reps: int) -> dict:
    """Time the reference's own CPU implementation of the path (its ATen
    backend, csrc/mxmac, built into oracle/_ref; kind "reference") on the same
    batch, and on config 1, the reference's CPU-runnable case. The fp32
    restatement (oracle.reference_port, kind "port") is timed beside it, and
    stands in for it where oracle/_ref was not built."""
    from mxflashattn_amd.workloads import CONFIGS
    from oracle import ref_aten

    # The host cores this process may use; a GPU box's share is capped by
    # OMP_NUM_THREADS whatever os.cpu_count() reports.
    cores = len(os.sched_getaffinity(0))
    cap = os.environ.get("OMP_NUM_THREADS", "")
    if cap.isdigit() and int(cap) > 0:
        cores = min(cores, int(cap))
    torch.set_num_threads(max(1, cores))
    ref = ref_aten.load()
    kind = "reference" if ref is not None else "port"
    med, b = _time_cpu(spec, reps, ref)
    med1, b1 = _time_cpu(CONFIGS["config1_cpu_ref"], 50, ref)
    res = {
        "value": round(b.kv_bytes() / med / 1e9, 3),
        "unit": "GB/s",
        "cores": torch.get_num_threads(),
        "kind": kind,
        "sample": (f"{name} full batch (B={b.batch}, {b.total_tokens()} tokens), "
                   f"median of {reps} calls after 1 warmup; {med * 1e3:.1f} ms per call"
                   + ("; the reference's csrc/mxmac flash_attn_with_kvcache built from its "
                      "sources (oracle/_ref)" if ref is not None else "")),
        "ms_per_call": round(med * 1e3, 2),
        "config1_cpu_ref": {
            "ms_per_call": round(med1 * 1e3, 3),
            "kv_gb_s": round(b1.kv_bytes() / med1 / 1e9, 3),
            "sample": f"B={b1.batch}, {b1.total_tokens()} tokens, median of 50 calls",
        },
    }
    if ref is not None:
        reps_p = min(reps, 3)
        med_p, _ = _time_cpu(spec, reps_p, None)
        res["port"] = {"ms_per_call": round(med_p * 1e3, 2),
                       "value": round(b.kv_bytes() / med_p / 1e9, 3),
                       "sample": (f"oracle.reference_port.attention_kvcache, same batch, median "
                                  f"of {reps_p} calls after 1 warmup")}
    return res


def host_overhead(device, calls: int = 100) -> dict:
    """Host microseconds per eager decode call (the time the call takes to
    return; the launches are asynchronous) at config 2, whose 107 us of GPU
    time per call keeps the host from ever waiting on the device:
    ``api`` flash_attn_with_kvcache (its fast path into the C++ operator),
    ``operator`` the C++ operator alone, ``binding`` native.paged_decode_split;
    ``*_ctypes`` the same with the operator switched off (the ctypes path)."""
    import mxflashattn_amd as mx
    from mxflashattn_amd import native
    from mxflashattn_amd.workloads import CONFIGS, make_paged_batch

    b = make_paged_batch(**CONFIGS["config2_qwen3_4b"], device=device)
    out = torch.empty_like(b.q)

    def api():
        mx.flash_attn_with_kvcache(b.q, b.k_cache, b.v_cache, cache_seqlens=b.cache_seqlens,
                                   block_table=b.block_table, out=out)

    def binding():
        native.paged_decode_split(b.q, b.k_cache, b.v_cache, b.block_table, b.cache_seqlens,
                                  b.scale, out=out)

    def timed(fn) -> float:
        for _ in range(10):
            fn()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(calls):
            fn()
        host = time.perf_counter() - t0
        torch.cuda.synchronize()
        return round(host * 1e6 / calls, 2)

    res = {"api": timed(api), "binding": timed(binding)}
    op = native.torch_op()
    if op is not None:
        res["operator"] = timed(lambda: op.decode(b.q, b.k_cache, b.v_cache, b.block_table,
                                                  b.cache_seqlens, b.scale, out, None, 0))
    native.USE_TORCH_OP = False
    try:
        res["api_ctypes"] = timed(api)
        res["binding_ctypes"] = timed(binding)
    finally:
        native.USE_TORCH_OP = True
    res["calls"] = calls
    del b
    torch.cuda.empty_cache()
    return res


def load_traffic(workload: str) -> float | None:
    path = REPO / "profiles" / f"traffic_{workload}.json"
    if not path.exists():
        return None
    try:
        return float(json.loads(path.read_text())["hbm_bytes_per_launch"])
    except (KeyError, ValueError, json.JSONDecodeError):
        return None


def main() -> int:
    args = parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported on this build "
              "(decode attention shards by sequence or kv head with no exchange, so the "
              "one-GPU figure is the per-GPU share)", file=sys.stderr)
        return 2
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 2
    from mxflashattn_amd import native
    from mxflashattn_amd.workloads import CELLS, CONFIGS, DEFAULT_SEED, WIDE

    native.library()  # fail loudly when the HIP library is missing
    device = torch.device("cuda", 0)
    if args.read_ceiling_bytes:
        sizes = {f"{int(n)}_bytes": int(n) for n in args.read_ceiling_bytes.split(",")}
        print(json.dumps({"read_ceiling": read_ceiling(device, sizes)}))
        return 0
    spec = {**CONFIGS, **CELLS, **WIDE}[args.workload]
    print(f"[bench] workload {args.workload}: steps={args.steps} warmup={args.warmup}",
          file=sys.stderr, flush=True)
    main_res = measure_workload(args.workload, spec, device, args.steps, args.warmup)
    print(f"[bench] {args.workload}: {main_res}", file=sys.stderr, flush=True)

    cells = {}
    if not args.no_cells:
        for name, cspec in {**CELLS, **CONFIGS}.items():
            if name == args.workload:
                continue
            cells[name] = measure_workload(name, cspec, device, 64, 10)
            print(f"[bench] {name}: {cells[name]}", file=sys.stderr, flush=True)

    wide = {}
    if not args.no_wide:
        for name, wspec in WIDE.items():
            wide[name] = measure_workload(name, wspec, device, 64, 10)
            print(f"[bench] {name}: {wide[name]}", file=sys.stderr, flush=True)

    ceiling = None
    if not args.no_read_ceiling:
        sizes = {args.workload: main_res["algorithmic_bytes"]}
        for name in ("cell_gq8_d64", "config3_highbatch_gq2_d64"):
            if name in cells:
                sizes[name] = cells[name]["algorithmic_bytes"]
        print("[bench] plain read ceiling", file=sys.stderr, flush=True)
        try:
            ceiling = read_ceiling(device, sizes)
        except Exception as exc:  # reported on stderr; the main metric still prints
            print(f"[bench] read ceiling failed: {exc!r}", file=sys.stderr, flush=True)
            ceiling = None
        print(f"[bench] read ceiling: {ceiling}", file=sys.stderr, flush=True)

    decode = None
    if not args.no_decode_step:
        from mxflashattn_amd.integrations.vllm import decode_step

        print("[bench] config5 decode step", file=sys.stderr, flush=True)
        try:
            decode = decode_step.run(device=device)
        except Exception as exc:  # reported in the line, the main metric still prints
            print(f"[bench] config5 decode step failed: {exc!r}", file=sys.stderr, flush=True)
            decode = {"error": repr(exc)}
        print(f"[bench] config5: {decode}", file=sys.stderr, flush=True)
        torch.cuda.empty_cache()
    decode_eager = None
    if not args.no_decode_step:
        print("[bench] config5 decode step, eager", file=sys.stderr, flush=True)
        try:
            decode_eager = decode_step.run(device=device, eager=True)
        except Exception as exc:
            print(f"[bench] eager decode step failed: {exc!r}", file=sys.stderr, flush=True)
            decode_eager = {"error": repr(exc)}
        print(f"[bench] config5 eager: {decode_eager}", file=sys.stderr, flush=True)
        torch.cuda.empty_cache()
    decode_fp8 = None
    if not args.no_decode_step and not args.no_wide:
        print("[bench] config5 decode step, fp8 KV cache", file=sys.stderr, flush=True)
        try:
            decode_fp8 = decode_step.run(device=device, kv_cache_dtype="fp8")
        except Exception as exc:
            print(f"[bench] fp8 decode step failed: {exc!r}", file=sys.stderr, flush=True)
            decode_fp8 = {"error": repr(exc)}
        print(f"[bench] config5 fp8: {decode_fp8}", file=sys.stderr, flush=True)
        torch.cuda.empty_cache()

    host = None
    if not args.no_host_overhead:
        print("[bench] host time per eager call", file=sys.stderr, flush=True)
        host = host_overhead(device)
        print(f"[bench] host: {host}", file=sys.stderr, flush=True)

    cpu = None
    if not args.no_cpu_baseline:
        print("[bench] cpu baseline", file=sys.stderr, flush=True)
        cpu = cpu_baseline(args.workload, spec, args.cpu_reps)

    # The partial kernel alone where its entry point takes the call (one
    # token, no window); otherwise the whole call, both kernels.
    achieved = main_res["partial_kernel_gb_s"]
    kernel, kernel_us = "split_partial_kernel", main_res["partial_kernel_us"]
    if main_res["num_splits"] == -1:  # SPLITS_PER_SEQUENCE: one kernel is the whole call
        kernel = "seq_decode_kernel"
    if achieved is None:
        achieved = main_res["alg_gb_s"]
        kernel, kernel_us = "split_partial_kernel + split_combine_kernel", main_res["us_per_call"]
    line = {
        "metric": METRIC,
        "value": main_res["kv_gb_s"],
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(main_res["us_per_call"] / 1e3, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16" if spec["dtype"] == torch.bfloat16 else "f16",
        "data": "synthetic",
        "config": {
            "workload": (f"{args.workload}: B={spec['batch']} HQ={spec['q_heads']} "
                         f"HKV={spec['kv_heads']} HD={spec['head_dim']} PS=16 "
                         f"L={spec['lengths']} seed={DEFAULT_SEED}"),
            "global_batch": spec["batch"],
            "parallelism": "single_gpu",
        },
        "us_per_call": main_res["us_per_call"],
        "timed_calls": main_res["timed_calls"],
        "timing": (f"median of 10 timed regions of exactly {args.steps} calls each, every region "
                   "one HIP-graph replay over the rotated KV pools, after "
                   f"{args.warmup} eager warmup calls and {WARM_MS:.0f} ms of untimed replays"),
        "us_per_call_eager": main_res["us_per_call_eager"],
        "kv_gb_s_eager": main_res["kv_gb_s_eager"],
        "us_per_call_warm": main_res["us_per_call_warm"],
        "kv_gb_s_warm": main_res["kv_gb_s_warm"],
        "pct_hbm_peak": main_res["pct_hbm_peak"],
        "num_splits": main_res["num_splits"],
        "roofline": {
            "bound": "hbm",
            "achieved": achieved,
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": load_traffic(args.workload),
            "kernel": kernel,
            "kernel_us": kernel_us,
            "algorithmic_bytes": main_res["algorithmic_bytes"],
            # The whole call (partial kernel, combine kernel and the launch
            # between them) against the same peak.
            "call_achieved": main_res["alg_gb_s"],
            "call_frac": round(main_res["alg_gb_s"] / HBM_PEAK_GBS, 4),
            # The plain read of the same byte count with no other work
            # (mxfa_stream_read_launch, best setting): what this device
            # streams, against which `achieved` is a fraction too.
            "read_ceiling_gb_s": ceiling[args.workload]["best_gb_s"] if ceiling else None,
            "frac_of_read_ceiling": (round(achieved / ceiling[args.workload]["best_gb_s"], 4)
                                     if ceiling else None),
        },
        "read_ceiling": ceiling,
        "cpu_baseline": cpu,
        "cells": cells,
        "wide": wide,
        "decode_step": decode,
        "decode_step_eager": decode_eager,
        "decode_step_fp8": decode_fp8,
        "host_us_per_call": host,
    }
    summary = {args.workload: main_res, **cells}
    for name in sorted(summary):
        res = summary[name]
        print(f"[cells] {name:28s} {res['us_per_call']:9.2f} us/call "
              f"{res['pct_hbm_peak']:6.2f} % of 8 TB/s", file=sys.stderr)
    sys.stderr.flush()
    print(json.dumps(line))
    return 0


if __name__ == "__main__":
    sys.exit(main())
