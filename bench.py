#!/usr/bin/env python3
"""Benchmark: Q4_K fused dequant-matvec, 4096 x 12288, batch 1, on one MI355X.

A step is one launch of the fused Q4_K matvec over one 28,311,552-byte
packed weight matrix (the FFN down projection of a Qwen3.5-9B-like model:
4096 outputs, 12288 inputs) with an f32 activation vector; weights and x are
resident in HBM before the timed region starts. The launches rotate over
enough distinct weight copies (>= 1 GiB) that the 256 MB Infinity Cache cannot
serve repeats, and run as one captured HIP graph so launch gaps do not bound
the measurement. Events are recorded on the stream the kernels run on.

Prints ONE JSON line (rank 0):
  value          packed-weight GB/s (weight bytes / mean time per launch)
  roofline       algorithmic bytes (weights + x + y) per launch over the mean
                 launch time, against MI355X's 8 TB/s; `traffic` is the HBM
                 bytes per launch measured with rocprofv3 counters, when a
                 summary exists under profiles/
  cpu_baseline   the reference's CPU path (the C restatement of ops::gemv,
                 single thread, sequential f64) timed on this host on a
                 bounded sample of the same workload
  extra          the other decode shapes (Q4_K 12288x4096 batch 1 and 8, Q8_0
                 4096x4096, Q6_K 151936x4096) measured the same way
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "strata-rs_amd"))

HBM_PEAK_GBS = 8000.0
ROTATE_BYTES = 1 << 30


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=400)
    ap.add_argument("--warmup", type=int, default=40)
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-extra", action="store_true")
    ap.add_argument("--only", default="", help="profile one shape: q4k_down|q4k_gate|q8|q6k")
    return ap.parse_args()


def timed_graph(torch, H, quant, rows, cols, w_host, batch, steps, warmup, flags=0):
    """Mean ms per launch over `steps` launches (graph replays), rotating over
    copies of the weights; returns (ms, n_copies, launches_timed)."""
    import numpy as np
    from strata_hip import synth as S

    nbytes = w_host.nbytes
    n_copies = max(2, min(64, -(-ROTATE_BYTES // nbytes)))
    dev = torch.device("cuda:0")
    base = torch.from_numpy(w_host).to(dev)
    copies = [base] + [base.clone() for _ in range(n_copies - 1)]
    x = torch.from_numpy(S.normal_f32(7, batch * cols)).to(dev)
    y = torch.empty(batch * rows, dtype=torch.float32, device=dev)
    stream = torch.cuda.Stream(dev)
    torch.cuda.synchronize()

    def launch_all(s):
        for c in copies:
            H.gemv_dev(quant, c.data_ptr(), rows, cols, x.data_ptr(), y.data_ptr(), batch, s, flags)

    # eager warm-up (also checks the launch is accepted before capture)
    with torch.cuda.stream(stream):
        launch_all(stream.cuda_stream)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        launch_all(torch.cuda.current_stream().cuda_stream)
    reps_w = max(1, -(-warmup // n_copies))
    reps = max(1, -(-steps // n_copies))
    with torch.cuda.stream(stream):
        for _ in range(reps_w):
            g.replay()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record(stream)
    with torch.cuda.stream(stream):
        for _ in range(reps):
            g.replay()
    end.record(stream)
    torch.cuda.synchronize()
    ms = start.elapsed_time(end) / (reps * n_copies)
    del g, copies, base
    torch.cuda.empty_cache()
    return ms, n_copies, reps * n_copies


def cpu_baseline(w, x, rows, cols, seconds):
    """The oracle (ops::gemv restated in C, one thread) on whole rows of the
    same matrix for about `seconds`; GB/s of packed weight bytes."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O

    rb = w.nbytes // rows
    # a row sample sized from a short probe so the leg stays bounded
    probe = 64
    t0 = time.perf_counter()
    O.gemv(O.Q4_K, probe, cols, w[: probe * rb], x)
    per_row = (time.perf_counter() - t0) / probe
    n_rows = int(max(probe, min(rows, seconds / max(per_row, 1e-9) / 5)))
    times = []
    for _ in range(5):
        t0 = time.perf_counter()
        O.gemv(O.Q4_K, n_rows, cols, w[: n_rows * rb], x)
        times.append(time.perf_counter() - t0)
    t = sorted(times)[2]
    gbs = n_rows * rb / t / 1e9
    nthreads = os.cpu_count() or 1
    t0 = time.perf_counter()
    O.gemv(O.Q4_K, rows, cols, w, x, threads=nthreads)
    t_mt = time.perf_counter() - t0
    return {
        "value": round(gbs, 4),
        "unit": "GB/s",
        "cores": 1,
        "kind": "port",
        "sample": f"{n_rows} of {rows} rows of the same Q4_K 4096x12288 matrix, median of 5 "
                  f"(ops::gemv restated in C: per-row dequant + sequential f64 dot, one thread, "
                  f"as the reference runs)",
        "all_cores": {"value": round(rows * rb / t_mt / 1e9, 4), "cores": nthreads,
                      "sample": "the whole matrix once, rows split over threads"},
    }


def load_traffic(name):
    p = os.path.join(ROOT, "profiles", name)
    if not os.path.exists(p):
        return None
    try:
        with open(p) as f:
            return json.load(f).get("traffic_bytes_per_launch")
    except (OSError, ValueError):
        return None


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only; --gpus must be 1"}))
        sys.exit(2)
    import numpy as np
    import torch

    import strata_hip as H
    from strata_hip import synth as S

    if not torch.cuda.is_available():
        print(json.dumps({"error": "no GPU visible"}))
        sys.exit(1)
    H.load_library()

    rows, cols = 4096, 12288
    w = S.matrix(S.Q4_K, 0x5EED0002, rows, cols)
    wbytes = w.nbytes
    print(f"[bench] Q4_K {rows}x{cols} ({wbytes} B) batch 1: warmup {args.warmup}, steps {args.steps}",
          file=sys.stderr, flush=True)
    ms, n_copies, launches = timed_graph(torch, H, S.Q4_K, rows, cols, w, 1, args.steps, args.warmup)
    gbs = wbytes / (ms * 1e-3) / 1e9
    alg = wbytes + 4 * cols + 4 * rows
    achieved = alg / (ms * 1e-3) / 1e9
    out = {
        "metric": "Q4_K fused matvec packed-weight GB/s + % HBM peak (4096x12288, batch 1)",
        "value": round(gbs, 2),
        "unit": "GB/s",
        "pct_hbm_peak": round(100.0 * gbs / HBM_PEAK_GBS, 2),
        "n_gpus": 1,
        "steps": launches,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": f"synthetic (seeded GGUF Q4_K blocks, x ~ N(0,1)); {n_copies} rotating weight copies "
                f"({n_copies * wbytes / 2**30:.2f} GiB), one HIP graph",
        "config": {"workload": "Q4_K fused dequant-matvec, W 4096x12288 (outputs x inputs), batch 1",
                   "rows": rows, "cols": cols, "batch": 1, "weight_bytes": wbytes},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": load_traffic("q4k_gemv_4096x12288_traffic.json")},
    }
    print(f"[bench] {ms * 1e3:.2f} us/launch, {gbs:.1f} GB/s", file=sys.stderr, flush=True)

    if not args.no_extra:
        extra = {}
        shapes = [("q4k_gate_12288x4096_b1", S.Q4_K, 12288, 4096, 1),
                  ("q4k_gate_12288x4096_b8", S.Q4_K, 12288, 4096, 8),
                  ("q8_0_4096x4096_b1", S.Q8_0, 4096, 4096, 1),
                  ("q6k_lm_head_151936x4096_b1", S.Q6_K, 151936, 4096, 1)]
        for name, q, r, c, b in shapes:
            wm = S.matrix(q, 0x5EED0000 + q + r, r, c)
            print(f"[bench] extra {name}", file=sys.stderr, flush=True)
            steps = max(40, min(args.steps, int(2e9 / wm.nbytes)))
            t, _, _ = timed_graph(torch, H, q, r, c, wm, b, steps, 10)
            extra[name] = {"us_per_launch": round(t * 1e3, 3),
                           "weight_GBps": round(wm.nbytes / (t * 1e-3) / 1e9, 1),
                           "pct_hbm_peak": round(100 * wm.nbytes / (t * 1e-3) / 1e9 / HBM_PEAK_GBS, 1)}
            del wm
        out["extra"] = extra

    if not args.no_cpu:
        print("[bench] cpu baseline", file=sys.stderr, flush=True)
        out["cpu_baseline"] = cpu_baseline(w, S.normal_f32(7, cols), rows, cols, args.cpu_seconds)
    else:
        out["cpu_baseline"] = None
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
