#!/usr/bin/env python3
"""Benchmark: Q4_K fused dequant-matvec, 4096 x 12288, batch 1, on one MI355X.

A step is one launch of the fused Q4_K matvec over one 28,311,552-byte
packed weight matrix (the FFN down projection of a Qwen3.5-9B-like model:
4096 outputs, 12288 inputs) with an f32 activation vector; weights and x are
resident in HBM before the timed region starts. The launches rotate over
enough distinct weight copies (>= 1 GiB) that the 256 MB Infinity Cache cannot
serve repeats, and are all queued behind a spin kernel before the GPU reaches
them, so host launch costs do not bound the measurement. Events are recorded
on the stream the kernels run on.

Prints ONE JSON line (rank 0):
  value          packed-weight GB/s (weight bytes / mean time per launch)
  roofline       algorithmic bytes (weights + x + y) per launch over the mean
                 launch time, against MI355X's 8 TB/s; `traffic` is the HBM
                 bytes per launch measured with rocprofv3 counters, when a
                 summary exists under profiles/; `measured_ceiling_GBps` is a
                 plain streaming read of the same bytes over the same rotating
                 copies in the same harness
  cpu_baseline   the reference's CPU path (the C restatement of ops::gemv,
                 single thread, sequential f64) timed on this host on a
                 bounded sample of the same workload
  extra          the other decode shapes (Q4_K 12288x4096 batch 1 and 8, Q8_0
                 4096x4096, Q6_K 151936x4096) measured the same way; the routed
                 MoE FFN (128 experts, hidden 2048, expert FFN 768, top-8; 1 and
                 16 tokens, routing varied per call, 3 copies of the expert
                 set rotated); the prefill matmul (Q4_K 12288x4096 times 512
                 tokens, bf16 and Q8 activation modes, activation pre-pass
                 included); the host-slice sh_gemv (the trait drop-in, PCIe
                 round trip included) at the headline shape
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
    ap.add_argument("--only", default="", choices=("", "headline", "moe", "prefill", "rowops", "ffn", "blaslt",
                                                    "batched", "decode", "hostslice"),
                    help="'headline': the Q4_K 4096x12288 line only (no extra shapes, no CPU leg); "
                         "'moe' / 'prefill' / 'rowops' / 'ffn' / 'blaslt': that extra alone, 'batched': the "
                         "batch-8 decode shapes (for profiling; prints its JSON), 'hostslice': sh_gemv on host "
                         "slices")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="first run a plain elementwise copy of 256 MiB (known bytes) 3 times, "
                         "to scale rocprofv3 FETCH_SIZE / WRITE_SIZE readings")
    return ap.parse_args()


_SPIN = {}


def _spin_cycles_per_us(torch, stream):
    """The rate of torch.cuda._sleep's cycle counter, measured once."""
    if "rate" not in _SPIN:
        a = torch.cuda.Event(enable_timing=True)
        b = torch.cuda.Event(enable_timing=True)
        with torch.cuda.stream(stream):
            torch.cuda._sleep(1000)  # the first launch of the spin kernel loads it
            a.record(stream)
            torch.cuda._sleep(1_000_000)
            b.record(stream)
        torch.cuda.synchronize()
        _SPIN["rate"] = 1_000_000 / (a.elapsed_time(b) * 1e3)
    return _SPIN["rate"]


def _time_queued_calls(torch, stream, calls, steps, warmup):
    """Runs `warmup` calls untimed, then times exactly `steps` calls with
    events on `stream`, cycling through `calls` (the timed calls continue
    where the warm-up stopped, so a rotation over weight copies never re-reads
    the copies just warmed). Every launch is queued before the GPU reaches
    it: the stream first runs a spin kernel (torch.cuda._sleep) long enough
    to cover the host's enqueueing (1 ms plus four times the host cost of
    the calls, measured on an eager pass; four times longer again on a retry
    if the host still fell behind, as under a tracer), so the timed region
    holds exactly the `steps` calls back to back and no host launch cost.
    A captured HIP graph would also do that, but a
    replay adds ~8 us of its own per timed region (measured at 20 and 400
    launches, and with the replays queued behind the same spin), 0.4 us a
    launch at 20. Raises if the host still fell behind after three tries.
    Returns ms per call."""
    with torch.cuda.stream(stream):  # eager pass: the calls are accepted
        for f in calls:
            f(stream.cuda_stream)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    with torch.cuda.stream(stream):
        for f in calls:
            f(stream.cuda_stream)
    host_us = (time.perf_counter() - t0) * 1e6 / len(calls)
    torch.cuda.synchronize()
    spin_us = 1000.0 + 4.0 * host_us * (warmup + steps)
    n = len(calls)
    for _attempt in range(3):
        cycles = int(spin_us * _spin_cycles_per_us(torch, stream))
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        with torch.cuda.stream(stream):
            h = stream.cuda_stream
            torch.cuda._sleep(cycles)
            for i in range(warmup):
                calls[i % n](h)
            start.record(stream)
            for i in range(steps):
                calls[(warmup + i) % n](h)
            end.record(stream)
            ahead = not start.query()  # still spinning: everything was queued in time
        torch.cuda.synchronize()
        if ahead:
            break
        spin_us *= 4.0  # the host was slower than measured (a tracer, a busy host): queue again
    if not ahead:
        raise RuntimeError("the host fell behind the GPU while queueing the timed calls")
    return start.elapsed_time(end) / steps


def timed_rotation(torch, H, quant, rows, cols, w_host, batch, steps, warmup, flags=0, ceiling=None):
    """Mean ms per launch over exactly `steps` launches (queued back to back)
    after `warmup` untimed ones, rotating over copies of the weights; returns
    (ms, n_copies, launches_timed). With `ceiling` (a dict), a plain
    streaming read of the same copies (sh_stream_read_dev) is timed the same
    way and its ms per launch stored under ceiling["ms"]."""
    from strata_hip import synth as S

    nbytes = w_host.nbytes
    n_copies = max(2, min(64, -(-ROTATE_BYTES // nbytes)))
    dev = torch.device("cuda:0")
    base = torch.from_numpy(w_host).to(dev)
    copies = [base] + [base.clone() for _ in range(n_copies - 1)]
    x = torch.from_numpy(S.normal_f32(7, batch * cols)).to(dev)
    y = torch.empty(batch * rows, dtype=torch.float32, device=dev)
    nws = H.gemv_workspace_bytes(quant, rows, cols, batch)
    ws = torch.empty(max(nws, 256), dtype=torch.uint8, device=dev)
    stream = torch.cuda.Stream(dev)
    torch.cuda.synchronize()

    def call(c):
        if nws:  # batches: the activations converted once per call into the workspace
            return lambda s: H.gemv_dev_ws(quant, c.data_ptr(), rows, cols, x.data_ptr(), y.data_ptr(), batch,
                                           ws.data_ptr(), nws, s, flags)
        return lambda s: H.gemv_dev(quant, c.data_ptr(), rows, cols, x.data_ptr(), y.data_ptr(), batch, s, flags)

    ms = _time_queued_calls(torch, stream, [call(c) for c in copies], steps, warmup)
    if ceiling is not None:
        folds = torch.empty(H.STREAM_READ_BLOCKS, dtype=torch.int32, device=dev)

        def read(c):
            return lambda s: H.stream_read_dev(c.data_ptr(), nbytes, folds.data_ptr(), s)

        ceiling["ms"] = _time_queued_calls(torch, stream, [read(c) for c in copies], steps, warmup)
    del copies, base
    torch.cuda.empty_cache()
    return ms, n_copies, steps


def time_calls(torch, calls, steps, warmup):
    """Mean ms per call of a list of enqueue functions f(stream_handle):
    exactly `steps` timed calls, cycled in order, after `warmup` untimed ones
    (the harness of _time_queued_calls)."""
    dev = torch.device("cuda:0")
    stream = torch.cuda.Stream(dev)
    torch.cuda.synchronize()
    return _time_queued_calls(torch, stream, calls, steps, warmup)


def bench_prefill(torch, H, S, w_host, rows, cols, m, steps):
    """Prefill matmul W[rows][cols] (Q4_K) x X[m][cols] -> Y[m][rows] in the
    bf16 mode and the int8 mode on 32-element Q8 activation blocks (the two
    variants of the prefill workload), plus the opt-in int8 mode on
    256-element blocks; TFLOP/s of 2 * m * rows * cols per call."""
    dev = torch.device("cuda:0")
    w = torch.from_numpy(w_host).to(dev)
    x = torch.from_numpy(S.normal_f32(0x5EED0006, m * cols)).to(dev)
    y = torch.empty(m * rows, dtype=torch.float32, device=dev)
    res = {}
    flops = 2.0 * m * rows * cols
    for mode, name, peak in ((H.MATMUL_BF16, "bf16", 2500.0), (H.MATMUL_Q8, "q8_int8", 5000.0),
                             (H.MATMUL_Q8K, "q8k_int8_256blocks", 5000.0)):
        nb = H.matmul_workspace_bytes(S.Q4_K, rows, cols, m, mode)
        ws = torch.empty(nb, dtype=torch.uint8, device=dev)
        call = (lambda st, mode=mode, ws=ws, nb=nb:
                H.matmul_dev(S.Q4_K, w.data_ptr(), rows, cols, x.data_ptr(), m, y.data_ptr(), mode,
                             ws.data_ptr(), nb, st))
        ms = time_calls(torch, [call], steps, 3)
        tf = flops / (ms * 1e-3) / 1e12
        res[f"prefill_q4k_12288x4096_m{m}_{name}"] = {
            "us_per_call": round(ms * 1e3, 2), "TFLOPs": round(tf, 1),
            "peak_TFLOPs": peak, "frac_of_peak": round(tf / peak, 4)}
        del ws
    del w, x, y
    # Q6_K weights of the same shape in both modes (the int8 mode on its
    # 16-element sub-block kernel)
    w6 = torch.from_numpy(S.matrix(S.Q6_K, 0x5EED0007, rows, cols)).to(dev)
    x = torch.from_numpy(S.normal_f32(0x5EED0006, m * cols)).to(dev)
    y = torch.empty(m * rows, dtype=torch.float32, device=dev)
    for mode, name, peak in ((H.MATMUL_BF16, "bf16", 2500.0), (H.MATMUL_Q8, "q8_int8", 5000.0)):
        nb = H.matmul_workspace_bytes(S.Q6_K, rows, cols, m, mode)
        ws = torch.empty(nb, dtype=torch.uint8, device=dev)
        call = (lambda st, mode=mode, ws=ws, nb=nb:
                H.matmul_dev(S.Q6_K, w6.data_ptr(), rows, cols, x.data_ptr(), m, y.data_ptr(), mode,
                             ws.data_ptr(), nb, st))
        ms = time_calls(torch, [call], steps, 3)
        tf = flops / (ms * 1e-3) / 1e12
        res[f"prefill_q6k_12288x4096_m{m}_{name}"] = {
            "us_per_call": round(ms * 1e3, 2), "TFLOPs": round(tf, 1),
            "peak_TFLOPs": peak, "frac_of_peak": round(tf / peak, 4)}
        del ws
    del w6, x, y
    return res


def bench_blaslt_reference(torch, steps):
    """The library GEMM the prefill kernel is measured beside: torch's bf16
    matmul (hipBLASLt, two-dimensional) of the same shape, X [512][4096] x
    W^T with W [12288][4096] already dequantized to bf16, the faster of two
    operand layouts, plus a 100 MB bf16 write, the least an unfused dequant
    pass of W costs. Random operands (the timing does not depend on them)."""
    dev = torch.device("cuda:0")
    m, n, k = 512, 12288, 4096
    g = torch.Generator(device=dev).manual_seed(7)
    x = torch.randn(m, k, device=dev, dtype=torch.float32, generator=g).to(torch.bfloat16)
    w = torch.randn(n, k, device=dev, dtype=torch.float32, generator=g).to(torch.bfloat16)
    wt = w.t().contiguous()
    out = torch.empty(m, n, device=dev, dtype=torch.bfloat16)
    # both operand layouts (W as [n][k], read transposed, or materialised
    # [k][n]); the faster one is the reference
    ms = min(time_calls(torch, [lambda st: torch.matmul(x, w.t(), out=out)], steps, 5),
             time_calls(torch, [lambda st: torch.matmul(x, wt, out=out)], steps, 5))
    fill = torch.empty(n * k, device=dev, dtype=torch.bfloat16)
    ms_fill = time_calls(torch, [lambda st: fill.fill_(1.0)], steps, 5)
    res = {"reference_hipblaslt_bf16_gemm_512x12288x4096": {
               "us_per_call": round(ms * 1e3, 2), "TFLOPs": round(2.0 * m * n * k / (ms * 1e-3) / 1e12, 1),
               "note": "torch.matmul on bf16 operands (hipBLASLt), weights pre-dequantized: no dequant in the time"},
           "reference_bf16_write_100MB": {
               "us_per_call": round(ms_fill * 1e3, 2),
               "note": "a 12288x4096 bf16 fill: the least an unfused dequant of W to bf16 adds"}}
    del x, w, wt, out, fill
    torch.cuda.empty_cache()
    return res


def bench_moe(torch, H, S, steps):
    """Routed MoE FFN at 128 experts, hidden 2048, expert FFN 768, top-8:
    gate/up Q4_K, down Q6_K; GB/s of the packed bytes of the experts each
    call routes to (each unique expert read once)."""
    import numpy as np
    E, n_embd, n_ff, top_k = 128, 2048, 768, 8
    gate = S.matrix(S.Q4_K, 0x5EED0041, E * n_embd, n_ff)
    up = S.matrix(S.Q4_K, 0x5EED0042, E * n_embd, n_ff)
    down = S.matrix(S.Q6_K, 0x5EED0043, E * n_ff, n_embd)
    per_expert = (gate.nbytes + up.nbytes + down.nbytes) // E
    dev = torch.device("cuda:0")
    sets = []
    for k in range(3):  # 3 x 391 MB: more than the Infinity Cache holds
        tg, tu, td = (torch.from_numpy(a).to(dev) for a in (gate, up, down))
        sets.append((tg, tu, td))
    del gate, up, down
    res = {}
    # the out-major (llama.cpp) stacks have the same byte counts, so the same
    # buffers serve both orientations
    for n_tok, om in ((1, 0), (16, 0), (1, H.FLAG_EXPERT_OUT_MAJOR), (16, H.FLAG_EXPERT_OUT_MAJOR)):
        variants = 8
        logits = [S.router_logits(0x5EED0044 + 97 * v + n_tok, n_tok, E) for v in range(variants)]
        uniq = []
        for lg in logits:
            # softmax preserves the order of the logits: the top-k ids are the
            # k largest logits (ties to the lower id)
            ids = set()
            for t in range(n_tok):
                ids.update(np.argsort(-lg[t], kind="stable")[:top_k].tolist())
            uniq.append(len(ids))
        tl = [torch.from_numpy(lg).to(dev) for lg in logits]
        x = torch.from_numpy(S.normal_f32(0x5EED0045 + n_tok, n_tok * n_embd)).to(dev)
        out = torch.empty(n_tok * n_embd, dtype=torch.float32, device=dev)
        nb = H.moe_workspace_bytes(n_tok, top_k, E, n_embd, n_ff, S.Q4_K, S.Q6_K)
        ws = torch.empty(nb, dtype=torch.uint8, device=dev)
        calls = []
        byts = 0
        for v in range(variants * len(sets)):
            tg, tu, td = sets[v % len(sets)]
            lgv = tl[v % variants]
            byts += uniq[v % variants] * per_expert
            calls.append(lambda st, tg=tg, tu=tu, td=td, lgv=lgv:
                         H.moe_ffn_dev((S.Q4_K, om, tg.data_ptr()), (S.Q4_K, om, tu.data_ptr()),
                                       (S.Q6_K, om, td.data_ptr()), E, n_embd, n_ff, lgv.data_ptr(), n_tok,
                                       top_k, x.data_ptr(), out.data_ptr(), ws.data_ptr(), nb, st))
        ms = time_calls(torch, calls, steps, len(calls))
        mean_bytes = byts / len(calls)
        res[f"moe_128x2048x768_top8_{n_tok}tok" + ("_out_major" if om else "")] = {
            "us_per_call": round(ms * 1e3, 2), "mean_unique_experts": round(sum(uniq) / variants, 2),
            "expert_bytes_GBps": round(mean_bytes / (ms * 1e-3) / 1e9, 1),
            "pct_hbm_peak": round(100 * mean_bytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 1)}
        del ws, tl, x, out
    del sets
    torch.cuda.empty_cache()
    return res


def bench_moe_layer(torch, H, S, steps):
    """The whole MoE layer (router on bf16(x), routed experts, shared expert
    and its gate) at the routed config plus a shared expert of width 768
    (gate/up Q4_K, down Q6_K) and F32 router / gate-input rows; GB/s of the
    packed bytes each call reads (the routed-to experts once each, the
    shared expert, the router and gate-input rows)."""
    import numpy as np
    E, n_embd, n_ff, n_sh, top_k = 128, 2048, 768, 768, 8
    gate = S.matrix(S.Q4_K, 0x5EED0041, E * n_embd, n_ff)
    up = S.matrix(S.Q4_K, 0x5EED0042, E * n_embd, n_ff)
    down = S.matrix(S.Q6_K, 0x5EED0043, E * n_ff, n_embd)
    router = S.normal_f32(0x5EED0047, E * n_embd)
    g_sh = S.matrix(S.Q4_K, 0x5EED0048, n_sh, n_embd)
    u_sh = S.matrix(S.Q4_K, 0x5EED0049, n_sh, n_embd)
    d_sh = S.matrix(S.Q6_K, 0x5EED004A, n_embd, n_sh)
    inp = S.normal_f32(0x5EED004B, n_embd)
    quants = [0, S.Q4_K, S.Q4_K, S.Q6_K, S.Q4_K, S.Q4_K, S.Q6_K, 0]
    host = [router.view(np.uint8), gate, up, down, g_sh, u_sh, d_sh, inp.view(np.uint8)]
    per_expert = (gate.nbytes + up.nbytes + down.nbytes) // E
    fixed = router.nbytes + g_sh.nbytes + u_sh.nbytes + d_sh.nbytes + inp.nbytes
    dev = torch.device("cuda:0")
    sets = [[torch.from_numpy(a).to(dev) for a in host] for _ in range(3)]  # 3 x ~395 MB
    rt = router.reshape(E, n_embd)
    del gate, up, down
    res = {}
    for n_tok in (1, 16):
        variants = 8
        xs = [S.normal_f32(0x5EED004C + 97 * v + n_tok, n_tok * n_embd).reshape(n_tok, n_embd)
              for v in range(variants)]
        uniq = []
        for xv in xs:
            # the experts each token routes to: top-k of router . bf16(x) (softmax keeps the order)
            bits = xv.view(np.uint32)
            xb = (((bits + 0x7FFF + ((bits >> 16) & 1)) >> 16) << 16).astype(np.uint32).view(np.float32)
            lg = xb.astype(np.float64) @ rt.T.astype(np.float64)
            ids = set()
            for t in range(n_tok):
                ids.update(np.argsort(-lg[t], kind="stable")[:top_k].tolist())
            uniq.append(len(ids))
        tx = [torch.from_numpy(xv).to(dev) for xv in xs]
        out = torch.empty(n_tok * n_embd, dtype=torch.float32, device=dev)
        nb = H.moe_layer_workspace_bytes(n_tok, top_k, E, n_embd, n_ff, n_sh, quants)
        ws = torch.empty(nb, dtype=torch.uint8, device=dev)
        calls, byts = [], 0
        for v in range(variants * len(sets)):
            ts, xv = sets[v % len(sets)], tx[v % variants]
            byts += uniq[v % variants] * per_expert + fixed
            calls.append(lambda st, ts=ts, xv=xv:
                         H.moe_layer_dev([(q, 0, t.data_ptr()) for q, t in zip(quants, ts)], E, n_embd, n_ff,
                                         n_sh, n_tok, top_k, xv.data_ptr(), out.data_ptr(), ws.data_ptr(), nb,
                                         st))
        ms = time_calls(torch, calls, steps, len(calls))
        mean_bytes = byts / len(calls)
        res[f"moe_layer_128x2048x768_top8_shexp768_{n_tok}tok"] = {
            "us_per_call": round(ms * 1e3, 2), "mean_unique_experts": round(sum(uniq) / variants, 2),
            "weight_GBps": round(mean_bytes / (ms * 1e-3) / 1e9, 1),
            "pct_hbm_peak": round(100 * mean_bytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 1)}
        del ws, tx, out
    del sets
    torch.cuda.empty_cache()
    return res


def bench_rowops(torch, H, S, steps):
    """The trait's elementwise methods at a decode step's shapes (hidden 4096,
    32 heads of 128 with 64 rotated dims, a 4096-long attention row per head)
    and a 16-token prefill's; launches of one method back to back; us per launch and GB/s of the bytes each launch reads and
    writes (the data stays in L2 between launches)."""
    import numpy as np
    dev = torch.device("cuda:0")
    res = {}

    def t(a):
        return torch.from_numpy(np.ascontiguousarray(a)).to(dev)

    w = t(S.normal_f32(0x5EED0061, 4096))
    cases = []
    for n_tok in (1, 16):
        x = t(S.normal_f32(0x5EED0062 + n_tok, n_tok * 4096))
        o = t(np.zeros(n_tok * 4096, np.float32))
        q = t(S.normal_f32(0x5EED0063 + n_tok, n_tok * 32 * 128))
        sc = t(S.normal_f32(0x5EED0064 + n_tok, n_tok * 32 * 4096))
        cfg = H.RopeCfg(pos=1000, n_rot=64, head_dim=128, freq_base=1e7)
        nb = 4 * n_tok * 4096
        cases += [
            (f"rms_norm_{n_tok}x4096", 2 * nb + 4 * 4096,
             lambda st, x=x, o=o, n=n_tok: H.rms_norm_dev(x.data_ptr(), w.data_ptr(), o.data_ptr(), n, 4096, 1e-6, st)),
            (f"rope_neox_{n_tok}x32x128_rot64", 2 * 4 * n_tok * 32 * 64,
             lambda st, q=q, n=n_tok: H.rope_neox_dev(q.data_ptr(), n * 32, 32, cfg, st)),
            (f"l2_norm_{n_tok}x32x128", 2 * 4 * n_tok * 32 * 128,
             lambda st, q=q, n=n_tok: H.l2_norm_dev(q.data_ptr(), n * 32, 128, 1e-6, st)),
            (f"softmax_{n_tok}x32x4096", 2 * 4 * n_tok * 32 * 4096,
             lambda st, sc=sc, n=n_tok: H.softmax_dev(sc.data_ptr(), n * 32, 4096, st)),
            (f"add_{n_tok}x4096", 3 * nb,
             lambda st, x=x, o=o, n=n_tok: H.add_dev(o.data_ptr(), x.data_ptr(), n * 4096, st)),
        ]
    for name, nbytes, f in cases:
        ms = time_calls(torch, [f], steps, 64)
        res[name] = {"us_per_call": round(ms * 1e3, 2), "GBps": round(nbytes / (ms * 1e-3) / 1e9, 1)}
    return res


def bench_ffn(torch, H, S, steps):
    """The dense FFN half of a layer (rms_norm, gate, up, silu * up, down,
    residual) at the dense config, Q4_K, hidden 4096, FFN 12288, one token,
    over rotating copies of the three matrices (3 x 28.3 MB); us per call and
    GB/s of the packed weights each call reads."""
    import numpy as np
    n_embd, n_ff = 4096, 12288
    mats = [S.matrix(S.Q4_K, 0x5EED0071 + i, *((n_ff, n_embd) if i < 2 else (n_embd, n_ff))) for i in range(3)]
    wbytes = sum(m.nbytes for m in mats)
    dev = torch.device("cuda:0")
    n_copies = 12  # 1.02 GB of weights: beyond the Infinity Cache
    sets = [[torch.from_numpy(m).to(dev) for m in mats]] + [None] * (n_copies - 1)
    for i in range(1, n_copies):
        sets[i] = [t.clone() for t in sets[0]]
    x = torch.from_numpy(S.normal_f32(0x5EED0074, n_embd)).to(dev)
    norm = torch.from_numpy(S.normal_f32(0x5EED0075, n_embd)).to(dev)
    out = torch.empty_like(x)
    nb = H.ffn_workspace_bytes(1, n_embd, n_ff)
    ws = torch.empty(nb, dtype=torch.uint8, device=dev)
    calls = [lambda st, ts=ts: H.ffn_dev([(S.Q4_K, 0, t.data_ptr()) for t in ts], n_embd, n_ff, 1, x.data_ptr(),
                                         norm.data_ptr(), 1e-6, out.data_ptr(), ws.data_ptr(), nb, st)
             for ts in sets]
    ms = time_calls(torch, calls, steps, len(calls))
    del sets, ws
    torch.cuda.empty_cache()
    return {"ffn_q4k_4096x12288_1tok": {"us_per_call": round(ms * 1e3, 2),
                                        "weight_GBps": round(wbytes / (ms * 1e-3) / 1e9, 1),
                                        "pct_hbm_peak": round(100 * wbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 1)}}


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
    nthreads = min(16, os.cpu_count() or 1)  # the box's CPU share per GPU
    times_mt = []
    for _ in range(5):
        t0 = time.perf_counter()
        O.gemv(O.Q4_K, rows, cols, w, x, threads=nthreads)
        times_mt.append(time.perf_counter() - t0)
    t_mt = sorted(times_mt)[2]
    return {
        "value": round(gbs, 4),
        "unit": "GB/s",
        "cores": 1,
        "kind": "port",
        "sample": f"{n_rows} of {rows} rows of the same Q4_K 4096x12288 matrix, median of 5 "
                  f"(ops::gemv restated in C: per-row dequant + sequential f64 dot, one thread, "
                  f"as the reference runs)",
        "all_cores": {"value": round(rows * rb / t_mt / 1e9, 4), "cores": nthreads,
                      "sample": "the whole matrix, rows split over threads, median of 5"},
        "cpu_model": cpu_model(),
        "nproc": os.cpu_count(),
    }


def cpu_model():
    """The host CPU as /proc/cpuinfo names it: model name plus family, model
    and stepping (the name alone can be as short as "AMD EPYC" under a
    hypervisor; family 25 is Zen 3/4, 26 Zen 5)."""
    info = {}
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if not line.strip():
                    break  # the first processor's block
                k, _, v = line.partition(":")
                info[k.strip()] = v.strip()
    except OSError:
        return None
    name = info.get("model name")
    if name is None:
        return None
    ids = [f"{k} {info[k]}" for k in ("cpu family", "model", "stepping") if k in info]
    return f"{name} ({', '.join(ids)})" if ids else name


def launch_sync_floor(torch, H, calls):
    """One launch of sh_stream_read_dev over 16 bytes (2048 workgroups, one
    lane of which loads anything) and a synchronisation of its stream, per
    call: about the round trip any synchronous host-slice call pays on top of
    its kernels; microseconds."""
    buf = torch.zeros(4, dtype=torch.int32, device="cuda")
    out = torch.zeros(2048, dtype=torch.int32, device="cuda")
    st = torch.cuda.current_stream()
    for _ in range(20):
        H.stream_read_dev(buf.data_ptr(), 16, out.data_ptr(), st.cuda_stream)
        st.synchronize()
    t0 = time.perf_counter()
    for _ in range(calls):
        H.stream_read_dev(buf.data_ptr(), 16, out.data_ptr(), st.cuda_stream)
        st.synchronize()
    return (time.perf_counter() - t0) / calls * 1e6


def host_slice_gemv(H, S, w, x, rows, cols, calls):
    """The trait drop-in path end to end: sh_gemv on host slices (x copied
    into mapped pinned staging, a copy kernel to the device, the matvec
    storing y into the staging, a synchronisation) with the weights already
    resident; microseconds per call, as (bare C-ABI call with its arguments
    built once -- what the crate's FFI call pays --, the same through the
    Python wrapper HipBackend.gemv)."""
    import ctypes as C
    import numpy as np
    y = np.empty(rows, np.float32)
    xv = np.ascontiguousarray(x, dtype=np.float32)
    with H.HipBackend(0) as be:
        t = H.QuantTensor("bench.host_slice", S.Q4_K, rows, cols, w)
        for _ in range(10):
            be.gemv(t, xv, y)
        wc = t._c()
        fn, ctx, wp = be._L.sh_gemv, be._ctx, C.byref(wc)
        xp, yp = xv.ctypes.data, y.ctypes.data
        t0 = time.perf_counter()
        for _ in range(calls):
            rc = fn(ctx, wp, xp, cols, yp, rows)
        bare = (time.perf_counter() - t0) / calls * 1e6
        H.check(rc)
        t0 = time.perf_counter()
        for _ in range(calls):
            be.gemv(t, xv, y)
        wrapped = (time.perf_counter() - t0) / calls * 1e6
    return bare, wrapped


# type ids: 8 Q8_0, 12 Q4_K, 13 Q5_K, 14 Q6_K
DECODE_SHAPES = (("q4k_gate_12288x4096_b1", 12, 12288, 4096, 1),
                 ("q4k_gate_12288x4096_b8", 12, 12288, 4096, 8),
                 ("q4k_down_4096x12288_b8", 12, 4096, 12288, 8),
                 ("q8_0_4096x4096_b1", 8, 4096, 4096, 1),
                 ("q5k_4096x12288_b1", 13, 4096, 12288, 1),
                 ("q5k_12288x4096_b8", 13, 12288, 4096, 8),
                 ("q5k_4096x12288_b8", 13, 4096, 12288, 8),
                 ("q6k_lm_head_151936x4096_b1", 14, 151936, 4096, 1))


def bench_decode_shapes(torch, H, S, steps_max, batched_only=False):
    """The other decode matvec shapes (Q4_K / Q5_K gate and down at batch 1
    and 8, Q8_0 attention-sized, the Q6_K head), each over rotating weight
    copies; microseconds per launch and GB/s of packed weights."""
    extra = {}
    for name, q, r, c, b in DECODE_SHAPES:
        if batched_only and b == 1:
            continue
        wm = S.matrix(q, 0x5EED0000 + q + r, r, c)
        print(f"[bench] extra {name}", file=sys.stderr, flush=True)
        steps = max(40, min(steps_max, int(2e9 / wm.nbytes)))
        t, _, _ = timed_rotation(torch, H, q, r, c, wm, b, steps, 10)
        extra[name] = {"us_per_launch": round(t * 1e3, 3),
                       "weight_GBps": round(wm.nbytes / (t * 1e-3) / 1e9, 1),
                       "pct_hbm_peak": round(100 * wm.nbytes / (t * 1e-3) / 1e9 / HBM_PEAK_GBS, 1)}
        if q == S.Q6_K:
            extra[name]["scale_reading"] = "u8, as strata-gguf reads the Q6_K sub-block scales (dequant.rs:211)"
        del wm
    return extra


def load_traffic(name):
    """(HBM bytes per launch, the kernel they were counted on) from a counter
    summary under profiles/, or (None, None)."""
    p = os.path.join(ROOT, "profiles", name)
    if not os.path.exists(p):
        return None, None
    try:
        with open(p) as f:
            d = json.load(f)
        return d.get("traffic_bytes_per_launch"), d.get("kernel")
    except (OSError, ValueError):
        return None, None


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "the benchmark runs on one GPU only; --gpus must be 1"}))
        sys.exit(2)
    import numpy as np
    import torch

    import strata_hip as H
    from strata_hip import synth as S

    if not torch.cuda.is_available():
        print(json.dumps({"error": "no GPU visible"}))
        sys.exit(1)
    H.load_library()

    if args.calibrate_copy:
        src = torch.ones(1 << 26, dtype=torch.float32, device="cuda:0")  # 256 MiB
        dst = torch.empty_like(src)
        for _ in range(3):
            torch.neg(src, out=dst)
        torch.cuda.synchronize()
        del src, dst
        print("[bench] copy calibration: 3 x 256 MiB read + 256 MiB written", file=sys.stderr, flush=True)
    if args.only == "headline":
        args.no_extra = True
        args.no_cpu = True
    elif args.only == "moe":
        res = bench_moe(torch, H, S, args.steps)
        res.update(bench_moe_layer(torch, H, S, args.steps))
        print(json.dumps(res), flush=True)
        return
    elif args.only == "ffn":
        print(json.dumps(bench_ffn(torch, H, S, args.steps)), flush=True)
        return
    elif args.only == "rowops":
        print(json.dumps(bench_rowops(torch, H, S, args.steps)), flush=True)
        return
    elif args.only == "batched":
        print(json.dumps(bench_decode_shapes(torch, H, S, args.steps, batched_only=True)), flush=True)
        return
    elif args.only == "decode":
        print(json.dumps(bench_decode_shapes(torch, H, S, args.steps)), flush=True)
        return
    elif args.only == "blaslt":
        print(json.dumps(bench_blaslt_reference(torch, args.steps)), flush=True)
        return
    elif args.only == "hostslice":
        w = S.matrix(S.Q4_K, 0x5EED0002, 4096, 12288)
        us, wrapped = host_slice_gemv(H, S, w, S.normal_f32(7, 12288), 4096, 12288, args.steps)
        floor = launch_sync_floor(torch, H, args.steps)
        print(json.dumps({"host_slice_gemv_q4k_4096x12288_b1": {"us_per_call": round(us, 2),
                                                                "us_per_call_python_wrapper": round(wrapped, 2),
                                                                "launch_sync_floor_us": round(floor, 2)}}),
              flush=True)
        return
    elif args.only == "prefill":
        wp = S.matrix(S.Q4_K, 0x5EED0000 + S.Q4_K + 12288, 12288, 4096)
        print(json.dumps(bench_prefill(torch, H, S, wp, 12288, 4096, 512, args.steps)), flush=True)
        return

    rows, cols = 4096, 12288
    w = S.matrix(S.Q4_K, 0x5EED0002, rows, cols)
    wbytes = w.nbytes
    print(f"[bench] Q4_K {rows}x{cols} ({wbytes} B) batch 1: warmup {args.warmup}, steps {args.steps}",
          file=sys.stderr, flush=True)
    ceiling = {}
    ms, n_copies, launches = timed_rotation(torch, H, S.Q4_K, rows, cols, w, 1, args.steps, args.warmup,
                                         ceiling=ceiling)
    gbs = wbytes / (ms * 1e-3) / 1e9
    alg = wbytes + 4 * cols + 4 * rows
    achieved = alg / (ms * 1e-3) / 1e9
    ceil_gbs = wbytes / (ceiling["ms"] * 1e-3) / 1e9
    traffic = load_traffic("gemv_q4k_4096x12288_b1.traffic.json")
    out = {
        "metric": "Q4_K fused matvec packed-weight GB/s + % HBM peak (4096x12288, batch 1)",
        "value": round(gbs, 2),
        "unit": "GB/s",
        "pct_hbm_peak": round(100.0 * gbs / HBM_PEAK_GBS, 2),
        "n_gpus": 1,
        "steps": launches,
        "steps_requested": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": f"synthetic (seeded GGUF Q4_K blocks, x ~ N(0,1)); {n_copies} rotating weight copies "
                f"({n_copies * wbytes / 2**30:.2f} GiB), launches queued behind a spin kernel",
        "config": {"workload": "Q4_K fused dequant-matvec, W 4096x12288 (outputs x inputs), batch 1",
                   "rows": rows, "cols": cols, "batch": 1, "weight_bytes": wbytes},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": traffic[0], "traffic_kernel": traffic[1],
                     "measured_ceiling_GBps": round(ceil_gbs, 2),
                     "frac_of_measured_ceiling": round(gbs / ceil_gbs, 4),
                     "ceiling": "plain streaming read of the same 28,311,552 bytes (sh_stream_read_dev: 16-byte "
                                "loads, 2048 x 256 threads) over the same rotating copies, same harness, "
                                f"{ceiling['ms'] * 1e3:.3f} us per launch"},
    }
    print(f"[bench] {ms * 1e3:.2f} us/launch, {gbs:.1f} GB/s", file=sys.stderr, flush=True)

    if not args.no_extra:
        extra = {}
        extra.update(bench_decode_shapes(torch, H, S, args.steps))
        print("[bench] extra prefill matmul", file=sys.stderr, flush=True)
        prefill_w = S.matrix(S.Q4_K, 0x5EED0000 + S.Q4_K + 12288, 12288, 4096)
        extra.update(bench_prefill(torch, H, S, prefill_w, 12288, 4096, 512, 50))
        extra.update(bench_blaslt_reference(torch, 50))
        del prefill_w
        print("[bench] extra moe", file=sys.stderr, flush=True)
        extra.update(bench_moe(torch, H, S, 240))
        print("[bench] extra moe layer", file=sys.stderr, flush=True)
        extra.update(bench_moe_layer(torch, H, S, 240))
        print("[bench] extra dense ffn", file=sys.stderr, flush=True)
        extra.update(bench_ffn(torch, H, S, 240))
        print("[bench] extra elementwise methods", file=sys.stderr, flush=True)
        extra.update(bench_rowops(torch, H, S, 200))
        print("[bench] extra host-slice gemv", file=sys.stderr, flush=True)
        us, wrapped = host_slice_gemv(H, S, w, S.normal_f32(7, cols), rows, cols, 200)
        extra["host_slice_gemv_q4k_4096x12288_b1"] = {
            "us_per_call": round(us, 2),
            "us_per_call_python_wrapper": round(wrapped, 2),
            "launch_sync_floor_us": round(launch_sync_floor(torch, H, 200), 2),
            "note": "sh_gemv on host slices (the ComputeBackend::gemv drop-in): x copied into mapped pinned "
                    "staging, a copy kernel in, the matvec storing y into the staging, synchronise; weights "
                    "resident; 200 calls, wall clock; us_per_call: the bare C-ABI call (arguments built "
                    "once, as an FFI caller holds them), us_per_call_python_wrapper: through "
                    "HipBackend.gemv. launch_sync_floor_us: one launch of a near-empty "
                    "kernel and a stream synchronisation, the round trip under every synchronous call"}
        out["extra"] = extra

    if not args.no_cpu:
        print("[bench] cpu baseline", file=sys.stderr, flush=True)
        out["cpu_baseline"] = cpu_baseline(w, S.normal_f32(7, cols), rows, cols, args.cpu_seconds)
    else:
        out["cpu_baseline"] = None
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
