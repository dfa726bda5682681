#!/usr/bin/env python3
"""Writes the golden fixtures of the quantized-weight path (data only).

reference_kats.json
    Known answers of the reference's own tests, transcribed as block bytes
    and expected values:
      crates/strata-gguf/tests/dequant_tests.rs:71-79   Q8_0 dequant
      crates/strata-gguf/tests/dequant_tests.rs:124-131 F16 conversion
      crates/strata-gguf/tests/dequant_tests.rs:161-169 Q6_K dequant
      crates/strata-core/tests/ops_tests.rs:44-61 and
      crates/strata-backend-cpu/src/lib.rs:102-120      Q8_0 gemv unit case
    plus hand-derived Q4_K answers (the reference has no Q4_K test), marked
    "derived": one for the direct (j < 4) and two for the split (j >= 4)
    6-bit scale packing of get_scale_min_k4 (dequant.rs:237-245).

seeded_cases.npz
    Small seeded cases with the oracle's outputs (the C restatement of the
    reference, sequential f64 sums): dequantized rows and gemv outputs for
    Q8_0, Q4_K, Q5_K and Q6_K (both scale readings), an expert gemv, MoE
    routing, the routed MoE FFN, the Q8 activation quantizer, and the
    elementwise methods (rms_norm, l2_norm, softmax, rope_neox) on rows. They let a machine
    without the oracle check the device path against fixed numbers. The MoE
    expert tensors are stored as the seeds of strata_hip.synth.matrix (their
    bytes would be most of the file); every other input is stored as data.

Run from the repository root:  python tests/golden/make_golden.py
"""
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "oracle"))
sys.path.insert(0, os.path.join(ROOT, "strata-rs_amd"))

import oracle as O  # noqa: E402
from strata_hip import synth as S  # noqa: E402


def f16b(v):
    return np.array([v], np.float32).astype(np.float16).view(np.uint8).tolist()


def hexs(b):
    return bytes(np.asarray(b, np.uint8)).hex()


def reference_kats():
    kats = []
    b = np.zeros(34, np.uint8)
    b[:2] = f16b(2.0)
    b[2] = 3
    b[3] = 256 - 4
    kats.append({"what": "dequant", "quant": 8, "n": 32, "block": hexs(b), "expect": {"0": 6.0, "1": -8.0},
                 "source": "crates/strata-gguf/tests/dequant_tests.rs:71-79"})
    b = np.zeros(210, np.uint8)
    b[208:210] = f16b(1.0)
    b[192] = 1
    kats.append({"what": "dequant", "quant": 14, "n": 256, "block": hexs(b), "expect": {"0": -32.0},
                 "source": "crates/strata-gguf/tests/dequant_tests.rs:161-169"})
    b = np.zeros(8, np.uint8)
    b[:2] = f16b(1.5)
    b[2:4] = f16b(-0.25)
    kats.append({"what": "f16", "bits": [int(b[0]) | int(b[1]) << 8, int(b[2]) | int(b[3]) << 8],
                 "expect": [1.5, -0.25], "source": "crates/strata-gguf/tests/dequant_tests.rs:124-131"})
    blk = np.zeros(34, np.uint8)
    blk[:2] = f16b(0.5)
    for j in range(32):
        blk[2 + j] = (j % 7 - 3) & 0xFF
    x = [i * 0.25 - 1.0 for i in range(32)]
    expect = sum(float(j % 7 - 3) * 0.5 * x[j] for j in range(32))
    kats.append({"what": "gemv", "quant": 8, "rows": 1, "cols": 32, "block": hexs(blk), "x": x,
                 "expect": [expect], "tol": 1e-4,
                 "source": "crates/strata-core/tests/ops_tests.rs:44-61, crates/strata-backend-cpu/src/lib.rs:102-120"})

    def q4k(d, dmin, sc, qs):
        b = np.zeros(144, np.uint8)
        b[0:2] = f16b(d)
        b[2:4] = f16b(dmin)
        b[4:16] = sc
        b[16:144] = qs
        return b

    sc = np.zeros(12, np.uint8); sc[0] = 3; sc[4] = 2
    qs = np.zeros(128, np.uint8); qs[0] = 0x5A
    kats.append({"what": "dequant", "quant": 12, "n": 256, "block": hexs(q4k(1.0, 0.5, sc, qs)),
                 "expect": {"0": 29.0, "1": -1.0, "32": 0.0}, "source": "derived: direct scales (j < 4)"})
    sc = np.zeros(12, np.uint8); sc[8] = 0x21; sc[0] = 0xC0; sc[4] = 0x80
    qs = np.zeros(128, np.uint8); qs[64] = 0x07
    kats.append({"what": "dequant", "quant": 12, "n": 256, "block": hexs(q4k(1.0, 0.5, sc, qs)),
                 "expect": {"128": 326.0, "0": 0.0}, "source": "derived: split scales, sub-block 4"})
    sc = np.zeros(12, np.uint8); sc[11] = 0xF3; sc[3] = 0x40; sc[7] = 0xC0
    qs = np.zeros(128, np.uint8); qs[127] = 0xF0
    kats.append({"what": "dequant", "quant": 12, "n": 256, "block": hexs(q4k(2.0, 0.25, sc, qs)),
                 "expect": {"255": 554.25, "224": -15.75}, "source": "derived: split scales, sub-block 7"})
    return kats


MOE_SEEDS = (0x601D0401, 0x601D0402, 0x601D0403)


def seeded_cases():
    out = {}
    for quant, rows, cols in ((8, 16, 256), (12, 16, 512), (14, 16, 512), (13, 16, 512)):
        w = S.matrix(quant, 0x601D0000 + quant, rows, cols)
        x = S.normal_f32(0x601D0100 + quant, cols)
        out[f"gemv_{quant}_w"] = w
        out[f"gemv_{quant}_x"] = x
        out[f"gemv_{quant}_y"] = O.gemv(quant, rows, cols, w, x)
        out[f"deq_{quant}"] = O.dequantize(quant, w, rows, cols)
    w = S.matrix(14, 0x601D0200, 16, 512)
    out["gemv_14s_w"] = w
    out["gemv_14s_x"] = S.normal_f32(0x601D0201, 512)
    out["gemv_14s_y"] = O.gemv(14, 16, 512, w, out["gemv_14s_x"], scale_mode=O.SCALE_I8)
    out["deq_14s"] = O.dequantize(14, w, 16, 512, O.SCALE_I8)
    # expert gemv: 3 experts of [64 in][256 out] Q4_K, expert 1
    ew = S.matrix(12, 0x601D0300, 3 * 64, 256)
    ex = S.normal_f32(0x601D0301, 64)
    ex[5] = 0.0
    out["expert_w"], out["expert_x"] = ew, ex
    out["expert_y"] = O.expert_gemv(12, 3, 64, 256, ew, 1, ex)
    # MoE routing and the routed FFN: 16 experts, hidden 256, expert FFN 256,
    # top-4, 3 tokens. The expert tensors are not stored (1.8 MB of random
    # bytes): they are S.matrix(quant, seed, rows, cols) with the seeds below.
    E, n_embd, n_ff, k, n_tok = 16, 256, 256, 4, 3
    lg = S.router_logits(0x601D0400, n_tok, E)
    g = S.matrix(12, MOE_SEEDS[0], E * n_embd, n_ff)
    u = S.matrix(12, MOE_SEEDS[1], E * n_embd, n_ff)
    d = S.matrix(14, MOE_SEEDS[2], E * n_ff, n_embd)
    xm = S.normal_f32(0x601D0404, n_tok * n_embd).reshape(n_tok, n_embd)
    ids, wts, ys = [], [], []
    for t in range(n_tok):
        i, wt = O.moe_route(lg[t], k)
        ids.append(i)
        wts.append(wt)
        ys.append(O.moe_routed(12, 12, 14, E, n_embd, n_ff, g, u, d, i, wt, xm[t]))
    out.update(moe_logits=lg, moe_seeds=np.array(MOE_SEEDS, np.uint64), moe_x=xm, moe_ids=np.array(ids, np.int64),
               moe_wts=np.array(wts, np.float32), moe_out=np.array(ys, np.float32))
    # Q8 activation blocks
    xa = S.normal_f32(0x601D0500, 32 * 24) * np.float32(4.0)
    xa[:32] = 0.0
    q, s, us = O.quantize_q8(xa)
    out.update(q8_x=xa, q8_codes=q, q8_scales=s, q8_sums=us)
    # the elementwise methods: 3 rows of 1024 (rms_norm, softmax), 8 heads of
    # 128 (l2_norm; rope with 64 rotated dims at position 4097, base 1e7)
    xr = S.normal_f32(0x601D0600, 3 * 1024).reshape(3, 1024) * np.float32(2.0)
    wr = S.normal_f32(0x601D0601, 1024)
    hr = S.normal_f32(0x601D0602, 8 * 128).reshape(8, 128)
    out.update(row_x=xr, row_w=wr, row_heads=hr, row_rms=O.rms_norm(xr, wr, 1e-6), row_softmax=O.softmax(xr),
               row_l2=O.l2_norm(hr, 1e-6), row_rope=O.rope_neox(hr, 4097, 64, 128, 1e7))
    return out


def main():
    with open(os.path.join(HERE, "reference_kats.json"), "w") as f:
        json.dump(reference_kats(), f, indent=1)
    np.savez_compressed(os.path.join(HERE, "seeded_cases.npz"), **seeded_cases())
    print("wrote", os.listdir(HERE))


if __name__ == "__main__":
    main()
