"""An independent vectorised numpy restatement of the reference dequant.

TEST INFRASTRUCTURE ONLY. Used to cross-check the C oracle bit for bit: it
is derived from the per-element index pattern of the block layouts rather
than from the block loops, so a slip in one of the two (a swapped nibble, a
wrong scale index, a fused multiply-add) shows up as a mismatch.

References: crates/strata-gguf/src/dequant.rs:123-128 (Q8_0), :208-234 (Q6_K),
:237-270 (Q4_K), :272-302 (Q5_K), :189-206 (IQ4_XS);
crates/strata-core/src/ops.rs:14-28 (gemv).
"""
from __future__ import annotations

import numpy as np

F32, F16, Q8_0, Q4_K, Q5_K, Q6_K, IQ4_XS, BF16 = 0, 1, 8, 12, 13, 14, 23, 30

# ggml's kvalues_iq4nl (crates/strata-gguf/src/tables.rs:2052-2054)
IQ4NL = np.array([-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113], np.float32)


def _f16(b: np.ndarray) -> np.ndarray:
    """Little-endian byte pairs (..., 2) -> f32 via numpy's binary16."""
    return np.ascontiguousarray(b).view(np.float16)[..., 0].astype(np.float32)


def q8_0(data: np.ndarray) -> np.ndarray:
    b = data.reshape(-1, 34)
    d = _f16(b[:, 0:2])
    q = b[:, 2:].view(np.int8).astype(np.float32)
    return (q * d[:, None]).astype(np.float32).reshape(-1)


def _k4_scales(sc: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """(n, 12) packed bytes -> (n, 8) scales and (n, 8) mins.

    Sub-blocks 0-3 keep their 6 bits in the low bits of bytes 0-3 (scale)
    and 4-7 (min). Sub-blocks 4-7 keep the low 4 bits in the nibbles of
    bytes 8-11 (scale low, min high) and borrow the top 2 bits of bytes 0-3
    (scale) and 4-7 (min)."""
    sc = sc.astype(np.uint16)
    top = sc[:, 0:8] >> 6                       # the borrowed 2-bit fields
    s = np.empty((sc.shape[0], 8), np.uint16)
    m = np.empty((sc.shape[0], 8), np.uint16)
    s[:, 0:4] = sc[:, 0:4] & 0x3F
    m[:, 0:4] = sc[:, 4:8] & 0x3F
    s[:, 4:8] = (sc[:, 8:12] & 0x0F) + 16 * top[:, 0:4]
    m[:, 4:8] = (sc[:, 8:12] >> 4) + 16 * top[:, 4:8]
    return s, m


def q4_k(data: np.ndarray) -> np.ndarray:
    b = data.reshape(-1, 144)
    n = b.shape[0]
    d = _f16(b[:, 0:2])
    dmin = _f16(b[:, 2:4])
    s, m = _k4_scales(b[:, 4:16])
    qs = b[:, 16:144]
    # element i: group g = i // 64, within-group k = i % 64; byte 32 g + k % 32,
    # low nibble for k < 32, high nibble otherwise; sub-block i // 32.
    i = np.arange(256)
    byte = 32 * (i // 64) + (i % 32)
    hi = (i % 64) >= 32
    q = np.where(hi[None, :], qs[:, byte] >> 4, qs[:, byte] & 0x0F).astype(np.float32)
    sub = i // 32
    dsc = (d[:, None] * s[:, sub].astype(np.float32)).astype(np.float32)
    mm = (dmin[:, None] * m[:, sub].astype(np.float32)).astype(np.float32)
    prod = (dsc * q).astype(np.float32)
    return (prod - mm).astype(np.float32).reshape(n * 256)


def q5_k(data: np.ndarray) -> np.ndarray:
    b = data.reshape(-1, 176)
    n = b.shape[0]
    d = _f16(b[:, 0:2])
    dmin = _f16(b[:, 2:4])
    s, m = _k4_scales(b[:, 4:16])
    qh = b[:, 16:48]
    qs = b[:, 48:176]
    # element i: sub-block i // 32; its nibble as Q4_K's; its fifth bit is
    # bit (i // 32) of qh[i % 32] (sub-block k reads bit k).
    i = np.arange(256)
    byte = 32 * (i // 64) + (i % 32)
    hi = (i % 64) >= 32
    nib = np.where(hi[None, :], qs[:, byte] >> 4, qs[:, byte] & 0x0F)
    fifth = (qh[:, i % 32] >> (i // 32)) & 1
    q = (nib + 16 * fifth).astype(np.float32)
    sub = i // 32
    dsc = (d[:, None] * s[:, sub].astype(np.float32)).astype(np.float32)
    mm = (dmin[:, None] * m[:, sub].astype(np.float32)).astype(np.float32)
    prod = (dsc * q).astype(np.float32)
    return (prod - mm).astype(np.float32).reshape(n * 256)


def q6_k(data: np.ndarray, signed_scales: bool = False) -> np.ndarray:
    b = data.reshape(-1, 210)
    n = b.shape[0]
    d = _f16(b[:, 208:210])
    sc = b[:, 192:208].view(np.int8) if signed_scales else b[:, 192:208]
    sc = sc.astype(np.float32)
    # element i: half h = i // 128, r = i % 128, quarter t = r // 32, l = r % 32.
    i = np.arange(256)
    h, r = i // 128, i % 128
    t, l = r // 32, r % 32
    ql_byte = 64 * h + l + 32 * (t % 2)
    low = np.where(t < 2, b[:, ql_byte] & 0x0F, b[:, ql_byte] >> 4).astype(np.int32)
    high = ((b[:, 128 + 32 * h + l] >> (2 * t)) & 3).astype(np.int32)
    q = (low | (high << 4)) - 32
    sidx = 8 * h + l // 16 + 2 * t
    ds = (d[:, None] * sc[:, sidx]).astype(np.float32)
    return (ds * q.astype(np.float32)).astype(np.float32).reshape(n * 256)


def iq4_xs(data: np.ndarray, ggml: bool = False) -> np.ndarray:
    """Element i of a super-block: sub-block ib = i // 32, position k = i % 32;
    code byte k % 16 of the first 16 qs bytes (the reference's reading) or of
    qs bytes [16 ib, +16) (ggml's), low nibble for k < 16, high otherwise;
    dl = d * (ls - 32) with the 6-bit ls split over scales_l (4 bits) and
    scales_h (2 bits)."""
    b = data.reshape(-1, 136)
    n = b.shape[0]
    d = _f16(b[:, 0:2])
    sh = b[:, 2].astype(np.uint32) | (b[:, 3].astype(np.uint32) << 8)
    ib = np.arange(8)
    lo4 = (b[:, 4 + ib // 2] >> (4 * (ib % 2))) & 0x0F
    ls = lo4.astype(np.int32) | (((sh[:, None] >> (2 * ib)) & 3).astype(np.int32) << 4)
    dl = (d[:, None] * (ls.astype(np.float32) - np.float32(32))).astype(np.float32)
    i = np.arange(256)
    k = i % 32
    byte = 8 + (16 * (i // 32) if ggml else 0) + k % 16
    nib = np.where(k[None, :] >= 16, b[:, byte] >> 4, b[:, byte] & 0x0F)
    return (dl[:, i // 32] * IQ4NL[nib]).astype(np.float32).reshape(n * 256)


def dequantize(quant: int, data: np.ndarray, rows: int, cols: int,
               signed_q6k_scales: bool = False, iq4xs_ggml: bool = False) -> np.ndarray:
    data = np.ascontiguousarray(data, dtype=np.uint8)
    if quant == Q8_0:
        flat = q8_0(data)
    elif quant == Q4_K:
        flat = q4_k(data)
    elif quant == Q5_K:
        flat = q5_k(data)
    elif quant == Q6_K:
        flat = q6_k(data, signed_q6k_scales)
    elif quant == IQ4_XS:
        flat = iq4_xs(data, iq4xs_ggml)
    elif quant == F32:
        flat = data.view(np.float32).copy()
    elif quant == F16:
        flat = data.view(np.float16).astype(np.float32)
    elif quant == BF16:
        flat = (data.view(np.uint16).astype(np.uint32) << 16).view(np.float32)
    else:
        raise ValueError(f"quant {quant}")
    return flat.reshape(rows, cols)


def gemv(quant: int, data: np.ndarray, rows: int, cols: int, x: np.ndarray) -> np.ndarray:
    """f64 products and sums (in BLAS order, not the reference's sequential
    order), rounded to f32 once."""
    w = dequantize(quant, data, rows, cols).astype(np.float64)
    return (w @ np.asarray(x, np.float64)).astype(np.float32)
