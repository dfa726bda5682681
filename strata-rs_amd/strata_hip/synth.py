"""Seeded synthetic workloads for the quantized matvec path.

A portable counter-based generator (splitmix64 over ``seed + (i + 1) * gamma``)
so that any element of any stream can be produced independently and the same
bytes come out on every machine. On top of it:

* ``normal_f32``   Box-Muller N(0, 1) from pairs of 53-bit uniforms,
* ``uniform_int``  ``lo + z % (hi - lo + 1)``,
* ``random_bytes`` the little-endian bytes of the stream,

and block builders for the three GGUF layouts the path reads
(crates/strata-gguf/src/quant.rs:138-164 for the sizes):

* Q8_0: 34-byte blocks ``[d: f16][q: i8 x 32]`` with d = f16(|N|*0.01) and
  q uniform in [-127, 127];
* Q4_K: 144-byte super-blocks ``[d: f16][dmin: f16][scales: 12][qs: 128]``
  with d, dmin = f16(|N|*0.01) and the 140 packed bytes uniform;
* Q6_K: 210-byte super-blocks ``[ql: 128][qh: 64][sc: 16][d: f16]`` with
  ql/qh uniform bytes, sc uniform int8 in [-64, 63] and d = f16(|N|*0.001);
* Q5_K: 176-byte super-blocks ``[d: f16][dmin: f16][scales: 12][qh: 32]
  [ql: 128]`` with d, dmin = f16(|N|*0.01) and the 172 packed bytes uniform;
* IQ4_XS: 136-byte super-blocks ``[d: f16][scales_h: u16][scales_l: 4]
  [qs: 128]`` with d = f16(|N|*0.01) and the 134 packed bytes uniform.

f32 -> f16 is numpy's round-to-nearest-even. Generation is chunked so a
510 MB tensor needs only a few hundred MB of temporaries.
"""
from __future__ import annotations

import numpy as np

GAMMA = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)
_CHUNK = 1 << 22

Q8_0, Q4_K, Q5_K, Q6_K, IQ4_XS = 8, 12, 13, 14, 23
BLOCK = {Q8_0: (32, 34), Q4_K: (256, 144), Q5_K: (256, 176), Q6_K: (256, 210), IQ4_XS: (256, 136)}


def _mix(z: np.ndarray) -> np.ndarray:
    z = (z ^ (z >> np.uint64(30))) * _M1
    z = (z ^ (z >> np.uint64(27))) * _M2
    return z ^ (z >> np.uint64(31))


def stream_u64(seed: int, n: int, start: int = 0) -> np.ndarray:
    """Elements ``start .. start+n`` of the splitmix64 stream of ``seed``."""
    with np.errstate(over="ignore"):
        idx = np.arange(start + 1, start + n + 1, dtype=np.uint64)
        return _mix(np.uint64(seed & 0xFFFFFFFFFFFFFFFF) + idx * GAMMA)


def sub_seed(seed: int, tag: int) -> int:
    """An independent stream for field ``tag`` of workload ``seed``."""
    with np.errstate(over="ignore"):
        return int(_mix(np.array([seed ^ (tag * 0xD1B54A32D192ED03 & 0xFFFFFFFFFFFFFFFF)],
                                 dtype=np.uint64))[0])


def random_bytes(seed: int, n: int) -> np.ndarray:
    out = np.empty(n, dtype=np.uint8)
    words = (n + 7) // 8
    for w0 in range(0, words, _CHUNK):
        w1 = min(words, w0 + _CHUNK)
        b = stream_u64(seed, w1 - w0, w0).view(np.uint8)
        lo = w0 * 8
        hi = min(n, w1 * 8)
        out[lo:hi] = b[: hi - lo]
    return out


def uniform_int(seed: int, n: int, lo: int, hi: int) -> np.ndarray:
    span = np.uint64(hi - lo + 1)
    out = np.empty(n, dtype=np.int64)
    for i0 in range(0, n, _CHUNK):
        i1 = min(n, i0 + _CHUNK)
        out[i0:i1] = (stream_u64(seed, i1 - i0, i0) % span).astype(np.int64) + lo
    return out


def normal_f32(seed: int, n: int) -> np.ndarray:
    out = np.empty(n, dtype=np.float32)
    scale = 2.0 ** -53
    for i0 in range(0, n, _CHUNK):
        i1 = min(n, i0 + _CHUNK)
        z = stream_u64(seed, 2 * (i1 - i0), 2 * i0)
        u1 = (z[0::2] >> np.uint64(11)).astype(np.float64) * scale
        u2 = (z[1::2] >> np.uint64(11)).astype(np.float64) * scale
        out[i0:i1] = (np.sqrt(-2.0 * np.log1p(-u1)) * np.cos(2.0 * np.pi * u2)).astype(np.float32)
    return out


def _f16_bytes(v: np.ndarray) -> np.ndarray:
    return v.astype(np.float32).astype(np.float16).view(np.uint8).reshape(-1, 2)


def q8_0_blocks(seed: int, n_blocks: int) -> np.ndarray:
    """``n_blocks`` Q8_0 blocks as a flat uint8 array."""
    b = np.empty((n_blocks, 34), dtype=np.uint8)
    b[:, 0:2] = _f16_bytes(np.abs(normal_f32(sub_seed(seed, 1), n_blocks)) * np.float32(0.01))
    q = uniform_int(sub_seed(seed, 2), n_blocks * 32, -127, 127).astype(np.int8)
    b[:, 2:34] = q.view(np.uint8).reshape(n_blocks, 32)
    return b.reshape(-1)


def q4_k_blocks(seed: int, n_blocks: int) -> np.ndarray:
    """``n_blocks`` Q4_K super-blocks as a flat uint8 array."""
    b = np.empty((n_blocks, 144), dtype=np.uint8)
    b[:, 0:2] = _f16_bytes(np.abs(normal_f32(sub_seed(seed, 1), n_blocks)) * np.float32(0.01))
    b[:, 2:4] = _f16_bytes(np.abs(normal_f32(sub_seed(seed, 2), n_blocks)) * np.float32(0.01))
    b[:, 4:144] = random_bytes(sub_seed(seed, 3), n_blocks * 140).reshape(n_blocks, 140)
    return b.reshape(-1)


def q6_k_blocks(seed: int, n_blocks: int) -> np.ndarray:
    """``n_blocks`` Q6_K super-blocks as a flat uint8 array."""
    b = np.empty((n_blocks, 210), dtype=np.uint8)
    b[:, 0:192] = random_bytes(sub_seed(seed, 3), n_blocks * 192).reshape(n_blocks, 192)
    sc = uniform_int(sub_seed(seed, 4), n_blocks * 16, -64, 63).astype(np.int8)
    b[:, 192:208] = sc.view(np.uint8).reshape(n_blocks, 16)
    b[:, 208:210] = _f16_bytes(np.abs(normal_f32(sub_seed(seed, 1), n_blocks)) * np.float32(0.001))
    return b.reshape(-1)


def q5_k_blocks(seed: int, n_blocks: int) -> np.ndarray:
    """``n_blocks`` Q5_K super-blocks as a flat uint8 array."""
    b = np.empty((n_blocks, 176), dtype=np.uint8)
    b[:, 0:2] = _f16_bytes(np.abs(normal_f32(sub_seed(seed, 1), n_blocks)) * np.float32(0.01))
    b[:, 2:4] = _f16_bytes(np.abs(normal_f32(sub_seed(seed, 2), n_blocks)) * np.float32(0.01))
    b[:, 4:176] = random_bytes(sub_seed(seed, 3), n_blocks * 172).reshape(n_blocks, 172)
    return b.reshape(-1)


def iq4_xs_blocks(seed: int, n_blocks: int) -> np.ndarray:
    """``n_blocks`` IQ4_XS super-blocks as a flat uint8 array."""
    b = np.empty((n_blocks, 136), dtype=np.uint8)
    b[:, 0:2] = _f16_bytes(np.abs(normal_f32(sub_seed(seed, 1), n_blocks)) * np.float32(0.01))
    b[:, 2:136] = random_bytes(sub_seed(seed, 3), n_blocks * 134).reshape(n_blocks, 134)
    return b.reshape(-1)


def blocks(quant: int, seed: int, n_blocks: int) -> np.ndarray:
    if quant == IQ4_XS:
        return iq4_xs_blocks(seed, n_blocks)
    if quant == Q5_K:
        return q5_k_blocks(seed, n_blocks)
    if quant == Q8_0:
        return q8_0_blocks(seed, n_blocks)
    if quant == Q4_K:
        return q4_k_blocks(seed, n_blocks)
    if quant == Q6_K:
        return q6_k_blocks(seed, n_blocks)
    raise ValueError(f"no synthetic generator for quant id {quant}")


def matrix(quant: int, seed: int, rows: int, cols: int) -> np.ndarray:
    """A ``rows x cols`` quantized matrix in GGUF row-major block layout."""
    bs, _ = BLOCK[quant]
    if cols % bs:
        raise ValueError(f"cols={cols} is not a multiple of the block size {bs}")
    return blocks(quant, seed, rows * (cols // bs))


def row_bytes(quant: int, cols: int) -> int:
    bs, ts = BLOCK[quant]
    return (cols + bs - 1) // bs * ts


def router_logits(seed: int, n_tok: int, n_expert: int) -> np.ndarray:
    return normal_f32(seed, n_tok * n_expert).reshape(n_tok, n_expert)
