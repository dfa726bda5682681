"""Pins the oracle's dequantizers.

* the reference's own known-answer tests
  (crates/strata-gguf/tests/dequant_tests.rs:71-79 Q8_0, :124-140 F16/BF16,
  :161-169 Q6_K) and its "finite values" fill (:187-244);
* hand-derived Q4_K known answers (the reference has none) covering the
  direct (j < 4) and split (j >= 4) 6-bit scale packings;
* hand-derived Q5_K known answers (none in the reference either) for the
  fifth bit of every sub-block;
* hand-derived negative Q6_K scales, u8 (reference) vs i8 (ggml) reading;
* hand-derived IQ4_XS known answers for both code-byte readings (the
  reference's first-16-bytes reading and ggml's 16 bytes per sub-block), the
  code book, the 6-bit scale split and the readings' agreement when the code
  bytes repeat;
* an encoder round trip for get_scale_min_k4 over every (j, sc, m);
* the exhaustive binary16 -> binary32 table against numpy;
* a bit-for-bit comparison with the independent numpy restatement.
"""
import numpy as np
import pytest

import np_oracle as N
from strata_hip import synth as S


def f16b(v):
    return np.array([v], np.float32).astype(np.float16).view(np.uint8).tolist()


# ---- the reference's own known answers -------------------------------------

def test_q8_0_known_answer(oracle):
    # dequant_tests.rs:71-79
    b = np.zeros(34, np.uint8)
    b[:2] = f16b(2.0)
    b[2] = 3
    b[3] = np.uint8(256 - 4)
    out = oracle.dequantize_row(oracle.Q8_0, b, 32)
    assert out[0] == 6.0
    assert out[1] == -8.0


def test_q6_k_known_answer(oracle):
    # dequant_tests.rs:161-169: fp16 scale last, all quants 0, sc[0] = 1 -> -32
    b = np.zeros(210, np.uint8)
    b[208:210] = f16b(1.0)
    b[192] = 1
    out = oracle.dequantize_row(oracle.Q6_K, b, 256)
    assert out[0] == -32.0


def test_f16_and_bf16_known_answers(oracle):
    # dequant_tests.rs:124-140
    b = np.zeros(8, np.uint8)
    b[0:2] = f16b(1.5)
    b[2:4] = f16b(-0.25)
    out = oracle.dequantize_row(oracle.F16, b, 4)
    assert out[0] == 1.5 and out[1] == -0.25
    bits = np.array([1.5], np.float32).view(np.uint32)[0] >> 16
    bb = np.array([bits & 0xFF, bits >> 8], np.uint8)
    assert oracle.dequantize_row(oracle.BF16, np.concatenate([bb, bb]), 2)[0] == 1.5


def _lcg_block(nbytes):
    # dequant_tests.rs:207-215: state = state * 1664525 + 1013904223, byte = state >> 16
    state = 0x12345678
    out = np.empty(nbytes, np.uint8)
    for i in range(nbytes):
        state = (state * 1664525 + 1013904223) & 0xFFFFFFFF
        out[i] = (state >> 16) & 0xFF
    return out


@pytest.mark.parametrize("quant,elems", [(8, 32), (12, 256), (13, 256), (14, 256)])
def test_every_type_decodes_finite(oracle, quant, elems):
    # dequant_tests.rs:187-244 with its fill and its f16 0.125 at bytes 0..1
    b = _lcg_block(oracle.byte_size(quant, elems))
    b[:2] = f16b(0.125)
    out = oracle.dequantize_row(quant, b, elems)
    assert np.all(np.isfinite(out))


# ---- hand-derived Q4_K known answers ----------------------------------------

def q4k_block(d, dmin, scales, qs):
    b = np.zeros(144, np.uint8)
    b[0:2] = f16b(d)
    b[2:4] = f16b(dmin)
    b[4:16] = scales
    b[16:144] = qs
    return b


def test_q4_k_direct_scales(oracle):
    sc = np.zeros(12, np.uint8)
    sc[0] = 3       # sub-block 0 scale
    sc[4] = 2       # sub-block 0 min
    qs = np.zeros(128, np.uint8)
    qs[0] = 0x5A    # element 0: low nibble 10; element 32: high nibble 5
    out = oracle.dequantize_row(oracle.Q4_K, q4k_block(1.0, 0.5, sc, qs), 256)
    assert out[0] == 29.0       # (1*3)*10 - 0.5*2
    assert out[1] == -1.0       # (1*3)*0 - 1
    assert out[32] == 0.0       # sub-block 1: scale 0, min 0


def test_q4_k_split_scales_low_groups(oracle):
    sc = np.zeros(12, np.uint8)
    sc[8] = 0x21    # sub-block 4: scale low nibble 1, min low nibble 2
    sc[0] = 0xC0    # top bits 3 -> scale 1 + 48 = 49; sub-block 0 scale 0
    sc[4] = 0x80    # top bits 2 -> min 2 + 32 = 34;   sub-block 0 min 0
    qs = np.zeros(128, np.uint8)
    qs[64] = 0x07   # element 128 = group 2, low nibble
    out = oracle.dequantize_row(oracle.Q4_K, q4k_block(1.0, 0.5, sc, qs), 256)
    assert out[128] == 326.0    # 49*7 - 0.5*34
    assert out[0] == 0.0


def test_q4_k_split_scales_last_subblock(oracle):
    sc = np.zeros(12, np.uint8)
    sc[11] = 0xF3   # sub-block 7: scale low 3, min low 15
    sc[3] = 0x40    # scale top bits 1 -> 19
    sc[7] = 0xC0    # min top bits 3 -> 63
    qs = np.zeros(128, np.uint8)
    qs[127] = 0xF0  # element 255 = group 3, high nibble 15
    out = oracle.dequantize_row(oracle.Q4_K, q4k_block(2.0, 0.25, sc, qs), 256)
    assert out[255] == 554.25   # (2*19)*15 - 0.25*63
    assert out[224] == -15.75   # same sub-block, q = 0


# ---- hand-derived Q5_K known answers ------------------------------------------

def q5k_block(d, dmin, scales, qh, qs):
    b = np.zeros(176, np.uint8)
    b[0:2] = f16b(d)
    b[2:4] = f16b(dmin)
    b[4:16] = scales
    b[16:48] = qh
    b[48:176] = qs
    return b


def test_q5_k_fifth_bit_per_subblock(oracle):
    """Sub-block k (elements 32k .. 32k+31) takes bit k of qh[l]: with scale
    1 and min 0 everywhere and every nibble 0, element 32k + l is 16 exactly
    when bit k of qh[l] is set."""
    sc = encode_scale_min_k4([1] * 8, [0] * 8)
    qh = np.zeros(32, np.uint8)
    qh[3] = 0b00000101      # sub-blocks 0 and 2 at l = 3
    qh[31] = 0b10000010     # sub-blocks 1 and 7 at l = 31
    out = oracle.dequantize_row(oracle.Q5_K, q5k_block(1.0, 0.0, sc, qh, np.zeros(128, np.uint8)), 256)
    want = np.zeros(256, np.float32)
    want[[3, 64 + 3, 32 + 31, 224 + 31]] = 16.0
    assert np.array_equal(out, want)


def test_q5_k_nibbles_scales_and_mins(oracle):
    sc = encode_scale_min_k4([3, 5, 0, 0, 0, 0, 0, 19], [2, 1, 0, 0, 0, 0, 0, 63])
    qh = np.zeros(32, np.uint8)
    qh[0] = 0x03            # element 0 and element 32 get +16
    qh[31] = 0x80           # element 255 gets +16
    qs = np.zeros(128, np.uint8)
    qs[0] = 0x5A            # element 0: low nibble 10; element 32: high nibble 5
    qs[127] = 0xF0          # element 255: high nibble 15, element 223: 0
    out = oracle.dequantize_row(oracle.Q5_K, q5k_block(2.0, 0.25, sc, qh, qs), 256)
    assert out[0] == 155.5      # (2*3)*(10+16) - 0.25*2
    assert out[1] == -0.5       # (2*3)*0 - 0.5
    assert out[32] == 209.75    # (2*5)*(5+16) - 0.25*1
    assert out[255] == 1162.25  # (2*19)*(15+16) - 0.25*63
    assert out[224] == -15.75   # same sub-block, q = 0


# ---- hand-derived Q6_K known answers, both scale readings -------------------

def q6k_kat_block():
    b = np.zeros(210, np.uint8)
    b[208:210] = f16b(0.5)
    b[0] = 0x05
    b[128] = 0x02        # element 0: q = (5 | 2<<4) - 32 = 5
    b[192] = 0xC0        # sc[0]: 192 as u8, -64 as i8
    b[32] = 0x0C         # element 32: q = 12 - 32 = -20 with sc[2]
    b[192 + 2] = 3
    b[16] = 0x01         # element 16: q = 1 - 32 = -31 with sc[1]
    b[192 + 1] = 7
    b[64] = 0x3F
    b[128 + 32] = 0xFF   # element 128: q = 63 - 32 = 31 with sc[8]; element 192: 51 - 32 = 19 with sc[12]
    b[192 + 8] = 1
    b[192 + 12] = 2
    return b


def test_q6_k_known_answers_u8(oracle):
    out = oracle.dequantize_row(oracle.Q6_K, q6k_kat_block(), 256)
    assert out[0] == 480.0      # (0.5*192)*5
    assert out[32] == -30.0     # (0.5*3)*-20
    assert out[16] == -108.5    # (0.5*7)*-31
    assert out[128] == 15.5     # (0.5*1)*31
    assert out[192] == 19.0     # (0.5*2)*19
    assert out[64] == 0.0       # sc[4] = 0


def test_q6_k_known_answers_i8(oracle):
    out = oracle.dequantize_row(oracle.Q6_K, q6k_kat_block(), 256, oracle.SCALE_I8)
    assert out[0] == -160.0     # (0.5*-64)*5
    assert out[32] == -30.0


# ---- hand-derived IQ4_XS known answers, both code-byte readings -------------

# ggml's kvalues_iq4nl as crates/strata-gguf/src/tables.rs:2052-2054 lists it
IQ4NL = [-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113]


def iq4xs_block(d, scales_h, scales_l, qs):
    b = np.zeros(136, np.uint8)
    b[0:2] = f16b(d)
    b[2:4] = [scales_h & 0xFF, scales_h >> 8]
    b[4:8] = scales_l
    b[8:136] = qs
    return b


def test_iq4_xs_code_book(oracle):
    """d = 1 and every ls = 33 (dl = 1): the outputs are the code book's
    values. qs[j] = j | (15 - j) << 4 puts index j at element j and index
    15 - j at element 16 + j of the first sub-block."""
    qs = np.zeros(128, np.uint8)
    qs[:16] = [j | ((15 - j) << 4) for j in range(16)]
    sl = [0x11] * 4                      # low 4 bits of every ls: 1
    sh = 0xAAAA                          # top 2 bits of every ls: 2 -> ls = 33
    for mode in (oracle.IQ4XS_REFERENCE, oracle.IQ4XS_GGML):
        out = oracle.dequantize_row(oracle.IQ4_XS, iq4xs_block(1.0, sh, sl, qs), 256, mode)
        assert out[:16].tolist() == IQ4NL
        assert out[16:32].tolist() == IQ4NL[::-1]


def iq4xs_kat_block():
    qs = np.zeros(128, np.uint8)
    qs[0] = 0x08                 # low nibble 8 (code 1), high nibble 0 (code -127)
    qs[112] = 0x3F               # sub-block 7 in ggml's reading: low 15 (113), high 3 (-65)
    sl = [0xF1, 0, 0, 0]         # ls low bits: sub-block 0 -> 1, 1 -> 15, 7 -> 0
    sh = 0x0002 | (3 << 2)       # ls high bits: sub-block 0 -> 2, 1 -> 3, 7 -> 0
    return iq4xs_block(0.5, sh, sl, qs)


def test_iq4_xs_known_answers_reference_reading(oracle):
    """Every sub-block reads qs[0..16]: ls0 = 33 (dl 0.5), ls1 = 63 (dl
    15.5), ls7 = 0 (dl -16)."""
    out = oracle.dequantize_row(oracle.IQ4_XS, iq4xs_kat_block(), 256)
    assert out[0] == 0.5         # 0.5 * 1
    assert out[16] == -63.5      # 0.5 * -127
    assert out[32] == 15.5       # 15.5 * 1 (qs[0] again)
    assert out[48] == -1968.5    # 15.5 * -127
    assert out[224] == -16.0     # -16 * 1
    assert out[240] == 2032.0    # -16 * -127
    assert out[1] == 0.5 * -127  # qs[1] = 0: code -127


def test_iq4_xs_known_answers_ggml_reading(oracle):
    """Sub-block ib reads qs[16 ib .. 16 ib + 16]: sub-block 1 sees zero
    bytes, sub-block 7 the 0x3F at qs[112]."""
    out = oracle.dequantize_row(oracle.IQ4_XS, iq4xs_kat_block(), 256, oracle.IQ4XS_GGML)
    assert out[0] == 0.5
    assert out[16] == -63.5
    assert out[32] == 15.5 * -127
    assert out[224] == -1808.0   # -16 * 113
    assert out[240] == 1040.0    # -16 * -65


def test_iq4_xs_readings_agree_when_code_bytes_repeat(oracle):
    for seed in range(20):
        blk = S.iq4_xs_blocks(3000 + seed, 1)
        blk[24:136] = np.tile(blk[8:24], 7)
        a = oracle.dequantize_row(oracle.IQ4_XS, blk, 256)
        b = oracle.dequantize_row(oracle.IQ4_XS, blk, 256, oracle.IQ4XS_GGML)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    # and differ when they do not
    blk = S.iq4_xs_blocks(3100, 1)
    assert not np.array_equal(oracle.dequantize_row(oracle.IQ4_XS, blk, 256),
                              oracle.dequantize_row(oracle.IQ4_XS, blk, 256, oracle.IQ4XS_GGML))


def test_iq4_xs_finite_fill(oracle):
    """dequant_tests.rs:187-244 for IQ4_XS: the LCG byte fill with an f16
    scale of 0.125 dequantizes to finite values."""
    state = 0x12345678
    blk = np.empty(136, np.uint8)
    for i in range(136):
        state = (state * 1664525 + 1013904223) & 0xFFFFFFFF
        blk[i] = (state >> 16) & 0xFF
    blk[0:2] = f16b(0.125)
    out = oracle.dequantize_row(oracle.IQ4_XS, blk, 256)
    assert np.all(np.isfinite(out))


# ---- get_scale_min_k4: round trip through an encoder ------------------------

def encode_scale_min_k4(sc, m):
    """Pack 8 (scale, min) 6-bit pairs into 12 bytes: j < 4 keeps them in the
    low 6 bits of bytes j and j+4; j >= 4 puts the low nibbles in byte j+4
    and the top 2 bits in the top bits of bytes j-4 (scale) and j (min)."""
    b = [0] * 12
    for j in range(8):
        if j < 4:
            b[j] |= sc[j]
            b[j + 4] |= m[j]
        else:
            b[j + 4] = (sc[j] & 0xF) | ((m[j] & 0xF) << 4)
            b[j - 4] |= (sc[j] >> 4) << 6
            b[j] |= (m[j] >> 4) << 6
    return np.array(b, np.uint8)


def test_scale_min_k4_round_trip_every_value(oracle):
    rng = np.random.default_rng(7)
    for j in range(8):
        for v in range(64):
            sc = rng.integers(0, 64, 8)
            m = rng.integers(0, 64, 8)
            sc[j] = v
            m[j] = 63 - v
            packed = encode_scale_min_k4(sc, m)
            for jj in range(8):
                assert oracle.get_scale_min_k4(jj, packed) == (sc[jj], m[jj])


def test_scale_min_k4_matches_numpy(oracle):
    rng = np.random.default_rng(3)
    raw = rng.integers(0, 256, (512, 12)).astype(np.uint8)
    s, m = N._k4_scales(raw)
    for i in range(raw.shape[0]):
        for j in range(8):
            assert oracle.get_scale_min_k4(j, raw[i]) == (s[i, j], m[i, j])


# ---- binary16 -----------------------------------------------------------------

def test_f16_to_f32_every_bit_pattern(oracle):
    bits = np.arange(65536, dtype=np.uint16)
    want = bits.view(np.float16).astype(np.float32)
    b = bits.view(np.uint8)
    got = oracle.dequantize_row(oracle.F16, b, 65536)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))
    # NaNs come out quiet with the payload in the top mantissa bits (half 2.7.1)
    gb = got[nan].view(np.uint32)
    assert np.all(gb & 0x00400000)
    assert np.array_equal((gb >> 13) & 0x3FF | 0x200, (bits[nan] & 0x3FF) | 0x200)


def test_f32_to_f16_round_to_nearest_even(oracle):
    rng = np.random.default_rng(11)
    vals = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * np.float32(0.01),
        rng.standard_normal(5000).astype(np.float32) * np.float32(1e-5),
        rng.standard_normal(5000).astype(np.float32) * np.float32(3e4),
        np.array([0.0, -0.0, 65504.0, 65519.0, 65520.0, 1e9, -1e9, 2.0 ** -24, 2.0 ** -25,
                  3 * 2.0 ** -26, 6.1e-5, 1.0 + 2.0 ** -11, 1.0 + 3 * 2.0 ** -11], np.float32),
    ])
    with np.errstate(over="ignore"):
        want = vals.astype(np.float16).view(np.uint16)
    got = np.array([oracle.f32_to_f16(float(v)) for v in vals], np.uint16)
    assert np.array_equal(got, want)


# ---- errors, geometry -----------------------------------------------------------

def test_geometry_constants(oracle):
    # quant.rs:125-164; a 4096x4096 Q8_0 tensor is 17,825,792 bytes
    assert (oracle.block_size(8), oracle.type_size(8)) == (32, 34)
    assert (oracle.block_size(12), oracle.type_size(12)) == (256, 144)
    assert (oracle.block_size(13), oracle.type_size(13)) == (256, 176)
    assert (oracle.block_size(14), oracle.type_size(14)) == (256, 210)
    assert (oracle.block_size(23), oracle.type_size(23)) == (256, 136)
    assert oracle.byte_size(8, 4096 * 4096) == 17_825_792
    assert oracle.byte_size(12, 4096 * 12288) == 28_311_552
    assert oracle.byte_size(14, 151936 * 4096) == 510_504_960


def test_truncated_rows(oracle):
    with pytest.raises(oracle.OracleError) as e:
        oracle.dequantize_row(oracle.Q4_K, np.zeros(143, np.uint8), 256)
    assert e.value.rc == oracle.TRUNCATED
    with pytest.raises(oracle.OracleError):
        oracle.dequantize_row(oracle.Q8_0, np.zeros(34, np.uint8), 33)


# ---- the independent numpy restatement --------------------------------------

@pytest.mark.parametrize("quant", [8, 12, 13, 14, 23])
def test_oracle_matches_numpy_restatement(oracle, quant):
    cols = 1024
    rows = 64
    w = S.matrix(quant, 4242 + quant, rows, cols)
    a = oracle.dequantize(quant, w, rows, cols)
    b = N.dequantize(quant, w, rows, cols)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    if quant == 14:
        a = oracle.dequantize(quant, w, rows, cols, oracle.SCALE_I8)
        b = N.dequantize(quant, w, rows, cols, signed_q6k_scales=True)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    if quant == 23:
        a = oracle.dequantize(quant, w, rows, cols, oracle.IQ4XS_GGML)
        b = N.dequantize(quant, w, rows, cols, iq4xs_ggml=True)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_q4_k_products_are_exact(oracle):
    """d1 = d*sc has at most 11 + 6 significant bits and d1*q at most 21, so
    both are exact in f32: d1*q - m1 rounds once whether or not it is fused.
    The oracle must equal that single-rounding value everywhere."""
    for seed in range(50):
        blk = S.q4_k_blocks(1000 + seed, 1)
        out = oracle.dequantize_row(oracle.Q4_K, blk, 256)
        d = np.float64(np.frombuffer(blk[0:2].tobytes(), np.float16)[0])
        dm = np.float64(np.frombuffer(blk[2:4].tobytes(), np.float16)[0])
        want = np.empty(256)
        for j in range(256):
            sub, k = j // 32, j % 64
            sc, m = oracle.get_scale_min_k4(sub, blk[4:16])
            byte = blk[16 + 32 * (j // 64) + (k % 32)]
            q = (byte & 0xF) if k < 32 else (byte >> 4)
            want[j] = d * sc * q - dm * m          # exact in f64
        assert np.array_equal(out, want.astype(np.float32))


def test_q5_k_products_are_exact(oracle):
    """As Q4_K: d1*q has at most 11 + 6 + 5 significant bits, exact in f32,
    so d1*q - m1 is one rounding of the exact value."""
    for seed in range(50):
        blk = S.q5_k_blocks(1500 + seed, 1)
        out = oracle.dequantize_row(oracle.Q5_K, blk, 256)
        d = np.float64(np.frombuffer(blk[0:2].tobytes(), np.float16)[0])
        dm = np.float64(np.frombuffer(blk[2:4].tobytes(), np.float16)[0])
        want = np.empty(256)
        for j in range(256):
            sub, k = j // 32, j % 64
            sc, m = oracle.get_scale_min_k4(sub, blk[4:16])
            byte = blk[48 + 32 * (j // 64) + (k % 32)]
            q = (byte & 0xF) if k < 32 else (byte >> 4)
            q += 16 * ((blk[16 + j % 32] >> sub) & 1)
            want[j] = d * sc * q - dm * m          # exact in f64
        assert np.array_equal(out, want.astype(np.float32))


@pytest.mark.parametrize("mode", [0, 1])
def test_q6_k_is_one_rounding_of_the_exact_value(oracle, mode):
    """d*sc has at most 11 + 8 bits, so (d*sc)*q rounds the exact product
    d*sc*q once, whatever the order: the oracle must equal f32(d*sc*q)
    computed exactly in f64, for the u8 (reference) and i8 scale readings."""
    for seed in range(50):
        blk = S.q6_k_blocks(2000 + seed, 1)
        out = oracle.dequantize_row(oracle.Q6_K, blk, 256, mode)
        d = np.float64(np.frombuffer(blk[208:210].tobytes(), np.float16)[0])
        j = np.arange(256)
        h, r = j // 128, j % 128
        t, l = r // 32, r % 32
        qlb = blk[64 * h + l + 32 * (t % 2)]
        low = np.where(t < 2, qlb & 0xF, qlb >> 4).astype(np.int64)
        high = ((blk[128 + 32 * h + l] >> (2 * t)) & 3).astype(np.int64)
        q = (low | (high << 4)) - 32
        raw = blk[192 + 8 * h + l // 16 + 2 * t]
        sc = raw.view(np.int8).astype(np.float64) if mode else raw.astype(np.float64)
        assert np.array_equal(out, (d * sc * q).astype(np.float32))


@pytest.mark.parametrize("mode", [0, 1])
def test_iq4_xs_products_are_exact(oracle, mode):
    """dl = d*(ls - 32) has at most 11 + 6 significant bits and dl*code at
    most 24, so both are exact in f32: the oracle must equal the exact value
    (f64) for both code-byte readings."""
    tab = np.array(IQ4NL, np.float64)
    for seed in range(30):
        blk = S.iq4_xs_blocks(3500 + seed, 1)
        out = oracle.dequantize_row(oracle.IQ4_XS, blk, 256, mode)
        d = np.float64(np.frombuffer(blk[0:2].tobytes(), np.float16)[0])
        sh = int(blk[2]) | (int(blk[3]) << 8)
        want = np.empty(256)
        for j in range(256):
            ib, k = j // 32, j % 32
            ls = ((int(blk[4 + ib // 2]) >> (4 * (ib % 2))) & 0xF) | (((sh >> (2 * ib)) & 3) << 4)
            byte = int(blk[8 + (16 * ib if mode else 0) + k % 16])
            want[j] = d * (ls - 32) * tab[(byte >> 4) if k >= 16 else (byte & 0xF)]
        assert np.array_equal(out, want.astype(np.float32))


def test_q8_0_is_one_rounding_of_the_exact_value(oracle):
    blk = S.q8_0_blocks(77, 64)
    out = oracle.dequantize_row(oracle.Q8_0, blk, 64 * 32)
    b = blk.reshape(64, 34)
    d = b[:, 0:2].copy().view(np.float16)[:, 0].astype(np.float64)
    q = b[:, 2:].view(np.int8).astype(np.float64)
    assert np.array_equal(out, (q * d[:, None]).astype(np.float32).reshape(-1))
