"""Device dequantization is bit-exact against the oracle (memcmp).

Through the C ABI: sh_dequantize_row (host slices) and sh_dequant_dev
(device pointers). Covers every binary16 scale pattern, the known-answer
blocks, random blocks at the configs' row widths, both Q6_K scale readings,
both IQ4_XS code-byte readings,
and the Truncated error of dequant.rs:50-55.
"""
import numpy as np
import pytest

import strata_hip as H
from strata_hip import synth as S

pytestmark = pytest.mark.gpu


def say(*a):
    print("[case]", *a, flush=True)


def same_bits(a, b):
    a = np.asarray(a, np.float32)
    b = np.asarray(b, np.float32)
    nan = np.isnan(b)
    return np.array_equal(np.isnan(a), nan) and np.array_equal(a[~nan].view(np.uint32),
                                                                b[~nan].view(np.uint32))


def test_every_f16_scale_pattern(backend, oracle):
    # 65536 Q8_0 blocks, block i has d = f16 bits i and q = (1, -1, 127, -127, 0, ...)
    say("dequant Q8_0 all f16 scales")
    n = 65536
    b = np.zeros((n, 34), np.uint8)
    b[:, 0:2] = np.arange(n, dtype=np.uint16).view(np.uint8).reshape(n, 2)
    q = np.zeros(32, np.int8)
    q[:4] = [1, -1, 127, -127]
    q[4:] = np.arange(28) - 14
    b[:, 2:] = q.view(np.uint8)
    flat = b.reshape(-1)
    got = np.empty(n * 32, np.float32)
    backend.dequantize_row(H.QuantType.Q8_0, flat, got)
    want = oracle.dequantize_row(oracle.Q8_0, flat, n * 32)
    assert same_bits(got, want)


@pytest.mark.parametrize("quant,cols", [(8, 4096), (12, 4096), (12, 12288), (14, 4096), (12, 768),
                                        (14, 2048), (13, 4096), (13, 768), (23, 4096), (23, 768)])
def test_random_rows_bit_exact(backend, oracle, quant, cols):
    say("dequant random rows", quant, cols)
    rows = 16
    w = S.matrix(quant, 900 + quant + cols, rows, cols)
    got = np.empty(rows * cols, np.float32)
    backend.dequantize_row(quant, w, got)
    want = oracle.dequantize_row(quant, w, rows * cols)
    assert same_bits(got, want)


def test_q6_k_signed_scales_bit_exact(backend, oracle):
    say("dequant Q6_K i8 scales")
    w = S.matrix(14, 5, 8, 4096)
    got = np.empty(8 * 4096, np.float32)
    backend.dequantize_row(14, w, got, flags=H.FLAG_Q6K_SIGNED_SCALES)
    want = oracle.dequantize_row(14, w, 8 * 4096, oracle.SCALE_I8)
    assert same_bits(got, want)
    # and the reading matters: u8 differs on negative scales
    got_u8 = np.empty_like(got)
    backend.dequantize_row(14, w, got_u8)
    assert not np.array_equal(got, got_u8)


def test_iq4_xs_ggml_reading_bit_exact(backend, oracle):
    say("dequant IQ4_XS ggml reading")
    w = S.matrix(23, 6, 8, 4096)
    got = np.empty(8 * 4096, np.float32)
    backend.dequantize_row(23, w, got, flags=H.FLAG_IQ4XS_GGML)
    assert same_bits(got, oracle.dequantize_row(23, w, 8 * 4096, oracle.IQ4XS_GGML))
    got_ref = np.empty_like(got)
    backend.dequantize_row(23, w, got_ref)
    assert same_bits(got_ref, oracle.dequantize_row(23, w, 8 * 4096))
    assert not np.array_equal(got, got_ref)


def test_iq4_xs_known_answer_blocks(backend):
    say("dequant IQ4_XS KAT blocks")
    from test_oracle_dequant import IQ4NL, iq4xs_block, iq4xs_kat_block
    out = np.empty(256, np.float32)
    backend.dequantize_row(23, iq4xs_kat_block(), out)
    assert (out[0], out[16], out[32], out[48], out[224], out[240]) == (0.5, -63.5, 15.5, -1968.5, -16.0, 2032.0)
    backend.dequantize_row(23, iq4xs_kat_block(), out, flags=H.FLAG_IQ4XS_GGML)
    assert (out[32], out[224], out[240]) == (15.5 * -127, -1808.0, 1040.0)
    # the code book: d = 1, every ls = 33
    qs = np.zeros(128, np.uint8)
    qs[:16] = [j | ((15 - j) << 4) for j in range(16)]
    backend.dequantize_row(23, iq4xs_block(1.0, 0xAAAA, [0x11] * 4, qs), out)
    assert out[:16].tolist() == IQ4NL and out[16:32].tolist() == IQ4NL[::-1]


def test_known_answer_blocks(backend, oracle):
    say("dequant KAT blocks")
    from test_oracle_dequant import q4k_block, q6k_kat_block
    sc = np.zeros(12, np.uint8)
    sc[11], sc[3], sc[7] = 0xF3, 0x40, 0xC0
    qs = np.zeros(128, np.uint8)
    qs[127] = 0xF0
    out = np.empty(256, np.float32)
    backend.dequantize_row(12, q4k_block(2.0, 0.25, sc, qs), out)
    assert out[255] == 554.25
    backend.dequantize_row(14, q6k_kat_block(), out)
    assert out[0] == 480.0 and out[16] == -108.5 and out[192] == 19.0


def test_truncated_and_unsupported(backend):
    say("dequant errors")
    out = np.empty(256, np.float32)
    with pytest.raises(H.TruncatedError):
        backend.dequantize_row(12, np.zeros(143, np.uint8), out)
    with pytest.raises(H.TruncatedError):
        backend.dequantize_row(8, np.zeros(68, np.uint8), np.empty(33, np.float32))
    with pytest.raises(H.UnsupportedQuantError):
        backend.dequantize_row(2, np.zeros(18, np.uint8), np.empty(32, np.float32))


def test_dev_pointer_dequant_full_matrix(oracle):
    import torch
    say("dequant_dev Q4_K 512x12288")
    rows, cols = 512, 12288
    w = S.matrix(12, 17, rows, cols)
    wd = torch.from_numpy(w).cuda()
    out = torch.empty(rows * cols, dtype=torch.float32, device="cuda")
    H.dequant_dev(12, wd.data_ptr(), rows, cols, out.data_ptr(), torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    want = oracle.dequantize_row(12, w, rows * cols)
    assert same_bits(out.cpu().numpy(), want)
