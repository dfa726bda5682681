"""The seeded synthetic workloads: deterministic, the documented ranges."""
import numpy as np

from strata_hip import synth as S


def test_stream_is_deterministic_and_offsettable():
    a = S.stream_u64(123, 100)
    b = S.stream_u64(123, 50, start=50)
    assert np.array_equal(a[50:], b)
    assert not np.array_equal(a, S.stream_u64(124, 100))
    # splitmix64 of seed 0: first output for state 0x9E3779B97F4A7C15
    assert int(S.stream_u64(0, 1)[0]) == 0xE220A8397B1DCDAF


def test_normal_moments():
    x = S.normal_f32(5, 200000).astype(np.float64)
    assert abs(x.mean()) < 0.01 and abs(x.std() - 1.0) < 0.01


def test_q8_0_ranges():
    b = S.q8_0_blocks(1, 4096).reshape(-1, 34)
    q = b[:, 2:].view(np.int8)
    assert q.min() >= -127 and q.max() <= 127 and q.min() < -120 and q.max() > 120
    d = b[:, :2].copy().view(np.float16).astype(np.float32)
    assert np.all(d >= 0) and 0.005 < float(d.mean()) < 0.011


def test_q6_k_ranges():
    b = S.q6_k_blocks(2, 2048).reshape(-1, 210)
    sc = b[:, 192:208].view(np.int8)
    assert sc.min() == -64 and sc.max() == 63
    d = b[:, 208:210].copy().view(np.float16).astype(np.float32)
    assert np.all(d >= 0) and 0.0005 < float(d.mean()) < 0.0011


def test_q4_k_layout_sizes():
    w = S.matrix(S.Q4_K, 3, 12, 4096)
    assert w.size == 12 * 16 * 144 == S.row_bytes(S.Q4_K, 4096) * 12
