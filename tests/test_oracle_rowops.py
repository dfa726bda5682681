"""Pins the oracle's restatement of the trait's elementwise methods
(crates/strata-core/src/backend.rs:38-50, CPU bodies ops.rs:46-165).

* the reference's own tests: ops_tests.rs:79-135 (rms_norm known values,
  unit l2 heads, rope at position 0 and one pair at freq_base 1, softmax
  sums to one and keeps the order) and strata-backend-cpu/src/lib.rs:121-151;
* closed forms that a plausible slip breaks: rms_norm of a constant row is
  w (drops the 1/n or the square root otherwise), eps inside the root after
  the mean, softmax of a uniform row is 1/n and is shift-invariant, rope
  pairs are (i, i + n_rot/2) (not adjacent), theta = base^(-2i/n_rot) at a
  base where the powers are exact, dims from n_rot on pass through, and a
  rotation keeps the pair's norm.
"""
import math

import numpy as np
import pytest


def f32(v):
    return float(np.float32(v))


# ---- the reference's own tests ----------------------------------------------

def test_rms_norm_known_values(oracle):
    # ops_tests.rs:79-88, strata-backend-cpu lib.rs:124-127
    x = oracle.rms_norm([3.0, 4.0], [2.0, 2.0], 0.0)
    s = 2.0 / math.sqrt(12.5)
    assert abs(x[0] - f32(3.0 * s)) < 1e-6 and abs(x[1] - f32(4.0 * s)) < 1e-6
    # and exactly the f64 expression the reference rounds once
    sc = 1.0 / math.sqrt(12.5)
    assert x[0] == f32(3.0 * sc * 2.0) and x[1] == f32(4.0 * sc * 2.0)


def test_l2_norm_unit_heads(oracle):
    # ops_tests.rs:90-96, lib.rs:143-145
    h = oracle.l2_norm([3.0, 4.0, 0.0], 0.0)
    assert abs(math.sqrt(float(np.sum(h.astype(np.float64) ** 2))) - 1.0) < 1e-6
    assert h[0] == np.float32(0.6) and h[1] == np.float32(0.8) and h[2] == 0.0


def test_rope_position_zero_is_identity(oracle):
    # ops_tests.rs:98-109, lib.rs:129-137
    h = oracle.rope_neox([1.0, 2.0, 3.0, 4.0], pos=0, n_rot=4, head_dim=4, freq_base=1e7)
    assert h.tolist() == [1.0, 2.0, 3.0, 4.0]


def test_rope_rotates_one_pair(oracle):
    # ops_tests.rs:111-125: one pair, theta = 1, angle = 1 rad
    h = oracle.rope_neox([1.0, 0.0], pos=1, n_rot=2, head_dim=2, freq_base=1.0)
    assert abs(h[0] - math.cos(1.0)) < 1e-6 and abs(h[1] - math.sin(1.0)) < 1e-6


def test_softmax_sums_to_one_in_order(oracle):
    # ops_tests.rs:127-134, lib.rs:139-141
    p = oracle.softmax([1.0, 2.0, 3.0, 0.5])
    assert abs(float(np.sum(p.astype(np.float64))) - 1.0) < 1e-6
    assert p[2] > p[1] > p[0] > p[3]


def test_add(oracle):
    # lib.rs:147-149
    assert oracle.add([1.0, 2.0], [10.0, 20.0]).tolist() == [11.0, 22.0]


# ---- closed forms -------------------------------------------------------------

def test_rms_norm_constant_row_gives_the_weights(oracle):
    rng = np.random.default_rng(1)
    for n in (1, 7, 64, 4096):
        for c in (3.0, -0.125, 1e-20, 7e30):
            w = rng.standard_normal(n).astype(np.float32)
            out = oracle.rms_norm(np.full(n, c, np.float32), w, 0.0)
            assert np.array_equal(out, np.sign(np.float32(c)) * w)


def test_rms_norm_eps_after_the_mean(oracle):
    # ss = mean(1) = 1; scale = 1 / sqrt(1 + 3) = 0.5
    w = np.array([1.0, -2.0, 4.0, 8.0], np.float32)
    assert oracle.rms_norm(np.ones(4, np.float32), w, 3.0).tolist() == [0.5, -1.0, 2.0, 4.0]


def test_rms_norm_rows_are_independent(oracle):
    rng = np.random.default_rng(2)
    x = rng.standard_normal((5, 96)).astype(np.float32)
    w = rng.standard_normal(96).astype(np.float32)
    both = oracle.rms_norm(x, w, 1e-6)
    for r in range(5):
        ss = float(np.sum(x[r].astype(np.float64) ** 2)) / 96
        sc = 1.0 / math.sqrt(ss + 1e-6)
        want = (x[r].astype(np.float64) * sc * w.astype(np.float64)).astype(np.float32)
        assert np.max(np.abs(both[r] - want)) <= 1e-6 * np.max(np.abs(want))


def test_l2_norm_eps(oracle):
    # inv = 1 / sqrt(25 + 11) = 1/6
    h = oracle.l2_norm([3.0, 4.0], 11.0)
    assert h[0] == np.float32(0.5) and h[1] == np.float32(4.0 / 6.0)


def test_softmax_uniform_and_shift(oracle):
    for n in (1, 2, 8, 1024):
        assert np.all(oracle.softmax(np.full(n, 5.0, np.float32)) == np.float32(1.0 / n))
    a = oracle.softmax([1000.0, 1000.0, 999.0])
    b = oracle.softmax([1.0, 1.0, 0.0])
    assert np.array_equal(a, b)
    # -inf entries get 0
    c = oracle.softmax([0.0, -np.inf, 0.0])
    assert c.tolist() == [0.5, 0.0, 0.5]


def test_softmax_two_elements_closed_form(oracle):
    for d in (0.5, 3.0, -7.25):
        p = oracle.softmax([0.0, d])
        assert abs(p[1] - 1.0 / (1.0 + math.exp(-d))) < 2e-7
        assert abs(p[0] - 1.0 / (1.0 + math.exp(d))) < 2e-7


def test_rope_pairs_half_apart_with_exact_thetas(oracle):
    # base 16, n_rot 4: theta_0 = 1, theta_1 = 16^(-1/2) = 1/4; pos 4 gives
    # angles 4 and 1. Pairs are (0, 2) and (1, 3); dims 4, 5 pass through.
    h0 = np.array([1.0, 2.0, 0.5, -1.0, 9.0, -9.0], np.float32)
    h = oracle.rope_neox(h0, pos=4, n_rot=4, head_dim=6, freq_base=16.0)
    for i, ang in ((0, 4.0), (1, 1.0)):
        a, b = float(h0[i]), float(h0[i + 2])
        assert h[i] == f32(a * math.cos(ang) - b * math.sin(ang))
        assert h[i + 2] == f32(a * math.sin(ang) + b * math.cos(ang))
    assert h[4] == 9.0 and h[5] == -9.0


def test_rope_keeps_norms_and_composes(oracle):
    rng = np.random.default_rng(3)
    heads = rng.standard_normal((8, 128)).astype(np.float32)
    out = oracle.rope_neox(heads, pos=37, n_rot=64, head_dim=128, freq_base=1e6)
    assert np.array_equal(out[:, 64:], heads[:, 64:])
    n0 = heads[:, :32].astype(np.float64) ** 2 + heads[:, 32:64].astype(np.float64) ** 2
    n1 = out[:, :32].astype(np.float64) ** 2 + out[:, 32:64].astype(np.float64) ** 2
    assert np.max(np.abs(n1 - n0) / np.maximum(n0, 1e-30)) < 1e-6
    # rotating by 20 then 17 is rotating by 37, to f32 rounding
    two = oracle.rope_neox(oracle.rope_neox(heads, 20, 64, 128, 1e6), 17, 64, 128, 1e6)
    assert np.max(np.abs(two - out)) < 1e-5


def test_rope_odd_n_rot_and_short_head(oracle):
    # r = min(n_rot, head_dim, len) & ~1: n_rot 5 rotates the same two pairs as 4
    h0 = np.arange(1, 7, dtype=np.float32)
    a = oracle.rope_neox(h0, pos=3, n_rot=5, head_dim=6, freq_base=1e4)
    b = oracle.rope_neox(h0, pos=3, n_rot=4, head_dim=6, freq_base=1e4)
    assert np.array_equal(a, b)
    assert a[4] == 5.0 and a[5] == 6.0


# ---- the dense FFN half of a layer (qwen35.rs:112-129) ---------------------------

def test_dense_ffn_hand_computed(oracle):
    # F32 identity matrices: mixed = x * w / rms, g = u = mixed,
    # h = silu(mixed) * mixed, out = x + h
    eye = np.eye(2, dtype=np.float32).view(np.uint8)
    x = np.array([3.0, 4.0], np.float32)
    out = oracle.dense_ffn([0, 0, 0], [eye, eye, eye], 2, 2, x, [2.0, 2.0], 0.0)
    for i, v in enumerate((3.0, 4.0)):
        m = v * 2.0 / math.sqrt(12.5)
        assert abs(out[i] - (v + m / (1 + math.exp(-m)) * m)) < 1e-5


def test_dense_ffn_zero_paths_give_x(oracle):
    from strata_hip import synth as S
    n_embd, n_ff = 256, 512
    gate = S.matrix(12, 1, n_ff, n_embd)
    up = S.matrix(12, 2, n_ff, n_embd)
    down = S.matrix(14, 3, n_embd, n_ff)
    x = S.normal_f32(4, n_embd)
    # a zero norm weight zeroes mixed, so g = u = h = 0 and out = x exactly
    out = oracle.dense_ffn([12, 12, 14], [gate, up, down], n_embd, n_ff, x, np.zeros(n_embd, np.float32), 1e-6)
    assert np.array_equal(out, x)
    # zero up rows (all-zero blocks decode to 0) also leave out = x
    out = oracle.dense_ffn([12, 12, 14], [gate, np.zeros_like(up), down], n_embd, n_ff, x, S.normal_f32(5, n_embd),
                           1e-6)
    assert np.array_equal(out, x)
