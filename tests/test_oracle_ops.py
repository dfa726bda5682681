"""Pins the oracle's gemv, expert_gemv and MoE routing/combine.

* the reference's unit tests: crates/strata-core/tests/ops_tests.rs:22-61,
  crates/strata-backend-cpu/src/lib.rs:88-120, and the wgpu parity shapes
  (crates/strata-backend-wgpu/src/gpu.rs:513-575) against manual dots;
* brute force with exact rational arithmetic on tiny shapes: the oracle's
  f64 sum may differ from the exact sum only by f64 rounding;
* the sequential f64 order (ops.rs:22-26): the oracle equals a Python loop
  of the same order bit for bit, and the threaded variant equals it too;
* MoE routing invariants (crates/strata-core/src/moe.rs:58-90): weights sum
  to one, ids ascending, ties to the lower id, uniform logits give uniform
  weights; the routed combine equals its composition from expert_gemv;
* the whole MoE layer (moe.rs:48-143): with the shared expert off it is the
  routed part on router . bf16(x) bit for bit; with the routed experts off
  and a zero gate input it is exactly half the shared expert's output; a
  tie that exists only after bf16 rounding routes to the lower id.
"""
from fractions import Fraction

import numpy as np
import pytest

import np_oracle as N
from strata_hip import synth as S


def f32_matrix(rows, cols, f):
    return np.array([[f(r, c) for c in range(cols)] for r in range(rows)], np.float32)


def test_gemv_matches_manual_dot(oracle):
    # ops_tests.rs:22-42
    rows, cols = 3, 4
    w = f32_matrix(rows, cols, lambda r, c: float(r * cols + c) + 1.0)
    x = np.array([1.0, 2.0, 3.0, 4.0], np.float32)
    y = oracle.gemv(oracle.F32, rows, cols, w.view(np.uint8), x)
    for r in range(rows):
        expect = sum(float(w[r, c]) * float(x[c]) for c in range(cols))
        assert abs(float(y[r]) - expect) < 1e-4


def test_cpu_backend_gemv_values(oracle):
    # crates/strata-backend-cpu/src/lib.rs:88-100: y = [14, 32]
    w = f32_matrix(2, 3, lambda r, c: float(r * 3 + c) + 1.0)
    y = oracle.gemv(oracle.F32, 2, 3, w.view(np.uint8), np.array([1, 2, 3], np.float32))
    assert abs(y[0] - 14.0) < 1e-4 and abs(y[1] - 32.0) < 1e-4


def q8_single_block():
    # ops_tests.rs:44-61 / lib.rs:102-120: d = 0.5, q = (j % 7) - 3
    b = np.zeros(34, np.uint8)
    b[:2] = np.array([0.5], np.float32).astype(np.float16).view(np.uint8)
    for j in range(32):
        b[2 + j] = np.uint8((j % 7 - 3) & 0xFF)
    x = np.array([i * 0.25 - 1.0 for i in range(32)], np.float32)
    return b, x


def test_gemv_q8_0_matches_dequant_dot(oracle):
    b, x = q8_single_block()
    y = oracle.gemv(oracle.Q8_0, 1, 32, b, x)
    expect = sum(float(j % 7 - 3) * 0.5 * float(x[j]) for j in range(32))
    assert abs(float(y[0]) - expect) < 1e-4


def test_expert_gemv_matches_transposed_dot(oracle):
    # gpu.rs:537-575: two experts of [rows = 5][cols = 8]
    n_expert, rows, cols = 2, 5, 8
    data = np.array([[[((e * 100 + r * 10 + c) % 13) * 0.2 - 1.0 for c in range(cols)]
                      for r in range(rows)] for e in range(n_expert)], np.float32)
    x = np.array([(i % 3) - 0.5 for i in range(rows)], np.float32)
    for e in range(n_expert):
        y = oracle.expert_gemv(oracle.F32, n_expert, rows, cols, data.view(np.uint8), e, x)
        for c in range(cols):
            expect = sum(float(data[e, i, c]) * float(x[i]) for i in range(rows))
            assert abs(float(y[c]) - expect) < 1e-6


def _exact_dot(wrow, x):
    return sum(Fraction(float(a)) * Fraction(float(b)) for a, b in zip(wrow, x))


@pytest.mark.parametrize("quant,rows,cols", [(8, 5, 64), (12, 3, 256), (14, 3, 512)])
def test_gemv_brute_force_exact(oracle, quant, rows, cols):
    w = S.matrix(quant, 99 + quant, rows, cols)
    x = S.normal_f32(5, cols)
    y = oracle.gemv(quant, rows, cols, w, x)
    deq = oracle.dequantize(quant, w, rows, cols)
    for r in range(rows):
        exact = _exact_dot(deq[r], x)
        mag = sum(abs(Fraction(float(a)) * Fraction(float(b))) for a, b in zip(deq[r], x))
        # f64 sequential sum of `cols` terms, then one f32 rounding
        bound = float(mag) * cols * 2.0 ** -52 + abs(float(exact)) * 2.0 ** -24
        assert abs(float(y[r]) - float(exact)) <= bound


def test_gemv_sequential_f64_order(oracle):
    rows, cols = 4, 512
    w = S.matrix(12, 31, rows, cols)
    x = S.normal_f32(32, cols)
    y = oracle.gemv(12, rows, cols, w, x)
    deq = oracle.dequantize(12, w, rows, cols)
    for r in range(rows):
        acc = 0.0
        for c in range(cols):
            acc += float(deq[r, c]) * float(x[c])
        assert np.float32(acc) == y[r]


@pytest.mark.parametrize("quant", [8, 12, 14])
def test_gemv_threads_identical_and_numpy_close(oracle, quant):
    rows, cols = 97, 1024
    w = S.matrix(quant, 7 + quant, rows, cols)
    x = S.normal_f32(8, cols)
    y1 = oracle.gemv(quant, rows, cols, w, x)
    y4 = oracle.gemv(quant, rows, cols, w, x, threads=4)
    assert np.array_equal(y1, y4)
    yn = N.gemv(quant, w, rows, cols, x)
    assert np.abs(y1 - yn).max() <= 1e-6 * np.abs(yn).max()


def test_expert_gemv_skips_zero_inputs(oracle):
    # ops.rs:182-184: a row whose x is 0 is not read, so a NaN weight there
    # does not poison the sum
    rows, cols, n_expert = 4, 256, 1
    w = S.matrix(12, 3, rows, cols).copy()
    w[144 * 2: 144 * 2 + 2] = [0x00, 0x7E]  # row 2's d = f16 NaN
    x = np.array([1.0, -2.0, 0.0, 0.5], np.float32)
    y = oracle.expert_gemv(12, n_expert, rows, cols, w, 0, x)
    assert np.all(np.isfinite(y))
    x[2] = 1.0
    assert np.all(np.isnan(oracle.expert_gemv(12, n_expert, rows, cols, w, 0, x)[:256]))


@pytest.mark.parametrize("quant,rows,cols", [(12, 16, 512), (14, 8, 512), (8, 8, 64)])
def test_expert_gemv_equals_transposed_gemv_exactly(oracle, quant, rows, cols):
    # both sum the same f64 products; the expert sum runs over rows i in order
    n_expert = 3
    w = S.matrix(quant, 11, n_expert * rows, cols)
    x = S.normal_f32(12, rows)
    deq = oracle.dequantize(quant, w, n_expert * rows, cols).reshape(n_expert, rows, cols)
    for e in range(n_expert):
        y = oracle.expert_gemv(quant, n_expert, rows, cols, w, e, x)
        for c in range(0, cols, 37):
            acc = 0.0
            for i in range(rows):
                acc += float(x[i]) * float(deq[e, i, c])
            assert np.float32(acc) == y[c]


# ---- MoE routing --------------------------------------------------------------

def test_route_invariants(oracle):
    for seed in range(20):
        logits = S.normal_f32(seed, 128)
        ids, w = oracle.moe_route(logits, 8)
        assert len(ids) == 8
        assert np.all(np.diff(ids) > 0)
        assert abs(float(np.sum(w.astype(np.float64))) - 1.0) < 1e-6
        # the selected set is the 8 largest logits (softmax is monotone)
        assert set(ids.tolist()) == set(np.argsort(-logits.astype(np.float64), kind="stable")[:8].tolist())


def test_route_ties_go_to_lower_ids(oracle):
    logits = np.zeros(16, np.float32)
    logits[[3, 9, 12]] = 1.0
    ids, w = oracle.moe_route(logits, 5)
    # the three 1.0 logits, then the two lowest ids among the zero logits
    assert ids.tolist() == [0, 1, 3, 9, 12]


def test_route_uniform_logits_give_uniform_weights(oracle):
    ids, w = oracle.moe_route(np.full(8, 0.3, np.float32), 8)
    assert ids.tolist() == list(range(8))
    assert np.all(w == np.float32(0.125))


def test_route_hand_computed(oracle):
    # logits [0, ln 3, ln 2] -> softmax [1/6, 1/2, 1/3]; top-2 ids [1, 2] with
    # renormalised weights [3/5, 2/5]
    logits = np.array([0.0, np.log(3.0), np.log(2.0)], np.float32)
    ids, w = oracle.moe_route(logits, 2)
    assert ids.tolist() == [1, 2]
    assert abs(w[0] - 0.6) < 1e-6 and abs(w[1] - 0.4) < 1e-6


def test_routed_combine_is_its_composition(oracle):
    n_expert, n_embd, n_ff = 4, 256, 512
    gate = S.matrix(12, 1, n_expert * n_embd, n_ff)
    up = S.matrix(12, 2, n_expert * n_embd, n_ff)
    down = S.matrix(14, 3, n_expert * n_ff, n_embd)
    x = S.normal_f32(4, n_embd)
    ids, w = oracle.moe_route(S.normal_f32(5, n_expert), 2)
    out = oracle.moe_routed(12, 12, 14, n_expert, n_embd, n_ff, gate, up, down, ids, w, x)
    want = np.zeros(n_embd, np.float32)
    for e, we in zip(ids, w):
        h = oracle.expert_gemv(12, n_expert, n_embd, n_ff, gate, int(e), x)
        p = oracle.expert_gemv(12, n_expert, n_embd, n_ff, up, int(e), x)
        a = np.array([np.float32(oracle.silu(float(v))) * p[i] for i, v in enumerate(h)], np.float32)
        d = oracle.expert_gemv(14, n_expert, n_ff, n_embd, down, int(e), a)
        want = (want + (np.float32(we) * d).astype(np.float32)).astype(np.float32)
    assert np.array_equal(out, want)


def test_routed_out_major_is_the_transposed_in_major(oracle):
    """F32 stacks can be transposed exactly: an out-major stack holding
    W_e^T gives bit for bit the in-major result (both sum x[i] * W_e[i][o]
    over i in f64 in the same order), which pins the out-major slice and
    row arithmetic."""
    n_expert, n_embd, n_ff = 5, 64, 96
    rng = np.random.default_rng(31)
    g_in = rng.standard_normal((n_expert, n_embd, n_ff)).astype(np.float32)
    u_in = rng.standard_normal((n_expert, n_embd, n_ff)).astype(np.float32)
    d_in = rng.standard_normal((n_expert, n_ff, n_embd)).astype(np.float32)
    x = rng.standard_normal(n_embd).astype(np.float32)
    ids, w = oracle.moe_route(rng.standard_normal(n_expert).astype(np.float32), 3)
    tr = lambda a: np.ascontiguousarray(a.transpose(0, 2, 1))
    a = oracle.moe_routed(0, 0, 0, n_expert, n_embd, n_ff, g_in.view(np.uint8), u_in.view(np.uint8),
                          d_in.view(np.uint8), ids, w, x)
    b = oracle.moe_routed(0, 0, 0, n_expert, n_embd, n_ff, tr(g_in).view(np.uint8), tr(u_in).view(np.uint8),
                          tr(d_in).view(np.uint8), ids, w, x, out_major=True)
    assert np.array_equal(a, b)
    # and the orientation matters for a stack that is not symmetric
    c = oracle.moe_routed(0, 0, 0, n_expert, n_embd, n_ff, tr(g_in).view(np.uint8), tr(u_in).view(np.uint8),
                          tr(d_in).view(np.uint8), ids, w, x)
    assert not np.array_equal(a, c)


def test_routed_out_major_quantized_is_gemv_of_slices(oracle):
    """Quantized out-major experts: gate_e . x is ops::gemv of rows
    [e * n_ff, (e + 1) * n_ff) of the stack (checked through the oracle's
    own gemv on the sliced bytes for one expert at weight 1)."""
    n_expert, n_embd, n_ff = 3, 256, 256
    gate = S.matrix(12, 41, n_expert * n_ff, n_embd)
    up = S.matrix(12, 42, n_expert * n_ff, n_embd)
    down = S.matrix(14, 43, n_expert * n_embd, n_ff)
    x = S.normal_f32(44, n_embd)
    rg, rd = S.row_bytes(12, n_embd), S.row_bytes(14, n_ff)
    e = 2
    out = oracle.moe_routed(12, 12, 14, n_expert, n_embd, n_ff, gate, up, down, np.array([e]),
                            np.array([1.0], np.float32), x, out_major=True)
    h = oracle.gemv(12, n_ff, n_embd, gate[e * n_ff * rg:(e + 1) * n_ff * rg], x)
    p = oracle.gemv(12, n_ff, n_embd, up[e * n_ff * rg:(e + 1) * n_ff * rg], x)
    a = np.array([np.float32(oracle.silu(float(v))) * p[i] for i, v in enumerate(h)], np.float32)
    d = oracle.gemv(14, n_embd, n_ff, down[e * n_embd * rd:(e + 1) * n_embd * rd], a)
    assert np.array_equal(out, d)


def test_silu_closed_form(oracle):
    for v in [-20.0, -1.0, 0.0, 0.5, 3.0, 40.0]:
        ref = v / (1.0 + np.exp(-v))
        assert abs(oracle.silu(v) - ref) <= 2e-7 * max(1.0, abs(ref))


# ---- prefill matmul and Q8 activation blocks --------------------------------

def test_matmul_is_stacked_gemv(oracle):
    # no reference matmul exists (generate.rs:116-117): the op is m gemvs
    rows, cols, m = 40, 512, 5
    w = S.matrix(12, 71, rows, cols)
    x = S.normal_f32(72, m * cols).reshape(m, cols)
    y = oracle.matmul(12, rows, cols, w, x, threads=3)
    for t in range(m):
        assert np.array_equal(y[t], oracle.gemv(12, rows, cols, w, x[t]))


def test_quantize_q8_known_answers(oracle):
    # block 0: max|x| = 127 -> s = 1 exactly, so codes are x rounded to
    # nearest even (2.5 -> 2, 3.5 -> 4, -2.5 -> -2, 0.5 -> 0, 1.5 -> 2);
    # block 1: all zero -> s = 0, codes 0; block 2: one non-zero value
    x = np.zeros(96, np.float32)
    x[:8] = [127.0, 2.5, 3.5, -2.5, -127.0, 0.5, 1.5, -0.49]
    x[64 + 7] = -3.0
    q, s, u = oracle.quantize_q8(x)
    assert s[0] == 1.0 and s[1] == 0.0 and s[2] == np.float32(3.0) / np.float32(127.0)
    assert q[:8].tolist() == [127, 2, 4, -2, -127, 0, 2, 0]
    assert not q[8:64].any()
    assert q[64 + 7] == -127 and np.count_nonzero(q[64:]) == 1
    assert u[0] == np.float32(sum(q[:32].astype(int)))
    assert u[1] == 0.0 and u[2] == np.float32(s[2] * np.float32(-127))


def test_quantize_q8_closed_form(oracle):
    # every code is within half a step of x / s, the block max maps to +-127,
    # and round-half-even agrees with numpy's rint
    x = S.normal_f32(73, 32 * 500) * np.float32(3.0)
    q, s, u = oracle.quantize_q8(x)
    xb = x.reshape(-1, 32).astype(np.float64)
    sb = s.astype(np.float64)[:, None]
    assert np.all(np.abs(xb / sb - q.reshape(-1, 32)) <= 0.5 + 1e-6)
    assert np.all(np.abs(q.reshape(-1, 32)).max(axis=1) == 127)
    ref = np.rint((x.reshape(-1, 32) / s[:, None]).astype(np.float32)).astype(np.int8)
    assert np.array_equal(q.reshape(-1, 32), ref)
    assert np.array_equal(u, (s * q.reshape(-1, 32).astype(np.int64).sum(axis=1).astype(np.float32)))


def test_quantize_q8k_known_answers(oracle):
    # block 0: max|x| = 127 anywhere in the 256 -> s = 1 exactly, codes are x
    # rounded to nearest even, sums per 32 elements; block 1: all zero
    x = np.zeros(512, np.float32)
    x[:6] = [2.5, 3.5, -2.5, 0.5, 1.5, -0.49]
    x[200] = -127.0
    x[33] = 7.0
    q, s, u = oracle.quantize_q8k(x)
    assert s.tolist() == [1.0, 0.0]
    assert q[:6].tolist() == [2, 4, -2, 0, 2, 0] and q[200] == -127 and q[33] == 7
    assert np.count_nonzero(q) == 6  # 0.5 and -0.49 round to 0
    assert u.tolist() == [6, 7, 0, 0, 0, 0, -127, 0] + [0] * 8


def test_quantize_q8k_is_q8_when_every_sub_block_holds_the_max(oracle):
    # with +-max|x| of the 256 in each of its 32-element sub-blocks, the one
    # super-block scale equals every block scale of the 32-element quantizer:
    # the codes agree and the integer sums are its u / s
    rng = np.random.default_rng(75)
    x = S.normal_f32(75, 256 * 40)
    xb = x.reshape(-1, 8, 32)
    amax = np.abs(xb).max(axis=(1, 2))
    for b in range(xb.shape[0]):
        for j in range(8):
            xb[b, j, rng.integers(32)] = amax[b] * (1 if rng.integers(2) else -1)
    q, s, u = oracle.quantize_q8k(x)
    q8, s8, u8 = oracle.quantize_q8(x)
    assert np.array_equal(q, q8)
    assert np.array_equal(np.repeat(s, 8), s8)
    assert np.array_equal(s8 * u.astype(np.float32), u8)


def test_quantize_q8k_closed_form(oracle):
    # one scale per 256 (not per 32): numpy restatement with f32 division and
    # rint, the max maps to +-127, sums over each 32-element sub-block
    x = S.normal_f32(76, 256 * 300) * np.float32(3.0)
    x[256 * 7: 256 * 8] = 0.0
    q, s, u = oracle.quantize_q8k(x)
    xb = x.reshape(-1, 256)
    sref = (np.abs(xb).max(axis=1) / np.float32(127.0)).astype(np.float32)
    assert np.array_equal(s, sref)
    with np.errstate(invalid="ignore", divide="ignore"):
        ref = np.where(sref[:, None] > 0, np.rint(xb / sref[:, None]), 0).astype(np.int8)
    assert np.array_equal(q.reshape(-1, 256), ref)
    assert np.all(np.abs(ref).max(axis=1)[sref > 0] == 127)
    assert np.array_equal(u, ref.reshape(-1, 32).astype(np.int64).sum(axis=1))


def test_bf16_round_matches_torch_and_scalar(oracle):
    import torch
    x = np.concatenate([S.normal_f32(74, 4096) * np.float32(100.0),
                        np.array([1.0 + 2.0 ** -8, 1.0 + 3 * 2.0 ** -8, -(1.0 + 2.0 ** -8), 0.0, -0.0,
                                  3.0e38, 1.0e-40], np.float32)])
    got = oracle.bf16_round_array(x)
    want = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    for v in x[-7:]:
        assert np.float32(oracle.lib().sho_bf16_round(float(v))) == oracle.bf16_round_array(np.float32(v))


def test_sigmoid_closed_form(oracle):
    # ops.rs:90-92: 1 / (1 + exp(-x)) in f32
    assert oracle.sigmoid(0.0) == 0.5
    assert oracle.sigmoid(100.0) == 1.0
    assert oracle.sigmoid(-100.0) < 1e-40
    for v in (-3.0, -0.5, 0.25, 2.0):
        assert abs(oracle.sigmoid(v) - 1.0 / (1.0 + np.exp(-v))) < 1e-7


def moe_layer_tensors(n_expert, n_embd, n_ff, n_sh, seed):
    f32 = lambda s, n: S.normal_f32(s, n).view(np.uint8)  # noqa: E731
    router = f32(seed, n_expert * n_embd)
    gate = S.matrix(12, seed + 1, n_expert * n_embd, n_ff)
    up = S.matrix(12, seed + 2, n_expert * n_embd, n_ff)
    down = S.matrix(14, seed + 3, n_expert * n_ff, n_embd)
    g_sh = S.matrix(8, seed + 4, n_sh, n_embd)
    u_sh = S.matrix(8, seed + 5, n_sh, n_embd)
    d_sh = S.matrix(12, seed + 6, n_embd, n_sh)
    inp = f32(seed + 7, n_embd)
    return [0, 12, 12, 14, 8, 8, 12, 0], [router, gate, up, down, g_sh, u_sh, d_sh, inp]


def test_moe_layer_without_shared_expert_is_the_routed_part(oracle):
    """moe.rs:48-127: with the shared down matrix zero the layer is route on
    router . bf16(x) plus the routed combine, bit for bit."""
    n_expert, n_embd, n_ff, n_sh, k = 16, 256, 256, 256, 4
    q, t = moe_layer_tensors(n_expert, n_embd, n_ff, n_sh, 8100)
    t[6] = np.zeros_like(t[6])
    x = S.normal_f32(8101, n_embd)
    got = oracle.moe_layer(q, t, n_expert, n_embd, n_ff, n_sh, x, k)
    xb = np.array([oracle.lib().sho_bf16_round(float(v)) for v in x], np.float32)
    logits = oracle.gemv(0, n_expert, n_embd, t[0], xb)
    ids, w = oracle.moe_route(logits, k)
    want = oracle.moe_routed(12, 12, 14, n_expert, n_embd, n_ff, t[1], t[2], t[3], ids, w, x)
    assert np.array_equal(got, want)


def test_moe_layer_shared_expert_half_gate(oracle):
    """moe.rs:129-142: with every routed down matrix zero and a zero gate
    input row (sigmoid(0) = 1/2 exactly), the layer is half the shared
    expert's output: down_sh . (silu(gate_sh . x) * (up_sh . x)) / 2."""
    n_expert, n_embd, n_ff, n_sh, k = 8, 256, 256, 512, 2
    q, t = moe_layer_tensors(n_expert, n_embd, n_ff, n_sh, 8200)
    t[3] = np.zeros_like(t[3])
    t[7] = np.zeros_like(t[7])
    x = S.normal_f32(8201, n_embd)
    got = oracle.moe_layer(q, t, n_expert, n_embd, n_ff, n_sh, x, k)
    g = oracle.gemv(8, n_sh, n_embd, t[4], x)
    u = oracle.gemv(8, n_sh, n_embd, t[5], x)
    h = np.array([oracle.silu(float(a)) for a in g], np.float32) * u
    d = oracle.gemv(12, n_embd, n_sh, t[6], h)
    assert np.array_equal(got, np.float32(0.5) * d)
    assert np.any(got != 0)


def test_moe_layer_routes_on_bf16_rounded_x(oracle):
    """moe.rs:55: the router sees bf16(x). Two experts whose logits are x[0]
    and x[1]; x[1] = 1 + 2^-9 rounds to 1.0 = x[0], so the tie goes to
    expert 0 (without the rounding expert 1 would win). Expert 1's down
    matrix is zero and the shared expert is off, so a nonzero output shows
    expert 0 was chosen."""
    n_expert, n_embd, n_ff, n_sh, k = 2, 256, 256, 256, 1
    q, t = moe_layer_tensors(n_expert, n_embd, n_ff, n_sh, 8300)
    router = np.zeros((n_expert, n_embd), np.float32)
    router[0, 0] = 1.0
    router[1, 1] = 1.0
    t[0] = router.view(np.uint8).reshape(-1)
    rb = S.row_bytes(14, n_embd)
    down = t[3].copy()
    down[n_ff * rb:] = 0  # expert 1
    t[3] = down
    t[6] = np.zeros_like(t[6])
    x = S.normal_f32(8301, n_embd)
    x[0], x[1] = 1.0, np.float32(1.0 + 2.0 ** -9)
    got = oracle.moe_layer(q, t, n_expert, n_embd, n_ff, n_sh, x, k)
    assert np.any(got != 0)
    want = oracle.moe_routed(12, 12, 14, n_expert, n_embd, n_ff, t[1], t[2], t[3], np.array([0]),
                             np.array([1.0], np.float32), x)
    assert np.array_equal(got, want)
