"""The trait's elementwise methods on the device vs the oracle
(ComputeBackend::{rms_norm, rope_neox, softmax, l2_norm, add},
crates/strata-core/src/backend.rs:38-50; CPU bodies ops.rs:46-165).

Tolerance, written per method: the device follows the CPU bodies operation
for operation, in f64 where they are, so outputs agree to the last f32 bit
except where the order of the f64 sums (butterfly instead of sequential) or
the device's pow / sin / cos (within an ulp of the platform libm's) or its
f32 exponential (the f64 one rounded once, against libm's expf) moves a
value across an f32 rounding boundary:
  rms_norm, l2_norm, rope   <= 1 ulp, >= 99% of elements bit-equal
  softmax                   <= 2 ulp, >= 99% bit-equal
  add                       bit-equal
Covers the reference's own unit cases (ops_tests.rs:79-135,
strata-backend-cpu lib.rs:121-151) through the host-slice entry points,
rows of 1 to 151,936 elements through the device entry points (one wave per
row up to 1024, four above), prefill rope over consecutive positions, empty
shapes, -inf logits, unaligned add and HIP graph replays.
"""
import math

import numpy as np
import pytest

import strata_hip as H
from strata_hip import synth as S

pytestmark = pytest.mark.gpu


def say(*a):
    print("[case]", *a, flush=True)


def ulps(a, b):
    """Per-element distance in f32 units in the last place (NaNs equal)."""
    a = np.ascontiguousarray(a, np.float32).view(np.int32).astype(np.int64)
    b = np.ascontiguousarray(b, np.float32).view(np.int32).astype(np.int64)
    # map to a monotone integer line: negative floats count down from 0
    a = np.where(a < 0, -(a & 0x7FFFFFFF), a)
    b = np.where(b < 0, -(b & 0x7FFFFFFF), b)
    return np.abs(a - b)


def close(got, want, max_ulp, min_exact):
    got = np.asarray(got, np.float32).reshape(-1)
    want = np.asarray(want, np.float32).reshape(-1)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    d = ulps(got[~nan], want[~nan])
    if d.size:
        assert d.max() <= max_ulp, (int(d.max()), int(np.argmax(d)))
        assert np.mean(d == 0) >= min_exact, float(np.mean(d == 0))


# ---- the reference's unit cases through the host-slice entry points --------

def test_reference_unit_cases(backend):
    say("elementwise reference unit cases")
    x = np.array([3.0, 4.0], np.float32)
    backend.rms_norm(x, [2.0, 2.0], 0.0)
    s = 2.0 / math.sqrt(12.5)
    assert abs(x[0] - np.float32(3.0 * s)) < 1e-6 and abs(x[1] - np.float32(4.0 * s)) < 1e-6

    h = np.array([1.0, 2.0, 3.0, 4.0], np.float32)
    backend.rope_neox(h, H.RopeCfg(pos=0, n_rot=4, head_dim=4, freq_base=1e7))
    assert h.tolist() == [1.0, 2.0, 3.0, 4.0]
    h = np.array([1.0, 0.0], np.float32)
    backend.rope_neox(h, H.RopeCfg(pos=1, n_rot=2, head_dim=2, freq_base=1.0))
    assert abs(h[0] - math.cos(1.0)) < 1e-6 and abs(h[1] - math.sin(1.0)) < 1e-6

    p = np.array([1.0, 2.0, 3.0, 0.5], np.float32)
    backend.softmax(p)
    assert abs(float(np.sum(p.astype(np.float64))) - 1.0) < 1e-6
    assert p[2] > p[1] > p[0] > p[3]

    h = np.array([3.0, 4.0, 0.0], np.float32)
    backend.l2_norm(h, 0.0)
    assert h[0] == np.float32(0.6) and h[1] == np.float32(0.8) and h[2] == 0.0

    a = np.array([1.0, 2.0], np.float32)
    backend.add(a, [10.0, 20.0])
    assert a.tolist() == [11.0, 22.0]


@pytest.mark.parametrize("n", [1, 5, 64, 1000, 1024, 1025, 2560, 4096, 5120])
def test_host_slices_match_oracle(backend, oracle, n):
    say("elementwise host slices", n)
    x = S.normal_f32(100 + n, n) * np.float32(3.0)
    w = S.normal_f32(200 + n, n)
    got = x.copy()
    backend.rms_norm(got, w, 1e-6)
    close(got, oracle.rms_norm(x, w, 1e-6), 1, 0.99)
    got = x.copy()
    backend.l2_norm(got, 1e-6)
    close(got, oracle.l2_norm(x, 1e-6), 1, 0.99)
    got = x.copy()
    backend.softmax(got)
    close(got, oracle.softmax(x), 2, 0.99)
    got = x.copy()
    cfg = H.RopeCfg(pos=777, n_rot=min(n, 64), head_dim=n, freq_base=1e6)
    backend.rope_neox(got, cfg)
    close(got, oracle.rope_neox(x, 777, min(n, 64), n, 1e6), 1, 0.99)
    got = x.copy()
    backend.add(got, w)
    assert np.array_equal(got, oracle.add(x, w))


def test_host_slice_errors_and_empty(backend):
    say("elementwise errors")
    with pytest.raises(H.ShapeError):
        backend.rms_norm(np.ones(4, np.float32), np.ones(3, np.float32), 0.0)
    with pytest.raises(H.ShapeError):
        backend.add(np.ones(4, np.float32), np.ones(5, np.float32))
    e = np.zeros(0, np.float32)
    backend.rms_norm(e, e, 0.0)
    backend.softmax(e)
    backend.l2_norm(e, 0.0)
    backend.add(e, e)
    backend.rope_neox(e, H.RopeCfg(pos=3, n_rot=4, head_dim=4, freq_base=1e4))


# ---- batched rows through the device entry points ---------------------------

def dev(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def stream():
    import torch
    return torch.cuda.current_stream().cuda_stream


def sync():
    import torch
    torch.cuda.synchronize()


@pytest.mark.parametrize("rows,n", [(1, 1), (3, 7), (32, 128), (16, 256), (33, 1024), (5, 1025),
                                    (16, 4096), (2, 5120), (1, 151936)])
def test_rms_and_l2_norm_rows(oracle, rows, n):
    say("rms_norm / l2_norm rows", rows, n)
    x = S.normal_f32(300 + rows + n, rows * n).reshape(rows, n)
    x[0, 0] = 40.0  # a dominant element
    w = S.normal_f32(400 + n, n)
    xd, wd = dev(x), dev(w)
    od = dev(np.zeros_like(x))
    H.rms_norm_dev(xd.data_ptr(), wd.data_ptr(), od.data_ptr(), rows, n, 1e-6, stream())
    H.rms_norm_dev(xd.data_ptr(), wd.data_ptr(), xd.data_ptr(), rows, n, 1e-6, stream())  # in place
    sync()
    want = oracle.rms_norm(x, w, 1e-6)
    close(od.cpu().numpy(), want, 1, 0.99)
    assert np.array_equal(xd.cpu().numpy(), od.cpu().numpy())
    ld = dev(x)
    H.l2_norm_dev(ld.data_ptr(), rows, n, 1e-6, stream())
    sync()
    close(ld.cpu().numpy(), oracle.l2_norm(x, 1e-6), 1, 0.99)


def test_rms_norm_eps_and_zero_rows(oracle):
    say("rms_norm eps / zero rows")
    x = np.zeros((4, 2048), np.float32)
    x[1] = 1.0
    x[2, :7] = -3.5
    w = S.normal_f32(5, 2048)
    xd, wd = dev(x), dev(w)  # held: a temporary's memory may be reused before the launch runs
    for eps in (1e-6, 3.0):
        od = dev(np.zeros_like(x))
        H.rms_norm_dev(xd.data_ptr(), wd.data_ptr(), od.data_ptr(), 4, 2048, eps, stream())
        sync()
        close(od.cpu().numpy(), oracle.rms_norm(x, w, eps), 1, 0.99)


@pytest.mark.parametrize("rows,n", [(1, 1), (4, 3), (32, 64), (32, 1024), (8, 1025), (32, 8192),
                                    (1, 151936)])
def test_softmax_rows(oracle, rows, n):
    say("softmax rows", rows, n)
    x = S.normal_f32(500 + rows + n, rows * n).reshape(rows, n) * np.float32(4.0)
    if n >= 3:
        x[:, 1] = -np.inf  # masked entries
        x[0, 2] = 60.0
    xd = dev(x)
    H.softmax_dev(xd.data_ptr(), rows, n, stream())
    sync()
    got = xd.cpu().numpy()
    close(got, oracle.softmax(x), 2, 0.99)
    if n >= 3:
        assert np.all(got[:, 1] == 0.0)


@pytest.mark.parametrize("n_tok,n_head,head_dim,n_rot,pos,base", [
    (1, 32, 128, 128, 0, 1e7), (1, 32, 128, 64, 4095, 1e7), (1, 16, 256, 64, 131071, 1e7),
    (7, 8, 128, 128, 100, 1e6), (16, 32, 128, 64, 30000, 5e6), (3, 4, 6, 5, 9, 1e4)])
def test_rope_heads_and_positions(oracle, n_tok, n_head, head_dim, n_rot, pos, base):
    say("rope", n_tok, n_head, head_dim, n_rot, pos, base)
    rows = n_tok * n_head
    x = S.normal_f32(600 + rows + head_dim, rows * head_dim).reshape(rows, head_dim)
    xd = dev(x)
    H.rope_neox_dev(xd.data_ptr(), rows, n_head, H.RopeCfg(pos, n_rot, head_dim, base), stream())
    sync()
    got = xd.cpu().numpy()
    want = np.concatenate([oracle.rope_neox(x[t * n_head:(t + 1) * n_head], pos + t, n_rot, head_dim, base)
                           for t in range(n_tok)])
    close(got, want, 1, 0.99)
    r = min(n_rot, head_dim) & ~1
    assert np.array_equal(got[:, r:], x[:, r:])


@pytest.mark.parametrize("n,off", [(1, 0), (1000, 0), (4096, 1), (1 << 22, 0), ((1 << 20) + 3, 3)])
def test_add_bit_exact(oracle, n, off):
    say("add", n, off)
    import torch
    a = S.normal_f32(700 + n, n + off)
    b = S.normal_f32(800 + n, n + off)
    ad, bd = dev(a), dev(b)
    H.add_dev(ad.data_ptr() + 4 * off, bd.data_ptr(), n, stream())
    sync()
    got = ad.cpu().numpy()
    assert np.array_equal(got[:off], a[:off])
    assert np.array_equal(got[off:], oracle.add(a[off:], b[:n]))
    del torch


def test_rowops_graph_replays(oracle):
    """A decode step's elementwise work captured once and replayed: every
    replay (inputs restored by a copy kernel between them) equals the eager
    result."""
    import torch
    say("rowops graph replays")
    n_head, head_dim, n_embd = 32, 128, 4096
    x0 = S.normal_f32(901, n_embd)
    w = S.normal_f32(902, n_embd)
    q0 = S.normal_f32(903, n_head * head_dim)
    xs, ws, qs = dev(x0), dev(w), dev(q0)
    out = dev(np.zeros(n_embd, np.float32))
    xin, qin = dev(x0), dev(q0)
    s = torch.cuda.Stream()

    def step(h):
        H.rms_norm_dev(xs.data_ptr(), ws.data_ptr(), out.data_ptr(), 1, n_embd, 1e-6, h)
        H.rope_neox_dev(qs.data_ptr(), n_head, n_head, H.RopeCfg(77, 64, head_dim, 1e7), h)
        H.l2_norm_dev(qs.data_ptr(), n_head, head_dim, 1e-6, h)
        H.softmax_dev(qs.data_ptr(), n_head, head_dim, h)
        H.add_dev(out.data_ptr(), xs.data_ptr(), n_embd, h)

    with torch.cuda.stream(s):
        step(s.cuda_stream)
    torch.cuda.synchronize()
    eager_out, eager_q = out.cpu().numpy(), qs.cpu().numpy()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        step(torch.cuda.current_stream().cuda_stream)
    for _ in range(3):
        qs.copy_(qin)
        xs.copy_(xin)
        out.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(out.cpu().numpy(), eager_out)
        assert np.array_equal(qs.cpu().numpy(), eager_q)
    want_q = oracle.softmax(oracle.l2_norm(oracle.rope_neox(q0.reshape(n_head, head_dim), 77, 64, head_dim, 1e7),
                                           1e-6))
    close(eager_q, want_q, 3, 0.98)
    want_out = oracle.add(oracle.rms_norm(x0, w, 1e-6), x0)
    close(eager_out, want_out, 1, 0.99)
