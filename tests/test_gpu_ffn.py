"""The dense FFN half of a layer on the device (sh_ffn_dev) vs the oracle's
sho_dense_ffn (crates/strata-core/src/qwen35.rs:112-129: rms_norm, gate, up,
silu * up, down, residual add).

Tolerance: the matvec bound, 1e-3, on out - x (the FFN's own output, which
the residual add would otherwise hide) relative to its largest magnitude,
and per element with the 1e-3 rms floor at 2e-3 (conftest.check_parity); the residual add itself is checked at
f32 rounding. Covers the config's dense shape (Q4_K, hidden 4096, FFN 12288)
on the fused one-token path (three launches), three tokens and mixed types
on the general path, in-place output, and Q8_0 / Q5_K / Q6_K fused.
"""
import numpy as np
import pytest

import strata_hip as H
from conftest import check_parity
from strata_hip import synth as S

pytestmark = pytest.mark.gpu
TOL = 1e-3


def say(*a):
    print("[case]", *a, flush=True)


def run_ffn(quants, mats, n_embd, n_ff, x, norm, eps, in_place=False):
    import torch
    dev = [torch.from_numpy(np.ascontiguousarray(m)).cuda() for m in mats]
    xd = torch.from_numpy(np.ascontiguousarray(x)).cuda()
    nd = torch.from_numpy(np.ascontiguousarray(norm)).cuda()
    n_tok = x.shape[0]
    out = xd if in_place else torch.empty_like(xd)
    nb = H.ffn_workspace_bytes(n_tok, n_embd, n_ff)
    ws = torch.empty(nb, dtype=torch.uint8, device="cuda")
    H.ffn_dev([(q, 0, t.data_ptr()) for q, t in zip(quants, dev)], n_embd, n_ff, n_tok, xd.data_ptr(),
              nd.data_ptr(), eps, out.data_ptr(), ws.data_ptr(), nb, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    return out.cpu().numpy()


def check(got, want, x):
    dg, dw = got.astype(np.float64) - x, want.astype(np.float64) - x
    check_parity(dg, dw, "ffn out - x")


@pytest.mark.parametrize("quants,n_embd,n_ff,n_tok,in_place", [
    ((12, 12, 12), 4096, 12288, 1, False),   # the dense config, fused
    ((12, 12, 12), 4096, 12288, 1, True),
    ((12, 12, 12), 2048, 4096, 3, False),    # general path
    ((12, 12, 14), 2048, 4096, 1, True),     # mixed types: general path
    ((8, 8, 8), 2048, 4096, 1, False),       # fused Q8_0
    ((13, 13, 13), 2048, 4096, 1, False),    # fused Q5_K
    ((14, 14, 14), 2048, 4096, 1, False),    # fused Q6_K
    ((14, 14, 14), 4096, 2048, 1, False),    # fused Q6_K, gate/up rows of one whole window (read whole)
    ((12, 12, 12), 8192, 1024, 1, False),    # fused, rows of two windows: h formed in down's staging
    ((14, 14, 14), 8192, 1024, 1, True),
])
def test_ffn_matches_oracle(oracle, quants, n_embd, n_ff, n_tok, in_place):
    say("ffn", quants, n_embd, n_ff, n_tok, in_place)
    mats = [S.matrix(quants[0], 31, n_ff, n_embd), S.matrix(quants[1], 32, n_ff, n_embd),
            S.matrix(quants[2], 33, n_embd, n_ff)]
    x = S.normal_f32(34 + n_tok, n_tok * n_embd).reshape(n_tok, n_embd)
    norm = S.normal_f32(35, n_embd)
    got = run_ffn(quants, mats, n_embd, n_ff, x, norm, 1e-6, in_place)
    want = oracle.dense_ffn(quants, mats, n_embd, n_ff, x, norm, 1e-6)
    check(got, want, x)


def test_ffn_errors():
    say("ffn errors")
    with pytest.raises(H.BackendError):
        H.ffn_workspace_bytes(0, 4096, 12288)
    with pytest.raises(H.BackendError):
        H.ffn_dev([(12, 0, 256), (12, 0, 256), (12, 0, 256)], 4096, 12288, 1, 16, 16, 1e-6, 16, 256, 0)


@pytest.mark.parametrize("n_tok", [1, 5])
def test_ffn_host_slices_match_device_path(backend, oracle, n_tok):
    """sh_ffn (host slices, resident weights, in place) against the oracle
    and bit for bit against sh_ffn_dev."""
    say("ffn host", n_tok)
    n_embd, n_ff = 2048, 4096
    mats = [S.matrix(12, 41, n_ff, n_embd), S.matrix(12, 42, n_ff, n_embd), S.matrix(14, 43, n_embd, n_ff)]
    x = S.normal_f32(44 + n_tok, n_tok * n_embd).reshape(n_tok, n_embd)
    norm = S.normal_f32(45, n_embd)
    got = x.copy()
    backend.ffn(H.QuantTensor("ffn.gate", 12, n_ff, n_embd, mats[0]), H.QuantTensor("ffn.up", 12, n_ff, n_embd, mats[1]),
                H.QuantTensor("ffn.down", 14, n_embd, n_ff, mats[2]), norm, 1e-6, got)
    check(got, oracle.dense_ffn((12, 12, 14), mats, n_embd, n_ff, x, norm, 1e-6), x)
    assert np.array_equal(got, run_ffn((12, 12, 14), mats, n_embd, n_ff, x, norm, 1e-6))


def test_ffn_budget_holding_two_of_three_refuses(oracle):
    """Three matrices against a budget that holds two: the call fails with
    OutOfMemoryError instead of evicting a matrix it already holds, and the
    context keeps working."""
    say("ffn budget two of three")
    n_embd, n_ff = 1024, 2048
    mats = [S.matrix(12, 51, n_ff, n_embd), S.matrix(12, 52, n_ff, n_embd), S.matrix(12, 53, n_embd, n_ff)]
    x = S.normal_f32(54, n_embd).reshape(1, n_embd)
    norm = S.normal_f32(55, n_embd)
    ts = (H.QuantTensor("bud.gate", 12, n_ff, n_embd, mats[0]), H.QuantTensor("bud.up", 12, n_ff, n_embd, mats[1]),
          H.QuantTensor("bud.down", 12, n_embd, n_ff, mats[2]))
    budget = mats[0].nbytes + mats[1].nbytes + mats[2].nbytes // 2
    with H.HipBackend(0, budget) as be:
        got = x.copy()
        with pytest.raises(H.OutOfMemoryError):
            be.ffn(*ts, norm, 1e-6, got)
        assert np.array_equal(got, x)  # untouched: nothing ran
        assert be.resident_bytes() <= budget
    with H.HipBackend(0, sum(m.nbytes for m in mats)) as be:
        got = x.copy()
        be.ffn(*ts, norm, 1e-6, got)
    check(got, oracle.dense_ffn((12, 12, 12), mats, n_embd, n_ff, x, norm, 1e-6), x)


def test_ffn_host_shape_errors(backend):
    say("ffn host shape errors")
    n_embd, n_ff = 1024, 2048
    mats = [S.matrix(12, 61, n_ff, n_embd), S.matrix(12, 62, n_ff, n_embd), S.matrix(12, 63, n_embd, n_ff)]
    ts = (H.QuantTensor("se.gate", 12, n_ff, n_embd, mats[0]), H.QuantTensor("se.up", 12, n_ff, n_embd, mats[1]),
          H.QuantTensor("se.down", 12, n_embd, n_ff, mats[2]))
    with pytest.raises(H.ShapeError):  # short post_norm
        backend.ffn(*ts, np.ones(n_embd - 4, np.float32), 1e-6, np.zeros(n_embd, np.float32))
    with pytest.raises(H.ShapeError):  # ragged x
        backend.ffn(*ts, np.ones(n_embd, np.float32), 1e-6, np.zeros(n_embd + 4, np.float32))
