"""Expert gather-matvec in the reference orientation vs ops::expert_gemv.

Expert tensors are [n_expert][rows = in][cols = out] with blocks along the
output axis (crates/strata-core/src/weights.rs:14-34). Shapes from the MoE
config (gate/up 2048 -> 768 Q4_K, down 768 -> 2048 Q6_K) plus ragged ones;
the x[i] == 0 skip of ops.rs:182-184 is checked with a NaN weight row.
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


@pytest.mark.parametrize("quant,n_expert,rows,cols", [
    (12, 128, 2048, 768), (14, 128, 768, 2048), (8, 4, 300, 512), (12, 3, 5, 256), (14, 2, 1, 256),
    (12, 2, 4096, 12288), (13, 128, 2048, 768), (13, 3, 5, 256), (13, 2, 1, 256), (13, 4, 300, 1024),
])
def test_expert_gemv(backend, oracle, quant, n_expert, rows, cols):
    say("expert_gemv", quant, n_expert, rows, cols)
    w = S.matrix(quant, 600 + rows + quant, n_expert * rows, cols)
    view = H.ExpertView(f"exps{quant}_{rows}_{cols}", quant, n_expert, rows, cols, w)
    for e in sorted({0, n_expert // 2, n_expert - 1}):
        x = S.normal_f32(e + 1, rows)
        y = np.empty(cols, np.float32)
        backend.expert_gemv(view, e, x, y)
        want = oracle.expert_gemv(quant, n_expert, rows, cols, w, e, x)
        check_parity(y, want, f"expert_gemv q{quant} {rows}x{cols} e{e}")
    backend.evict(view.name)


def test_expert_gemv_skips_zero_inputs(backend):
    say("expert_gemv zero skip")
    rows, cols = 4, 256
    w = S.matrix(12, 3, rows, cols).copy()
    w[144 * 2: 144 * 2 + 2] = [0x00, 0x7E]  # row 2's d = f16 NaN
    view = H.ExpertView("nanrow", 12, 1, rows, cols, w)
    y = np.empty(cols, np.float32)
    backend.expert_gemv(view, 0, np.array([1.0, -2.0, 0.0, 0.5], np.float32), y)
    assert np.all(np.isfinite(y))


def test_expert_gemv_errors(backend):
    say("expert_gemv errors")
    w = S.matrix(12, 3, 2 * 8, 256)
    view = H.ExpertView("errs", 12, 2, 8, 256, w)
    with pytest.raises(H.ShapeError):
        backend.expert_gemv(view, 2, np.zeros(8, np.float32), np.zeros(256, np.float32))
    with pytest.raises(H.ShapeError):
        backend.expert_gemv(view, 0, np.zeros(9, np.float32), np.zeros(256, np.float32))
    with pytest.raises(H.TruncatedError):
        short = H.ExpertView("errs_short", 12, 2, 8, 256, w[:-144])
        backend.expert_gemv(short, 0, np.zeros(8, np.float32), np.zeros(256, np.float32))



@pytest.mark.parametrize("quant", [12, 8, 13, 14])
def test_expert_gemv_ggml_orientation(backend, oracle, quant):
    """SH_FLAG_EXPERT_OUT_MAJOR: experts stored as llama.cpp GGUFs do,
    [n_expert][out][in], each expert an ordinary matvec of its slice."""
    n_expert, rows, cols = 4, 768, 2048
    w = S.matrix(quant, 8800 + quant, n_expert * rows, cols)
    x = S.normal_f32(8900 + quant, cols)
    v = H.ExpertView(f"ggml{quant}", quant, n_expert, rows, cols, w, flags=H.FLAG_EXPERT_OUT_MAJOR)
    rb = S.row_bytes(quant, cols)
    for e in (0, 3):
        y = np.empty(rows, np.float32)
        backend.expert_gemv(v, e, x, y)
        want = oracle.gemv(quant, rows, cols, w[e * rows * rb:(e + 1) * rows * rb], x)
        check_parity(y, want, f"expert_gemv out-major q{quant} e{e}")
