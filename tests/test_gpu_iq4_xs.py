"""IQ4_XS beyond the batch-1 matvec: the expert gather-matvec in both
orientations, the fused MoE with IQ4_XS gate / up (and down), the batched
matvec (one weight read for every vector of the batch) and the prefill
matmul, each in both code-byte readings.

The reference's dequantizer reads the first 16 qs bytes for every sub-block
(crates/strata-gguf/src/dequant.rs:189-206, its qs slice never advances);
ggml's reads 16 bytes per sub-block (SH_FLAG_IQ4XS_GGML). The oracle's
restatement takes either reading (its dequant is pinned against both in the
CPU suite), and every device result here is checked against the oracle under
the same reading -- and, where the shape allows, shown to differ from the
other reading, so a test cannot pass on the wrong bytes.

Bars as the other formats': the matvec, expert and MoE paths at
max|y - r| / max|r| <= 1e-3 plus the per-element bar; the matmul's bf16
mode at 2e-2 against the f32 oracle and 1e-3 against the same sums on
bf16-rounded operands; its q8 mode (32-element activation blocks) at 1e-3
and the strict bar against the oracle on x rounded through the blocks, 2e-2
against the f32 oracle.
"""
import numpy as np
import pytest

import strata_hip as H
from conftest import STRICT_TOL, check_parity, rel_err
from strata_hip import synth as S

pytestmark = pytest.mark.gpu
IQ = 23
Q6K = 14
OM = H.FLAG_EXPERT_OUT_MAJOR
TOL_F32 = 2e-2
TOL_EXACT_OPERANDS = 1e-3


def say(*a):
    print("[case]", *a, flush=True)


def reading(oracle, ggml):
    return (oracle.IQ4XS_GGML if ggml else oracle.IQ4XS_REFERENCE), (H.FLAG_IQ4XS_GGML if ggml else 0)


def flags_for(quant, ggml):
    return H.FLAG_IQ4XS_GGML if (quant == IQ and ggml) else 0


def mode_for(oracle, quant, ggml):
    return oracle.IQ4XS_GGML if (quant == IQ and ggml) else 0


# ------------------------------------------------------------------ expert --

@pytest.mark.parametrize("ggml", [False, True])
@pytest.mark.parametrize("n_expert,rows,cols", [(128, 2048, 768), (128, 768, 2048), (4, 300, 512),
                                                (3, 5, 256), (2, 1, 256), (2, 4096, 12288)])
def test_expert_gemv_iq4_xs(backend, oracle, ggml, n_expert, rows, cols):
    """In-major experts [n_expert][rows = in][cols = out] (weights.rs:14-34)
    against ops::expert_gemv (ops.rs:169-195) under the reading."""
    say("expert_gemv IQ4_XS", "ggml" if ggml else "reference", n_expert, rows, cols)
    mode, flags = reading(oracle, ggml)
    w = S.matrix(IQ, 11000 + rows + cols, n_expert * rows, cols)
    view = H.ExpertView(f"iq4exps{int(ggml)}_{rows}_{cols}", IQ, n_expert, rows, cols, w, flags=flags)
    for e in sorted({0, n_expert // 2, n_expert - 1}):
        x = S.normal_f32(11100 + e, rows)
        y = np.empty(cols, np.float32)
        backend.expert_gemv(view, e, x, y)
        want = oracle.expert_gemv(IQ, n_expert, rows, cols, w, e, x, mode=mode)
        check_parity(y, want, f"expert_gemv iq4_xs {rows}x{cols} e{e}")
        if rows >= 5:
            other = oracle.expert_gemv(IQ, n_expert, rows, cols, w, e, x, mode=1 - mode)
            assert rel_err(y, other) > 1e-2, "the two readings must differ on random code bytes"
    backend.evict(view.name)


@pytest.mark.parametrize("ggml", [False, True])
def test_expert_gemv_iq4_xs_out_major(backend, oracle, ggml):
    """Out-major experts (llama.cpp's [n_expert][out][in]): each expert an
    ops::gemv of its slice."""
    say("expert_gemv IQ4_XS out-major", ggml)
    mode, flags = reading(oracle, ggml)
    n_expert, rows, cols = 4, 768, 2048
    w = S.matrix(IQ, 11200, n_expert * rows, cols)
    x = S.normal_f32(11300, cols)
    v = H.ExpertView(f"iq4om{int(ggml)}", IQ, n_expert, rows, cols, w, flags=OM | flags)
    rb = S.row_bytes(IQ, cols)
    for e in (0, 3):
        y = np.empty(rows, np.float32)
        backend.expert_gemv(v, e, x, y)
        want = oracle.gemv(IQ, rows, cols, w[e * rows * rb:(e + 1) * rows * rb], x, scale_mode=mode)
        check_parity(y, want, f"expert_gemv out-major iq4_xs e{e}")
    backend.evict(v.name)


# --------------------------------------------------------------------- MoE --

def oracle_moe(oracle, qg, qd, n_expert, n_embd, n_ff, gate, up, down, logits, x, top_k, out_major, modes):
    out = np.empty_like(x)
    for t in range(x.shape[0]):
        ids, w = oracle.moe_route(logits[t], top_k)
        out[t] = oracle.moe_routed(qg, qg, qd, n_expert, n_embd, n_ff, gate, up, down, ids, w, x[t],
                                   out_major=out_major, modes=modes)
    return out


def moe_tensors(n_expert, n_embd, n_ff, qg, qd, seed, out_major):
    if out_major:  # gate / up [E][n_ff][n_embd], down [E][n_embd][n_ff]
        return (S.matrix(qg, seed, n_expert * n_ff, n_embd), S.matrix(qg, seed + 1, n_expert * n_ff, n_embd),
                S.matrix(qd, seed + 2, n_expert * n_embd, n_ff))
    return (S.matrix(qg, seed, n_expert * n_embd, n_ff), S.matrix(qg, seed + 1, n_expert * n_embd, n_ff),
            S.matrix(qd, seed + 2, n_expert * n_ff, n_embd))


def moe_views(name, qg, qd, n_expert, n_embd, n_ff, gate, up, down, out_major, ggml):
    o = OM if out_major else 0
    fg, fd = flags_for(qg, ggml), flags_for(qd, ggml)
    if out_major:
        return (H.ExpertView(f"{name}.g", qg, n_expert, n_ff, n_embd, gate, flags=o | fg),
                H.ExpertView(f"{name}.u", qg, n_expert, n_ff, n_embd, up, flags=o | fg),
                H.ExpertView(f"{name}.d", qd, n_expert, n_embd, n_ff, down, flags=o | fd))
    return (H.ExpertView(f"{name}.g", qg, n_expert, n_embd, n_ff, gate, flags=fg),
            H.ExpertView(f"{name}.u", qg, n_expert, n_embd, n_ff, up, flags=fg),
            H.ExpertView(f"{name}.d", qd, n_expert, n_ff, n_embd, down, flags=fd))


def run_moe(backend, oracle, name, qg, qd, n_expert, n_embd, n_ff, top_k, n_tok, tensors, out_major, ggml, seed,
            check_other=False):
    gate, up, down = tensors
    logits = S.router_logits(seed + 10, n_tok, n_expert)
    x = S.normal_f32(seed + 20, n_tok * n_embd).reshape(n_tok, n_embd)
    views = moe_views(name, qg, qd, n_expert, n_embd, n_ff, gate, up, down, out_major, ggml)
    out = backend.moe_ffn(*views, logits, x, top_k)
    modes = (mode_for(oracle, qg, ggml), mode_for(oracle, qg, ggml), mode_for(oracle, qd, ggml))
    ref = oracle_moe(oracle, qg, qd, n_expert, n_embd, n_ff, gate, up, down, logits, x, top_k, out_major, modes)
    for t in range(n_tok):
        check_parity(out[t], ref[t], f"moe iq4_xs {name} t{t}")
    if check_other:
        other = tuple(1 - m if q == IQ else m for m, q in zip(modes, (qg, qg, qd)))
        alt = oracle_moe(oracle, qg, qd, n_expert, n_embd, n_ff, gate, up, down, logits[:1], x[:1], top_k,
                         out_major, other)
        assert rel_err(out[0], alt[0]) > 1e-2, "the two readings must differ on random code bytes"
    for v in views:
        backend.evict(v.name)


@pytest.fixture(scope="module")
def iq4_config_in_major():
    # 128 experts, hidden 2048, expert intermediate 768: gate / up IQ4_XS, down Q6_K
    return moe_tensors(128, 2048, 768, IQ, Q6K, 12000, False)


@pytest.fixture(scope="module")
def iq4_config_out_major():
    return moe_tensors(128, 2048, 768, IQ, Q6K, 12100, True)


@pytest.mark.parametrize("ggml", [False, True])
@pytest.mark.parametrize("n_tok", [1, 16])
def test_moe_ffn_iq4_xs_config_in_major(backend, oracle, iq4_config_in_major, ggml, n_tok):
    """The MoE config (128 experts, top-8, 2048 x 768) with IQ4_XS gate / up
    and Q6_K down in the reference orientation (moe.rs:108-127)."""
    say("moe ffn IQ4_XS config in-major", "ggml" if ggml else "reference", n_tok)
    run_moe(backend, oracle, f"iqcfg_in{int(ggml)}{n_tok}", IQ, Q6K, 128, 2048, 768, 8, n_tok,
            iq4_config_in_major, False, ggml, 12200 + n_tok, check_other=True)


@pytest.mark.parametrize("ggml", [False, True])
@pytest.mark.parametrize("n_tok", [1, 16])
def test_moe_ffn_iq4_xs_config_out_major(backend, oracle, iq4_config_out_major, ggml, n_tok):
    """The same configuration over llama.cpp's out-major stacks."""
    say("moe ffn IQ4_XS config out-major", "ggml" if ggml else "reference", n_tok)
    run_moe(backend, oracle, f"iqcfg_om{int(ggml)}{n_tok}", IQ, Q6K, 128, 2048, 768, 8, n_tok,
            iq4_config_out_major, True, ggml, 12300 + n_tok, check_other=True)


@pytest.mark.parametrize("out_major", [False, True])
@pytest.mark.parametrize("ggml", [False, True])
@pytest.mark.parametrize("qg,qd,n_tok", [(IQ, IQ, 1), (IQ, IQ, 5), (12, IQ, 3), (IQ, 8, 2)])
def test_moe_ffn_iq4_xs_formats(backend, oracle, out_major, ggml, qg, qd, n_tok):
    """IQ4_XS down, and IQ4_XS next to the other formats, one and several
    tokens, both orientations and readings."""
    say("moe ffn IQ4_XS formats", qg, qd, n_tok, "om" if out_major else "im", ggml)
    n_expert, n_embd, n_ff, top_k = 16, 512, 256, 4
    seed = 12400 + 10 * qg + qd + n_tok + 100 * int(out_major)
    t = moe_tensors(n_expert, n_embd, n_ff, qg, qd, seed, out_major)
    run_moe(backend, oracle, f"iqf{qg}_{qd}_{n_tok}_{int(out_major)}{int(ggml)}", qg, qd, n_expert, n_embd, n_ff,
            top_k, n_tok, t, out_major, ggml, seed)


@pytest.mark.parametrize("out_major", [False, True])
@pytest.mark.parametrize("n_tok", [1, 4])
def test_moe_layer_iq4_xs(backend, oracle, out_major, n_tok):
    """The whole layer (router, routed experts, shared expert and its
    sigmoid gate; moe.rs:48-143) with IQ4_XS routed gate / up / down and
    shared gate / up in ggml's reading, Q8_0 router and shared down."""
    say("moe layer IQ4_XS", n_tok, "om" if out_major else "im")
    n_expert, n_embd, n_ff, n_sh, top_k = 16, 512, 256, 256, 4
    q = [8, IQ, IQ, IQ, IQ, IQ, 8, 8]
    seed = 12600 + n_tok + 50 * int(out_major)
    gr, gc = (n_ff, n_embd) if out_major else (n_embd, n_ff)
    dims = [(n_expert, n_embd), (n_expert * gr, gc), (n_expert * gr, gc), (n_expert * gc, gr),
            (n_sh, n_embd), (n_sh, n_embd), (n_embd, n_sh), (1, n_embd)]
    ts = [S.matrix(q[i], seed + i, r, c) for i, (r, c) in enumerate(dims)]
    modes = [oracle.IQ4XS_GGML if qi == IQ else 0 for qi in q]
    x = S.normal_f32(seed + 9, n_tok * n_embd).reshape(n_tok, n_embd)
    o = OM if out_major else 0
    g = H.FLAG_IQ4XS_GGML
    views = (H.QuantTensor(f"iql{seed}.r", 8, n_expert, n_embd, ts[0]),
             H.ExpertView(f"iql{seed}.g", IQ, n_expert, gr, gc, ts[1], flags=o | g),
             H.ExpertView(f"iql{seed}.u", IQ, n_expert, gr, gc, ts[2], flags=o | g),
             H.ExpertView(f"iql{seed}.d", IQ, n_expert, gc, gr, ts[3], flags=o | g),
             H.QuantTensor(f"iql{seed}.gs", IQ, n_sh, n_embd, ts[4], flags=g),
             H.QuantTensor(f"iql{seed}.us", IQ, n_sh, n_embd, ts[5], flags=g),
             H.QuantTensor(f"iql{seed}.ds", 8, n_embd, n_sh, ts[6]),
             H.QuantTensor(f"iql{seed}.gi", 8, 1, n_embd, ts[7]))
    out = backend.moe_layer(*views, x, top_k)
    for t in range(n_tok):
        ref = oracle.moe_layer(q, ts, n_expert, n_embd, n_ff, n_sh, x[t], top_k, out_major=out_major, modes=modes)
        check_parity(out[t], ref, f"moe layer iq4_xs t{t}")


# ------------------------------------------------------------ batched gemv --

@pytest.mark.parametrize("ggml", [False, True])
@pytest.mark.parametrize("rows,cols,batch", [(96, 4096, 2), (37, 256, 4), (300, 2048, 5), (4096, 4096, 8),
                                             (129, 12288, 7)])
def test_gemv_batch_iq4_xs(backend, oracle, ggml, rows, cols, batch):
    """Batches of 2-8 vectors over one read of the weights (the multi-vector
    matvec kernel), each vector against its own ops::gemv."""
    say("gemv batch IQ4_XS", "ggml" if ggml else "reference", rows, cols, batch)
    mode, flags = reading(oracle, ggml)
    w = S.matrix(IQ, 12700 + rows + cols, rows, cols)
    x = S.normal_f32(12800 + cols + batch, batch * cols).reshape(batch, cols)
    t = H.QuantTensor(f"iqb{int(ggml)}_{rows}_{cols}_{batch}", IQ, rows, cols, w, flags)
    y = backend.gemv_batch(t, x, batch)
    for b in range(batch):
        check_parity(y[b], oracle.gemv(IQ, rows, cols, w, x[b], scale_mode=mode), f"iq4_xs batch b{b}")
    backend.evict(t.name)


# ------------------------------------------------------------------ matmul --

def bf16_operand_ref(oracle, rows, cols, w, x, mode):
    W = oracle.dequantize(IQ, w, rows, cols, mode)
    Wb = oracle.bf16_round_array(W).astype(np.float64)
    xb = oracle.bf16_round_array(x).astype(np.float64)
    return (xb @ Wb.T).astype(np.float32)


def check_rows(got, want, tol, strict_tol=None):
    for t in range(want.shape[0]):
        check_parity(got[t], want[t], f"row {t}", norm_tol=tol, strict_tol=strict_tol)


@pytest.mark.parametrize("ggml", [False, True])
@pytest.mark.parametrize("rows,cols,m", [(96, 256, 1), (200, 512, 37), (100, 768, 300), (192, 1024, 513),
                                         (97, 2048, 33)])
def test_matmul_iq4_xs(backend, oracle, ggml, rows, cols, m):
    """Both MFMA modes: bf16 operands, and int8 codes on 32-element Q8
    activation blocks (the code-book values are the int8 weight codes, the
    sub-block scale d * (ls - 32) the per-block weight scale)."""
    say("matmul IQ4_XS", "ggml" if ggml else "reference", rows, cols, m)
    mode, flags = reading(oracle, ggml)
    w = S.matrix(IQ, 12900 + rows + cols, rows, cols)
    x = S.normal_f32(13000 + m, m * cols).reshape(m, cols)
    f32_ref = oracle.matmul(IQ, rows, cols, w, x, threads=8, mode=mode)
    t = H.QuantTensor(f"iqm{int(ggml)}_{rows}_{cols}_{m}", IQ, rows, cols, w, flags)
    y = backend.matmul(t, x)
    check_rows(y, bf16_operand_ref(oracle, rows, cols, w, x, mode), TOL_EXACT_OPERANDS)
    check_rows(y, f32_ref, TOL_F32)
    yq = backend.matmul(t, x, mode=H.MATMUL_Q8)
    xq = oracle.q8_activations_for(H.MATMUL_Q8, x)
    check_rows(yq, oracle.matmul(IQ, rows, cols, w, xq, threads=8, mode=mode), TOL_EXACT_OPERANDS, STRICT_TOL)
    check_rows(yq, f32_ref, TOL_F32)
    other = oracle.matmul(IQ, rows, cols, w, x[:1], threads=8, mode=1 - mode)
    assert rel_err(yq[0], other[0]) > 1e-2, "the two readings must differ on random code bytes"
    backend.evict(t.name)


def test_matmul_iq4_xs_q8k_refused(backend):
    """The 256-element activation mode is defined for Q4_K / Q5_K weights
    (one scale per K-quant super-block); IQ4_XS is refused there."""
    say("matmul IQ4_XS q8k refused")
    w = S.matrix(IQ, 13100, 96, 256)
    with pytest.raises(H.UnsupportedQuantError):
        backend.matmul(H.QuantTensor("iqm_q8k", IQ, 96, 256, w), np.zeros((4, 256), np.float32),
                       mode=H.MATMUL_Q8K)
