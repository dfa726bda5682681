"""The fused MoE over out-major expert stacks (SH_FLAG_EXPERT_OUT_MAJOR):
llama.cpp's [n_expert][out][in] layout, gate / up [n_expert][n_ff][n_embd]
and down [n_expert][n_embd][n_ff], each expert an ops::gemv of its slice
(crates/strata-core/src/ops.rs:14-28; the reference itself only defines the
in-major orientation, weights.rs:14-34).

Against the oracle's out-major composition (sho_moe_routed_o): the MoE
configuration (128 experts, 2048 x 768, top-8) for 1 and 16 tokens, every
type pair, rows wider than one 64-lane pass, the fused and separate routing
launches, the whole layer with the shared expert, the device-pointer entry
points, and the refusals (mixed orientation, mismatched views).
"""
import numpy as np
import pytest

import strata_hip as H
from conftest import check_parity
from strata_hip import synth as S

pytestmark = pytest.mark.gpu
OM = H.FLAG_EXPERT_OUT_MAJOR


def say(*a):
    print("[case]", *a, flush=True)


def om_tensors(n_expert, n_embd, n_ff, qg, qd, seed):
    gate = S.matrix(qg, seed, n_expert * n_ff, n_embd)
    up = S.matrix(qg, seed + 1, n_expert * n_ff, n_embd)
    down = S.matrix(qd, seed + 2, n_expert * n_embd, n_ff)
    return gate, up, down


def om_views(name, qg, qd, n_expert, n_embd, n_ff, gate, up, down):
    return (H.ExpertView(f"{name}.g", qg, n_expert, n_ff, n_embd, gate, flags=OM),
            H.ExpertView(f"{name}.u", qg, n_expert, n_ff, n_embd, up, flags=OM),
            H.ExpertView(f"{name}.d", qd, n_expert, n_embd, n_ff, down, flags=OM))


def oracle_om(oracle, qg, qd, n_expert, n_embd, n_ff, gate, up, down, logits, x, top_k):
    out = np.empty_like(x)
    for t in range(x.shape[0]):
        ids, w = oracle.moe_route(logits[t], top_k)
        out[t] = oracle.moe_routed(qg, qg, qd, n_expert, n_embd, n_ff, gate, up, down, ids, w, x[t],
                                   out_major=True)
    return out


def run(backend, oracle, name, qg, qd, n_expert, n_embd, n_ff, top_k, n_tok, seed):
    gate, up, down = om_tensors(n_expert, n_embd, n_ff, qg, qd, seed)
    logits = S.router_logits(seed + 10, n_tok, n_expert)
    x = S.normal_f32(seed + 20, n_tok * n_embd).reshape(n_tok, n_embd)
    views = om_views(name, qg, qd, n_expert, n_embd, n_ff, gate, up, down)
    out = backend.moe_ffn(*views, logits, x, top_k)
    ref = oracle_om(oracle, qg, qd, n_expert, n_embd, n_ff, gate, up, down, logits, x, top_k)
    for t in range(n_tok):
        check_parity(out[t], ref[t], f"moe out-major {name} t{t}")
    for v in views:
        backend.evict(v.name)


@pytest.fixture(scope="module")
def om_config_tensors():
    # 128 experts, hidden 2048, expert intermediate 768, as llama.cpp stores them
    return om_tensors(128, 2048, 768, 12, 14, 9000)


@pytest.mark.parametrize("n_tok", [1, 16])
def test_moe_ffn_out_major_config(backend, oracle, om_config_tensors, n_tok):
    n_expert, n_embd, n_ff, top_k = 128, 2048, 768, 8
    say("moe ffn out-major config", n_tok)
    gate, up, down = om_config_tensors
    logits = S.router_logits(9100 + n_tok, n_tok, n_expert)
    x = S.normal_f32(9200 + n_tok, n_tok * n_embd).reshape(n_tok, n_embd)
    views = om_views("omcfg", 12, 14, n_expert, n_embd, n_ff, gate, up, down)
    out = backend.moe_ffn(*views, logits, x, top_k)
    ref = oracle_om(oracle, 12, 14, n_expert, n_embd, n_ff, gate, up, down, logits, x, top_k)
    for t in range(n_tok):
        check_parity(out[t], ref[t], "moe out-major")


@pytest.mark.parametrize("qg,qd", [(12, 14), (8, 8), (13, 13), (14, 12), (12, 8), (8, 13)])
@pytest.mark.parametrize("n_tok", [1, 5])
def test_moe_ffn_out_major_formats(backend, oracle, qg, qd, n_tok):
    say("moe ffn out-major formats", qg, qd, n_tok)
    run(backend, oracle, f"omf{qg}{qd}{n_tok}", qg, qd, 16, 512, 256, 4, n_tok, 9300 + 10 * qg + qd + n_tok)


@pytest.mark.parametrize("n_embd,n_ff,n_tok", [(5120, 256, 2), (256, 5120, 1), (1024, 768, 3)])
def test_moe_ffn_out_major_row_widths(backend, oracle, n_embd, n_ff, n_tok):
    """Rows wider than 64 units (each lane takes several), and narrow down
    rows of 12 units (16 lanes a row, four rows a wave)."""
    say("moe ffn out-major widths", n_embd, n_ff, n_tok)
    run(backend, oracle, f"omw{n_embd}_{n_ff}", 12, 14, 8, n_embd, n_ff, 3, n_tok, 9400 + n_embd + n_ff)


def test_moe_ffn_out_major_separate_route(backend, oracle):
    """One token over 300 experts: routed by the route launch (the fused
    routing takes at most 256 experts)."""
    say("moe ffn out-major 300 experts")
    run(backend, oracle, "om300", 12, 14, 300, 256, 256, 8, 1, 9500)


def layer_om_tensors(n_expert, n_embd, n_ff, n_sh, seed):
    quants = [0, 12, 12, 14, 12, 12, 14, 0]
    tensors = [S.normal_f32(seed, n_expert * n_embd).view(np.uint8),
               S.matrix(12, seed + 1, n_expert * n_ff, n_embd), S.matrix(12, seed + 2, n_expert * n_ff, n_embd),
               S.matrix(14, seed + 3, n_expert * n_embd, n_ff),
               S.matrix(12, seed + 4, n_sh, n_embd), S.matrix(12, seed + 5, n_sh, n_embd),
               S.matrix(14, seed + 6, n_embd, n_sh), S.normal_f32(seed + 7, n_embd).view(np.uint8)]
    return quants, tensors


def layer_om_views(name, q, t, n_expert, n_embd, n_ff, n_sh):
    return (H.QuantTensor(f"{name}.router", q[0], n_expert, n_embd, t[0]),
            H.ExpertView(f"{name}.gate", q[1], n_expert, n_ff, n_embd, t[1], flags=OM),
            H.ExpertView(f"{name}.up", q[2], n_expert, n_ff, n_embd, t[2], flags=OM),
            H.ExpertView(f"{name}.down", q[3], n_expert, n_embd, n_ff, t[3], flags=OM),
            H.QuantTensor(f"{name}.gate_sh", q[4], n_sh, n_embd, t[4]),
            H.QuantTensor(f"{name}.up_sh", q[5], n_sh, n_embd, t[5]),
            H.QuantTensor(f"{name}.down_sh", q[6], n_embd, n_sh, t[6]),
            H.QuantTensor(f"{name}.inp_sh", q[7], 1, n_embd, t[7]))


@pytest.mark.parametrize("n_tok", [1, 3])
def test_moe_layer_out_major(backend, oracle, n_tok):
    """The whole layer (moe.rs:48-143) with out-major routed stacks."""
    n_expert, n_embd, n_ff, n_sh, top_k = 32, 512, 256, 256, 6
    say("moe layer out-major", n_tok)
    q, t = layer_om_tensors(n_expert, n_embd, n_ff, n_sh, 9600 + n_tok)
    x = S.normal_f32(9700 + n_tok, n_tok * n_embd).reshape(n_tok, n_embd)
    out = backend.moe_layer(*layer_om_views(f"LO{n_tok}", q, t, n_expert, n_embd, n_ff, n_sh), x, top_k)
    for i in range(n_tok):
        ref = oracle.moe_layer(q, t, n_expert, n_embd, n_ff, n_sh, x[i], top_k, out_major=True)
        check_parity(out[i], ref, "moe layer out-major")


def test_moe_ffn_dev_out_major_matches_host_path(backend):
    import torch
    n_expert, n_embd, n_ff, top_k, n_tok = 32, 512, 256, 8, 4
    say("moe ffn dev out-major")
    gate, up, down = om_tensors(n_expert, n_embd, n_ff, 12, 14, 9800)
    logits = S.router_logits(9810, n_tok, n_expert)
    x = S.normal_f32(9820, n_tok * n_embd).reshape(n_tok, n_embd)
    host = backend.moe_ffn(*om_views("omdev", 12, 14, n_expert, n_embd, n_ff, gate, up, down), logits, x, top_k)
    dev = torch.device("cuda:0")
    tg, tu, td = (torch.from_numpy(a).to(dev) for a in (gate, up, down))
    tl, tx = torch.from_numpy(logits).to(dev), torch.from_numpy(x).to(dev)
    out = torch.empty((n_tok, n_embd), dtype=torch.float32, device=dev)
    nb = H.moe_workspace_bytes(n_tok, top_k, n_expert, n_embd, n_ff, 12, 14)
    ws = torch.empty(nb, dtype=torch.uint8, device=dev)
    H.moe_ffn_dev((12, OM, tg.data_ptr()), (12, OM, tu.data_ptr()), (14, OM, td.data_ptr()), n_expert, n_embd,
                  n_ff, tl.data_ptr(), n_tok, top_k, tx.data_ptr(), out.data_ptr(), ws.data_ptr(), nb,
                  torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy(), host)


@pytest.mark.parametrize("n_tok", [1, 5])
def test_moe_ffn_out_major_graph_replays(backend, n_tok):
    """Captured in a HIP graph (route, gate/up, down, combine), every replay,
    with eager calls of other inputs between replays, equals the eager
    result."""
    import torch
    n_expert, n_embd, n_ff, top_k = 32, 512, 256, 8
    say("moe ffn out-major graph", n_tok)
    gate, up, down = om_tensors(n_expert, n_embd, n_ff, 12, 14, 9850 + n_tok)
    dev = torch.device("cuda:0")
    tg, tu, td = (torch.from_numpy(a).to(dev) for a in (gate, up, down))
    tls = [torch.from_numpy(S.router_logits(9860 + i, n_tok, n_expert)).to(dev) for i in range(2)]
    txs = [torch.from_numpy(S.normal_f32(9870 + i, n_tok * n_embd)).to(dev) for i in range(2)]
    out = torch.empty((n_tok, n_embd), dtype=torch.float32, device=dev)
    nb = H.moe_workspace_bytes(n_tok, top_k, n_expert, n_embd, n_ff, 12, 14)
    ws = torch.empty(nb, dtype=torch.uint8, device=dev)

    def call(i, stream):
        H.moe_ffn_dev((12, OM, tg.data_ptr()), (12, OM, tu.data_ptr()), (14, OM, td.data_ptr()), n_expert, n_embd,
                      n_ff, tls[i].data_ptr(), n_tok, top_k, txs[i].data_ptr(), out.data_ptr(), ws.data_ptr(), nb,
                      stream)

    eager = []
    for i in range(2):
        call(i, torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        eager.append(out.cpu().numpy().copy())
    assert not np.array_equal(eager[0], eager[1])
    s = torch.cuda.Stream(dev)
    with torch.cuda.stream(s):
        call(0, s.cuda_stream)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        call(0, torch.cuda.current_stream().cuda_stream)
    for rep in range(3):
        out.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(out.cpu().numpy(), eager[0]), rep
        call(1, torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        assert np.array_equal(out.cpu().numpy(), eager[1]), rep


def test_moe_layer_dev_out_major_matches_host_path(backend):
    import torch
    n_expert, n_embd, n_ff, n_sh, top_k, n_tok = 32, 512, 256, 256, 6, 2
    say("moe layer dev out-major")
    q, t = layer_om_tensors(n_expert, n_embd, n_ff, n_sh, 9900)
    x = S.normal_f32(9910, n_tok * n_embd).reshape(n_tok, n_embd)
    host = backend.moe_layer(*layer_om_views("LOdev", q, t, n_expert, n_embd, n_ff, n_sh), x, top_k)
    dev = torch.device("cuda:0")
    bufs = [torch.from_numpy(np.ascontiguousarray(a)).to(dev) for a in t]
    flags = [0, OM, OM, OM, 0, 0, 0, 0]
    tx = torch.from_numpy(x).to(dev)
    out = torch.empty((n_tok, n_embd), dtype=torch.float32, device=dev)
    nb = H.moe_layer_workspace_bytes(n_tok, top_k, n_expert, n_embd, n_ff, n_sh, q)
    ws = torch.empty(nb, dtype=torch.uint8, device=dev)
    H.moe_layer_dev([(q[i], flags[i], bufs[i].data_ptr()) for i in range(8)], n_expert, n_embd, n_ff, n_sh, n_tok,
                    top_k, tx.data_ptr(), out.data_ptr(), ws.data_ptr(), nb, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy(), host)


def test_moe_out_major_refusals(backend):
    n_expert, n_embd, n_ff, top_k = 8, 256, 512, 2
    say("moe out-major refusals")
    gate, up, down = om_tensors(n_expert, n_embd, n_ff, 12, 14, 9950)
    logits = S.router_logits(9960, 1, n_expert)
    x = S.normal_f32(9970, n_embd).reshape(1, n_embd)
    g, u, d = om_views("omref", 12, 14, n_expert, n_embd, n_ff, gate, up, down)
    # one stack without the flag: mixed orientations are refused
    d_in = H.ExpertView("omref.d_in", 14, n_expert, n_embd, n_ff, down)
    with pytest.raises(H.UnsupportedShapeError):
        backend.moe_ffn(g, u, d_in, logits, x, top_k)
    # down not the transpose of gate's [out][in]
    d_bad = H.ExpertView("omref.d_bad", 14, n_expert, n_ff, n_embd, down, flags=OM)
    with pytest.raises(H.ShapeError):
        backend.moe_ffn(g, u, d_bad, logits, x, top_k)
    # x as wide as the in-major reading would have it
    with pytest.raises(H.ShapeError):
        backend.moe_ffn(g, u, d, logits, np.zeros((1, n_ff), np.float32), top_k)
