"""Routed MoE FFN on the device vs the oracle (crates/strata-core/src/moe.rs).

Routing: ids must equal the oracle's (softmax, stable top-k, ascending ids)
and weights agree to f32 rounding (the device exp differs from glibc's by at
most an ulp). The FFN output is checked with max|out - ref| / max|ref| <=
1e-3 at the MoE config's shapes (128 experts, top-8, hidden 2048, expert
intermediate 768; gate/up Q4_K, down Q6_K) for 1 and 16 tokens, and on a
small Q8_0 / signed-scale variant.
"""
import numpy as np
import pytest

import strata_hip as H
from conftest import check_parity, rel_err
from strata_hip import synth as S

pytestmark = pytest.mark.gpu


def say(*a):
    print("[case]", *a, flush=True)


@pytest.mark.parametrize("n_tok,n_expert,top_k", [(1, 128, 8), (16, 128, 8), (5, 64, 4), (3, 8, 8),
                                                  (2, 1000, 32)])
def test_route_matches_oracle(backend, oracle, n_tok, n_expert, top_k):
    say("route", n_tok, n_expert, top_k)
    logits = S.router_logits(100 + n_tok + n_expert, n_tok, n_expert)
    ids, w = backend.moe_route(logits, top_k)
    for t in range(n_tok):
        oid, ow = oracle.moe_route(logits[t], top_k)
        assert ids[t].tolist() == oid.tolist()
        assert np.abs(w[t] - ow).max() <= 4e-7
        assert abs(float(w[t].astype(np.float64).sum()) - 1.0) < 1e-5


def test_route_ties_and_uniform(backend, oracle):
    say("route ties")
    lg = np.zeros((2, 16), np.float32)
    lg[0, [3, 9, 12]] = 1.0
    ids, w = backend.moe_route(lg, 5)
    assert ids[0].tolist() == [0, 1, 3, 9, 12]
    assert ids[1].tolist() == [0, 1, 2, 3, 4]
    assert np.all(w[1] == np.float32(0.2))


def expert_tensors(n_expert, n_embd, n_ff, qg, qd, seed):
    gate = S.matrix(qg, seed, n_expert * n_embd, n_ff)
    up = S.matrix(qg, seed + 1, n_expert * n_embd, n_ff)
    down = S.matrix(qd, seed + 2, n_expert * n_ff, n_embd)
    return gate, up, down


def oracle_moe(oracle, qg, qd, n_expert, n_embd, n_ff, gate, up, down, logits, x, top_k, q6_signed=False):
    out = np.empty_like(x)
    for t in range(x.shape[0]):
        ids, w = oracle.moe_route(logits[t], top_k)
        out[t] = oracle.moe_routed(qg, qg, qd, n_expert, n_embd, n_ff, gate, up, down, ids, w, x[t])
    return out


@pytest.fixture(scope="module")
def moe_config_tensors():
    # 128 experts, hidden 2048, expert intermediate 768 (about 26 s to synthesise)
    return expert_tensors(128, 2048, 768, 12, 14, 4000)


@pytest.mark.parametrize("n_tok", [1, 16])
def test_moe_ffn_config_shapes(backend, oracle, moe_config_tensors, n_tok):
    n_expert, n_embd, n_ff, top_k = 128, 2048, 768, 8
    say("moe ffn", n_tok, "tokens", n_expert, n_embd, n_ff)
    gate, up, down = moe_config_tensors
    logits = S.router_logits(4100 + n_tok, n_tok, n_expert)
    x = S.normal_f32(4200 + n_tok, n_tok * n_embd).reshape(n_tok, n_embd)
    g = H.ExpertView("blk.0.ffn_gate_exps.weight", 12, n_expert, n_embd, n_ff, gate)
    u = H.ExpertView("blk.0.ffn_up_exps.weight", 12, n_expert, n_embd, n_ff, up)
    d = H.ExpertView("blk.0.ffn_down_exps.weight", 14, n_expert, n_ff, n_embd, down)
    out = backend.moe_ffn(g, u, d, logits, x, top_k)
    ref = oracle_moe(oracle, 12, 14, n_expert, n_embd, n_ff, gate, up, down, logits, x, top_k)
    for t in range(n_tok):
        check_parity(out[t], ref[t], "moe")


def test_moe_ffn_q8_gate_up_small(backend, oracle):
    n_expert, n_embd, n_ff, top_k, n_tok = 16, 256, 128, 4, 6
    say("moe ffn q8 small")
    gate, up, down = expert_tensors(n_expert, n_embd, n_ff, 8, 14, 5000)
    logits = S.router_logits(5100, n_tok, n_expert)
    x = S.normal_f32(5200, n_tok * n_embd).reshape(n_tok, n_embd)
    out = backend.moe_ffn(H.ExpertView("g8", 8, n_expert, n_embd, n_ff, gate),
                          H.ExpertView("u8", 8, n_expert, n_embd, n_ff, up),
                          H.ExpertView("d8", 14, n_expert, n_ff, n_embd, down), logits, x, top_k)
    ref = oracle_moe(oracle, 8, 14, n_expert, n_embd, n_ff, gate, up, down, logits, x, top_k)
    check_parity(out, ref, "moe")


def test_moe_ffn_dev_matches_host_path(backend):
    import torch
    n_expert, n_embd, n_ff, top_k, n_tok = 32, 512, 256, 8, 4
    say("moe ffn dev")
    gate, up, down = expert_tensors(n_expert, n_embd, n_ff, 12, 14, 6000)
    logits = S.router_logits(6100, n_tok, n_expert)
    x = S.normal_f32(6200, n_tok * n_embd).reshape(n_tok, n_embd)
    host = backend.moe_ffn(H.ExpertView("gd", 12, n_expert, n_embd, n_ff, gate),
                           H.ExpertView("ud", 12, n_expert, n_embd, n_ff, up),
                           H.ExpertView("dd", 14, n_expert, n_ff, n_embd, down), logits, x, top_k)
    dev = torch.device("cuda:0")
    tg, tu, td = (torch.from_numpy(a).to(dev) for a in (gate, up, down))
    tl, tx = torch.from_numpy(logits).to(dev), torch.from_numpy(x).to(dev)
    out = torch.empty((n_tok, n_embd), dtype=torch.float32, device=dev)
    nb = H.moe_workspace_bytes(n_tok, top_k, n_expert, n_embd, n_ff, 12, 14)
    ws = torch.empty(nb, dtype=torch.uint8, device=dev)
    H.moe_ffn_dev((12, 0, tg.data_ptr()), (12, 0, tu.data_ptr()), (14, 0, td.data_ptr()), n_expert, n_embd,
                  n_ff, tl.data_ptr(), n_tok, top_k, tx.data_ptr(), out.data_ptr(), ws.data_ptr(), nb,
                  torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy(), host)


def test_moe_ffn_one_token_many_experts(backend, oracle):
    """One token over more than 256 experts: routed by the route kernel rather
    than inside gate/up (which takes up to 256)."""
    n_expert, n_embd, n_ff, top_k, n_tok = 320, 256, 256, 6, 1
    say("moe ffn one token", n_expert, "experts")
    gate, up, down = expert_tensors(n_expert, n_embd, n_ff, 12, 14, 6600)
    logits = S.router_logits(6700, n_tok, n_expert)
    x = S.normal_f32(6800, n_tok * n_embd).reshape(n_tok, n_embd)
    out = backend.moe_ffn(H.ExpertView("gm", 12, n_expert, n_embd, n_ff, gate),
                          H.ExpertView("um", 12, n_expert, n_embd, n_ff, up),
                          H.ExpertView("dm", 14, n_expert, n_ff, n_embd, down), logits, x, top_k)
    ref = oracle_moe(oracle, 12, 14, n_expert, n_embd, n_ff, gate, up, down, logits, x, top_k)
    check_parity(out, ref, "moe")


@pytest.mark.parametrize("n_tok", [1, 4])
def test_moe_ffn_dev_unaligned_tensors_match(backend, n_tok):
    """Expert tensors 2 bytes off a 16-byte boundary (allowed for Q4_K/Q6_K)
    take the register-staged row stream instead of the global_load_lds ring;
    both apply the rows in the same order, so the outputs are identical."""
    import torch
    n_expert, n_embd, n_ff, top_k = 32, 512, 256, 8
    say("moe ffn dev unaligned", n_tok)
    gate, up, down = expert_tensors(n_expert, n_embd, n_ff, 12, 14, 6300)
    logits = S.router_logits(6400 + n_tok, n_tok, n_expert)
    x = S.normal_f32(6500 + n_tok, n_tok * n_embd).reshape(n_tok, n_embd)
    dev = torch.device("cuda:0")
    tl, tx = torch.from_numpy(logits).to(dev), torch.from_numpy(x).to(dev)
    nb = H.moe_workspace_bytes(n_tok, top_k, n_expert, n_embd, n_ff, 12, 14)
    ws = torch.empty(nb, dtype=torch.uint8, device=dev)
    outs = []
    for shift in (0, 2):
        bufs = []
        for a in (gate, up, down):
            t = torch.zeros(a.nbytes + 16, dtype=torch.uint8, device=dev)
            t[shift:shift + a.nbytes] = torch.from_numpy(a.view(np.uint8).reshape(-1)).to(dev)
            bufs.append(t)
        assert (bufs[0].data_ptr() + shift) % 16 == shift
        out = torch.empty((n_tok, n_embd), dtype=torch.float32, device=dev)
        H.moe_ffn_dev((12, 0, bufs[0].data_ptr() + shift), (12, 0, bufs[1].data_ptr() + shift),
                      (14, 0, bufs[2].data_ptr() + shift), n_expert, n_embd, n_ff, tl.data_ptr(), n_tok,
                      top_k, tx.data_ptr(), out.data_ptr(), ws.data_ptr(), nb,
                      torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        outs.append(out.cpu().numpy())
    assert np.all(np.isfinite(outs[0]))
    assert np.array_equal(outs[0], outs[1])


@pytest.mark.parametrize("qg,qd", [(12, 14), (8, 8), (14, 12), (12, 8), (8, 14), (13, 13), (13, 14), (12, 13)])
def test_moe_ffn_one_token_formats(backend, oracle, qg, qd):
    """One token (routed inside the gate/up launch) over aligned tensors whose
    sizes are multiples of 16 bytes (the global_load_lds copy ring), for each
    gate/up x down type pair."""
    n_expert, n_embd, n_ff, top_k = 24, 512, 256, 6
    say("moe ffn one token", qg, qd)
    gate, up, down = expert_tensors(n_expert, n_embd, n_ff, qg, qd, 7000 + 10 * qg + qd)
    assert all(a.nbytes % 16 == 0 for a in (gate, up, down))
    logits = S.router_logits(7100 + qg, 1, n_expert)
    x = S.normal_f32(7200 + qd, n_embd).reshape(1, n_embd)
    out = backend.moe_ffn(H.ExpertView(f"gf{qg}{qd}", qg, n_expert, n_embd, n_ff, gate),
                          H.ExpertView(f"uf{qg}{qd}", qg, n_expert, n_embd, n_ff, up),
                          H.ExpertView(f"df{qg}{qd}", qd, n_expert, n_ff, n_embd, down), logits, x, top_k)
    ref = oracle_moe(oracle, qg, qd, n_expert, n_embd, n_ff, gate, up, down, logits, x, top_k)
    check_parity(out, ref, "moe")


def test_moe_ffn_one_token_repeat_and_graph(backend):
    """Back-to-back one-token calls on one workspace (which starts out
    filled with garbage), with new logits each time, and replays of a
    captured HIP graph (eager work between replays) all equal the eager
    result of the same inputs: nothing carries over between calls."""
    import torch
    n_expert, n_embd, n_ff, top_k = 64, 1024, 512, 8
    say("moe ffn one token repeat + graph")
    gate, up, down = expert_tensors(n_expert, n_embd, n_ff, 12, 14, 7300)
    dev = torch.device("cuda:0")
    tg, tu, td = (torch.from_numpy(a).to(dev) for a in (gate, up, down))
    x = torch.from_numpy(S.normal_f32(7400, n_embd)).to(dev)
    lgs = [torch.from_numpy(S.router_logits(7500 + i, 1, n_expert)).to(dev) for i in range(3)]
    nb = H.moe_workspace_bytes(1, top_k, n_expert, n_embd, n_ff, 12, 14)
    ws = torch.empty(nb, dtype=torch.uint8, device=dev)
    ws.fill_(0xA5)
    out = torch.empty(n_embd, dtype=torch.float32, device=dev)

    def call(lg, stream):
        H.moe_ffn_dev((12, 0, tg.data_ptr()), (12, 0, tu.data_ptr()), (14, 0, td.data_ptr()), n_expert, n_embd,
                      n_ff, lg.data_ptr(), 1, top_k, x.data_ptr(), out.data_ptr(), ws.data_ptr(), nb, stream)

    eager = []
    for lg in lgs + lgs:
        call(lg, torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        eager.append(out.cpu().numpy().copy())
    for i in range(3):
        assert np.all(np.isfinite(eager[i]))
        assert np.array_equal(eager[i], eager[i + 3])
    assert not np.array_equal(eager[0], eager[1])
    s = torch.cuda.Stream(dev)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        call(lgs[2], s.cuda_stream)  # warm-up outside capture
    torch.cuda.synchronize()
    with torch.cuda.graph(g, stream=s):
        call(lgs[2], torch.cuda.current_stream().cuda_stream)
    for rep in range(3):
        out.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(out.cpu().numpy(), eager[2]), rep
        call(lgs[0], torch.cuda.current_stream().cuda_stream)  # eager work between replays
        torch.cuda.synchronize()
        assert np.array_equal(out.cpu().numpy(), eager[0]), rep


def test_moe_errors(backend):
    say("moe errors")
    g = H.ExpertView("eg", 12, 4, 256, 256, S.matrix(12, 1, 4 * 256, 256))
    d_bad = H.ExpertView("ed", 14, 4, 256, 512, S.matrix(14, 1, 4 * 256, 512))
    with pytest.raises(H.ShapeError):
        backend.moe_ffn(g, g, d_bad, np.zeros((1, 4), np.float32), np.zeros((1, 256), np.float32), 2)
    with pytest.raises(H.BackendError):
        backend.moe_route(np.zeros((1, 4), np.float32), 5)  # top_k > n_expert


def layer_tensors(n_expert, n_embd, n_ff, n_sh, seed, q_router=0, q_inp=0, q_sh=(12, 12, 14)):
    """Router and gate-input rows as plain floats (F32, or BF16 when asked),
    experts as the MoE config (gate/up Q4_K, down Q6_K), the shared expert
    in the given types."""
    def plain(q, s, n):
        if q not in (0, 30):  # a quantized router or gate input: rows of n_embd
            return S.matrix(q, s, n // n_embd, n_embd)
        v = S.normal_f32(s, n)
        if q == 0:
            return v.view(np.uint8)
        bits = v.view(np.uint32)
        return ((bits + 0x7FFF + ((bits >> 16) & 1)) >> 16).astype(np.uint16).view(np.uint8)
    quants = [q_router, 12, 12, 14, q_sh[0], q_sh[1], q_sh[2], q_inp]
    tensors = [plain(q_router, seed, n_expert * n_embd),
               S.matrix(12, seed + 1, n_expert * n_embd, n_ff), S.matrix(12, seed + 2, n_expert * n_embd, n_ff),
               S.matrix(14, seed + 3, n_expert * n_ff, n_embd),
               S.matrix(q_sh[0], seed + 4, n_sh, n_embd), S.matrix(q_sh[1], seed + 5, n_sh, n_embd),
               S.matrix(q_sh[2], seed + 6, n_embd, n_sh), plain(q_inp, seed + 7, n_embd)]
    return quants, tensors


def layer_views(name, quants, tensors, n_expert, n_embd, n_ff, n_sh):
    q, t = quants, tensors
    return (H.QuantTensor(f"{name}.router", q[0], n_expert, n_embd, t[0]),
            H.ExpertView(f"{name}.gate", q[1], n_expert, n_embd, n_ff, t[1]),
            H.ExpertView(f"{name}.up", q[2], n_expert, n_embd, n_ff, t[2]),
            H.ExpertView(f"{name}.down", q[3], n_expert, n_ff, n_embd, t[3]),
            H.QuantTensor(f"{name}.gate_sh", q[4], n_sh, n_embd, t[4]),
            H.QuantTensor(f"{name}.up_sh", q[5], n_sh, n_embd, t[5]),
            H.QuantTensor(f"{name}.down_sh", q[6], n_embd, n_sh, t[6]),
            H.QuantTensor(f"{name}.inp_sh", q[7], 1, n_embd, t[7]))


@pytest.mark.parametrize("n_tok,q_router,q_inp,q_sh", [(1, 0, 0, (12, 12, 14)), (3, 30, 0, (8, 8, 8)),
                                                       (9, 0, 30, (14, 14, 12)), (2, 8, 13, (13, 13, 14)),
                                                       (1, 12, 0, (12, 12, 14)), (1, 30, 30, (14, 14, 12)),
                                                       (1, 0, 30, (13, 13, 8)), (1, 0, 0, (8, 8, 13))])
def test_moe_layer_matches_oracle(backend, oracle, n_tok, q_router, q_inp, q_sh):
    """The whole layer (moe.rs:48-143): router matvec on bf16(x) (F32 or
    BF16 rows with f64 sums, rounding x as they load it; or quantized rows
    after a rounding pass), routing, the routed experts and the shared
    expert with its sigmoid gate, against the oracle token by token; 9
    tokens take two 8-token matvec launches. One token with gate and up of
    one type runs the shared expert in two launches (gate and up rows paired
    in one matvec that stores silu(g) * u, then down), and a router and
    gate input of one plain type share a launch."""
    n_expert, n_embd, n_ff, n_sh, top_k = 32, 512, 256, 256, 6
    say("moe layer", n_tok, q_router, q_inp, q_sh)
    q, t = layer_tensors(n_expert, n_embd, n_ff, n_sh, 8400 + n_tok, q_router, q_inp, q_sh)
    x = S.normal_f32(8500 + n_tok, n_tok * n_embd).reshape(n_tok, n_embd)
    views = layer_views(f"L{n_tok}", q, t, n_expert, n_embd, n_ff, n_sh)
    out = backend.moe_layer(*views, x, top_k)
    for i in range(n_tok):
        ref = oracle.moe_layer(q, t, n_expert, n_embd, n_ff, n_sh, x[i], top_k)
        check_parity(out[i], ref, "moe")


@pytest.mark.parametrize("q_sh", [(12, 12, 14), (13, 13, 8)])
def test_moe_layer_wide_rows(backend, oracle, q_sh):
    """One token with rows of more than one 4096-column window: the shared
    expert's gate and up run as one 2 n_ff-row matvec and down forms
    silu(g) * u as it stages its x (the paired mode takes one window)."""
    n_expert, n_embd, n_ff, n_sh, top_k = 8, 8192, 256, 256, 2
    say("moe layer wide", q_sh)
    q, t = layer_tensors(n_expert, n_embd, n_ff, n_sh, 8700, 0, 0, q_sh)
    x = S.normal_f32(8701, n_embd).reshape(1, n_embd)
    views = layer_views("Lw", q, t, n_expert, n_embd, n_ff, n_sh)
    out = backend.moe_layer(*views, x, top_k)
    check_parity(out[0], oracle.moe_layer(q, t, n_expert, n_embd, n_ff, n_sh, x[0], top_k), "moe")


@pytest.fixture(scope="module")
def layer_config_tensors():
    # the MoE config (128 experts, hidden 2048, expert FFN 768, top-8) with a
    # shared expert of width 768 (Q4_K gate/up, Q6_K down) and F32 router and
    # gate-input rows
    return layer_tensors(128, 2048, 768, 768, 8600)


@pytest.mark.parametrize("n_tok", [1, 16])
def test_moe_layer_config_shapes(backend, oracle, layer_config_tensors, n_tok):
    n_expert, n_embd, n_ff, n_sh, top_k = 128, 2048, 768, 768, 8
    say("moe layer config", n_tok)
    q, t = layer_config_tensors
    x = S.normal_f32(8700 + n_tok, n_tok * n_embd).reshape(n_tok, n_embd)
    out = backend.moe_layer(*layer_views("Lcfg", q, t, n_expert, n_embd, n_ff, n_sh), x, top_k)
    for i in range(n_tok):
        ref = oracle.moe_layer(q, t, n_expert, n_embd, n_ff, n_sh, x[i], top_k)
        check_parity(out[i], ref, "moe")


def test_moe_layer_dev_matches_host_path(backend):
    import torch
    n_expert, n_embd, n_ff, n_sh, top_k, n_tok = 32, 512, 256, 256, 8, 4
    say("moe layer dev")
    q, t = layer_tensors(n_expert, n_embd, n_ff, n_sh, 8800)
    x = S.normal_f32(8801, n_tok * n_embd).reshape(n_tok, n_embd)
    host = backend.moe_layer(*layer_views("Ldev", q, t, n_expert, n_embd, n_ff, n_sh), x, top_k)
    dev = torch.device("cuda:0")
    td = [torch.from_numpy(a).to(dev) for a in t]
    tx = torch.from_numpy(x).to(dev)
    out = torch.empty((n_tok, n_embd), dtype=torch.float32, device=dev)
    nb = H.moe_layer_workspace_bytes(n_tok, top_k, n_expert, n_embd, n_ff, n_sh, q)
    ws = torch.empty(nb, dtype=torch.uint8, device=dev)
    H.moe_layer_dev([(qq, 0, a.data_ptr()) for qq, a in zip(q, td)], n_expert, n_embd, n_ff, n_sh, n_tok,
                    top_k, tx.data_ptr(), out.data_ptr(), ws.data_ptr(), nb, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy(), host)


@pytest.mark.parametrize("n_tok", [3, 1])
def test_moe_layer_graph_replays(backend, n_tok):
    """The layer forks its shared expert onto a second stream and joins it
    back: captured in a HIP graph (two parallel branches), every replay, with
    eager calls of other inputs between replays, equals the eager result
    (1 token: the shared expert's two-launch form)."""
    import torch
    n_expert, n_embd, n_ff, n_sh, top_k = 32, 512, 256, 256, 8
    say("moe layer graph", n_tok)
    q, t = layer_tensors(n_expert, n_embd, n_ff, n_sh, 9000)
    dev = torch.device("cuda:0")
    td = [torch.from_numpy(a).to(dev) for a in t]
    xs = [torch.from_numpy(S.normal_f32(9001 + i, n_tok * n_embd)).to(dev) for i in range(2)]
    out = torch.empty((n_tok, n_embd), dtype=torch.float32, device=dev)
    nb = H.moe_layer_workspace_bytes(n_tok, top_k, n_expert, n_embd, n_ff, n_sh, q)
    ws = torch.empty(nb, dtype=torch.uint8, device=dev)

    def call(x, stream):
        H.moe_layer_dev([(qq, 0, a.data_ptr()) for qq, a in zip(q, td)], n_expert, n_embd, n_ff, n_sh, n_tok,
                        top_k, x.data_ptr(), out.data_ptr(), ws.data_ptr(), nb, stream)

    eager = []
    for x in xs:
        call(x, torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        eager.append(out.cpu().numpy().copy())
    assert not np.array_equal(eager[0], eager[1])
    s = torch.cuda.Stream(dev)
    with torch.cuda.stream(s):
        call(xs[0], s.cuda_stream)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        call(xs[0], torch.cuda.current_stream().cuda_stream)
    for rep in range(3):
        out.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(out.cpu().numpy(), eager[0]), rep
        call(xs[1], torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        assert np.array_equal(out.cpu().numpy(), eager[1]), rep


def test_moe_layer_errors(backend):
    say("moe layer errors")
    n_expert, n_embd, n_ff, n_sh = 8, 256, 256, 256
    q, t = layer_tensors(n_expert, n_embd, n_ff, n_sh, 8900)
    views = list(layer_views("Lerr", q, t, n_expert, n_embd, n_ff, n_sh))
    x = np.zeros((1, n_embd), np.float32)
    bad = list(views)
    bad[0] = H.QuantTensor("Lerr.router_bad", 0, n_expert + 1, n_embd,
                           S.normal_f32(1, (n_expert + 1) * n_embd).view(np.uint8))
    with pytest.raises(H.ShapeError):
        backend.moe_layer(*bad, x, 2)
    bad = list(views)
    bad[4] = H.QuantTensor("Lerr.gsh_q40", 2, n_sh, n_embd, np.zeros(n_sh * n_embd // 32 * 18, np.uint8))
    with pytest.raises(H.UnsupportedQuantError):
        backend.moe_layer(*bad, x, 2)


@pytest.mark.parametrize("seed", range(4))
def test_moe_ffn_random_configs(backend, oracle, seed):
    """Seeded random routed-FFN configurations: 4..128 experts, hidden and
    expert widths of several multiples of 256, top-1..8, 1..12 tokens,
    Q4_K / Q8_0 gate-up with Q6_K / Q4_K / Q8_0 down, against the oracle."""
    rng = np.random.default_rng(7000 + seed)
    n_expert = int(rng.choice([4, 16, 64, 128]))
    n_embd = 256 * int(rng.integers(1, 5))
    n_ff = 256 * int(rng.integers(1, 4))
    top_k = int(rng.integers(1, min(8, n_expert) + 1))
    n_tok = int(rng.integers(1, 13))
    qa = int(rng.choice([12, 8]))
    qd = int(rng.choice([14, 12, 8]))
    say("moe random", seed, n_expert, n_embd, n_ff, top_k, n_tok, qa, qd)
    gate, up, down = expert_tensors(n_expert, n_embd, n_ff, qa, qd, 7100 + seed)
    logits = S.router_logits(7200 + seed, n_tok, n_expert)
    x = S.normal_f32(7300 + seed, n_tok * n_embd).reshape(n_tok, n_embd)
    out = backend.moe_ffn(H.ExpertView(f"rg{seed}", qa, n_expert, n_embd, n_ff, gate),
                          H.ExpertView(f"ru{seed}", qa, n_expert, n_embd, n_ff, up),
                          H.ExpertView(f"rd{seed}", qd, n_expert, n_ff, n_embd, down), logits, x, top_k)
    ref = oracle_moe(oracle, qa, qd, n_expert, n_embd, n_ff, gate, up, down, logits, x, top_k)
    for t in range(n_tok):
        check_parity(out[t], ref[t], "moe")
    for name in (f"rg{seed}", f"ru{seed}", f"rd{seed}"):
        backend.evict(name)


@pytest.mark.parametrize("n_tok", [2, 7])
def test_moe_ffn_q5_k(backend, oracle, n_tok):
    """Q5_K experts (gate/up and down) over several tokens: the two-token
    work items and the route launch."""
    n_expert, n_embd, n_ff, top_k = 16, 1024, 512, 4
    say("moe ffn q5_k", n_tok)
    gate, up, down = expert_tensors(n_expert, n_embd, n_ff, 13, 13, 7400 + n_tok)
    logits = S.router_logits(7500 + n_tok, n_tok, n_expert)
    x = S.normal_f32(7600 + n_tok, n_tok * n_embd).reshape(n_tok, n_embd)
    out = backend.moe_ffn(H.ExpertView(f"q5g{n_tok}", 13, n_expert, n_embd, n_ff, gate),
                          H.ExpertView(f"q5u{n_tok}", 13, n_expert, n_embd, n_ff, up),
                          H.ExpertView(f"q5d{n_tok}", 13, n_expert, n_ff, n_embd, down), logits, x, top_k)
    ref = oracle_moe(oracle, 13, 13, n_expert, n_embd, n_ff, gate, up, down, logits, x, top_k)
    for t in range(n_tok):
        check_parity(out[t], ref[t], "moe q5_k")
    for name in (f"q5g{n_tok}", f"q5u{n_tok}", f"q5d{n_tok}"):
        backend.evict(name)


def test_moe_ffn_budget_holding_two_of_three_refuses(oracle, moe_config_tensors):
    # gate and up (Q4_K, 113 MB each) and down (Q6_K, 165 MB) of the MoE
    # config; the budget holds any two of them but not all three, so the
    # call must fail before any launch rather than evict a tensor it holds
    gate, up, down = moe_config_tensors
    n_expert, n_embd, n_ff, top_k = 128, 2048, 768, 8
    say("moe ffn budget two of three")
    budget = gate.nbytes + down.nbytes
    assert budget < gate.nbytes + up.nbytes + down.nbytes
    logits = S.router_logits(4150, 1, n_expert)
    x = S.normal_f32(4250, n_embd).reshape(1, n_embd)
    g = H.ExpertView("bud.gate", 12, n_expert, n_embd, n_ff, gate)
    u = H.ExpertView("bud.up", 12, n_expert, n_embd, n_ff, up)
    d = H.ExpertView("bud.down", 14, n_expert, n_ff, n_embd, down)
    with H.HipBackend(0, budget) as be:
        for _ in range(2):  # the second attempt starts with gate and up resident
            with pytest.raises(H.OutOfMemoryError):
                be.moe_ffn(g, u, d, logits, x, top_k)
            assert be.resident_bytes() <= budget
        # the context still serves calls that fit: expert 5 of down alone
        xe = S.normal_f32(4260, n_ff)
        y = np.empty(n_embd, np.float32)
        be.expert_gemv(d, 5, xe, y)
        want = oracle.expert_gemv(14, n_expert, n_ff, n_embd, down, 5, xe)
        check_parity(y, want, "moe")
    # and a budget that holds all three runs the call
    with H.HipBackend(0, gate.nbytes + up.nbytes + down.nbytes) as be:
        out = be.moe_ffn(g, u, d, logits, x, top_k)
    ref = oracle_moe(oracle, 12, 14, n_expert, n_embd, n_ff, gate, up, down, logits, x, top_k)
    check_parity(out, ref, "moe")
