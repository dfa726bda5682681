"""The device path against the committed golden fixtures (tests/golden/).

Dequantization and the Q8 activation quantizer are checked bit for bit;
gemv, expert gemv and the MoE FFN within max|y - r| / max|r| <= 1e-3 of the
stored reference outputs; routing ids exactly and weights to 4e-7.
"""
import json
import os

import numpy as np
import pytest

import strata_hip as H
from conftest import check_parity
from strata_hip import synth as S

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def say(*a):
    print("[case]", *a, flush=True)


def cases():
    return np.load(os.path.join(GOLDEN, "seeded_cases.npz"), allow_pickle=False)


def test_reference_dequant_kats(backend):
    with open(os.path.join(GOLDEN, "reference_kats.json")) as f:
        kats = json.load(f)
    say("golden reference kats")
    for kat in kats:
        if kat["what"] != "dequant":
            continue
        out = np.empty(kat["n"], np.float32)
        backend.dequantize_row(kat["quant"], bytes.fromhex(kat["block"]), out)
        for i, v in kat["expect"].items():
            assert out[int(i)] == v, (kat["source"], i)


@pytest.mark.parametrize("quant,rows,cols", [(8, 16, 256), (12, 16, 512), (14, 16, 512), (13, 16, 512)])
def test_golden_gemv_and_dequant(backend, quant, rows, cols):
    say("golden gemv", quant)
    c = cases()
    w, x = c[f"gemv_{quant}_w"], c[f"gemv_{quant}_x"]
    y = np.empty(rows, np.float32)
    backend.gemv(H.QuantTensor(f"golden{quant}", quant, rows, cols, w), x, y)
    check_parity(y, c[f"gemv_{quant}_y"], "golden")
    rb = H.byte_size(quant, cols)
    for r in range(rows):
        out = np.empty(cols, np.float32)
        backend.dequantize_row(quant, w[r * rb:(r + 1) * rb], out)
        assert np.array_equal(out.view(np.uint32), c[f"deq_{quant}"][r].view(np.uint32))


def test_golden_q6k_signed_gemv(backend):
    say("golden q6k signed")
    c = cases()
    y = np.empty(16, np.float32)
    backend.gemv(H.QuantTensor("golden14s", 14, 16, 512, c["gemv_14s_w"], flags=H.FLAG_Q6K_SIGNED_SCALES),
                 c["gemv_14s_x"], y)
    check_parity(y, c["gemv_14s_y"], "golden")


def test_golden_expert_and_moe(backend):
    say("golden expert + moe")
    c = cases()
    y = np.empty(256, np.float32)
    backend.expert_gemv(H.ExpertView("golden_exp", 12, 3, 64, 256, c["expert_w"]), 1, c["expert_x"], y)
    check_parity(y, c["expert_y"], "golden")
    ids, w = backend.moe_route(c["moe_logits"], 4)
    assert ids.tolist() == c["moe_ids"].tolist()
    assert np.abs(w - c["moe_wts"]).max() <= 4e-7
    g, u, d = (S.matrix(q, int(sd), 16 * 256, 256) for q, sd in zip((12, 12, 14), c["moe_seeds"]))
    out = backend.moe_ffn(H.ExpertView("gg", 12, 16, 256, 256, g), H.ExpertView("gu", 12, 16, 256, 256, u),
                          H.ExpertView("gd", 14, 16, 256, 256, d), c["moe_logits"], c["moe_x"], 4)
    for t in range(3):
        check_parity(out[t], c["moe_out"][t], "golden")


def test_golden_q8_quantizer(backend):
    import torch
    say("golden q8 quantizer")
    c = cases()
    x = c["q8_x"]
    dev = torch.device("cuda:0")
    tx = torch.from_numpy(x).to(dev)
    q = torch.empty(x.size, dtype=torch.int8, device=dev)
    s = torch.empty(x.size // 32, dtype=torch.float32, device=dev)
    u = torch.empty(x.size // 32, dtype=torch.float32, device=dev)
    H.quantize_q8_dev(tx.data_ptr(), x.size, q.data_ptr(), s.data_ptr(), u.data_ptr(),
                      torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert np.array_equal(q.cpu().numpy(), c["q8_codes"])
    assert np.array_equal(s.cpu().numpy().view(np.uint32), c["q8_scales"].view(np.uint32))
    assert np.array_equal(u.cpu().numpy().view(np.uint32), c["q8_sums"].view(np.uint32))


def test_golden_row_methods(backend):
    """The elementwise methods on the host-slice entry points against the
    fixtures: within one ulp (softmax two), as their parity tests."""
    say("golden row methods")
    c = cases()

    def ulps(a, b):
        a = np.ascontiguousarray(a, np.float32).view(np.int32).astype(np.int64)
        b = np.ascontiguousarray(b, np.float32).view(np.int32).astype(np.int64)
        a = np.where(a < 0, -(a & 0x7FFFFFFF), a)
        b = np.where(b < 0, -(b & 0x7FFFFFFF), b)
        return int(np.abs(a - b).max())

    for r in range(3):
        x = c["row_x"][r].copy()
        backend.rms_norm(x, c["row_w"], 1e-6)
        assert ulps(x, c["row_rms"][r]) <= 1
        x = c["row_x"][r].copy()
        backend.softmax(x)
        assert ulps(x, c["row_softmax"][r]) <= 2
    for h in range(8):
        x = c["row_heads"][h].copy()
        backend.l2_norm(x, 1e-6)
        assert ulps(x, c["row_l2"][h]) <= 1
        x = c["row_heads"][h].copy()
        backend.rope_neox(x, H.RopeCfg(pos=4097, n_rot=64, head_dim=128, freq_base=1e7))
        assert ulps(x, c["row_rope"][h]) <= 1
