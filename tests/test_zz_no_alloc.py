"""sh_ffn_dev_noalloc (the allocation-free form of sh_ffn_dev, its
intermediates in the library's fixed device scratch) against sh_ffn_dev
with a caller workspace: the same kernels in the same order, so the outputs
must be equal bit for bit. Two calls in a row, the second with a smaller
input, so a second call finds the scratch holding the first call's data.
Also checked against the oracle's dense FFN at the matvec bound (1e-3)."""
import numpy as np
import pytest

import strata_hip as H
from strata_hip import synth as S

pytestmark = pytest.mark.gpu


def say(*a):
    print("[case]", *a, flush=True)


def run(torch, quants, mats, n_embd, n_ff, x, norm, noalloc):
    dev = [torch.from_numpy(np.ascontiguousarray(m)).cuda() for m in mats]
    xd = torch.from_numpy(np.ascontiguousarray(x)).cuda()
    nd = torch.from_numpy(np.ascontiguousarray(norm)).cuda()
    out = torch.full_like(xd, float("nan"))
    n_tok = x.shape[0]
    s = torch.cuda.current_stream().cuda_stream
    tens = [(q, 0, t.data_ptr()) for q, t in zip(quants, dev)]
    if noalloc:
        H.ffn_dev_noalloc(tens, n_embd, n_ff, n_tok, xd.data_ptr(), nd.data_ptr(), 1e-6, out.data_ptr(), s)
    else:
        nb = H.ffn_workspace_bytes(n_tok, n_embd, n_ff)
        ws = torch.empty(nb, dtype=torch.uint8, device="cuda")
        H.ffn_dev(tens, n_embd, n_ff, n_tok, xd.data_ptr(), nd.data_ptr(), 1e-6, out.data_ptr(), ws.data_ptr(), nb, s)
    torch.cuda.synchronize()
    return out.cpu().numpy()


def test_ffn_dev_noalloc_equals_workspace_path(oracle):
    import torch
    from conftest import rel_err
    cases = [((12, 12, 12), 4096, 12288, 3),   # general path, three tokens: 2.2 MB of scratch
             ((12, 12, 14), 2048, 4096, 1)]    # then a smaller call (mixed types)
    for quants, n_embd, n_ff, n_tok in cases:
        say("ffn noalloc", quants, n_embd, n_ff, n_tok)
        mats = [S.matrix(quants[0], 71 + n_ff, n_ff, n_embd), S.matrix(quants[1], 72 + n_ff, n_ff, n_embd),
                S.matrix(quants[2], 73 + n_ff, n_embd, n_ff)]
        x = S.normal_f32(74 + n_tok, n_tok * n_embd).reshape(n_tok, n_embd)
        norm = S.normal_f32(75, n_embd)
        got = run(torch, quants, mats, n_embd, n_ff, x, norm, True)
        want = run(torch, quants, mats, n_embd, n_ff, x, norm, False)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
        ref = oracle.dense_ffn(quants, mats, n_embd, n_ff, x, norm, 1e-6)
        assert rel_err(got.astype(np.float64) - x, ref.astype(np.float64) - x) <= 1e-3


def test_ffn_dev_noalloc_refuses_shapes_beyond_the_scratch():
    say("ffn noalloc limit")
    assert H.ffn_workspace_bytes(24, 4096, 12288) > 4 << 20
    assert H.ffn_workspace_bytes(23, 4096, 12288) <= 4 << 20
    tens = [(12, 0, 1 << 20)] * 3  # never dereferenced: refused on the host
    with pytest.raises(H.UnsupportedShapeError):
        H.ffn_dev_noalloc(tens, 4096, 12288, 24, 1 << 20, 1 << 20, 1e-6, 1 << 20, 0)
