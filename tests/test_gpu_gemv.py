"""Fused dequant-matvec on the device vs the oracle (ops::gemv).

Tolerance (conftest.check_parity): max|y - ref| / max|ref| <= 1e-3 (the
path's stated bound under f32 accumulation), and per element
|y_i - ref_i| / max(|ref_i|, 1e-3 rms(ref)) <= 2e-3 (f32 arithmetic itself
scores about 6e-4 there at 12288 inputs). Covers the reference's own gemv unit test, ragged row counts,
one- and multi-window rows, batches 1..8 (Q5_K too), the Q6_K scale readings, IQ4_XS in
both code-byte readings, the
configs' full shapes (the lm_head on a row sample) and the device-pointer
entry point.
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


def check(got, want, label=""):
    check_parity(got, want, label)


def test_reference_q8_0_unit_case(backend):
    # ops_tests.rs:44-61 as the reference runs it: one 34-byte Q8_0 block
    # (d = 0.5, q = j % 7 - 3), a 32-element x, one output row
    from test_oracle_ops import q8_single_block
    b, x = q8_single_block()
    w = H.QuantTensor("q8unit", H.QuantType.Q8_0, 1, 32, b)
    y = np.zeros(1, np.float32)
    say("gemv reference Q8_0 unit case (one block)")
    backend.gemv(w, x, y)
    expect = sum(float(j % 7 - 3) * 0.5 * float(x[j]) for j in range(32))
    assert abs(float(y[0]) - expect) < 1e-4


@pytest.mark.parametrize("rows,cols,batch", [(1, 32, 1), (7, 96, 1), (300, 4128, 1), (33, 12320, 3),
                                             (1000, 4064, 8), (5, 32, 8)])
def test_gemv_q8_0_odd_block_rows(backend, oracle, rows, cols, batch):
    """Q8_0 rows of an odd number of 32-element blocks (any multiple of 32
    columns, as quant.rs:125-136 allows): 34-byte rows alternate 4- and
    2-byte alignment, every batch size."""
    say("gemv Q8_0 odd blocks", rows, cols, batch)
    w = S.matrix(8, 4000 + rows + cols, rows, cols)
    x = S.normal_f32(4001 + cols, batch * cols).reshape(batch, cols)
    y = backend.gemv_batch(H.QuantTensor(f"q8odd_{rows}_{cols}", 8, rows, cols, w), x, batch)
    for i in range(batch):
        check(y[i], oracle.gemv(8, rows, cols, w, x[i]), f"q8 odd b{i}")


@pytest.mark.parametrize("quant,rows,cols", [
    (12, 37, 256), (12, 1, 4096), (12, 129, 4096), (12, 64, 12288), (12, 33, 8192 + 256),
    (8, 37, 64), (8, 129, 4096), (8, 17, 4160), (8, 5, 12288),
    (14, 37, 256), (14, 129, 4096), (14, 9, 12288), (14, 3, 2048 + 256),
    (13, 37, 256), (13, 129, 4096), (13, 9, 12288), (13, 3, 2048 + 256), (13, 4096, 4096),
])
def test_gemv_shapes(backend, oracle, quant, rows, cols):
    say("gemv", quant, rows, cols)
    w = S.matrix(quant, 31 * rows + cols + quant, rows, cols)
    x = S.normal_f32(rows + 7, cols)
    y = np.empty(rows, np.float32)
    backend.gemv(H.QuantTensor(f"t{quant}_{rows}_{cols}", quant, rows, cols, w), x, y)
    check(y, oracle.gemv(quant, rows, cols, w, x))


@pytest.mark.parametrize("quant,rows,cols", [(12, 12288, 4096), (12, 4096, 12288), (8, 4096, 4096)])
def test_gemv_config_shapes(backend, oracle, quant, rows, cols):
    say("gemv config shape", quant, rows, cols)
    w = S.matrix(quant, 2024 + quant, rows, cols)
    x = S.normal_f32(3, cols)
    y = np.empty(rows, np.float32)
    backend.gemv(H.QuantTensor(f"cfg{quant}_{rows}_{cols}", quant, rows, cols, w), x, y)
    check(y, oracle.gemv(quant, rows, cols, w, x, threads=8))
    backend.evict(f"cfg{quant}_{rows}_{cols}")


@pytest.mark.parametrize("signed", [False, True])
def test_lm_head_q6_k_full_shape(backend, oracle, signed):
    # 151936 x 4096 Q6_K (510 MB): the device computes every row, the oracle
    # checks 4096 rows spread over the matrix
    rows, cols = 151936, 4096
    say("gemv Q6_K lm_head", "signed" if signed else "u8")
    w = S.matrix(14, 77, rows, cols)
    x = S.normal_f32(78, cols)
    y = np.empty(rows, np.float32)
    flags = H.FLAG_Q6K_SIGNED_SCALES if signed else 0
    backend.gemv(H.QuantTensor("lm_head" + ("_i8" if signed else ""), 14, rows, cols, w, flags), x, y)
    rb = S.row_bytes(14, cols)
    idx = np.linspace(0, rows - 1, 4096).astype(np.int64)
    sub = np.concatenate([w[i * rb:(i + 1) * rb] for i in idx])
    mode = oracle.SCALE_I8 if signed else oracle.SCALE_U8
    want = oracle.gemv(14, len(idx), cols, sub, x, scale_mode=mode)
    check(y[idx], want)
    backend.evict("lm_head" + ("_i8" if signed else ""))


@pytest.mark.parametrize("quant,cols", [(12, 4096), (12, 12288), (8, 4096), (14, 4096), (13, 4096),
                                        (13, 12288)])
@pytest.mark.parametrize("batch", [1, 2, 3, 8])
def test_gemv_batch(backend, oracle, quant, cols, batch):
    rows = 96
    say("gemv batch", quant, cols, batch)
    w = S.matrix(quant, 5 + cols + quant, rows, cols)
    x = S.normal_f32(batch * 13 + cols, batch * cols).reshape(batch, cols)
    y = backend.gemv_batch(H.QuantTensor(f"b{quant}_{cols}", quant, rows, cols, w), x, batch)
    for b in range(batch):
        check(y[b], oracle.gemv(quant, rows, cols, w, x[b]))


@pytest.mark.parametrize("quant", [12, 13])
@pytest.mark.parametrize("rows,cols,batch", [(100, 4096, 5), (17, 256, 8), (1, 512, 2), (12288, 4096, 8),
                                             (4099, 1024, 7), (16400, 1024, 8), (4096, 12288, 8),
                                             (37, 4096 + 256, 3), (300, 8192 + 1024, 2)])
def test_gemv_batch_kquant_mfma_shapes(backend, oracle, quant, rows, cols, batch):
    # the batched Q4_K / Q5_K path on int8 MFMA: partial 16-row tiles, shares
    # of super-blocks with nothing to do, odd batches, a tall matrix (16400
    # rows: four row tiles per workgroup and three shares, one of them empty),
    # rows of several 4096-column windows (the last one partial)
    say("gemv batch mfma", quant, rows, cols, batch)
    w = S.matrix(quant, 77 + rows + cols, rows, cols)
    x = S.normal_f32(batch * 17 + rows, batch * cols).reshape(batch, cols)
    y = backend.gemv_batch(H.QuantTensor(f"bm{quant}_{rows}_{cols}", quant, rows, cols, w), x, batch)
    idx = np.unique(np.linspace(0, rows - 1, min(rows, 512)).astype(np.int64))
    rb = S.row_bytes(quant, cols)
    sub = np.concatenate([w[i * rb:(i + 1) * rb] for i in idx])
    for b in range(batch):
        check(y[b][idx], oracle.gemv(quant, len(idx), cols, sub, x[b]))


def test_gemv_batch_q4k_mixed_block_magnitudes(backend, oracle):
    """The batched Q4_K path scales each 256-element super-block of x by one
    power of two: 32-element blocks whose magnitudes differ by up to 10^8
    within a super-block still meet the tolerance against the f64 sums."""
    rows, cols, batch = 256, 2048, 8
    say("gemv batch q4k mixed block magnitudes")
    w = S.matrix(12, 4321, rows, cols)
    x = S.normal_f32(4322, batch * cols).reshape(batch, cols)
    rng = np.random.default_rng(4323)
    scale = (10.0 ** rng.uniform(-4, 4, size=(batch, cols // 32))).astype(np.float32)
    x = (x.reshape(batch, cols // 32, 32) * scale[:, :, None]).reshape(batch, cols).astype(np.float32)
    y = backend.gemv_batch(H.QuantTensor("bm_mixed", 12, rows, cols, w), x, batch)
    for b in range(batch):
        check(y[b], oracle.gemv(12, rows, cols, w, x[b]))


def test_gemv_shape_errors(backend):
    say("gemv errors")
    w = S.matrix(12, 1, 4, 256)
    t = H.QuantTensor("err", 12, 4, 256, w)
    with pytest.raises(H.ShapeError):
        backend.gemv(t, np.zeros(255, np.float32), np.zeros(4, np.float32))
    with pytest.raises(H.ShapeError):
        backend.gemv(t, np.zeros(256, np.float32), np.zeros(5, np.float32))
    with pytest.raises(H.TruncatedError):
        backend.gemv(H.QuantTensor("short", 12, 4, 256, w[:-1]), np.zeros(256, np.float32),
                     np.zeros(4, np.float32))
    with pytest.raises(H.UnsupportedQuantError):
        q4_0 = np.zeros(4 * 18, np.uint8)  # Q4_0: not on this path
        backend.gemv(H.QuantTensor("q4_0", 2, 4, 32, q4_0), np.zeros(32, np.float32), np.zeros(4, np.float32))


@pytest.mark.parametrize("ggml", [False, True])
@pytest.mark.parametrize("rows,cols,batch", [(37, 256, 1), (129, 4096, 1), (9, 12288, 1), (4096, 4096, 1),
                                             (33, 8192 + 256, 1), (96, 4096, 3), (64, 12288, 8)])
def test_gemv_iq4_xs(backend, oracle, ggml, rows, cols, batch):
    """IQ4_XS in both code-byte readings (strata-gguf's first 16 bytes for
    every sub-block, ggml's 16 bytes per sub-block): one- and multi-window
    rows, batches."""
    say("gemv IQ4_XS", "ggml" if ggml else "reference", rows, cols, batch)
    w = S.matrix(23, 6100 + rows + cols, rows, cols)
    x = S.normal_f32(6200 + cols + batch, batch * cols).reshape(batch, cols)
    flags = H.FLAG_IQ4XS_GGML if ggml else 0
    t = H.QuantTensor(f"iq4_{int(ggml)}_{rows}_{cols}", 23, rows, cols, w, flags)
    y = backend.gemv_batch(t, x, batch)
    mode = oracle.IQ4XS_GGML if ggml else oracle.IQ4XS_REFERENCE
    for b in range(batch):
        check(y[b], oracle.gemv(23, rows, cols, w, x[b], scale_mode=mode), f"iq4_xs b{b}")
    if batch == 1 and rows <= 129:
        # the two readings differ on random code bytes
        other = oracle.gemv(23, rows, cols, w, x[0], scale_mode=1 - mode)
        assert np.abs(y[0] - other).max() > 1e-2 * np.abs(other).max()
    backend.evict(t.name)


def test_gemv_empty_shapes(backend):
    say("gemv empty")
    y = np.full(3, 7.0, np.float32)
    backend.gemv(H.QuantTensor("empty_cols", 12, 3, 0, np.zeros(0, np.uint8)), np.zeros(0, np.float32), y)
    assert np.all(y == 0.0)  # ops::gemv writes 0 for an empty row


def test_gemv_dev_pointers_on_torch_stream(oracle):
    import torch
    rows, cols = 4096, 12288
    say("gemv_dev Q4_K", rows, cols)
    w = S.matrix(12, 55, rows, cols)
    x = S.normal_f32(56, cols)
    wd = torch.from_numpy(w).cuda()
    xd = torch.from_numpy(x).cuda()
    yd = torch.empty(rows, dtype=torch.float32, device="cuda")
    s = torch.cuda.current_stream().cuda_stream
    H.gemv_dev(12, wd.data_ptr(), rows, cols, xd.data_ptr(), yd.data_ptr(), 1, s)
    torch.cuda.synchronize()
    check(yd.cpu().numpy(), oracle.gemv(12, rows, cols, w, x, threads=8))


@pytest.mark.parametrize("cols", [4096, 12288])
@pytest.mark.parametrize("offset", [0, 2, 8, 16])
def test_gemv_q6k_base_offsets(oracle, cols, offset):
    """Q6_K rows of whole 4096-column windows from weight buffers starting 0,
    2, 8 and 16 bytes into an allocation: 16-byte boundaries read each window
    whole through LDS, the others the unit loads (2: every other block two
    bytes below a dword boundary); both readings of the scales."""
    import torch
    rows = 300
    say("gemv_dev Q6_K offset", rows, cols, offset)
    w = S.matrix(14, 57 + offset, rows, cols)
    x = S.normal_f32(58, cols)
    buf = torch.zeros(w.nbytes + 64, dtype=torch.uint8, device="cuda")
    buf[offset:offset + w.nbytes] = torch.from_numpy(w).cuda()
    xd = torch.from_numpy(x).cuda()
    s = torch.cuda.current_stream().cuda_stream
    for signed in (False, True):
        yd = torch.empty(rows, dtype=torch.float32, device="cuda")
        flags = H.FLAG_Q6K_SIGNED_SCALES if signed else 0
        H.gemv_dev(14, buf.data_ptr() + offset, rows, cols, xd.data_ptr(), yd.data_ptr(), 1, s, flags)
        torch.cuda.synchronize()
        mode = oracle.SCALE_I8 if signed else oracle.SCALE_U8
        check(yd.cpu().numpy(), oracle.gemv(14, rows, cols, w, x, scale_mode=mode), f"signed {signed}")


def plain_matrix(quant, seed, rows, cols):
    """F32 / F16 / BF16 rows of N(0, 1) values, as packed bytes."""
    v = S.normal_f32(seed, rows * cols)
    if quant == H.QuantType.F32:
        return v.view(np.uint8)
    if quant == H.QuantType.F16:
        return v.astype(np.float16).view(np.uint8)
    bits = v.view(np.uint32)
    rne = ((bits + 0x7FFF + ((bits >> 16) & 1)) >> 16).astype(np.uint16)  # round to nearest even
    return rne.view(np.uint8)


@pytest.mark.parametrize("quant", [H.QuantType.F32, H.QuantType.F16, H.QuantType.BF16])
@pytest.mark.parametrize("rows,cols,batch", [(128, 2048, 1), (1, 2048, 1), (300, 2049, 3), (5, 1, 8),
                                             (4096, 4096, 2)])
def test_gemv_plain_types(backend, oracle, quant, rows, cols, batch):
    """Plain-float rows (router and shared-expert gate tensors): products and
    sums in f64 as ops::gemv, so the f32 results equal the oracle's except
    where the two summation orders straddle a rounding boundary (1 ulp)."""
    say("gemv plain", int(quant), rows, cols, batch)
    w = plain_matrix(quant, 900 + rows + cols, rows, cols)
    x = S.normal_f32(901 + cols, batch * cols).reshape(batch, cols)
    t = H.QuantTensor(f"p{int(quant)}_{rows}_{cols}", int(quant), rows, cols, w)
    if batch == 1:
        y = np.empty(rows, np.float32)
        backend.gemv(t, x[0], y)
        y = y[None]
    else:
        y = backend.gemv_batch(t, x, batch)
    for b in range(batch):
        ref = oracle.gemv(int(quant), rows, cols, w, x[b])
        ulp = np.abs(y[b].view(np.int32).astype(np.int64) - ref.view(np.int32).astype(np.int64))
        assert ulp.max() <= 1, (b, int(ulp.max()))
        assert np.mean(y[b] == ref) >= 0.99


@pytest.mark.parametrize("seed", range(6))
def test_gemv_random_shapes(backend, oracle, seed):
    """Seeded random shapes across every matvec type and batch 1..8: rows
    1..3000, columns any multiple of the type's block (and of 64) up to
    20480, so partial 16-row tiles, partial windows and several windows all
    occur against the oracle."""
    rng = np.random.default_rng(9000 + seed)
    for case in range(8):
        quant = int(rng.choice([8, 12, 13, 14, 0, 1, 30]))
        step = 256 if quant in (12, 13, 14) else 32 if quant == 8 else 64
        cols = step * int(rng.integers(1, 20480 // step + 1))
        rows = int(rng.integers(1, 3001))
        batch = int(rng.integers(1, 9))
        say("gemv random", seed, case, quant, rows, cols, batch)
        if quant in (0, 1, 30):
            w = plain_matrix(quant, seed * 100 + case, rows, cols)
        else:
            w = S.matrix(quant, seed * 100 + case, rows, cols)
        x = S.normal_f32(seed * 100 + case + 7, batch * cols).reshape(batch, cols)
        t = H.QuantTensor(f"rand{seed}_{case}", quant, rows, cols, w)
        y = backend.gemv_batch(t, x, batch)
        for b in range(batch):
            check(y[b], oracle.gemv(quant, rows, cols, w, x[b], threads=8))
        backend.evict(f"rand{seed}_{case}")



@pytest.mark.parametrize("quant,rows,cols,batch", [(12, 4096, 12288, 8), (13, 4096, 12288, 3), (12, 4096, 8192, 2),
                                                   (12, 33, 8192 + 256, 7), (13, 1000, 20480, 8),
                                                   (12, 12288, 4096, 8), (13, 12288, 4096, 8), (12, 500, 2048, 5),
                                                   (13, 16384, 4096, 2)])
def test_gemv_dev_ws_batches(oracle, quant, rows, cols, batch):
    """sh_gemv_dev_ws: batches convert their activations once per call into
    the workspace, each workgroup copying its window; rows wider than one
    window (2048 to 4096 columns by shape) run split-K, the windows' sums
    added in window order by the last workgroup of each row block: the same
    call twice gives the same bits (no dependence on which workgroup
    finished last), against the oracle at the parity bars; two activation
    sets on one workspace."""
    import torch
    say("gemv_dev_ws", quant, rows, cols, batch)
    w = S.matrix(quant, 91 + rows + cols, rows, cols)
    nb = H.gemv_workspace_bytes(quant, rows, cols, batch)
    assert nb > 0
    wd = torch.from_numpy(w).cuda()
    ws = torch.empty(nb, dtype=torch.uint8, device="cuda")
    s = torch.cuda.current_stream().cuda_stream
    for seed in (92, 93):
        x = S.normal_f32(seed + cols, batch * cols).reshape(batch, cols)
        xd = torch.from_numpy(x).cuda()
        y1 = torch.empty(batch * rows, dtype=torch.float32, device="cuda")
        y2 = torch.empty_like(y1)
        H.gemv_dev_ws(quant, wd.data_ptr(), rows, cols, xd.data_ptr(), y1.data_ptr(), batch, ws.data_ptr(), nb, s)
        H.gemv_dev_ws(quant, wd.data_ptr(), rows, cols, xd.data_ptr(), y2.data_ptr(), batch, ws.data_ptr(), nb, s)
        torch.cuda.synchronize()
        a, b = y1.cpu().numpy(), y2.cpu().numpy()
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
        a = a.reshape(batch, rows)
        for i in sorted({0, batch - 1}):
            check(a[i], oracle.gemv(quant, rows, cols, w, x[i], threads=8), f"dev_ws b{i}")


def test_gemv_workspace_sizes():
    say("gemv workspace sizes")
    assert H.gemv_workspace_bytes(12, 4096, 12288, 1) == 0      # batch 1: none
    assert H.gemv_workspace_bytes(14, 4096, 12288, 8) == 0      # no batched MFMA kernel for Q6_K
    assert H.gemv_workspace_bytes(12, 4096, 12288, 8) > 0
    assert H.gemv_workspace_bytes(12, 12288, 4096, 8) > 0       # one window: converted once, copied
    with pytest.raises(H.BackendError):
        H.gemv_dev_ws(12, 1 << 20, 4096, 12288, 1 << 20, 1 << 20, 8, 1 << 20, 16)  # workspace too small
