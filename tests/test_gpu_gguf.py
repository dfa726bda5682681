"""GGUF tensors admitted straight into the resident store
(sh_upload_gguf_tensor) and used by the matvec entry points.

Each call afterwards passes a zero-filled stand-in of the right size under
the same key: the results still match the oracle on the file's real bytes,
so the kernels read what the upload put on the device (a re-upload of the
stand-in would give zeros). The Q8_0 tensor (17.8 MB) crosses several
8 MiB staging chunks. Tolerance as the matvec tests: 1e-3.
"""
import numpy as np
import pytest

import strata_hip as H
from conftest import check_parity
from gguf_writer import STRING, U32, Writer
from strata_hip import synth as S

pytestmark = pytest.mark.gpu
TOL = 1e-3


def say(*a):
    print("[case]", *a, flush=True)


def check(got, want):
    check_parity(got, want, "gguf")


def test_upload_from_gguf_then_matvec(tmp_path, oracle):
    say("gguf upload + gemv / expert_gemv")
    q4 = S.matrix(12, 11, 1024, 4096)            # [cols 4096, rows 1024]
    q8 = S.matrix(8, 12, 4096, 4096)             # 17.8 MB: three staging chunks
    q5 = S.matrix(13, 13, 300, 2048)
    ex = S.matrix(14, 14, 4 * 256, 512)          # 4 experts, 256 inputs, 512 outputs
    router = S.normal_f32(15, 128 * 2048)
    iq = S.matrix(23, 16, 2, 256)                # IQ4_XS: matvec only
    nl = np.zeros(18 * 2, np.uint8)              # IQ4_NL: no device kernel
    w = Writer()
    w.kv("general.architecture", STRING, "qwen4exp").kv("general.alignment", U32, 32)
    w.tensor("blk.0.ffn_down.weight", [4096, 1024], 12, q4.tobytes())
    w.tensor("blk.0.attn_q.weight", [4096, 4096], 8, q8.tobytes())
    w.tensor("blk.0.ffn_up.weight", [2048, 300], 13, q5.tobytes())
    w.tensor("blk.0.ffn_down_exps.weight", [512, 256, 4], 14, ex.tobytes())
    w.tensor("blk.0.ffn_gate_inp.weight", [2048, 128], 0, router.tobytes())
    w.tensor("blk.0.iq.weight", [256, 2], 23, iq.tobytes())
    w.tensor("blk.0.nl.weight", [32, 2], 20, nl.tobytes())
    w.tensor("blk.0.four_d.weight", [32, 1, 1, 1], 0, b"\0" * 128)
    path = tmp_path / "model.gguf"
    path.write_bytes(w.finish())

    be = H.HipBackend(0, 1 << 30)
    try:
        with H.GgufFile(str(path)) as f:
            before = be.resident_bytes()
            names = ("blk.0.ffn_down.weight", "blk.0.attn_q.weight", "blk.0.ffn_up.weight",
                     "blk.0.ffn_down_exps.weight", "blk.0.ffn_gate_inp.weight", "blk.0.iq.weight")
            for name in names:
                be.upload_gguf(f, f.find(name), name)
            total = sum(f.tensor(f.find(n)).nbytes for n in names)
            assert be.resident_bytes() - before == total
            with pytest.raises(H.UnsupportedQuantError):
                be.upload_gguf(f, f.find("blk.0.nl.weight"), "nl")
            with pytest.raises(H.BackendError):
                be.upload_gguf(f, f.find("blk.0.four_d.weight"), "four_d")

        for name, quant, rows, cols, real in (("blk.0.ffn_down.weight", 12, 1024, 4096, q4),
                                              ("blk.0.attn_q.weight", 8, 4096, 4096, q8),
                                              ("blk.0.ffn_up.weight", 13, 300, 2048, q5),
                                              ("blk.0.ffn_gate_inp.weight", 0, 128, 2048,
                                               router.view(np.uint8)),
                                              ("blk.0.iq.weight", 23, 2, 256, iq)):
            x = S.normal_f32(rows + 3, cols)
            y = np.empty(rows, np.float32)
            be.gemv(H.QuantTensor(name, quant, rows, cols, np.zeros(real.nbytes, np.uint8)), x, y)
            check(y, oracle.gemv(quant, rows, cols, real, x, threads=8))

        x = S.normal_f32(77, 256)
        y = np.empty(512, np.float32)
        view = H.ExpertView("blk.0.ffn_down_exps.weight", 14, 4, 256, 512, np.zeros(ex.nbytes, np.uint8))
        be.expert_gemv(view, 2, x, y)
        check(y, oracle.expert_gemv(14, 4, 256, 512, ex, 2, x))
    finally:
        be.close()


def test_weight_upload_pitched_and_idempotent(oracle):
    """sh_weight_upload: rows given with a pitch (16 pad bytes after each
    2304-byte Q4_K row) are stored packed; a second upload of the key is a
    no-op; later calls pass a zero stand-in and still read the real rows."""
    say("weight upload, pitched rows")
    rows, cols = 96, 4096
    w = S.matrix(12, 21, rows, cols)
    rb = S.row_bytes(12, cols)
    pitched = np.zeros((rows, rb + 16), np.uint8)
    pitched[:, :rb] = w.reshape(rows, rb)
    pitched[:, rb:] = 0xAB
    be = H.HipBackend(0, 1 << 30)
    try:
        be.upload("pitched", 12, 1, rows, cols, pitched, row_pitch=rb + 16)
        before = be.resident_bytes()
        assert before == rows * rb
        be.upload("pitched", 12, 1, rows, cols, pitched, row_pitch=rb + 16)
        assert be.resident_bytes() == before
        x = S.normal_f32(22, cols)
        y = np.empty(rows, np.float32)
        be.gemv(H.QuantTensor("pitched", 12, rows, cols, np.zeros(w.nbytes, np.uint8)), x, y)
        check(y, oracle.gemv(12, rows, cols, w, x))
        with pytest.raises(H.BackendError):
            be.upload("bad", 12, 1, rows, cols, pitched, row_pitch=rb - 1)
        with pytest.raises(H.UnsupportedQuantError):
            be.upload("nl", 20, 1, 2, 32, np.zeros(36, np.uint8))  # IQ4_NL: no device kernel
    finally:
        be.close()
