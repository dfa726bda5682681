"""Backend behaviour around the kernels: the resident weight store (LRU under
a byte budget, crates/strata-backend-wgpu/src/gpu.rs:577-599), re-upload on a
changed tensor, and one context shared by several threads (the trait is
Send + Sync, crates/strata-core/src/backend.rs:20)."""
import threading

import numpy as np
import pytest

import strata_hip as H
from conftest import rel_err
from strata_hip import synth as S

pytestmark = pytest.mark.gpu


def say(*a):
    print("[case]", *a, flush=True)


def test_name_is_hip(backend):
    assert backend.name() == "hip"


def test_weight_cache_evicts_when_over_budget():
    # gpu.rs:577-599: a 24 MiB budget and three 10 MiB matrices: the first goes
    say("LRU eviction")
    rows, cols = 4552, 4096          # 4552 * 2304 B ~= 10 MiB of Q4_K
    w = S.matrix(12, 1, rows, cols)
    x = S.normal_f32(2, cols)
    y = np.empty(rows, np.float32)
    with H.HipBackend(0, 24 << 20) as be:
        for i in range(3):
            be.gemv(H.QuantTensor(f"big{i}", 12, rows, cols, w), x, y)
        assert be.resident_bytes() <= 2 * w.nbytes
        assert be.resident_bytes() >= w.nbytes


def test_changed_tensor_under_the_same_name_is_reuploaded(backend, oracle):
    say("re-upload on change")
    rows, cols = 64, 4096
    x = S.normal_f32(9, cols)
    y = np.empty(rows, np.float32)
    w1 = S.matrix(12, 10, rows, cols)
    backend.gemv(H.QuantTensor("same", 12, rows, cols, w1), x, y)
    assert rel_err(y, oracle.gemv(12, rows, cols, w1, x)) <= 1e-3
    w2 = S.matrix(8, 11, rows, cols)  # same name, another type and size
    backend.gemv(H.QuantTensor("same", 8, rows, cols, w2), x, y)
    assert rel_err(y, oracle.gemv(8, rows, cols, w2, x)) <= 1e-3


def test_threads_share_one_context(backend, oracle):
    say("threads")
    rows, cols = 256, 4096
    ws = [S.matrix(12, 20 + i, rows, cols) for i in range(4)]
    xs = [S.normal_f32(30 + i, cols) for i in range(4)]
    wants = [oracle.gemv(12, rows, cols, ws[i], xs[i]) for i in range(4)]
    errors = []

    def work(i):
        try:
            for _ in range(5):
                y = np.empty(rows, np.float32)
                backend.gemv(H.QuantTensor(f"thr{i}", 12, rows, cols, ws[i]), xs[i], y)
                if rel_err(y, wants[i]) > 1e-3:
                    errors.append(i)
        except Exception as e:  # pragma: no cover - reported below
            errors.append(repr(e))

    ts = [threading.Thread(target=work, args=(i,)) for i in range(4)]
    for t in ts:
        t.start()
    for t in ts:
        t.join()
    assert not errors


def test_stream_read_folds_every_word():
    """sh_stream_read_dev (the bandwidth ceiling the benchmark reports): the
    XOR of its per-workgroup folds equals the XOR of every 32-bit word, so
    every byte is read (a ragged length that is not a multiple of the grid's
    stride included)."""
    import torch
    say("stream read")
    for n in (16, 4096 * 16 + 48, 28_311_552):
        data = np.random.default_rng(n).integers(0, 2**32, n // 4, dtype=np.uint32)
        d = torch.from_numpy(data.view(np.int32)).cuda()
        out = torch.zeros(H.STREAM_READ_BLOCKS, dtype=torch.int32, device="cuda")
        H.stream_read_dev(d.data_ptr(), n, out.data_ptr(), torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        got = np.bitwise_xor.reduce(out.cpu().numpy().view(np.uint32))
        assert int(got) == int(np.bitwise_xor.reduce(data))
