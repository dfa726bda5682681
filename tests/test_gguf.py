"""The GGUF weight source: the library's reader (sh_gguf_*) against the
oracle's restatement of crates/strata-gguf/src/reader.rs, and both against
the reference's own reader tests (reader_tests.rs:195-230 read-back,
:274-280 bad magic) and hand-made byte-level cases. CPU only: the reader
is host code (the device upload is tested in test_gpu_gguf.py).

The oracle itself is pinned by the reference's known answers and by cases
whose outcome the format fixes (alignment rounding, truncation at every
prefix, each header error), so a slip in either reader shows up as a
disagreement or a failed known answer.
"""
import struct

import numpy as np
import pytest

import gguf_oracle as G
import strata_hip as H
from gguf_writer import (ARRAY, BOOL, F32, F64, I8, I16, I32, I64, STRING, U8, U16, U32, U64, Writer, gstr)


def f16b(v):
    return np.array([v], np.float32).astype(np.float16).tobytes()


def write(tmp_path, name, data: bytes):
    p = tmp_path / f"{name}.gguf"
    p.write_bytes(data)
    return str(p)


def qwen4exp_metadata(w: Writer):
    # reader_tests.rs:139-193
    w.kv("general.architecture", STRING, "qwen4exp")
    w.kv("general.alignment", U32, 32)
    w.kv("qwen4exp.block_count", U32, 48)
    w.kv("qwen4exp.embedding_length", U32, 2560)
    w.kv("qwen4exp.expert_count", U32, 512)
    w.kv("qwen4exp.expert_used_count", U32, 10)
    w.kv("qwen4exp.attention.head_count", U32, 24)
    w.kv("qwen4exp.attention.head_count_kv", U32, 2)
    w.kv("qwen4exp.attention.layer_norm_rms_epsilon", F32, 1e-6)
    w.kv("qwen4exp.attention.compress_ratios", ARRAY, (I32, [4 if l % 4 == 3 else 0 for l in range(48)]))
    w.kv("tokenizer.ggml.tokens", ARRAY, (STRING, ["<|endoftext|>", "hello", " world"]))
    w.kv("tokenizer.ggml.model", STRING, "gpt2")


def compare(path, data: bytes):
    """Both readers on the same file: the same outcome, field for field."""
    try:
        want = G.parse(data)
        werr = None
    except G.GgufError as e:
        want, werr = None, e.kind
    try:
        got = H.GgufFile(path)
        gerr = None
    except H.FormatError:
        got, gerr = None, "format"
    except H.TruncatedError:
        got, gerr = None, "truncated"
    assert gerr == werr, (gerr, werr)
    if got is None:
        return None
    assert (got.version, got.n_tensors, got.n_kv) == (want.version, len(want.tensors), want.n_kv)
    assert (got.alignment, got.data_start, got.file_size) == (want.alignment, want.data_start, want.size)
    for k, m in want.meta.items():
        assert got.meta_type(k) == (m.ty, m.elem if m.ty == ARRAY else got.meta_type(k)[1],
                                    m.count if m.ty == ARRAY else got.meta_type(k)[2])
        assert got.get_int(k) == m.as_int()
        gf, wf = got.get_float(k), m.as_float()
        assert (gf is None and wf is None) or gf == wf or (gf != gf and wf != wf)
        assert got.get_str(k) == m.as_str()
    for i, t in enumerate(want.tensors):
        gt = got.tensor(i)
        assert (gt.name, gt.shape, gt.type, gt.offset) == (t.name, t.shape, t.ty, t.offset)
        assert got.find(t.name) == i
        try:
            wd = want.tensor_data(t)
            wkind = None
        except G.GgufError as e:
            wd, wkind = None, e.kind
        try:
            gd = got.tensor_data(i)
            gkind = None
        except H.TruncatedError:
            gd, gkind = None, "truncated"
        except H.UnsupportedQuantError:
            gd, gkind = None, "unsupported_quant"
        assert gkind == wkind, (t.name, gkind, wkind)
        if wd is not None:
            assert gd.tobytes() == wd
            assert gt.nbytes == len(wd)
    return got


# ---- the reference's own reader tests ----------------------------------------

def test_reads_back_metadata_and_tensors(tmp_path, oracle):
    # reader_tests.rs:195-230
    w = Writer()
    qwen4exp_metadata(w)
    data = bytearray(34)
    data[:2] = f16b(2.0)
    data[2] = 5
    w.tensor("blk.0.attn_q.weight", [32], 8, bytes(data))
    raw = w.finish()
    path = write(tmp_path, "read-back", raw)
    with H.GgufFile(path) as f:
        assert f.version == 3
        assert f.get_str("general.architecture") == "qwen4exp"
        assert f.get_int("qwen4exp.block_count") == 48
        assert f.meta_type("tokenizer.ggml.tokens")[2] == 3
        assert abs(f.get_float("qwen4exp.attention.layer_norm_rms_epsilon") - 1e-6) < 1e-12
        i = f.find("blk.0.attn_q.weight")
        t = f.tensor(i)
        assert t.shape == [32] and t.type == 8
        td = f.tensor_data(i)
        assert td[2] == 5
        out = oracle.dequantize_row(oracle.Q8_0, td[:34].copy(), 32)
        assert out[0] == 10.0
    compare(path, raw)


def test_bad_magic_is_refused(tmp_path):
    # reader_tests.rs:274-280
    path = write(tmp_path, "bad-magic", b"NOTGGUF and more bytes................")
    with pytest.raises(H.FormatError):
        H.GgufFile(path)
    with pytest.raises(G.GgufError) as e:
        G.parse(b"NOTGGUF and more bytes................")
    assert e.value.kind == "format"


def test_metadata_only_file(tmp_path):
    # reader_tests.rs:232-255 (a file with metadata and no tensors)
    w = Writer()
    qwen4exp_metadata(w)
    raw = w.finish()
    f = compare(write(tmp_path, "meta-only", raw), raw)
    assert f.n_tensors == 0 and f.data_start == len(raw)


def test_missing_file():
    with pytest.raises(H.IoError):
        H.GgufFile("/nonexistent/dir/model.gguf")


# ---- every metadata type, and the differential over random files -----------

def test_every_value_type(tmp_path):
    w = Writer()
    vals = [("u8", U8, 200), ("i8", I8, -100), ("u16", U16, 60000), ("i16", I16, -30000), ("u32", U32, 4000000000),
            ("i32", I32, -2000000000), ("f32", F32, 1.5), ("bool", BOOL, 1), ("str", STRING, "héllo ✓"),
            ("u64", U64, 2**63 + 5), ("i64", I64, -2**62), ("f64", F64, -2.25),
            ("arr", ARRAY, (ARRAY, [(U8, [1, 2]), (U8, [])])), ("empty", ARRAY, (F32, []))]
    for k, t, v in vals:
        w.kv(k, t, v)
    raw = w.finish()
    f = compare(write(tmp_path, "types", raw), raw)
    assert f.get_int("u8") == 200 and f.get_int("i8") == -100 and f.get_int("u32") == 4000000000
    assert f.get_int("bool") == 1 and f.get_str("str") == "héllo ✓"
    assert f.get_int("u64") == 0  # MetaValue::as_int reads the int field, 0 for u64
    assert f.get_float("f32") == 1.5 and f.get_float("i16") == -30000.0
    assert f.get_int("f64") is None and f.get_str("u8") is None
    assert f.meta_type("arr") == (ARRAY, ARRAY, 2)


def rand_value(rng, ty, depth=0):
    if ty in (U8, BOOL):
        return int(rng.integers(0, 256)) if ty == U8 else int(rng.integers(0, 2))
    if ty == I8:
        return int(rng.integers(-128, 128))
    if ty == U16:
        return int(rng.integers(0, 65536))
    if ty == I16:
        return int(rng.integers(-32768, 32768))
    if ty == U32:
        return int(rng.integers(0, 2**32))
    if ty == I32:
        return int(rng.integers(-2**31, 2**31))
    if ty == U64:
        return int(rng.integers(0, 2**63))
    if ty == I64:
        return int(rng.integers(-2**62, 2**62))
    if ty in (F32, F64):
        return float(np.float32(rng.standard_normal())) if ty == F32 else float(rng.standard_normal())
    if ty == STRING:
        return "".join(chr(int(c)) for c in rng.integers(32, 0x2FFF, int(rng.integers(0, 12))))
    elem = int(rng.choice([U8, I32, F32, STRING, U64] + ([ARRAY] if depth < 1 else [])))
    return (elem, [rand_value(rng, elem, depth + 1) for _ in range(int(rng.integers(0, 5)))])


@pytest.mark.parametrize("seed", range(12))
def test_random_files_agree_with_oracle(tmp_path, seed):
    rng = np.random.default_rng(seed)
    align = int(rng.choice([1, 8, 32, 64, 4096]))
    w = Writer(alignment=align)
    if align != 32 or rng.integers(0, 2):
        w.kv("general.alignment", U32, align)
    for k in range(int(rng.integers(0, 20))):
        ty = int(rng.integers(0, 13))
        w.kv(f"key.{k}", ty, rand_value(rng, ty))
    for k in range(int(rng.integers(0, 6))):
        ty = int(rng.choice([0, 1, 8, 12, 13, 14, 30, 2, 23]))
        block, size = G.GEOMETRY[ty]
        nd = int(rng.integers(1, 4))
        shape = [block * int(rng.integers(1, 4))] + [int(rng.integers(1, 4)) for _ in range(nd - 1)]
        n = int(np.prod(shape)) // block * size
        w.tensor(f"blk.{k}.weight", shape, ty, rng.integers(0, 256, n).astype(np.uint8).tobytes(), pad_to=align)
    raw = w.finish()
    compare(write(tmp_path, f"rand{seed}", raw), raw)


# ---- alignment ------------------------------------------------------------------

@pytest.mark.parametrize("ty,val,want", [(U32, 64, 64), (U8, 16, 16), (I32, -5, 32), (U32, 0, 32),
                                         (F32, 64.0, 32), (U64, 64, 32), (STRING, "64", 32), (BOOL, 1, 1)])
def test_alignment_rules(tmp_path, ty, val, want):
    w = Writer(alignment=max(want, 1))
    w.kv("general.alignment", ty, val)
    w.tensor("t", [32], 0, b"\x01" * 128, pad_to=max(want, 1))
    raw = w.finish()
    f = compare(write(tmp_path, "align", raw), raw)
    assert f.alignment == want and f.data_start % want == 0
    assert f.tensor_data(0)[0] == 1


# ---- errors -------------------------------------------------------------------

def small_file():
    w = Writer()
    w.kv("general.architecture", STRING, "qwen4exp")
    w.kv("arr", ARRAY, (STRING, ["a", "bc"]))
    w.tensor("a.weight", [64, 2], 8, bytes(range(136)))
    return w.finish()


def test_every_truncation_agrees(tmp_path):
    raw = small_file()
    p = tmp_path / "trunc.gguf"
    for n in range(len(raw) + 1):
        p.write_bytes(raw[:n])
        compare(str(p), raw[:n])


def test_header_errors(tmp_path):
    cases = {
        "version": Writer(version=2).finish(),
        "key_len": Writer().raw_kv(struct.pack("<Q", 65536) + b"k" * 65536 + struct.pack("<IB", U8, 1)).finish(),
        "utf8": Writer().raw_kv(gstr(b"bad\xff") + struct.pack("<IB", U8, 1)).finish(),
        "surrogate": Writer().kv("s", STRING, "ok").raw_kv(gstr(b"\xed\xa0\x80") + struct.pack("<IB", U8, 1)).finish(),
        "value_type": Writer().raw_kv(gstr("k") + struct.pack("<I", 13)).finish(),
        "elem_type": Writer().raw_kv(gstr("k") + struct.pack("<IIQ", ARRAY, 99, 0)).finish(),
        "array_len": Writer().raw_kv(gstr("k") + struct.pack("<IIQ", ARRAY, U8, (1 << 24) + 1)).finish(),
        "depth": Writer().kv("k", ARRAY, (ARRAY, [(ARRAY, [(U8, [1])])])).finish(),
        "dims0": Writer().raw_info(gstr("t") + struct.pack("<IIQ", 0, 0, 0)).finish(),
        "dims5": Writer().raw_info(gstr("t") + struct.pack("<I5QIQ", 5, 1, 1, 1, 1, 1, 0, 0)).finish(),
        "duplicate": Writer().tensor("t", [32], 0, b"\0" * 128).tensor("t", [32], 0, b"\0" * 128).finish(),
    }
    for name, raw in cases.items():
        with pytest.raises(G.GgufError) as e:
            G.parse(raw)
        assert e.value.kind == "format", name
        with pytest.raises(H.FormatError):
            H.GgufFile(write(tmp_path, name, raw))
    # two array levels are allowed
    ok = Writer().kv("k", ARRAY, (ARRAY, [(U8, [1, 2])])).finish()
    compare(write(tmp_path, "depth2", ok), ok)


def test_payload_errors(tmp_path):
    w = Writer()
    w.tensor("short", [256], 12, b"\0" * 144)
    w.tensor("unknown", [32], 5, b"", offset=0)        # type id 5 does not exist
    w.tensor("zero", [0, 4], 0, b"", offset=0)
    w.tensor("past_end", [256, 2], 12, b"", offset=144)  # needs 288 bytes from 144
    raw = w.finish()
    f = compare(write(tmp_path, "payload", raw), raw)
    assert f.tensor_data(0).size == 144
    with pytest.raises(H.UnsupportedQuantError):
        f.tensor_data(1)
    with pytest.raises(H.TruncatedError):
        f.tensor_data(2)
    with pytest.raises(H.TruncatedError):
        f.tensor_data(3)
    assert f.tensor(1).nbytes == 0


def test_last_key_wins(tmp_path):
    raw = Writer().kv("k", U32, 1).kv("k", STRING, "two").finish()
    f = compare(write(tmp_path, "dupkey", raw), raw)
    assert f.get_str("k") == "two" and f.n_kv == 2


# ---- split models (reader.rs:450-572) ------------------------------------------

def test_split_paths_resolves_siblings(tmp_path):
    # reader_tests.rs:282-290, with the library's model open as the probe
    single = str(tmp_path / "qwen4exp-q2_0.gguf")
    assert G.split_paths(single) == [single]
    missing = str(tmp_path / "model-00001-of-00002.gguf")
    with pytest.raises(G.GgufError) as e:
        G.split_paths(missing)
    assert e.value.kind == "io"
    (tmp_path / "model-00001-of-00002.gguf").write_bytes(Writer().finish())
    with pytest.raises(H.IoError) as e:
        H.GgufModel(missing)
    assert "00002" in str(e.value)
    # shapes that are not a split suffix are single files
    for odd in ("m-00001-of-0000x.gguf", "m-00003-of-00002.gguf", "m-00000-of-00002.gguf", "m00001-of-00002.gguf",
                "m-00001-of-00002.ggml", "m-0001-of-00002.gguf"):
        assert G.split_paths(str(tmp_path / odd)) == [str(tmp_path / odd)]


def test_multi_shard_model_reads_tensors_across_shards(tmp_path):
    # reader_tests.rs:292-331
    w1 = Writer()
    qwen4exp_metadata(w1)
    w1.kv("split.count", U32, 2).kv("split.no", U32, 0).kv("split.tensors.count", U32, 2)
    w1.tensor("token_embd.weight", [32], 0, b"\0" * 128)
    w2 = Writer()
    w2.kv("split.count", U32, 2).kv("split.no", U32, 1).kv("split.tensors.count", U32, 2)
    w2.tensor("output.weight", [32], 0, b"\1" * 128)
    p1 = tmp_path / "strata-rs-test-model-00001-of-00002.gguf"
    p2 = tmp_path / "strata-rs-test-model-00002-of-00002.gguf"
    p1.write_bytes(w1.finish())
    p2.write_bytes(w2.finish())
    assert G.split_paths(str(p2)) == [str(p1), str(p2)]
    with H.GgufModel(str(p2)) as m:
        assert m.n_shards == 2
        assert m.meta().get_str("general.architecture") == "qwen4exp"
        assert m.find("token_embd.weight") == (0, 0)
        assert m.find("output.weight") == (1, 0)
        assert m.find("nope") is None
        assert m.tensor_data("output.weight")[0] == 1
    # a name in both shards is refused
    w3 = Writer().kv("split.no", U32, 1).tensor("token_embd.weight", [32], 0, b"\0" * 128)
    p2.write_bytes(w3.finish())
    with pytest.raises(H.FormatError):
        H.GgufModel(str(p1))


# ---- malformed files: random byte mutations ------------------------------------

@pytest.mark.parametrize("seed", range(4))
def test_mutated_files_agree_with_oracle(tmp_path, seed):
    """Random byte flips in the header, metadata and directory of a valid
    file: the library's reader never reads out of bounds or disagrees with the
    oracle about the outcome (the error kind, or every parsed field)."""
    w = Writer()
    qwen4exp_metadata(w)
    w.kv("arr.nested", ARRAY, (ARRAY, [(U8, [1, 2, 3]), (STRING, ["x", "yz"])]))
    w.tensor("a.weight", [64, 2], 8, bytes(range(136)))
    w.tensor("b.weight", [256], 12, bytes(144))
    base = bytearray(w.finish())
    head = len(base) - 136 - 8 - 144 - 16  # mutate the header, metadata and directory
    rng = np.random.default_rng(seed)
    p = tmp_path / "mut.gguf"
    for _ in range(150):
        b = bytearray(base)
        for _ in range(int(rng.integers(1, 4))):
            i = int(rng.integers(0, head))
            b[i] = int(rng.integers(0, 256))
        if rng.integers(0, 4) == 0:
            b = b[:int(rng.integers(0, len(b)))]
        p.write_bytes(bytes(b))
        try:
            compare(str(p), bytes(b))
        except H.UnsupportedQuantError:
            pass  # a flipped type id: both readers refuse the payload (checked in compare)
