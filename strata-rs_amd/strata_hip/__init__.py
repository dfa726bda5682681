"""Python host mirror of strata-core's ComputeBackend over libstrata_hip.

Names and argument meanings follow the reference interface
(crates/strata-core/src/backend.rs:20-51 and :117-153,
crates/strata-core/src/weights.rs:14-34):

* ``QuantTensor(name, quant, rows, cols, data)`` -- a packed row-major matrix;
* ``ExpertView(name, quant, n_expert, rows, cols, data)`` -- expert-major
  ``[n_expert][rows = in][cols = out]``;
* ``HipBackend.gemv(w, x, y, scratch)`` / ``expert_gemv(w, e, x, y, scratch)``
  write ``y`` in place, like the trait methods; ``scratch`` is accepted and
  ignored, as a device backend may (crates/strata-backend-wgpu/src/gpu.rs:270).

Errors raise ``BackendError`` (the trait's ``Error::Backend``), with
``ShapeError`` for the length mismatches the reference asserts on
(crates/strata-core/src/ops.rs:15-17) and ``TruncatedError`` for
strata-gguf's ``Error::Truncated`` (crates/strata-gguf/src/dequant.rs:50-55).

Every call goes through the C ABI in ``include/strata_hip.h``; there is no
fallback: if the library is not built or no device exists, construction
fails loudly.
"""
from __future__ import annotations

import ctypes as C
import enum
import os
from dataclasses import dataclass, field

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
PKG_ROOT = os.path.dirname(HERE)
LIB_PATH = os.path.join(PKG_ROOT, "lib", "libstrata_hip.so")

SH_OK = 0
SH_ERR_INVALID_ARGUMENT = -1
SH_ERR_SHAPE = -2
SH_ERR_TRUNCATED = -3
SH_ERR_UNSUPPORTED_QUANT = -4
SH_ERR_UNSUPPORTED_SHAPE = -5
SH_ERR_NO_DEVICE = -6
SH_ERR_DEVICE = -7
SH_ERR_OUT_OF_MEMORY = -8
SH_ERR_FORMAT = -9
SH_ERR_IO = -10
SH_ERR_NOT_FOUND = -11

FLAG_Q6K_SIGNED_SCALES = 1
FLAG_EXPERT_OUT_MAJOR = 2
FLAG_IQ4XS_GGML = 4
MATMUL_BF16 = 0
MATMUL_Q8 = 1
MATMUL_Q8K = 2

# Every symbol include/strata_hip.h declares (kept in step with the header).
EXPORTS = (
    "sh_abi_version", "sh_last_error", "sh_device_count", "sh_quant_geometry",
    "sh_create", "sh_destroy", "sh_name", "sh_resident_bytes", "sh_evict",
    "sh_gemv", "sh_gemv_batch", "sh_expert_gemv", "sh_dequantize_row",
    "sh_moe_route", "sh_moe_ffn", "sh_moe_layer", "sh_matmul",
    "sh_moe_workspace_bytes", "sh_moe_ffn_dev", "sh_matmul_workspace_bytes", "sh_matmul_dev",
    "sh_quantize_q8_dev", "sh_quantize_q8k_dev", "sh_moe_layer_workspace_bytes", "sh_moe_layer_dev", "sh_dequant_dev",
    "sh_gemv_dev", "sh_rms_norm", "sh_rope_neox", "sh_softmax", "sh_l2_norm", "sh_add", "sh_rms_norm_dev",
    "sh_l2_norm_dev", "sh_softmax_dev", "sh_rope_neox_dev", "sh_add_dev", "sh_gguf_open", "sh_gguf_close",
    "sh_gguf_header", "sh_gguf_tensor", "sh_gguf_find", "sh_gguf_tensor_data", "sh_gguf_meta_type",
    "sh_gguf_meta_int", "sh_gguf_meta_float", "sh_gguf_meta_str", "sh_upload_gguf_tensor", "sh_gguf_model_open",
    "sh_gguf_model_close", "sh_gguf_model_shards", "sh_gguf_model_shard", "sh_gguf_model_find", "sh_weight_upload",
    "sh_ffn_workspace_bytes", "sh_ffn_dev", "sh_ffn", "sh_ffn_dev_noalloc", "sh_stream_read_dev",
    "sh_gemv_workspace_bytes", "sh_gemv_dev_ws",
)


class QuantType(enum.IntEnum):
    """Strata's ggml type ids (crates/strata-gguf/src/quant.rs:15-43)."""
    F32 = 0
    F16 = 1
    Q8_0 = 8
    Q4_K = 12
    Q5_K = 13
    Q6_K = 14
    IQ4_XS = 23
    BF16 = 30


class BackendError(RuntimeError):
    def __init__(self, code: int, message: str):
        super().__init__(f"backend error ({code}): {message}")
        self.code = code


class ShapeError(BackendError):
    pass


class TruncatedError(BackendError):
    pass


class UnsupportedQuantError(BackendError):
    pass


class NoDeviceError(BackendError):
    pass


class FormatError(BackendError):
    """A malformed GGUF file (the reference reader's header errors)."""


class NotFoundError(BackendError):
    pass


class IoError(BackendError):
    pass


class UnsupportedShapeError(BackendError):
    pass


class OutOfMemoryError(BackendError):
    """A device or pinned allocation failed, or the weight budget cannot hold
    the tensors one call needs at once."""


_ERRORS = {
    SH_ERR_SHAPE: ShapeError,
    SH_ERR_TRUNCATED: TruncatedError,
    SH_ERR_UNSUPPORTED_QUANT: UnsupportedQuantError,
    SH_ERR_NO_DEVICE: NoDeviceError,
    SH_ERR_FORMAT: FormatError,
    SH_ERR_IO: IoError,
    SH_ERR_NOT_FOUND: NotFoundError,
    SH_ERR_UNSUPPORTED_SHAPE: UnsupportedShapeError,
    SH_ERR_OUT_OF_MEMORY: OutOfMemoryError,
}


class _QuantTensorC(C.Structure):
    _fields_ = [("key", C.c_uint64), ("quant", C.c_uint32), ("flags", C.c_uint32),
                ("rows", C.c_uint64), ("cols", C.c_uint64), ("data", C.c_void_p),
                ("nbytes", C.c_uint64)]


class _ExpertDevC(C.Structure):
    _fields_ = [("quant", C.c_uint32), ("flags", C.c_uint32), ("data", C.c_void_p)]


class _ExpertViewC(C.Structure):
    _fields_ = [("key", C.c_uint64), ("quant", C.c_uint32), ("flags", C.c_uint32),
                ("n_expert", C.c_uint64), ("rows", C.c_uint64), ("cols", C.c_uint64),
                ("data", C.c_void_p), ("nbytes", C.c_uint64)]


class _GgufTensorInfoC(C.Structure):
    _fields_ = [("name", C.c_char_p), ("n_dims", C.c_uint32), ("type", C.c_uint32), ("shape", C.c_uint64 * 4),
                ("offset", C.c_uint64), ("nbytes", C.c_uint64)]


class _RopeCfgC(C.Structure):
    _fields_ = [("pos", C.c_uint64), ("n_rot", C.c_uint64), ("head_dim", C.c_uint64), ("freq_base", C.c_double)]


@dataclass
class RopeCfg:
    """backend.rs:158-167."""
    pos: int
    n_rot: int
    head_dim: int
    freq_base: float

    def _c(self) -> _RopeCfgC:
        return _RopeCfgC(self.pos, self.n_rot, self.head_dim, self.freq_base)


_lib = None


def library_path() -> str:
    return LIB_PATH


def load_library() -> C.CDLL:
    """The C-ABI library; raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(f"{LIB_PATH} is not built: run __graft_entry__.build() "
                           f"(or make -C strata-rs_amd)")
    L = C.CDLL(LIB_PATH)
    vp, u32, u64, f32p = C.c_void_p, C.c_uint32, C.c_uint64, C.c_void_p
    L.sh_abi_version.restype = C.c_int
    L.sh_last_error.restype = C.c_char_p
    L.sh_device_count.argtypes = [C.POINTER(C.c_int)]
    L.sh_quant_geometry.argtypes = [u32, C.POINTER(C.c_uint32), C.POINTER(C.c_uint32)]
    L.sh_create.argtypes = [C.c_int, u64, C.POINTER(vp)]
    L.sh_destroy.argtypes = [vp]
    L.sh_name.argtypes = [vp]
    L.sh_name.restype = C.c_char_p
    L.sh_resident_bytes.argtypes = [vp, C.POINTER(C.c_uint64)]
    L.sh_evict.argtypes = [vp, u64]
    L.sh_gemv.argtypes = [vp, C.POINTER(_QuantTensorC), f32p, u64, f32p, u64]
    L.sh_gemv_batch.argtypes = [vp, C.POINTER(_QuantTensorC), f32p, f32p, u32]
    L.sh_expert_gemv.argtypes = [vp, C.POINTER(_ExpertViewC), u64, f32p, u64, f32p, u64]
    L.sh_dequantize_row.argtypes = [vp, u32, u32, vp, u64, f32p, u64]
    L.sh_moe_route.argtypes = [vp, f32p, u32, u32, u32, vp, f32p]
    L.sh_moe_ffn.argtypes = [vp, C.POINTER(_ExpertViewC), C.POINTER(_ExpertViewC),
                             C.POINTER(_ExpertViewC), f32p, u32, u32, f32p, f32p]
    L.sh_moe_workspace_bytes.argtypes = [u32, u32, u64, u64, u64, u32, u32, C.POINTER(C.c_uint64)]
    L.sh_moe_ffn_dev.argtypes = [C.POINTER(_ExpertDevC), C.POINTER(_ExpertDevC), C.POINTER(_ExpertDevC),
                                 u64, u64, u64, vp, u32, u32, vp, vp, vp, u64, vp]
    L.sh_moe_layer.argtypes = [vp, C.POINTER(_QuantTensorC), C.POINTER(_ExpertViewC), C.POINTER(_ExpertViewC),
                               C.POINTER(_ExpertViewC), C.POINTER(_QuantTensorC), C.POINTER(_QuantTensorC),
                               C.POINTER(_QuantTensorC), C.POINTER(_QuantTensorC), f32p, u32, u32, f32p]
    L.sh_moe_layer_workspace_bytes.argtypes = [u32, u32, u64, u64, u64, u64, C.POINTER(C.c_uint32),
                                               C.POINTER(C.c_uint64)]
    L.sh_moe_layer_dev.argtypes = [C.POINTER(_ExpertDevC), u64, u64, u64, u64, u32, u32, vp, vp, vp, u64, vp]
    L.sh_matmul.argtypes = [vp, C.POINTER(_QuantTensorC), f32p, u32, f32p, u32]
    L.sh_matmul_workspace_bytes.argtypes = [u32, u64, u64, u32, u32, C.POINTER(C.c_uint64)]
    L.sh_matmul_dev.argtypes = [u32, u32, vp, u64, u64, vp, u32, vp, u32, vp, u64, vp]
    L.sh_quantize_q8_dev.argtypes = [vp, u64, vp, vp, vp, vp]
    L.sh_quantize_q8k_dev.argtypes = [vp, u64, vp, vp, vp, vp]
    L.sh_dequant_dev.argtypes = [u32, u32, vp, u64, u64, vp, vp]
    L.sh_gemv_dev.argtypes = [u32, u32, vp, u64, u64, vp, vp, u32, vp]
    L.sh_stream_read_dev.argtypes = [vp, u64, vp, vp]
    L.sh_gemv_workspace_bytes.argtypes = [u32, u64, u64, u32, C.POINTER(C.c_uint64)]
    L.sh_gemv_dev_ws.argtypes = [u32, u32, vp, u64, u64, vp, vp, u32, vp, u64, vp]
    dbl, ropep = C.c_double, C.POINTER(_RopeCfgC)
    L.sh_rms_norm.argtypes = [vp, f32p, f32p, u64, dbl]
    L.sh_rope_neox.argtypes = [vp, f32p, u64, ropep]
    L.sh_softmax.argtypes = [vp, f32p, u64]
    L.sh_l2_norm.argtypes = [vp, f32p, u64, dbl]
    L.sh_add.argtypes = [vp, f32p, f32p, u64]
    L.sh_rms_norm_dev.argtypes = [vp, vp, vp, u64, u64, dbl, vp]
    L.sh_l2_norm_dev.argtypes = [vp, u64, u64, dbl, vp]
    L.sh_softmax_dev.argtypes = [vp, u64, u64, vp]
    L.sh_rope_neox_dev.argtypes = [vp, u64, u64, ropep, vp]
    L.sh_add_dev.argtypes = [vp, vp, u64, vp]
    u64p, u32p = C.POINTER(C.c_uint64), C.POINTER(C.c_uint32)
    L.sh_gguf_open.argtypes = [C.c_char_p, C.POINTER(vp)]
    L.sh_gguf_close.argtypes = [vp]
    L.sh_gguf_header.argtypes = [vp, u32p, u64p, u64p, u64p, u64p, u64p]
    L.sh_gguf_tensor.argtypes = [vp, u64, C.POINTER(_GgufTensorInfoC)]
    L.sh_gguf_find.argtypes = [vp, C.c_char_p, u64p]
    L.sh_gguf_tensor_data.argtypes = [vp, u64, C.POINTER(vp), u64p]
    L.sh_gguf_meta_type.argtypes = [vp, C.c_char_p, u32p, u32p, u64p]
    L.sh_gguf_meta_int.argtypes = [vp, C.c_char_p, C.POINTER(C.c_int64)]
    L.sh_gguf_meta_float.argtypes = [vp, C.c_char_p, C.POINTER(C.c_double)]
    L.sh_gguf_meta_str.argtypes = [vp, C.c_char_p, C.POINTER(C.c_char_p), u64p]
    L.sh_upload_gguf_tensor.argtypes = [vp, vp, u64, u64]
    L.sh_gguf_model_open.argtypes = [C.c_char_p, C.POINTER(vp)]
    L.sh_gguf_model_close.argtypes = [vp]
    L.sh_gguf_model_shards.argtypes = [vp, u64p]
    L.sh_gguf_model_shard.argtypes = [vp, u64, C.POINTER(vp)]
    L.sh_gguf_model_find.argtypes = [vp, C.c_char_p, u64p, u64p]
    L.sh_weight_upload.argtypes = [vp, u64, u32, u64, u64, u64, vp, u64]
    L.sh_ffn_workspace_bytes.argtypes = [u32, u64, u64, u64p]
    L.sh_ffn_dev.argtypes = [C.POINTER(_ExpertDevC), u64, u64, u32, vp, vp, dbl, vp, vp, u64, vp]
    L.sh_ffn_dev_noalloc.argtypes = [C.POINTER(_ExpertDevC), u64, u64, u32, vp, vp, dbl, vp, vp]
    L.sh_ffn.argtypes = [vp, C.POINTER(_QuantTensorC), C.POINTER(_QuantTensorC), C.POINTER(_QuantTensorC), f32p, dbl,
                         u32, f32p]
    _lib = L
    return L


def last_error() -> str:
    return load_library().sh_last_error().decode()


def check(rc: int) -> None:
    if rc != SH_OK:
        raise _ERRORS.get(rc, BackendError)(rc, last_error())


def device_count() -> int:
    n = C.c_int(0)
    check(load_library().sh_device_count(C.byref(n)))
    return n.value


def quant_geometry(quant: int) -> tuple[int, int]:
    bs, ts = C.c_uint32(), C.c_uint32()
    check(load_library().sh_quant_geometry(int(quant), C.byref(bs), C.byref(ts)))
    return bs.value, ts.value


def byte_size(quant: int, n: int) -> int:
    """QuantType::byte_size (crates/strata-gguf/src/quant.rs:173-181)."""
    bs, ts = quant_geometry(quant)
    return (n + bs - 1) // bs * ts


def name_key(name: str) -> int:
    """64-bit FNV-1a of a tensor name: the key the Rust shim derives."""
    h = 0xCBF29CE484222325
    for b in name.encode():
        h = ((h ^ b) * 0x100000001B3) & 0xFFFFFFFFFFFFFFFF
    return h


def _bytes(data) -> np.ndarray:
    if isinstance(data, (bytes, bytearray, memoryview)):
        return np.frombuffer(data, dtype=np.uint8)
    return np.ascontiguousarray(data).view(np.uint8).reshape(-1)


@dataclass
class QuantTensor:
    """backend.rs:117-153: ``rows`` rows of ``cols`` elements in ``quant``."""
    name: str
    quant: int
    rows: int
    cols: int
    data: object
    flags: int = 0
    _buf: np.ndarray = field(init=False, repr=False)

    def __post_init__(self):
        self._buf = _bytes(self.data)

    def row_bytes(self) -> int:
        return byte_size(self.quant, self.cols)

    def _c(self) -> _QuantTensorC:
        return _QuantTensorC(name_key(self.name), int(self.quant), self.flags, self.rows, self.cols,
                             self._buf.ctypes.data, self._buf.nbytes)


@dataclass
class ExpertView:
    """weights.rs:14-34: expert-major ``[n_expert][rows = in][cols = out]``; with
    ``FLAG_EXPERT_OUT_MAJOR`` llama.cpp's ``[n_expert][rows = out][cols = in]``."""
    name: str
    quant: int
    n_expert: int
    rows: int
    cols: int
    data: object
    flags: int = 0
    _buf: np.ndarray = field(init=False, repr=False)

    def __post_init__(self):
        self._buf = _bytes(self.data)

    def _c(self) -> _ExpertViewC:
        return _ExpertViewC(name_key(self.name), int(self.quant), self.flags, self.n_expert, self.rows,
                            self.cols, self._buf.ctypes.data, self._buf.nbytes)


def _f32_in(a, n: int | None = None) -> np.ndarray:
    v = np.ascontiguousarray(a, dtype=np.float32)
    return v


def _f32_out(y) -> np.ndarray:
    if not (isinstance(y, np.ndarray) and y.dtype == np.float32 and y.flags.c_contiguous):
        raise TypeError("output must be a C-contiguous float32 numpy array")
    return y


@dataclass
class GgufTensorInfo:
    """TensorInfo (crates/strata-gguf/src/reader.rs:179-197) and its payload size."""
    name: str
    shape: list
    type: int
    offset: int
    nbytes: int


class GgufFile:
    """GgufFile (reader.rs:200-445) over the library's reader: the file is
    mapped until close(); tensor_data() views point into the mapping."""

    def __init__(self, path: str | None = None, _borrowed=None):
        self._L = load_library()
        self._owned = _borrowed is None
        if self._owned:
            h = C.c_void_p()
            check(self._L.sh_gguf_open(os.fsencode(path), C.byref(h)))
        else:
            h = _borrowed
        self._h = h
        v, nt, nkv, al, ds, fs = C.c_uint32(), *(C.c_uint64() for _ in range(5))
        check(self._L.sh_gguf_header(h, C.byref(v), C.byref(nt), C.byref(nkv), C.byref(al), C.byref(ds),
                                     C.byref(fs)))
        self.version, self.n_tensors, self.n_kv = v.value, nt.value, nkv.value
        self.alignment, self.data_start, self.file_size = al.value, ds.value, fs.value

    def close(self) -> None:
        if self._h and self._owned:
            self._L.sh_gguf_close(self._h)
        self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def tensor(self, index: int) -> GgufTensorInfo:
        t = _GgufTensorInfoC()
        check(self._L.sh_gguf_tensor(self._h, index, C.byref(t)))
        return GgufTensorInfo(t.name.decode(), list(t.shape[:t.n_dims]), t.type, t.offset, t.nbytes)

    def tensors(self) -> list:
        return [self.tensor(i) for i in range(self.n_tensors)]

    def find(self, name: str) -> int | None:
        i = C.c_uint64()
        rc = self._L.sh_gguf_find(self._h, name.encode(), C.byref(i))
        if rc == SH_ERR_NOT_FOUND:
            return None
        check(rc)
        return i.value

    def tensor_data(self, index: int) -> np.ndarray:
        p, n = C.c_void_p(), C.c_uint64()
        check(self._L.sh_gguf_tensor_data(self._h, index, C.byref(p), C.byref(n)))
        if n.value == 0:
            return np.zeros(0, np.uint8)
        v = np.ctypeslib.as_array((C.c_uint8 * n.value).from_address(p.value))
        v.flags.writeable = False
        return v

    def meta_type(self, key: str):
        t, e, c = C.c_uint32(), C.c_uint32(), C.c_uint64()
        rc = self._L.sh_gguf_meta_type(self._h, key.encode(), C.byref(t), C.byref(e), C.byref(c))
        if rc == SH_ERR_NOT_FOUND:
            return None
        check(rc)
        return t.value, e.value, c.value

    def get_int(self, key: str):
        v = C.c_int64()
        rc = self._L.sh_gguf_meta_int(self._h, key.encode(), C.byref(v))
        return None if rc == SH_ERR_NOT_FOUND else (check(rc), v.value)[1]

    def get_float(self, key: str):
        v = C.c_double()
        rc = self._L.sh_gguf_meta_float(self._h, key.encode(), C.byref(v))
        return None if rc == SH_ERR_NOT_FOUND else (check(rc), v.value)[1]

    def get_str(self, key: str):
        s, n = C.c_char_p(), C.c_uint64()
        rc = self._L.sh_gguf_meta_str(self._h, key.encode(), C.byref(s), C.byref(n))
        return None if rc == SH_ERR_NOT_FOUND else (check(rc), C.string_at(s, n.value).decode())[1]


class GgufModel:
    """GgufModel (reader.rs:450-522): every shard of a split model, one name
    index; shard(i) lends a GgufFile valid until close()."""

    def __init__(self, any_shard: str):
        self._L = load_library()
        h = C.c_void_p()
        check(self._L.sh_gguf_model_open(os.fsencode(any_shard), C.byref(h)))
        self._h = h
        n = C.c_uint64()
        check(self._L.sh_gguf_model_shards(h, C.byref(n)))
        self._shards = []
        for i in range(n.value):
            sh = C.c_void_p()
            check(self._L.sh_gguf_model_shard(h, i, C.byref(sh)))
            self._shards.append(GgufFile(_borrowed=sh))

    @property
    def n_shards(self) -> int:
        return len(self._shards)

    def shard(self, i: int) -> GgufFile:
        return self._shards[i]

    def meta(self) -> GgufFile:
        return self._shards[0]

    def find(self, name: str):
        si, ti = C.c_uint64(), C.c_uint64()
        rc = self._L.sh_gguf_model_find(self._h, name.encode(), C.byref(si), C.byref(ti))
        if rc == SH_ERR_NOT_FOUND:
            return None
        check(rc)
        return si.value, ti.value

    def tensor_data(self, name: str):
        f = self.find(name)
        return None if f is None else self._shards[f[0]].tensor_data(f[1])

    def close(self) -> None:
        if self._h:
            for sh in self._shards:
                sh.close()
            self._L.sh_gguf_model_close(self._h)
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class HipBackend:
    """The HIP backend: the quantized primitives of ComputeBackend on one GPU.

    ``weight_budget`` bounds resident packed weights (LRU eviction), like
    ``WgpuBackend::probe_with_budget`` (crates/strata-backend-wgpu/src/gpu.rs:164).
    """

    def __init__(self, device: int = 0, weight_budget: int = 0):
        L = load_library()
        ctx = C.c_void_p()
        check(L.sh_create(device, weight_budget, C.byref(ctx)))
        self._ctx = ctx
        self._L = L

    def close(self) -> None:
        if self._ctx:
            self._L.sh_destroy(self._ctx)
            self._ctx = C.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def name(self) -> str:
        return self._L.sh_name(self._ctx).decode()

    def resident_bytes(self) -> int:
        v = C.c_uint64()
        check(self._L.sh_resident_bytes(self._ctx, C.byref(v)))
        return v.value

    def evict(self, name: str) -> None:
        check(self._L.sh_evict(self._ctx, name_key(name)))

    def gemv(self, w: QuantTensor, x, y: np.ndarray, scratch=None) -> None:
        """``y = W x`` (backend.rs:25; ops.rs:14-28)."""
        xv, yv = _f32_in(x), _f32_out(y)
        wc = w._c()
        check(self._L.sh_gemv(self._ctx, C.byref(wc), xv.ctypes.data, xv.size, yv.ctypes.data, yv.size))

    def gemv_batch(self, w: QuantTensor, x, batch: int) -> np.ndarray:
        """``batch`` gemvs sharing one weight read: x ``[batch][cols]``."""
        xv = _f32_in(x)
        if xv.size != batch * w.cols:
            raise ShapeError(SH_ERR_SHAPE, f"x has {xv.size} elements, want {batch}x{w.cols}")
        y = np.empty((batch, w.rows), dtype=np.float32)
        wc = w._c()
        check(self._L.sh_gemv_batch(self._ctx, C.byref(wc), xv.ctypes.data, y.ctypes.data, batch))
        return y

    def expert_gemv(self, w: ExpertView, e: int, x, y: np.ndarray, scratch=None) -> None:
        """``y = W_e x`` in the in-major orientation (backend.rs:28-35; ops.rs:169-195)."""
        xv, yv = _f32_in(x), _f32_out(y)
        wc = w._c()
        check(self._L.sh_expert_gemv(self._ctx, C.byref(wc), e, xv.ctypes.data, xv.size,
                                     yv.ctypes.data, yv.size))

    def moe_route(self, logits, top_k: int) -> tuple[np.ndarray, np.ndarray]:
        """MoeLayer::route from router logits (crates/strata-core/src/moe.rs:58-90):
        ids (ascending) and renormalised weights, ``[n_tok][top_k]`` each."""
        lg = np.ascontiguousarray(logits, dtype=np.float32)
        if lg.ndim == 1:
            lg = lg[None, :]
        n_tok, n_expert = lg.shape
        ids = np.empty((n_tok, top_k), np.int32)
        w = np.empty((n_tok, top_k), np.float32)
        check(self._L.sh_moe_route(self._ctx, lg.ctypes.data, n_tok, n_expert, top_k, ids.ctypes.data,
                                   w.ctypes.data))
        return ids, w

    def moe_ffn(self, gate: ExpertView, up: ExpertView, down: ExpertView, logits, x,
                top_k: int) -> np.ndarray:
        """Routed MoE FFN (moe.rs:108-127) for ``x [n_tok][n_embd]`` from router
        ``logits [n_tok][n_expert]``; returns ``[n_tok][n_embd]``."""
        lg = np.ascontiguousarray(logits, dtype=np.float32)
        xv = np.ascontiguousarray(x, dtype=np.float32)
        if xv.ndim == 1:
            xv, lg = xv[None, :], lg.reshape(1, -1)
        n_tok = xv.shape[0]
        n_embd = gate.cols if gate.flags & FLAG_EXPERT_OUT_MAJOR else gate.rows
        if xv.ndim != 2 or xv.shape[1] != n_embd or lg.shape != (n_tok, gate.n_expert):
            raise ShapeError(SH_ERR_SHAPE, f"x {xv.shape} and logits {lg.shape} do not fit "
                                           f"{gate.n_expert} experts of width {n_embd}")
        out = np.empty_like(xv)
        g, u, d = gate._c(), up._c(), down._c()
        check(self._L.sh_moe_ffn(self._ctx, C.byref(g), C.byref(u), C.byref(d), lg.ctypes.data, n_tok,
                                 top_k, xv.ctypes.data, out.ctypes.data))
        return out

    def moe_layer(self, router: QuantTensor, gate: ExpertView, up: ExpertView, down: ExpertView,
                  gate_shexp: QuantTensor, up_shexp: QuantTensor, down_shexp: QuantTensor,
                  gate_inp_shexp: QuantTensor, x, top_k: int) -> np.ndarray:
        """MoeLayer::route + MoeLayer::combine (moe.rs:48-143) for ``x [n_tok][n_embd]``:
        router logits on bf16(x), the routed experts, and the shared expert
        added with its sigmoid gate; returns ``[n_tok][n_embd]``."""
        xv = np.ascontiguousarray(x, dtype=np.float32)
        if xv.ndim == 1:
            xv = xv[None, :]
        if xv.ndim != 2 or xv.shape[1] != router.cols:
            raise ShapeError(SH_ERR_SHAPE, f"x has shape {xv.shape}, want [n_tok][{router.cols}]")
        out = np.empty_like(xv)
        cs = [t._c() for t in (router, gate, up, down, gate_shexp, up_shexp, down_shexp, gate_inp_shexp)]
        check(self._L.sh_moe_layer(self._ctx, *(C.byref(c) for c in cs), xv.ctypes.data, xv.shape[0], top_k,
                                   out.ctypes.data))
        return out

    def matmul(self, w: QuantTensor, x, mode: int = MATMUL_BF16) -> np.ndarray:
        """Prefill matmul ``y[t] = W x[t]`` for ``x [m][cols]`` -> ``[m][rows]``:
        m gemvs (ops.rs:14-28) with bf16 or Q8-block activations (``mode``)."""
        xv = _f32_in(x)
        if xv.ndim == 1:
            xv = xv[None, :]
        if xv.ndim != 2 or xv.shape[1] != w.cols:
            raise ShapeError(SH_ERR_SHAPE, f"x has shape {xv.shape}, want [m][{w.cols}]")
        m = xv.shape[0]
        y = np.empty((m, w.rows), dtype=np.float32)
        wc = w._c()
        check(self._L.sh_matmul(self._ctx, C.byref(wc), xv.ctypes.data, m, y.ctypes.data, int(mode)))
        return y

    # ---- the trait's elementwise methods (backend.rs:38-50), in place ----
    def rms_norm(self, x: np.ndarray, w, eps: float) -> None:
        xv = _f32_out(x)
        wv = _f32_in(w)
        if wv.size != xv.size:
            raise ShapeError(SH_ERR_SHAPE, f"w has {wv.size} elements, x {xv.size}")
        check(self._L.sh_rms_norm(self._ctx, xv.ctypes.data, wv.ctypes.data, xv.size, float(eps)))

    def rope_neox(self, head: np.ndarray, cfg: RopeCfg) -> None:
        hv = _f32_out(head)
        c = cfg._c()
        check(self._L.sh_rope_neox(self._ctx, hv.ctypes.data, hv.size, C.byref(c)))

    def softmax(self, xs: np.ndarray) -> None:
        xv = _f32_out(xs)
        check(self._L.sh_softmax(self._ctx, xv.ctypes.data, xv.size))

    def l2_norm(self, head: np.ndarray, eps: float) -> None:
        hv = _f32_out(head)
        check(self._L.sh_l2_norm(self._ctx, hv.ctypes.data, hv.size, float(eps)))

    def add(self, a: np.ndarray, b) -> None:
        av = _f32_out(a)
        bv = _f32_in(b)
        if bv.size != av.size:
            raise ShapeError(SH_ERR_SHAPE, f"b has {bv.size} elements, a {av.size}")
        check(self._L.sh_add(self._ctx, av.ctypes.data, bv.ctypes.data, av.size))

    def ffn(self, gate: QuantTensor, up: QuantTensor, down: QuantTensor, post_norm, eps: float, x: np.ndarray) -> None:
        """The dense FFN half of a layer (qwen35.rs:112-129) in place on
        ``x [n_tok][n_embd]`` (float32, C-contiguous)."""
        xv = _f32_out(x)
        nv = _f32_in(post_norm)
        if nv.size != gate.cols:
            raise ShapeError(SH_ERR_SHAPE, f"post_norm has {nv.size} elements, n_embd is {gate.cols}")
        if gate.cols == 0 or xv.size == 0 or xv.size % gate.cols != 0:
            raise ShapeError(SH_ERR_SHAPE, f"x has {xv.size} elements, not a positive multiple of {gate.cols}")
        n_tok = xv.size // gate.cols
        g, u, d = gate._c(), up._c(), down._c()
        check(self._L.sh_ffn(self._ctx, C.byref(g), C.byref(u), C.byref(d), nv.ctypes.data, float(eps), n_tok,
                             xv.ctypes.data))

    def upload(self, name: str, quant: int, n_expert: int, rows: int, cols: int, data, row_pitch: int = 0) -> None:
        """Admits a packed tensor under `name` ahead of its first use
        (idempotent per name and shape); `row_pitch` bytes between row starts
        in `data` (0: packed)."""
        b = _bytes(data)
        check(self._L.sh_weight_upload(self._ctx, name_key(name), int(quant), n_expert, rows, cols, b.ctypes.data,
                                       row_pitch))

    def upload_gguf(self, f: GgufFile, index: int, name: str) -> None:
        """Admits tensor `index` of an open GGUF file into the resident store
        under `name` (the key later QuantTensor / ExpertView calls use)."""
        check(self._L.sh_upload_gguf_tensor(self._ctx, f._h, index, name_key(name)))

    def dequantize_row(self, quant: int, block, out: np.ndarray, flags: int = 0) -> None:
        """dequantize_row (crates/strata-gguf/src/dequant.rs:45-61) on the device."""
        b = _bytes(block)
        o = _f32_out(out)
        check(self._L.sh_dequantize_row(self._ctx, int(quant), flags, b.ctypes.data, b.nbytes,
                                        o.ctypes.data, o.size))


# ---- device-pointer entry points (pointers and a hipStream_t as ints) ------

def dequant_dev(quant: int, w_ptr: int, rows: int, cols: int, out_ptr: int, stream: int = 0,
                flags: int = 0) -> None:
    check(load_library().sh_dequant_dev(int(quant), flags, w_ptr, rows, cols, out_ptr, stream or None))


STREAM_READ_BLOCKS = 2048


def stream_read_dev(data_ptr: int, nbytes: int, out_ptr: int, stream: int = 0) -> None:
    """sh_stream_read_dev: a plain streaming read (the bandwidth ceiling);
    out_ptr receives STREAM_READ_BLOCKS uint32 XOR folds."""
    check(load_library().sh_stream_read_dev(data_ptr, nbytes, out_ptr, stream or None))


def gemv_dev(quant: int, w_ptr: int, rows: int, cols: int, x_ptr: int, y_ptr: int, batch: int = 1,
             stream: int = 0, flags: int = 0) -> None:
    check(load_library().sh_gemv_dev(int(quant), flags, w_ptr, rows, cols, x_ptr, y_ptr, batch,
                                     stream or None))


def gemv_workspace_bytes(quant: int, rows: int, cols: int, batch: int) -> int:
    v = C.c_uint64()
    check(load_library().sh_gemv_workspace_bytes(int(quant), rows, cols, batch, C.byref(v)))
    return v.value


def gemv_dev_ws(quant: int, w_ptr: int, rows: int, cols: int, x_ptr: int, y_ptr: int, batch: int,
                ws_ptr: int, ws_bytes: int, stream: int = 0, flags: int = 0) -> None:
    """sh_gemv_dev_ws: batches of 2..8 convert their activations once per
    call into the workspace."""
    check(load_library().sh_gemv_dev_ws(int(quant), flags, w_ptr, rows, cols, x_ptr, y_ptr, batch,
                                        ws_ptr or None, ws_bytes, stream or None))


def moe_workspace_bytes(n_tok: int, top_k: int, n_expert: int, n_embd: int, n_ff: int,
                        quant_gate_up: int, quant_down: int) -> int:
    v = C.c_uint64()
    check(load_library().sh_moe_workspace_bytes(n_tok, top_k, n_expert, n_embd, n_ff, int(quant_gate_up),
                                                int(quant_down), C.byref(v)))
    return v.value


def moe_ffn_dev(gate: tuple, up: tuple, down: tuple, n_expert: int, n_embd: int, n_ff: int,
                logits_ptr: int, n_tok: int, top_k: int, x_ptr: int, out_ptr: int, ws_ptr: int,
                ws_bytes: int, stream: int = 0) -> None:
    """gate/up/down: (quant, flags, device pointer)."""
    g, u, d = (_ExpertDevC(int(q), f, p) for q, f, p in (gate, up, down))
    check(load_library().sh_moe_ffn_dev(C.byref(g), C.byref(u), C.byref(d), n_expert, n_embd, n_ff,
                                        logits_ptr, n_tok, top_k, x_ptr, out_ptr, ws_ptr, ws_bytes,
                                        stream or None))


def moe_layer_workspace_bytes(n_tok: int, top_k: int, n_expert: int, n_embd: int, n_ff: int, n_ff_shexp: int,
                              quants) -> int:
    """quants: the 8 types (router, gate, up, down, gate_shexp, up_shexp, down_shexp, gate_inp_shexp)."""
    q = (C.c_uint32 * 8)(*[int(v) for v in quants])
    v = C.c_uint64()
    check(load_library().sh_moe_layer_workspace_bytes(n_tok, top_k, n_expert, n_embd, n_ff, n_ff_shexp, q,
                                                      C.byref(v)))
    return v.value


def moe_layer_dev(tensors, n_expert: int, n_embd: int, n_ff: int, n_ff_shexp: int, n_tok: int, top_k: int,
                  x_ptr: int, out_ptr: int, ws_ptr: int, ws_bytes: int, stream: int = 0) -> None:
    """tensors: 8 (quant, flags, device pointer) in sh_moe_layer_dev's order."""
    arr = (_ExpertDevC * 8)(*[_ExpertDevC(int(q), f, p) for q, f, p in tensors])
    check(load_library().sh_moe_layer_dev(arr, n_expert, n_embd, n_ff, n_ff_shexp, n_tok, top_k, x_ptr, out_ptr,
                                          ws_ptr, ws_bytes, stream or None))


def matmul_workspace_bytes(quant: int, rows: int, cols: int, m: int, mode: int = MATMUL_BF16) -> int:
    v = C.c_uint64()
    check(load_library().sh_matmul_workspace_bytes(int(quant), rows, cols, m, int(mode), C.byref(v)))
    return v.value


def matmul_dev(quant: int, w_ptr: int, rows: int, cols: int, x_ptr: int, m: int, y_ptr: int, mode: int,
               ws_ptr: int, ws_bytes: int, stream: int = 0, flags: int = 0) -> None:
    check(load_library().sh_matmul_dev(int(quant), flags, w_ptr, rows, cols, x_ptr, m, y_ptr, int(mode),
                                       ws_ptr, ws_bytes, stream or None))


def quantize_q8_dev(x_ptr: int, n: int, codes_ptr: int, scales_ptr: int, sums_ptr: int,
                    stream: int = 0) -> None:
    check(load_library().sh_quantize_q8_dev(x_ptr, n, codes_ptr, scales_ptr, sums_ptr, stream or None))


def quantize_q8k_dev(x_ptr: int, n: int, codes_ptr: int, scales_ptr: int, sums_ptr: int,
                     stream: int = 0) -> None:
    check(load_library().sh_quantize_q8k_dev(x_ptr, n, codes_ptr, scales_ptr, sums_ptr, stream or None))


def rms_norm_dev(x_ptr: int, w_ptr: int, out_ptr: int, rows: int, n: int, eps: float, stream: int = 0) -> None:
    check(load_library().sh_rms_norm_dev(x_ptr, w_ptr, out_ptr, rows, n, float(eps), stream or None))


def l2_norm_dev(x_ptr: int, rows: int, n: int, eps: float, stream: int = 0) -> None:
    check(load_library().sh_l2_norm_dev(x_ptr, rows, n, float(eps), stream or None))


def softmax_dev(x_ptr: int, rows: int, n: int, stream: int = 0) -> None:
    check(load_library().sh_softmax_dev(x_ptr, rows, n, stream or None))


def rope_neox_dev(x_ptr: int, rows: int, heads_per_pos: int, cfg: RopeCfg, stream: int = 0) -> None:
    c = cfg._c()
    check(load_library().sh_rope_neox_dev(x_ptr, rows, heads_per_pos, C.byref(c), stream or None))


def add_dev(a_ptr: int, b_ptr: int, n: int, stream: int = 0) -> None:
    check(load_library().sh_add_dev(a_ptr, b_ptr, n, stream or None))


def ffn_workspace_bytes(n_tok: int, n_embd: int, n_ff: int) -> int:
    v = C.c_uint64()
    check(load_library().sh_ffn_workspace_bytes(n_tok, n_embd, n_ff, C.byref(v)))
    return v.value


def ffn_dev(tensors, n_embd: int, n_ff: int, n_tok: int, x_ptr: int, norm_ptr: int, eps: float, out_ptr: int,
            ws_ptr: int, ws_bytes: int, stream: int = 0) -> None:
    """The dense FFN half of a layer (qwen35.rs:112-129); tensors: gate, up,
    down as (quant, flags, device pointer)."""
    arr = (_ExpertDevC * 3)(*[_ExpertDevC(int(q), f, p) for q, f, p in tensors])
    check(load_library().sh_ffn_dev(arr, n_embd, n_ff, n_tok, x_ptr, norm_ptr, float(eps), out_ptr, ws_ptr, ws_bytes,
                                    stream or None))


def ffn_dev_noalloc(tensors, n_embd: int, n_ff: int, n_tok: int, x_ptr: int, norm_ptr: int, eps: float, out_ptr: int,
                    stream: int = 0) -> None:
    """ffn_dev with the library's fixed device scratch (no allocation; at
    most 4 MiB of intermediates; overlapping calls on one GPU race)."""
    arr = (_ExpertDevC * 3)(*[_ExpertDevC(int(q), f, p) for q, f, p in tensors])
    check(load_library().sh_ffn_dev_noalloc(arr, n_embd, n_ff, n_tok, x_ptr, norm_ptr, float(eps), out_ptr,
                                            stream or None))
