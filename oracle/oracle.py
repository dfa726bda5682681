"""ctypes binding of the CPU oracle (liboracle.so, built by oracle/Makefile).

TEST INFRASTRUCTURE ONLY: imported by tests/, the smoke check and the CPU
baseline leg of bench.py, as the checker or the timed CPU reference. The
product library never loads it.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

F32, F16, Q8_0, Q4_K, Q5_K, Q6_K, IQ4_XS, BF16 = 0, 1, 8, 12, 13, 14, 23, 30
# the two readings of formats that have them (the `scale_mode` arguments):
# Q6_K sub-block scales as u8 (the reference) or i8 (ggml); IQ4_XS code
# bytes the first 16 for every sub-block (the reference) or 16 per sub-block
# (ggml)
SCALE_U8, SCALE_I8 = 0, 1
IQ4XS_REFERENCE, IQ4XS_GGML = 0, 1
OK, TRUNCATED, UNSUPPORTED = 0, -1, -2

_lib = None


def build() -> None:
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is not built (run `make -C oracle`)")
        L = C.CDLL(LIB_PATH)
        u8p, f32p, i64p = C.c_void_p, C.c_void_p, C.c_void_p
        L.sho_f16_to_f32.argtypes = [C.c_uint16]
        L.sho_f16_to_f32.restype = C.c_float
        L.sho_f32_to_f16.argtypes = [C.c_float]
        L.sho_f32_to_f16.restype = C.c_uint16
        L.sho_bf16_round.argtypes = [C.c_float]
        L.sho_bf16_round.restype = C.c_float
        for fn in ("sho_block_size", "sho_type_size"):
            getattr(L, fn).argtypes = [C.c_uint32]
            getattr(L, fn).restype = C.c_int64
        L.sho_byte_size.argtypes = [C.c_uint32, C.c_int64]
        L.sho_byte_size.restype = C.c_int64
        L.sho_get_scale_min_k4.argtypes = [C.c_int, u8p, C.POINTER(C.c_uint8), C.POINTER(C.c_uint8)]
        L.sho_dequantize_row.argtypes = [C.c_uint32, u8p, C.c_size_t, f32p, C.c_size_t]
        L.sho_dequantize_row_q6k_mode.argtypes = [u8p, C.c_size_t, f32p, C.c_size_t, C.c_int]
        L.sho_dequantize_row_mode.argtypes = [C.c_uint32, u8p, C.c_size_t, f32p, C.c_size_t, C.c_int]
        L.sho_gemv_mode.argtypes = [C.c_uint32, C.c_int64, C.c_int64, u8p, C.c_size_t, f32p, f32p, C.c_int]
        L.sho_gemv.argtypes = [C.c_uint32, C.c_int64, C.c_int64, u8p, C.c_size_t, f32p, f32p]
        L.sho_gemv_q6k_mode.argtypes = [C.c_int64, C.c_int64, u8p, C.c_size_t, f32p, f32p, C.c_int]
        L.sho_gemv_threads.argtypes = [C.c_uint32, C.c_int64, C.c_int64, u8p, C.c_size_t, f32p, f32p,
                                       C.c_int]
        L.sho_expert_gemv.argtypes = [C.c_uint32, C.c_int64, C.c_int64, C.c_int64, u8p, C.c_size_t,
                                      C.c_int64, f32p, f32p]
        L.sho_expert_gemv_mode.argtypes = [C.c_uint32, C.c_int64, C.c_int64, C.c_int64, u8p, C.c_size_t,
                                           C.c_int64, f32p, f32p, C.c_int]
        ip = C.POINTER(C.c_int)
        L.sho_moe_routed_m.argtypes = [C.c_uint32, C.c_uint32, C.c_uint32, C.c_int64, C.c_int64,
                                       C.c_int64, u8p, C.c_size_t, u8p, C.c_size_t, u8p, C.c_size_t,
                                       i64p, f32p, C.c_int64, f32p, f32p, C.c_int, ip]
        L.sho_moe_layer_m.argtypes = [C.POINTER(C.c_uint32), C.POINTER(C.c_void_p), C.POINTER(C.c_size_t),
                                      C.c_int64, C.c_int64, C.c_int64, C.c_int64, C.c_int64, f32p, f32p, C.c_int,
                                      ip]
        L.sho_matmul_mode.argtypes = [C.c_uint32, C.c_int64, C.c_int64, u8p, C.c_size_t, f32p, C.c_int64,
                                      f32p, C.c_int, C.c_int]
        L.sho_silu.argtypes = [C.c_float]
        L.sho_silu.restype = C.c_float
        L.sho_moe_route.argtypes = [f32p, C.c_int64, C.c_int64, i64p, f32p]
        L.sho_moe_routed.argtypes = [C.c_uint32, C.c_uint32, C.c_uint32, C.c_int64, C.c_int64,
                                     C.c_int64, u8p, C.c_size_t, u8p, C.c_size_t, u8p, C.c_size_t,
                                     i64p, f32p, C.c_int64, f32p, f32p]
        L.sho_moe_routed_o.argtypes = [C.c_uint32, C.c_uint32, C.c_uint32, C.c_int64, C.c_int64,
                                       C.c_int64, u8p, C.c_size_t, u8p, C.c_size_t, u8p, C.c_size_t,
                                       i64p, f32p, C.c_int64, f32p, f32p, C.c_int]
        L.sho_moe_layer_o.argtypes = [C.POINTER(C.c_uint32), C.POINTER(C.c_void_p), C.POINTER(C.c_size_t),
                                      C.c_int64, C.c_int64, C.c_int64, C.c_int64, C.c_int64, f32p, f32p, C.c_int]
        L.sho_sigmoid.argtypes = [C.c_float]
        L.sho_sigmoid.restype = C.c_float
        L.sho_moe_layer.argtypes = [C.POINTER(C.c_uint32), C.POINTER(C.c_void_p), C.POINTER(C.c_size_t),
                                    C.c_int64, C.c_int64, C.c_int64, C.c_int64, C.c_int64, f32p, f32p]
        L.sho_matmul.argtypes = [C.c_uint32, C.c_int64, C.c_int64, u8p, C.c_size_t, f32p, C.c_int64, f32p,
                                 C.c_int]
        L.sho_quantize_q8.argtypes = [f32p, C.c_size_t, u8p, f32p, f32p]
        L.sho_quantize_q8k.argtypes = [f32p, C.c_size_t, u8p, f32p, C.c_void_p]
        L.sho_rms_norm.argtypes = [f32p, f32p, C.c_size_t, C.c_double, f32p]
        L.sho_rms_norm.restype = None
        L.sho_l2_norm.argtypes = [f32p, C.c_size_t, C.c_double]
        L.sho_l2_norm.restype = None
        L.sho_softmax.argtypes = [f32p, C.c_size_t]
        L.sho_softmax.restype = None
        L.sho_rope_neox.argtypes = [f32p, C.c_size_t, C.c_uint64, C.c_size_t, C.c_size_t, C.c_double]
        L.sho_rope_neox.restype = None
        L.sho_add.argtypes = [f32p, f32p, C.c_size_t]
        L.sho_add.restype = None
        L.sho_dense_ffn.argtypes = [C.POINTER(C.c_uint32), C.POINTER(C.c_void_p), C.POINTER(C.c_size_t),
                                    C.c_int64, C.c_int64, f32p, f32p, C.c_double, f32p]
        _lib = L
    return _lib


def _ptr(a: np.ndarray) -> int:
    return a.ctypes.data


def _u8(a) -> np.ndarray:
    return np.ascontiguousarray(np.frombuffer(bytes(a), np.uint8) if isinstance(a, (bytes, bytearray))
                                else a, dtype=np.uint8)


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


class OracleError(RuntimeError):
    def __init__(self, rc: int, what: str):
        name = {TRUNCATED: "truncated", UNSUPPORTED: "unsupported quant"}.get(rc, str(rc))
        super().__init__(f"{what}: {name}")
        self.rc = rc


def _check(rc: int, what: str) -> None:
    if rc != OK:
        raise OracleError(rc, what)


def f16_to_f32(h: int) -> float:
    return lib().sho_f16_to_f32(h)


def f32_to_f16(f: float) -> int:
    return lib().sho_f32_to_f16(f)


def block_size(q: int) -> int:
    return lib().sho_block_size(q)


def type_size(q: int) -> int:
    return lib().sho_type_size(q)


def byte_size(q: int, n: int) -> int:
    return lib().sho_byte_size(q, n)


def get_scale_min_k4(j: int, scales) -> tuple[int, int]:
    s = _u8(scales)
    sc, m = C.c_uint8(), C.c_uint8()
    lib().sho_get_scale_min_k4(j, _ptr(s), C.byref(sc), C.byref(m))
    return sc.value, m.value


def dequantize_row(quant: int, block, n: int, scale_mode: int = SCALE_U8) -> np.ndarray:
    b = _u8(block)
    out = np.zeros(n, dtype=np.float32)
    if scale_mode != 0:
        rc = lib().sho_dequantize_row_mode(quant, _ptr(b), b.nbytes, _ptr(out), n, scale_mode)
    else:
        rc = lib().sho_dequantize_row(quant, _ptr(b), b.nbytes, _ptr(out), n)
    _check(rc, "dequantize_row")
    return out


def dequantize(quant: int, data, rows: int, cols: int, scale_mode: int = SCALE_U8) -> np.ndarray:
    """All rows of a ``rows x cols`` matrix, row by row through dequantize_row."""
    b = _u8(data)
    rb = byte_size(quant, cols)
    out = np.empty((rows, cols), dtype=np.float32)
    for r in range(rows):
        out[r] = dequantize_row(quant, b[r * rb:(r + 1) * rb], cols, scale_mode)
    return out


def gemv(quant: int, rows: int, cols: int, data, x, scale_mode: int = SCALE_U8,
         threads: int = 1) -> np.ndarray:
    b, xv = _u8(data), _f32(x)
    assert xv.size == cols
    y = np.empty(rows, dtype=np.float32)
    if scale_mode != 0:
        rc = lib().sho_gemv_mode(quant, rows, cols, _ptr(b), b.nbytes, _ptr(xv), _ptr(y), scale_mode)
    elif threads > 1:
        rc = lib().sho_gemv_threads(quant, rows, cols, _ptr(b), b.nbytes, _ptr(xv), _ptr(y), threads)
    else:
        rc = lib().sho_gemv(quant, rows, cols, _ptr(b), b.nbytes, _ptr(xv), _ptr(y))
    _check(rc, "gemv")
    return y


def expert_gemv(quant: int, n_expert: int, rows: int, cols: int, data, e: int, x,
                mode: int = 0) -> np.ndarray:
    """``mode``: the reading of a two-reading format (Q6_K scales, IQ4_XS
    code bytes), as ``dequantize``'s."""
    b, xv = _u8(data), _f32(x)
    assert xv.size == rows
    y = np.empty(cols, dtype=np.float32)
    _check(lib().sho_expert_gemv_mode(quant, n_expert, rows, cols, _ptr(b), b.nbytes, e, _ptr(xv), _ptr(y),
                                      mode), "expert_gemv")
    return y


def silu(x: float) -> float:
    return lib().sho_silu(x)


def moe_route(logits, top_k: int) -> tuple[np.ndarray, np.ndarray]:
    lg = _f32(logits)
    ids = np.zeros(top_k, dtype=np.int64)
    w = np.zeros(top_k, dtype=np.float32)
    k = lib().sho_moe_route(_ptr(lg), lg.size, top_k, _ptr(ids), _ptr(w))
    return ids[:k], w[:k]


def moe_routed(gate_q: int, up_q: int, down_q: int, n_expert: int, n_embd: int, n_ff: int,
               gate, up, down, ids, weights, x, out_major: bool = False, modes=(0, 0, 0)) -> np.ndarray:
    """The routed experts of one token; ``out_major``: the stacks are
    llama.cpp's [n_expert][out][in] (each expert an ops::gemv of its slice)
    instead of the reference's [n_expert][in][out]; ``modes``: the readings
    of gate, up and down."""
    g, u, d = _u8(gate), _u8(up), _u8(down)
    idv = np.ascontiguousarray(ids, dtype=np.int64)
    wv, xv = _f32(weights), _f32(x)
    out = np.empty(n_embd, dtype=np.float32)
    md = (C.c_int * 3)(*[int(v) for v in modes])
    _check(lib().sho_moe_routed_m(gate_q, up_q, down_q, n_expert, n_embd, n_ff, _ptr(g), g.nbytes,
                                  _ptr(u), u.nbytes, _ptr(d), d.nbytes, _ptr(idv), _ptr(wv), idv.size,
                                  _ptr(xv), _ptr(out), int(out_major), md), "moe_routed")
    return out


def sigmoid(x: float) -> float:
    return lib().sho_sigmoid(x)


# ---- the trait's elementwise methods (ops.rs:46-165), row by row -----------

def _rows(x, n: int | None = None) -> np.ndarray:
    v = np.array(x, dtype=np.float32, copy=True)
    return v.reshape(-1, n if n is not None else v.shape[-1])


def rms_norm(x, w, eps: float) -> np.ndarray:
    """ops::rms_norm on each row of x ([rows][n]) with the weights w [n]."""
    v = _rows(x)
    wv = _f32(w)
    assert wv.size == v.shape[1]
    for r in range(v.shape[0]):
        row = v[r]
        lib().sho_rms_norm(_ptr(row), _ptr(wv), row.size, float(eps),
                           _ptr(row))
    return v.reshape(np.shape(x))


def l2_norm(x, eps: float) -> np.ndarray:
    """ops::l2_norm on each row (head) of x."""
    v = _rows(x)
    for r in range(v.shape[0]):
        lib().sho_l2_norm(_ptr(v[r]), v.shape[1], float(eps))
    return v.reshape(np.shape(x))


def softmax(x) -> np.ndarray:
    """ops::softmax on each row of x."""
    v = _rows(x)
    for r in range(v.shape[0]):
        lib().sho_softmax(_ptr(v[r]), v.shape[1])
    return v.reshape(np.shape(x))


def rope_neox(x, pos: int, n_rot: int, head_dim: int, freq_base: float) -> np.ndarray:
    """ops::rope_neox on each head_dim-long head of x (the whole buffer is
    a run of heads, as the attention code passes them one at a time)."""
    v = _rows(x, head_dim)
    for r in range(v.shape[0]):
        lib().sho_rope_neox(_ptr(v[r]), head_dim, int(pos), int(n_rot), int(head_dim),
                            float(freq_base))
    return v.reshape(np.shape(x))


def add(a, b) -> np.ndarray:
    """ops::add_into: a + b in f32."""
    av = np.array(a, dtype=np.float32, copy=True).reshape(-1)
    bv = _f32(b).reshape(-1)
    assert av.size == bv.size
    lib().sho_add(_ptr(av), _ptr(bv), av.size)
    return av.reshape(np.shape(a))


def moe_layer(quants, tensors, n_expert: int, n_embd: int, n_ff: int, n_ff_sh: int, x, top_k: int,
              out_major: bool = False, modes=(0,) * 8) -> np.ndarray:
    """The whole MoE layer for one token (moe.rs:48-143): router matvec on
    bf16(x), route, routed experts, then the shared expert added with its
    sigmoid gate. quants / tensors / modes (readings): router, gate, up,
    down, gate_sh, up_sh, down_sh, gate_inp."""
    bufs = [_u8(t) for t in tensors]
    xv = _f32(x)
    assert xv.size == n_embd and len(bufs) == 8
    out = np.empty(n_embd, dtype=np.float32)
    q = (C.c_uint32 * 8)(*[int(v) for v in quants])
    tp = (C.c_void_p * 8)(*[_ptr(b) for b in bufs])
    nb = (C.c_size_t * 8)(*[b.nbytes for b in bufs])
    md = (C.c_int * 8)(*[int(v) for v in modes])
    _check(lib().sho_moe_layer_m(q, tp, nb, n_expert, n_embd, n_ff, n_ff_sh, top_k, _ptr(xv), _ptr(out),
                                 int(out_major), md), "moe_layer")
    return out


def matmul(quant: int, rows: int, cols: int, data, x, threads: int = 1, mode: int = 0) -> np.ndarray:
    """y[t] = gemv(W, x[t]) for every row t of x ([m][cols] -> [m][rows])
    under reading ``mode``."""
    b, xv = _u8(data), _f32(x)
    m = xv.size // cols
    assert xv.size == m * cols
    y = np.empty((m, rows), dtype=np.float32)
    _check(lib().sho_matmul_mode(quant, rows, cols, _ptr(b), b.nbytes, _ptr(xv), m, _ptr(y), threads, mode),
           "matmul")
    return y


def quantize_q8(x) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """(codes int8 [n], scales f32 [n/32], scale * code sums f32 [n/32])."""
    xv = _f32(x).reshape(-1)
    q = np.empty(xv.size, dtype=np.int8)
    s = np.empty(xv.size // 32, dtype=np.float32)
    u = np.empty(xv.size // 32, dtype=np.float32)
    _check(lib().sho_quantize_q8(_ptr(xv), xv.size, _ptr(q), _ptr(s), _ptr(u)), "quantize_q8")
    return q, s, u


def dequantize_q8_activations(x) -> np.ndarray:
    """x rounded through Q8 blocks: scale * code per element (f32 product)."""
    xv = _f32(x)
    q, s, _ = quantize_q8(xv)
    return (np.repeat(s, 32) * q.astype(np.float32)).astype(np.float32).reshape(xv.shape)


def quantize_q8k(x) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """(codes int8 [n], scales f32 [n/256], code sums int32 [n/32]): blocks of
    256 with one scale, the q8 matmul mode's rounding for K-quant weights."""
    xv = _f32(x).reshape(-1)
    q = np.empty(xv.size, dtype=np.int8)
    s = np.empty(xv.size // 256, dtype=np.float32)
    u = np.empty(xv.size // 32, dtype=np.int32)
    _check(lib().sho_quantize_q8k(_ptr(xv), xv.size, _ptr(q), _ptr(s), _ptr(u)), "quantize_q8k")
    return q, s, u


def dequantize_q8k_activations(x) -> np.ndarray:
    """x rounded through 256-element Q8 blocks: scale * code per element (f32 product)."""
    xv = _f32(x)
    q, s, _ = quantize_q8k(xv)
    return (np.repeat(s, 256) * q.astype(np.float32)).astype(np.float32).reshape(xv.shape)


def q8_activations_for(mode: int, x) -> np.ndarray:
    """The activation rounding of an int8 matmul mode: Q8 blocks of 32
    elements (mode 1, every weight type) or of 256 elements (mode 2, one
    scale per K-quant super-block)."""
    return dequantize_q8k_activations(x) if mode == 2 else dequantize_q8_activations(x)


def bf16_round_array(a) -> np.ndarray:
    """Round f32 to bf16 (nearest even) and back, elementwise (matches sho_bf16_round for finite values)."""
    u = _f32(a).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000).astype(np.uint32)
    return r.view(np.float32).reshape(np.shape(a))


def dense_ffn(quants, tensors, n_embd: int, n_ff: int, x, post_norm, eps: float) -> np.ndarray:
    """The dense FFN half of a layer for each row of x (qwen35.rs:112-129);
    quants / tensors: gate, up, down."""
    bufs = [_u8(t) for t in tensors]
    q = (C.c_uint32 * 3)(*[int(v) for v in quants])
    ptrs = (C.c_void_p * 3)(*[b.ctypes.data for b in bufs])
    nbs = (C.c_size_t * 3)(*[b.nbytes for b in bufs])
    xv = np.array(x, dtype=np.float32, copy=True).reshape(-1, n_embd)
    nw = _f32(post_norm)
    out = np.empty_like(xv)
    for r in range(xv.shape[0]):
        row = np.ascontiguousarray(xv[r])
        o = np.empty(n_embd, np.float32)
        _check(lib().sho_dense_ffn(q, ptrs, nbs, n_embd, n_ff, _ptr(row), _ptr(nw), float(eps), _ptr(o)), "dense_ffn")
        out[r] = o
    return out.reshape(np.shape(x))
