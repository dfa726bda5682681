//! The C ABI of libstrata_hip, one for one with include/strata_hip.h:
//! status codes, type ids, flags, the plain-data structs and every entry
//! point. Pointers are the header's; ownership and lifetimes are documented
//! there. Nothing here is safe to call without reading that contract.
#![allow(non_camel_case_types, dead_code)]

use std::os::raw::{c_char, c_int, c_void};

pub const SH_ABI_VERSION: c_int = 1;

// ---- status codes
pub const SH_OK: c_int = 0;
pub const SH_ERR_INVALID_ARGUMENT: c_int = -1;
pub const SH_ERR_SHAPE: c_int = -2;
pub const SH_ERR_TRUNCATED: c_int = -3;
pub const SH_ERR_UNSUPPORTED_QUANT: c_int = -4;
pub const SH_ERR_UNSUPPORTED_SHAPE: c_int = -5;
pub const SH_ERR_NO_DEVICE: c_int = -6;
pub const SH_ERR_DEVICE: c_int = -7;
pub const SH_ERR_OUT_OF_MEMORY: c_int = -8;
pub const SH_ERR_FORMAT: c_int = -9;
pub const SH_ERR_IO: c_int = -10;
pub const SH_ERR_NOT_FOUND: c_int = -11;

// ---- quant type ids (strata-gguf's QuantType discriminants)
pub const SH_QUANT_F32: u32 = 0;
pub const SH_QUANT_F16: u32 = 1;
pub const SH_QUANT_Q8_0: u32 = 8;
pub const SH_QUANT_Q4_K: u32 = 12;
pub const SH_QUANT_Q5_K: u32 = 13;
pub const SH_QUANT_Q6_K: u32 = 14;
pub const SH_QUANT_IQ4_XS: u32 = 23;
pub const SH_QUANT_BF16: u32 = 30;

// ---- tensor flags
pub const SH_FLAG_Q6K_SIGNED_SCALES: u32 = 1;
pub const SH_FLAG_EXPERT_OUT_MAJOR: u32 = 2;
pub const SH_FLAG_IQ4XS_GGML: u32 = 4;

// ---- matmul modes
pub const SH_MATMUL_BF16: u32 = 0;
pub const SH_MATMUL_Q8: u32 = 1;
pub const SH_MATMUL_Q8K: u32 = 2;

/// Opaque: one device, its stream, pinned staging and resident weights.
#[repr(C)]
pub struct ShContext {
    _opaque: [u8; 0],
}

/// Opaque: a memory-mapped GGUF file.
#[repr(C)]
pub struct ShGguf {
    _opaque: [u8; 0],
}

/// Opaque: a GGUF model split over shards.
#[repr(C)]
pub struct ShGgufModel {
    _opaque: [u8; 0],
}

#[repr(C)]
#[derive(Debug, Clone, Copy)]
pub struct ShQuantTensor {
    pub key: u64,
    pub quant: u32,
    pub flags: u32,
    pub rows: u64,
    pub cols: u64,
    pub data: *const u8,
    pub nbytes: u64,
}

#[repr(C)]
#[derive(Debug, Clone, Copy)]
pub struct ShExpertView {
    pub key: u64,
    pub quant: u32,
    pub flags: u32,
    pub n_expert: u64,
    pub rows: u64,
    pub cols: u64,
    pub data: *const u8,
    pub nbytes: u64,
}

#[repr(C)]
#[derive(Debug, Clone, Copy)]
pub struct ShRopeCfg {
    pub pos: u64,
    pub n_rot: u64,
    pub head_dim: u64,
    pub freq_base: f64,
}

#[repr(C)]
#[derive(Debug, Clone, Copy)]
pub struct ShGgufTensorInfo {
    pub name: *const c_char,
    pub n_dims: u32,
    pub type_: u32,
    pub shape: [u64; 4],
    pub offset: u64,
    pub nbytes: u64,
}

#[repr(C)]
#[derive(Debug, Clone, Copy)]
pub struct ShExpertDev {
    pub quant: u32,
    pub flags: u32,
    pub data: *const c_void,
}

extern "C" {
    pub fn sh_abi_version() -> c_int;
    pub fn sh_last_error() -> *const c_char;
    pub fn sh_device_count(count: *mut c_int) -> c_int;
    pub fn sh_quant_geometry(quant: u32, block_size: *mut u32, type_size: *mut u32) -> c_int;
    pub fn sh_create(device: c_int, weight_budget_bytes: u64, out: *mut *mut ShContext) -> c_int;
    pub fn sh_destroy(ctx: *mut ShContext) -> c_int;
    pub fn sh_name(ctx: *const ShContext) -> *const c_char;
    pub fn sh_resident_bytes(ctx: *mut ShContext, bytes: *mut u64) -> c_int;
    pub fn sh_evict(ctx: *mut ShContext, key: u64) -> c_int;
    pub fn sh_gemv(ctx: *mut ShContext, w: *const ShQuantTensor, x: *const f32, x_len: u64, y: *mut f32,
        y_len: u64) -> c_int;
    pub fn sh_gemv_batch(ctx: *mut ShContext, w: *const ShQuantTensor, x: *const f32, y: *mut f32,
        batch: u32) -> c_int;
    pub fn sh_expert_gemv(ctx: *mut ShContext, w: *const ShExpertView, e: u64, x: *const f32, x_len: u64,
        y: *mut f32, y_len: u64) -> c_int;
    pub fn sh_weight_upload(ctx: *mut ShContext, key: u64, quant: u32, n_expert: u64, rows: u64, cols: u64,
        data: *const u8, src_row_pitch: u64) -> c_int;
    pub fn sh_rms_norm(ctx: *mut ShContext, x: *mut f32, w: *const f32, n: u64, eps: f64) -> c_int;
    pub fn sh_rope_neox(ctx: *mut ShContext, head: *mut f32, n: u64, cfg: *const ShRopeCfg) -> c_int;
    pub fn sh_softmax(ctx: *mut ShContext, xs: *mut f32, n: u64) -> c_int;
    pub fn sh_l2_norm(ctx: *mut ShContext, head: *mut f32, n: u64, eps: f64) -> c_int;
    pub fn sh_add(ctx: *mut ShContext, a: *mut f32, b: *const f32, n: u64) -> c_int;
    pub fn sh_dequantize_row(ctx: *mut ShContext, quant: u32, flags: u32, block: *const u8, nbytes: u64,
        out: *mut f32, n: u64) -> c_int;
    pub fn sh_moe_route(ctx: *mut ShContext, logits: *const f32, n_tok: u32, n_expert: u32, top_k: u32,
        ids: *mut i32, weights: *mut f32) -> c_int;
    pub fn sh_moe_ffn(ctx: *mut ShContext, gate: *const ShExpertView, up: *const ShExpertView,
        down: *const ShExpertView, logits: *const f32, n_tok: u32, top_k: u32, x: *const f32,
        out: *mut f32) -> c_int;
    pub fn sh_moe_layer(ctx: *mut ShContext, router: *const ShQuantTensor, gate: *const ShExpertView,
        up: *const ShExpertView, down: *const ShExpertView, gate_shexp: *const ShQuantTensor,
        up_shexp: *const ShQuantTensor, down_shexp: *const ShQuantTensor,
        gate_inp_shexp: *const ShQuantTensor, x: *const f32, n_tok: u32, top_k: u32, out: *mut f32) -> c_int;
    pub fn sh_matmul(ctx: *mut ShContext, w: *const ShQuantTensor, x: *const f32, m: u32, y: *mut f32,
        mode: u32) -> c_int;
    pub fn sh_matmul_workspace_bytes(quant: u32, rows: u64, cols: u64, m: u32, mode: u32,
        bytes: *mut u64) -> c_int;
    pub fn sh_matmul_dev(quant: u32, flags: u32, w: *const c_void, rows: u64, cols: u64, x: *const f32,
        m: u32, y: *mut f32, mode: u32, workspace: *mut c_void, workspace_bytes: u64,
        stream: *mut c_void) -> c_int;
    pub fn sh_quantize_q8_dev(x: *const f32, n: u64, codes: *mut i8, scales: *mut f32, code_sums: *mut f32,
        stream: *mut c_void) -> c_int;
    pub fn sh_quantize_q8k_dev(x: *const f32, n: u64, codes: *mut i8, scales: *mut f32, sub_sums: *mut i32,
        stream: *mut c_void) -> c_int;
    pub fn sh_moe_workspace_bytes(n_tok: u32, top_k: u32, n_expert: u64, n_embd: u64, n_ff: u64,
        quant_gate_up: u32, quant_down: u32, bytes: *mut u64) -> c_int;
    pub fn sh_moe_ffn_dev(gate: *const ShExpertDev, up: *const ShExpertDev, down: *const ShExpertDev,
        n_expert: u64, n_embd: u64, n_ff: u64, logits: *const f32, n_tok: u32, top_k: u32, x: *const f32,
        out: *mut f32, workspace: *mut c_void, workspace_bytes: u64, stream: *mut c_void) -> c_int;
    pub fn sh_moe_layer_workspace_bytes(n_tok: u32, top_k: u32, n_expert: u64, n_embd: u64, n_ff: u64,
        n_ff_shexp: u64, quants: *const u32, bytes: *mut u64) -> c_int;
    pub fn sh_moe_layer_dev(tensors: *const ShExpertDev, n_expert: u64, n_embd: u64, n_ff: u64,
        n_ff_shexp: u64, n_tok: u32, top_k: u32, x: *const f32, out: *mut f32, workspace: *mut c_void,
        workspace_bytes: u64, stream: *mut c_void) -> c_int;
    pub fn sh_dequant_dev(quant: u32, flags: u32, w: *const c_void, rows: u64, cols: u64, out: *mut f32,
        stream: *mut c_void) -> c_int;
    pub fn sh_gemv_dev(quant: u32, flags: u32, w: *const c_void, rows: u64, cols: u64, x: *const f32,
        y: *mut f32, batch: u32, stream: *mut c_void) -> c_int;
    pub fn sh_gemv_workspace_bytes(quant: u32, rows: u64, cols: u64, batch: u32, bytes: *mut u64) -> c_int;
    pub fn sh_gemv_dev_ws(quant: u32, flags: u32, w: *const c_void, rows: u64, cols: u64, x: *const f32,
        y: *mut f32, batch: u32, workspace: *mut c_void, workspace_bytes: u64, stream: *mut c_void) -> c_int;
    pub fn sh_stream_read_dev(data: *const c_void, nbytes: u64, out: *mut u32, stream: *mut c_void) -> c_int;
    pub fn sh_gguf_open(path: *const c_char, out: *mut *mut ShGguf) -> c_int;
    pub fn sh_gguf_close(gguf: *mut ShGguf) -> c_int;
    pub fn sh_gguf_header(gguf: *const ShGguf, version: *mut u32, n_tensors: *mut u64, n_kv: *mut u64,
        alignment: *mut u64, data_start: *mut u64, file_size: *mut u64) -> c_int;
    pub fn sh_gguf_tensor(gguf: *const ShGguf, index: u64, out: *mut ShGgufTensorInfo) -> c_int;
    pub fn sh_gguf_find(gguf: *const ShGguf, name: *const c_char, index: *mut u64) -> c_int;
    pub fn sh_gguf_tensor_data(gguf: *const ShGguf, index: u64, data: *mut *const u8,
        nbytes: *mut u64) -> c_int;
    pub fn sh_gguf_meta_type(gguf: *const ShGguf, key: *const c_char, type_: *mut u32, elem: *mut u32,
        count: *mut u64) -> c_int;
    pub fn sh_gguf_meta_int(gguf: *const ShGguf, key: *const c_char, value: *mut i64) -> c_int;
    pub fn sh_gguf_meta_float(gguf: *const ShGguf, key: *const c_char, value: *mut f64) -> c_int;
    pub fn sh_gguf_meta_str(gguf: *const ShGguf, key: *const c_char, s: *mut *const c_char,
        len: *mut u64) -> c_int;
    pub fn sh_gguf_model_open(any_shard: *const c_char, out: *mut *mut ShGgufModel) -> c_int;
    pub fn sh_gguf_model_close(model: *mut ShGgufModel) -> c_int;
    pub fn sh_gguf_model_shards(model: *const ShGgufModel, n_shards: *mut u64) -> c_int;
    pub fn sh_gguf_model_shard(model: *mut ShGgufModel, i: u64, shard: *mut *mut ShGguf) -> c_int;
    pub fn sh_gguf_model_find(model: *const ShGgufModel, name: *const c_char, shard: *mut u64,
        index: *mut u64) -> c_int;
    pub fn sh_upload_gguf_tensor(ctx: *mut ShContext, gguf: *const ShGguf, index: u64, key: u64) -> c_int;
    pub fn sh_ffn_workspace_bytes(n_tok: u32, n_embd: u64, n_ff: u64, bytes: *mut u64) -> c_int;
    pub fn sh_ffn(ctx: *mut ShContext, gate: *const ShQuantTensor, up: *const ShQuantTensor,
        down: *const ShQuantTensor, post_norm: *const f32, eps: f64, n_tok: u32, x: *mut f32) -> c_int;
    pub fn sh_ffn_dev(tensors: *const ShExpertDev, n_embd: u64, n_ff: u64, n_tok: u32, x: *const f32,
        post_norm: *const f32, eps: f64, out: *mut f32, workspace: *mut c_void, workspace_bytes: u64,
        stream: *mut c_void) -> c_int;
    pub fn sh_ffn_dev_noalloc(tensors: *const ShExpertDev, n_embd: u64, n_ff: u64, n_tok: u32, x: *const f32,
        post_norm: *const f32, eps: f64, out: *mut f32, stream: *mut c_void) -> c_int;
    pub fn sh_rms_norm_dev(x: *const f32, w: *const f32, out: *mut f32, rows: u64, n: u64, eps: f64,
        stream: *mut c_void) -> c_int;
    pub fn sh_l2_norm_dev(x: *mut f32, rows: u64, n: u64, eps: f64, stream: *mut c_void) -> c_int;
    pub fn sh_softmax_dev(x: *mut f32, rows: u64, n: u64, stream: *mut c_void) -> c_int;
    pub fn sh_rope_neox_dev(x: *mut f32, rows: u64, heads_per_pos: u64, cfg: *const ShRopeCfg,
        stream: *mut c_void) -> c_int;
    pub fn sh_add_dev(a: *mut f32, b: *const f32, n: u64, stream: *mut c_void) -> c_int;
}
