//! # strata-backend-hip
//!
//! The HIP implementation of [`strata_core::backend::ComputeBackend`] for AMD
//! Instinct MI355X (gfx950). GGUF weights stay packed in device memory in
//! their block layout, admitted on first use under a byte budget and evicted
//! least-recently-used; the hand-written kernels of libstrata_hip
//! (`include/strata_hip.h`) dequantize in registers. Besides the trait's
//! methods the backend offers the batched entry points the trait has no slot
//! for: several tokens against one weight read, the fused MoE FFN and layer,
//! the dense FFN half of a layer, and the prefill matmul.
//!
//! Types or shapes the device path does not take run on the CPU backend
//! instead, as the wgpu backend does for what it does not accelerate
//! (crates/strata-backend-wgpu/src/gpu.rs:306-325). Device failures are
//! returned as `Error::Backend`, as the wgpu backend propagates its own
//! (gpu.rs:331-365); they are never retried on the CPU.

pub mod ffi;

use std::ffi::{CStr, CString};
use std::fmt;
use std::os::raw::c_int;
use std::path::Path;

use strata_backend_cpu::CpuBackend;
use strata_core::backend::{ComputeBackend, QuantTensor, RopeCfg};
use strata_core::error::{Error, Result};
use strata_core::weights::ExpertView;
use strata_gguf::quant::QuantType;

/// The 64-bit FNV-1a hash of a tensor name: the key under which the library
/// keeps a tensor resident.
pub fn name_key(name: &str) -> u64 {
    name.bytes()
        .fold(0xcbf2_9ce4_8422_2325_u64, |h, b| (h ^ u64::from(b)).wrapping_mul(0x0100_0000_01b3))
}

/// Device, budget, and the readings of the formats that have two.
#[derive(Debug, Clone, Copy, Default)]
pub struct HipOptions {
    /// HIP device ordinal.
    pub device: i32,
    /// Resident-weight budget in bytes; 0 takes the library's default (4 GiB).
    pub weight_budget: u64,
    /// Q6_K sub-block scales as ggml's int8 (strata-gguf reads them as u8,
    /// crates/strata-gguf/src/dequant.rs:211,224-227).
    pub q6k_signed_scales: bool,
    /// IQ4_XS code bytes in ggml's layout (strata-gguf reads the first 16
    /// for every sub-block, dequant.rs:189-206).
    pub iq4xs_ggml: bool,
    /// Expert stacks in llama.cpp's `[n_expert][out][in]` orientation:
    /// `ExpertView::rows` is then the output width and `cols` the input.
    pub expert_out_major: bool,
}

impl HipOptions {
    /// The flags passed with a 2-D tensor of type `q`.
    pub fn tensor_flags(&self, q: QuantType) -> u32 {
        match q {
            QuantType::Q6K if self.q6k_signed_scales => ffi::SH_FLAG_Q6K_SIGNED_SCALES,
            QuantType::Iq4Xs if self.iq4xs_ggml => ffi::SH_FLAG_IQ4XS_GGML,
            _ => 0,
        }
    }

    /// The flags passed with an expert stack of type `q`.
    pub fn expert_flags(&self, q: QuantType) -> u32 {
        let orientation = if self.expert_out_major { ffi::SH_FLAG_EXPERT_OUT_MAJOR } else { 0 };
        self.tensor_flags(q) | orientation
    }
}

/// Types the matvec (and dequant) kernels read.
fn gemv_quant(q: QuantType) -> bool {
    matches!(
        q,
        QuantType::Q8_0
            | QuantType::Q4K
            | QuantType::Q5K
            | QuantType::Q6K
            | QuantType::Iq4Xs
            | QuantType::F32
            | QuantType::F16
            | QuantType::Bf16
    )
}

/// Types the expert, MoE and matmul kernels read.
fn device_quant(q: QuantType) -> bool {
    matches!(q, QuantType::Q8_0 | QuantType::Q4K | QuantType::Q5K | QuantType::Q6K | QuantType::Iq4Xs)
}

fn last_error() -> String {
    // SAFETY: sh_last_error returns null or a NUL-terminated thread-local string.
    let p = unsafe { ffi::sh_last_error() };
    if p.is_null() {
        String::new()
    } else {
        // SAFETY: non-null, NUL-terminated, valid until the next call on this thread.
        unsafe { CStr::from_ptr(p) }.to_string_lossy().into_owned()
    }
}

/// A status code as the engine's error (crates/strata-core/src/error.rs:31-32).
fn check(rc: c_int) -> Result<()> {
    if rc == ffi::SH_OK {
        Ok(())
    } else {
        Err(Error::Backend { message: format!("hip ({rc}): {}", last_error()) })
    }
}

/// Where a trait call goes after the library returned `rc`.
#[derive(Debug, Clone, Copy, PartialEq, Eq)]
enum Route {
    /// The device computed the result.
    Done,
    /// The CPU backend computes it (or reports the caller's error its way).
    Cpu,
}

/// The status of a trait call, mapped as the reference's backends behave:
/// - `SH_OK`: the device result stands;
/// - `SH_ERR_UNSUPPORTED_QUANT`, `SH_ERR_UNSUPPORTED_SHAPE`: a type or shape
///   the kernels do not take; the CPU backend computes it, as the wgpu
///   backend does for what it does not accelerate (gpu.rs:306-325);
/// - `SH_ERR_SHAPE`, `SH_ERR_TRUNCATED`: the caller's arguments are wrong;
///   the CPU body reports them the reference's way (the length asserts of
///   crates/strata-core/src/ops.rs:15-17, `Error::Truncated` of
///   crates/strata-gguf/src/dequant.rs:50-55), so the caller sees the same
///   failure as with the CPU backend;
/// - anything else (`SH_ERR_DEVICE`, `SH_ERR_OUT_OF_MEMORY`,
///   `SH_ERR_INVALID_ARGUMENT`, ...): `Error::Backend`, as the wgpu backend
///   propagates its device errors (gpu.rs:331-365); no CPU retry.
fn route(rc: c_int, what: &str) -> Result<Route> {
    match rc {
        ffi::SH_OK => Ok(Route::Done),
        ffi::SH_ERR_UNSUPPORTED_QUANT | ffi::SH_ERR_UNSUPPORTED_SHAPE | ffi::SH_ERR_SHAPE | ffi::SH_ERR_TRUNCATED => {
            tracing::debug!("{what} ({rc}): {}; on the CPU", last_error());
            Ok(Route::Cpu)
        }
        _ => Err(Error::Backend { message: format!("hip {what} ({rc}): {}", last_error()) }),
    }
}

fn len_u32(n: usize, what: &str) -> Result<u32> {
    u32::try_from(n).map_err(|_| Error::Backend { message: format!("{what} {n} does not fit the ABI") })
}

/// One HIP device with its resident weights.
pub struct HipBackend {
    ctx: *mut ffi::ShContext,
    opts: HipOptions,
    cpu: CpuBackend,
}

// SAFETY: the library serialises every call on a context with its own lock
// (include/strata_hip.h, "Conventions"), so the handle may be shared and sent
// between threads; it is destroyed exactly once, in Drop.
unsafe impl Send for HipBackend {}
unsafe impl Sync for HipBackend {}

impl fmt::Debug for HipBackend {
    fn fmt(&self, f: &mut fmt::Formatter<'_>) -> fmt::Result {
        f.debug_struct("HipBackend").field("opts", &self.opts).finish_non_exhaustive()
    }
}

impl Drop for HipBackend {
    fn drop(&mut self) {
        // SAFETY: ctx came from sh_create and is not used after this.
        unsafe {
            ffi::sh_destroy(self.ctx);
        }
    }
}

impl HipBackend {
    /// Opens the device; `SH_ERR_NO_DEVICE` (no usable GPU) comes back as an
    /// error, and the caller keeps the CPU backend.
    pub fn probe(opts: HipOptions) -> Result<Self> {
        let mut ctx = std::ptr::null_mut();
        // SAFETY: `ctx` is a valid out-pointer.
        check(unsafe { ffi::sh_create(opts.device, opts.weight_budget, &mut ctx) })?;
        Ok(Self { ctx, opts, cpu: CpuBackend::new() })
    }

    /// Device 0 with a weight budget and the reference's readings.
    pub fn probe_with_budget(max_weight_bytes: u64) -> Result<Self> {
        Self::probe(HipOptions { weight_budget: max_weight_bytes, ..HipOptions::default() })
    }

    pub fn options(&self) -> HipOptions {
        self.opts
    }

    fn tensor(&self, w: &QuantTensor<'_>) -> ffi::ShQuantTensor {
        ffi::ShQuantTensor {
            key: name_key(w.name),
            quant: w.quant as u32,
            flags: self.opts.tensor_flags(w.quant),
            rows: w.rows as u64,
            cols: w.cols as u64,
            data: w.data.as_ptr(),
            nbytes: w.data.len() as u64,
        }
    }

    fn view(&self, w: &ExpertView<'_>) -> ffi::ShExpertView {
        ffi::ShExpertView {
            key: name_key(w.name),
            quant: w.quant as u32,
            flags: self.opts.expert_flags(w.quant),
            n_expert: w.n_expert as u64,
            rows: w.rows as u64,
            cols: w.cols as u64,
            data: w.data.as_ptr(),
            nbytes: w.data.len() as u64,
        }
    }

    /// Bytes of weights resident on the device.
    pub fn resident_bytes(&self) -> Result<u64> {
        let mut b = 0u64;
        // SAFETY: valid context and out-pointer.
        check(unsafe { ffi::sh_resident_bytes(self.ctx, &mut b) })?;
        Ok(b)
    }

    /// Drops one resident tensor (no-op when absent).
    pub fn evict(&self, name: &str) -> Result<()> {
        // SAFETY: valid context.
        check(unsafe { ffi::sh_evict(self.ctx, name_key(name)) })
    }

    /// Admits the named tensors of a GGUF file before the first token, packed,
    /// through pinned staging (names missing from the file are skipped).
    pub fn preload(&self, path: &Path, names: &[&str]) -> Result<()> {
        let p = CString::new(path.as_os_str().as_encoded_bytes())
            .map_err(|_| Error::Backend { message: "path holds a NUL byte".to_string() })?;
        let mut g = std::ptr::null_mut();
        // SAFETY: NUL-terminated path, valid out-pointer.
        check(unsafe { ffi::sh_gguf_open(p.as_ptr(), &mut g) })?;
        let mut result = Ok(());
        for name in names {
            let Ok(n) = CString::new(*name) else { continue };
            let mut index = 0u64;
            // SAFETY: g is open; NUL-terminated name; valid out-pointer.
            if unsafe { ffi::sh_gguf_find(g, n.as_ptr(), &mut index) } == ffi::SH_OK {
                // SAFETY: valid context, open file, an index the file holds.
                result = check(unsafe { ffi::sh_upload_gguf_tensor(self.ctx, g, index, name_key(name)) });
                if result.is_err() {
                    break;
                }
            }
        }
        // SAFETY: g came from sh_gguf_open.
        unsafe {
            ffi::sh_gguf_close(g);
        }
        result
    }

    /// `batch` (1..8) gemvs against one weight read: x is `[batch][cols]`,
    /// y `[batch][rows]`.
    pub fn gemv_batch(&self, w: &QuantTensor<'_>, x: &[f32], batch: usize, y: &mut [f32]) -> Result<()> {
        if x.len() != batch * w.cols || y.len() != batch * w.rows {
            return Err(Error::Backend { message: format!("gemv_batch: {batch} x {} shape mismatch", w.name) });
        }
        let t = self.tensor(w);
        // SAFETY: slices of the checked lengths; the library copies before returning.
        check(unsafe { ffi::sh_gemv_batch(self.ctx, &t, x.as_ptr(), y.as_mut_ptr(), len_u32(batch, "batch")?) })
    }

    /// The routed MoE FFN (crates/strata-core/src/moe.rs:58-127) for `n_tok`
    /// tokens: x and out `[n_tok][n_embd]`, logits `[n_tok][n_expert]`.
    #[allow(clippy::too_many_arguments)]
    pub fn moe_ffn(
        &self,
        gate: &ExpertView<'_>,
        up: &ExpertView<'_>,
        down: &ExpertView<'_>,
        logits: &[f32],
        n_tok: usize,
        top_k: usize,
        x: &[f32],
        out: &mut [f32],
    ) -> Result<()> {
        let n_embd = if self.opts.expert_out_major { gate.cols } else { gate.rows };
        if x.len() != n_tok * n_embd || out.len() != x.len() || logits.len() != n_tok * gate.n_expert {
            return Err(Error::Backend { message: "moe_ffn: shape mismatch".to_string() });
        }
        let (g, u, d) = (self.view(gate), self.view(up), self.view(down));
        // SAFETY: slices of the checked lengths; views over the caller's bytes.
        check(unsafe {
            ffi::sh_moe_ffn(
                self.ctx,
                &g,
                &u,
                &d,
                logits.as_ptr(),
                len_u32(n_tok, "n_tok")?,
                len_u32(top_k, "top_k")?,
                x.as_ptr(),
                out.as_mut_ptr(),
            )
        })
    }

    /// The whole MoE layer (moe.rs:48-143): router matvec on bf16(x),
    /// routing, routed experts, and the shared expert with its sigmoid gate.
    #[allow(clippy::too_many_arguments)]
    pub fn moe_layer(
        &self,
        router: &QuantTensor<'_>,
        gate: &ExpertView<'_>,
        up: &ExpertView<'_>,
        down: &ExpertView<'_>,
        gate_shexp: &QuantTensor<'_>,
        up_shexp: &QuantTensor<'_>,
        down_shexp: &QuantTensor<'_>,
        gate_inp_shexp: &QuantTensor<'_>,
        x: &[f32],
        n_tok: usize,
        top_k: usize,
        out: &mut [f32],
    ) -> Result<()> {
        if x.len() != n_tok * router.cols || out.len() != x.len() {
            return Err(Error::Backend { message: "moe_layer: shape mismatch".to_string() });
        }
        let (r, gs, us, ds, gi) = (
            self.tensor(router),
            self.tensor(gate_shexp),
            self.tensor(up_shexp),
            self.tensor(down_shexp),
            self.tensor(gate_inp_shexp),
        );
        let (g, u, d) = (self.view(gate), self.view(up), self.view(down));
        // SAFETY: slices of the checked lengths; views over the caller's bytes.
        check(unsafe {
            ffi::sh_moe_layer(
                self.ctx,
                &r,
                &g,
                &u,
                &d,
                &gs,
                &us,
                &ds,
                &gi,
                x.as_ptr(),
                len_u32(n_tok, "n_tok")?,
                len_u32(top_k, "top_k")?,
                out.as_mut_ptr(),
            )
        })
    }

    /// The dense FFN half of a layer in place on `x` `[n_tok][n_embd]`
    /// (crates/strata-core/src/qwen35.rs:112-129): rms_norm with
    /// `post_norm`, gate and up matvecs, silu(gate) * up, the down matvec and
    /// the residual add.
    pub fn dense_ffn(
        &self,
        gate: &QuantTensor<'_>,
        up: &QuantTensor<'_>,
        down: &QuantTensor<'_>,
        post_norm: &[f32],
        eps: f64,
        n_tok: usize,
        x: &mut [f32],
    ) -> Result<()> {
        if post_norm.len() != gate.cols || x.len() != n_tok * gate.cols {
            return Err(Error::Backend { message: "dense_ffn: shape mismatch".to_string() });
        }
        let (g, u, d) = (self.tensor(gate), self.tensor(up), self.tensor(down));
        // SAFETY: slices of the checked lengths.
        check(unsafe {
            ffi::sh_ffn(self.ctx, &g, &u, &d, post_norm.as_ptr(), eps, len_u32(n_tok, "n_tok")?, x.as_mut_ptr())
        })
    }

    /// Prefill: `y[t] = W x[t]` for `m` tokens (x `[m][cols]`, y `[m][rows]`);
    /// `mode` is `ffi::SH_MATMUL_BF16`, `ffi::SH_MATMUL_Q8` (32-element Q8
    /// activation blocks) or `ffi::SH_MATMUL_Q8K` (256-element blocks, K-quants).
    pub fn matmul(&self, w: &QuantTensor<'_>, x: &[f32], m: usize, y: &mut [f32], mode: u32) -> Result<()> {
        if x.len() != m * w.cols || y.len() != m * w.rows {
            return Err(Error::Backend { message: format!("matmul: {m} x {} shape mismatch", w.name) });
        }
        let t = self.tensor(w);
        // SAFETY: slices of the checked lengths.
        check(unsafe { ffi::sh_matmul(self.ctx, &t, x.as_ptr(), len_u32(m, "m")?, y.as_mut_ptr(), mode) })
    }

    /// expert_gemv on the CPU in the configured orientation: out-major
    /// experts are ops::gemv of their `[rows][cols]` slice.
    fn cpu_expert_gemv(&self, w: &ExpertView<'_>, e: usize, x: &[f32], y: &mut [f32], s: &mut [f32]) -> Result<()> {
        if !self.opts.expert_out_major {
            return self.cpu.expert_gemv(w, e, x, y, s);
        }
        let rb = w.quant.byte_size(w.cols);
        let slice = &w.data[e * w.rows * rb..(e + 1) * w.rows * rb];
        let t = QuantTensor { name: w.name, quant: w.quant, rows: w.rows, cols: w.cols, data: slice };
        self.cpu.gemv(&t, x, y, s)
    }
}

impl ComputeBackend for HipBackend {
    fn name(&self) -> &'static str {
        "hip"
    }

    fn gemv(&self, w: &QuantTensor<'_>, x: &[f32], y: &mut [f32], scratch: &mut [f32]) -> Result<()> {
        if !gemv_quant(w.quant) {
            return self.cpu.gemv(w, x, y, scratch); // legacy and IQ2/IQ3 types stay on the CPU
        }
        let t = self.tensor(w);
        // SAFETY: the library checks x_len / y_len against the tensor.
        let rc = unsafe { ffi::sh_gemv(self.ctx, &t, x.as_ptr(), x.len() as u64, y.as_mut_ptr(), y.len() as u64) };
        match route(rc, "gemv")? {
            Route::Done => Ok(()),
            Route::Cpu => self.cpu.gemv(w, x, y, scratch),
        }
    }

    fn expert_gemv(
        &self,
        w: &ExpertView<'_>,
        e: usize,
        x: &[f32],
        y: &mut [f32],
        scratch: &mut [f32],
    ) -> Result<()> {
        let on_device = if self.opts.expert_out_major { gemv_quant(w.quant) } else { device_quant(w.quant) };
        if !on_device {
            return self.cpu_expert_gemv(w, e, x, y, scratch);
        }
        let v = self.view(w);
        // SAFETY: the library checks e, x_len and y_len against the view.
        let rc = unsafe {
            ffi::sh_expert_gemv(self.ctx, &v, e as u64, x.as_ptr(), x.len() as u64, y.as_mut_ptr(), y.len() as u64)
        };
        match route(rc, "expert_gemv")? {
            Route::Done => Ok(()),
            Route::Cpu => self.cpu_expert_gemv(w, e, x, y, scratch),
        }
    }

    // The elementwise methods run on the device; a host-slice call is one
    // upload, one launch and one readback, so they pay off once a layer's
    // activations stay on the device (the library's *_dev forms). The slices
    // are written only when a call succeeds, so a call routed to the CPU runs
    // its body on the untouched input.
    fn rms_norm(&self, x: &mut [f32], w: &[f32], eps: f64) -> Result<()> {
        let rc = if w.len() == x.len() {
            // SAFETY: equal lengths, checked above.
            unsafe { ffi::sh_rms_norm(self.ctx, x.as_mut_ptr(), w.as_ptr(), x.len() as u64, eps) }
        } else {
            ffi::SH_ERR_SHAPE
        };
        match route(rc, "rms_norm")? {
            Route::Done => Ok(()),
            Route::Cpu => self.cpu.rms_norm(x, w, eps),
        }
    }

    fn rope_neox(&self, head: &mut [f32], cfg: &RopeCfg) -> Result<()> {
        let c = ffi::ShRopeCfg {
            pos: cfg.pos as u64,
            n_rot: cfg.n_rot as u64,
            head_dim: cfg.head_dim as u64,
            freq_base: cfg.freq_base,
        };
        // SAFETY: the library checks n against the rope shape.
        let rc = unsafe { ffi::sh_rope_neox(self.ctx, head.as_mut_ptr(), head.len() as u64, &c) };
        match route(rc, "rope_neox")? {
            Route::Done => Ok(()),
            Route::Cpu => self.cpu.rope_neox(head, cfg),
        }
    }

    fn softmax(&self, xs: &mut [f32]) -> Result<()> {
        // SAFETY: one slice of its own length.
        let rc = unsafe { ffi::sh_softmax(self.ctx, xs.as_mut_ptr(), xs.len() as u64) };
        match route(rc, "softmax")? {
            Route::Done => Ok(()),
            Route::Cpu => self.cpu.softmax(xs),
        }
    }

    fn l2_norm(&self, head: &mut [f32], eps: f64) -> Result<()> {
        // SAFETY: one slice of its own length.
        let rc = unsafe { ffi::sh_l2_norm(self.ctx, head.as_mut_ptr(), head.len() as u64, eps) };
        match route(rc, "l2_norm")? {
            Route::Done => Ok(()),
            Route::Cpu => self.cpu.l2_norm(head, eps),
        }
    }

    fn add(&self, a: &mut [f32], b: &[f32]) -> Result<()> {
        let rc = if b.len() == a.len() {
            // SAFETY: equal lengths, checked above.
            unsafe { ffi::sh_add(self.ctx, a.as_mut_ptr(), b.as_ptr(), a.len() as u64) }
        } else {
            ffi::SH_ERR_SHAPE
        };
        match route(rc, "add")? {
            Route::Done => Ok(()),
            Route::Cpu => self.cpu.add(a, b),
        }
    }
}

#[cfg(test)]
mod tests {
    use super::*;

    #[test]
    fn name_key_is_fnv1a() {
        assert_eq!(name_key(""), 0xcbf2_9ce4_8422_2325);
        assert_eq!(name_key("a"), 0xaf63_dc4c_8601_ec8c);
    }

    #[test]
    fn flags_follow_the_options() {
        let o = HipOptions { q6k_signed_scales: true, expert_out_major: true, ..HipOptions::default() };
        assert_eq!(o.tensor_flags(QuantType::Q6K), ffi::SH_FLAG_Q6K_SIGNED_SCALES);
        assert_eq!(o.tensor_flags(QuantType::Q4K), 0);
        assert_eq!(o.expert_flags(QuantType::Q4K), ffi::SH_FLAG_EXPERT_OUT_MAJOR);
        assert_eq!(HipOptions { iq4xs_ggml: true, ..o }.tensor_flags(QuantType::Iq4Xs), ffi::SH_FLAG_IQ4XS_GGML);
    }

    #[test]
    fn abi_version_matches() {
        // SAFETY: no arguments.
        assert_eq!(unsafe { ffi::sh_abi_version() }, ffi::SH_ABI_VERSION);
    }

    #[test]
    fn no_device_keeps_the_cpu_backend() {
        let mut n: c_int = 0;
        // SAFETY: valid out-pointer.
        unsafe { ffi::sh_device_count(&mut n) };
        if n == 0 {
            assert!(HipBackend::probe(HipOptions::default()).is_err());
        }
    }
}
