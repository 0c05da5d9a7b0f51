//! qbk-sys -- Rust binding of libqbk (`include/qbk.h`), the MI355X (gfx950)
//! implementation of quantibbler-kernels' two hot paths.
//!
//! The raw `extern "C"` declarations mirror the header one for one; the safe
//! wrappers keep the reference's Rust names and contracts so that the engine
//! and the kernels crate can swap their device faces in:
//!
//! * `GpuContext::{init, init_at, packed_matvec, attention, attention_sage}`
//!   -- crates/quantibbler-kernels/src/gpu.rs:76-189, gpu_attention.rs:451-756;
//! * `attention_sage_decode` -- the decode call site's row 0
//!   (crates/quantibbler-server/src/engine/mod.rs:984-1030), in O(seq);
//! * `FactorLayer` -- engine/mod.rs:313-481 PackedLayer, uploaded once;
//! * `LmHead` -- engine/mod.rs:781-800 Engine::logits;
//! * `pack_bits`, `unpack_bits`, `joint_itq` -- core.rs, host code.
//!
//! Errors come back as `KernelError(String)` holding the reference's text
//! (`qbk_last_error`).  Link with `-L<dir of libqbk.so> -lqbk` (build.rs).
#![allow(clippy::too_many_arguments)]

use std::ffi::CStr;
use std::os::raw::{c_char, c_int, c_void};

pub const QBK_OK: c_int = 0;
pub const QBK_ERR_VALIDATION: c_int = 1;
pub const QBK_ERR_DEVICE: c_int = 2;
pub const QBK_ERR_INIT: c_int = 3;
pub const QBK_F64: c_int = 0;
pub const QBK_F32: c_int = 1;
pub const QBK_BF16: c_int = 2;
pub const QBK_ATTN_SAGE: c_int = 0;
pub const QBK_ATTN_EXACT: c_int = 1;

#[repr(C)]
pub struct QbkCtx {
    _p: [u8; 0],
}
#[repr(C)]
pub struct QbkFactor {
    _p: [u8; 0],
}
#[repr(C)]
pub struct QbkHead {
    _p: [u8; 0],
}
#[repr(C)]
pub struct QbkFactorSet {
    _p: [u8; 0],
}
#[repr(C)]
pub struct QbkBlock {
    _p: [u8; 0],
}

/// gpu_attention.rs:402-411 AttentionShape, field for field.
#[repr(C)]
#[derive(Clone, Copy, Debug, PartialEq, Eq)]
pub struct AttentionShape {
    pub batch: usize,
    pub n_heads: usize,
    pub n_kv_heads: usize,
    pub seq_q: usize,
    pub seq_kv: usize,
    pub head_dim: usize,
    pub val_dim: usize,
}

extern "C" {
    pub fn qbk_backend_version() -> *const c_char;
    pub fn qbk_last_error() -> *const c_char;
    pub fn qbk_pack_bits(factor: *const i8, factor_len: usize, n_rows: usize, n_cols: usize, out: *mut u8) -> c_int;
    pub fn qbk_unpack_bits(packed: *const u8, packed_len: usize, n_rows: usize, n_bits: usize, out: *mut i8) -> c_int;
    pub fn qbk_joint_itq(u_hat: *const f64, u_len: usize, v_hat: *const f64, v_len: usize, dout: usize, din: usize,
                         rank: usize, max_iter: usize, tol: f64, seed: u64, u_t: *mut i8, v_t: *mut i8,
                         n_iter: *mut usize, converged: *mut c_int) -> c_int;
    pub fn qbk_ctx_create(device_index: c_int, out: *mut *mut QbkCtx) -> c_int;
    pub fn qbk_ctx_destroy(ctx: *mut QbkCtx);
    pub fn qbk_gpu_available() -> c_int;
    pub fn qbk_packed_matvec(ctx: *mut QbkCtx, dtype: c_int, packed: *const u8, packed_len: usize, n_rows: usize,
                             n_bits: usize, vec: *const c_void, vec_len: usize, out: *mut c_void) -> c_int;
    pub fn qbk_packed_matmul(ctx: *mut QbkCtx, dtype: c_int, packed: *const u8, packed_len: usize, n_rows: usize,
                             n_bits: usize, mat: *const c_void, mat_len: usize, n_cols: usize,
                             out: *mut c_void) -> c_int;
    pub fn qbk_factor_from_qpk1(ctx: *mut QbkCtx, stream: *const u8, len: usize, out: *mut *mut QbkFactor) -> c_int;
    pub fn qbk_factor_destroy(layer: *mut QbkFactor);
    pub fn qbk_factor_dims(layer: *const QbkFactor, dout: *mut usize, din: *mut usize, r: *mut usize) -> c_int;
    pub fn qbk_factor_apply(ctx: *mut QbkCtx, layer: *const QbkFactor, serving: c_int, x: *const f32, batch: usize,
                            y: *mut f32) -> c_int;
    pub fn qbk_factor_workspace_size(layer: *const QbkFactor, batch: usize) -> usize;
    pub fn qbk_factor_linear_dev(ctx: *mut QbkCtx, layer: *const QbkFactor, x: *const u16, batch: usize,
                                 y: *mut c_void, y_dtype: c_int, workspace: *mut c_void, workspace_size: usize,
                                 stream: *mut c_void) -> c_int;
    pub fn qbk_attention(ctx: *mut QbkCtx, shape: *const AttentionShape, q: *const f32, q_len: usize, k: *const f32,
                         k_len: usize, v: *const f32, v_len: usize, causal: c_int, out: *mut f32) -> c_int;
    pub fn qbk_attention_sage(ctx: *mut QbkCtx, shape: *const AttentionShape, q: *const f32, q_len: usize,
                              k: *const f32, k_len: usize, v: *const f32, v_len: usize, causal: c_int,
                              block_size: usize, out: *mut f32) -> c_int;
    pub fn qbk_attention_sage_decode(ctx: *mut QbkCtx, shape: *const AttentionShape, q: *const f32, q_len: usize,
                                     k: *const f32, k_len: usize, v: *const f32, v_len: usize, block_size: usize,
                                     out: *mut f32, out_len: usize) -> c_int;
    pub fn qbk_head_create(ctx: *mut QbkCtx, head: *const f32, head_len: usize, vocab: usize, d_model: usize,
                           out: *mut *mut QbkHead) -> c_int;
    pub fn qbk_head_destroy(head: *mut QbkHead);
    pub fn qbk_head_logits(ctx: *mut QbkCtx, head: *const QbkHead, hidden: *const f32, hidden_len: usize,
                           logits: *mut f32, logits_len: usize) -> c_int;
}

// The device-pointer faces (`_dev`: device buffers in and out, work queued
// on the caller's HIP stream, no copies), layer sets, the decoder block, the
// trunk pieces and the remaining host helpers -- the rest of include/qbk.h.
extern "C" {
    pub fn qbk_dtype_from_name(name: *const c_char, dtype_out: *mut c_int) -> c_int;
    pub fn qbk_validate_packed(packed_len: usize, n_rows: usize, n_bits: usize, n_words: *mut usize) -> c_int;
    pub fn qbk_sign_estimate(x: *const f64, n: usize, out: *mut i8);
    pub fn qbk_packed_matvec_dev(ctx: *mut QbkCtx, dtype: c_int, packed: *const u8, n_rows: usize, n_bits: usize,
                                 vec: *const c_void, out: *mut c_void, stream: *mut c_void) -> c_int;
    pub fn qbk_packed_matmul_dev(ctx: *mut QbkCtx, dtype: c_int, packed: *const u8, n_rows: usize, n_bits: usize,
                                 mat: *const c_void, k_cols: usize, n_cols: usize, out: *mut c_void,
                                 stream: *mut c_void) -> c_int;
    pub fn qbk_factor_from_rows(ctx: *mut QbkCtx, dout: usize, din: usize, r: usize, ub_rows: *const u8,
                                vb_t_rows: *const u8, s1: *const f32, s2: *const f32, bias: *const f32,
                                out: *mut *mut QbkFactor) -> c_int;
    pub fn qbk_factor_linear_noalloc_dev(ctx: *mut QbkCtx, layer: *const QbkFactor, x: *const u16, batch: usize,
                                         y: *mut c_void, y_dtype: c_int, stream: *mut c_void) -> c_int;
    pub fn qbk_factor_set_create(ctx: *mut QbkCtx, layers: *const *const QbkFactor, n_layers: usize,
                                 out: *mut *mut QbkFactorSet) -> c_int;
    pub fn qbk_factor_set_destroy(set: *mut QbkFactorSet);
    pub fn qbk_factor_set_workspace_size(set: *const QbkFactorSet) -> usize;
    pub fn qbk_factor_set_decode_dev(ctx: *mut QbkCtx, set: *const QbkFactorSet, x: *const u16, y: *mut u16,
                                     workspace: *mut c_void, workspace_size: usize, stream: *mut c_void) -> c_int;
    pub fn qbk_factor_set_stage_dev(ctx: *mut QbkCtx, set: *const QbkFactorSet, stage: c_int, x: *const u16,
                                    y: *mut u16, workspace: *mut c_void, workspace_size: usize,
                                    stream: *mut c_void) -> c_int;
    pub fn qbk_factor_set_workspace_size_batch(set: *const QbkFactorSet, n: usize) -> usize;
    pub fn qbk_factor_set_shared_workspace_size(set: *const QbkFactorSet, n: usize) -> usize;
    pub fn qbk_factor_set_shared_dev(ctx: *mut QbkCtx, set: *const QbkFactorSet, n: usize, x: *const u16,
                                     y: *mut u16, workspace: *mut c_void, workspace_size: usize,
                                     stream: *mut c_void) -> c_int;
    pub fn qbk_factor_set_decode_batch_dev(ctx: *mut QbkCtx, set: *const QbkFactorSet, n: usize, x: *const u16,
                                           y: *mut u16, workspace: *mut c_void, workspace_size: usize,
                                           stream: *mut c_void) -> c_int;
    pub fn qbk_block_create(ctx: *mut QbkCtx, layers: *const *const QbkFactor, input_norm: *const f32,
                            input_norm_len: usize, post_norm: *const f32, post_norm_len: usize, q_norm: *const f32,
                            k_norm: *const f32, qk_norm_len: usize, n_heads: usize, n_kv_heads: usize,
                            head_dim: usize, rope_theta: f64, rms_norm_eps: f64, capacity: usize, block_size: usize,
                            out: *mut *mut QbkBlock) -> c_int;
    pub fn qbk_block_destroy(block: *mut QbkBlock);
    pub fn qbk_block_decode_dev(ctx: *mut QbkCtx, block: *mut QbkBlock, h: *mut f32, pos: usize,
                                stream: *mut c_void) -> c_int;
    pub fn qbk_block_reset(block: *mut QbkBlock) -> c_int;
    pub fn qbk_block_prefill_workspace_size(block: *const QbkBlock, n_tokens: usize) -> usize;
    pub fn qbk_block_prefill_dev(ctx: *mut QbkCtx, block: *mut QbkBlock, h: *mut f32, n_tokens: usize,
                                 workspace: *mut c_void, workspace_size: usize, stream: *mut c_void) -> c_int;
    pub fn qbk_block_cache(block: *const QbkBlock, k_cache: *mut *mut f32, v_cache: *mut *mut f32) -> c_int;
    pub fn qbk_block_create_seqs(ctx: *mut QbkCtx, layers: *const *const QbkFactor, input_norm: *const f32,
                                 input_norm_len: usize, post_norm: *const f32, post_norm_len: usize,
                                 q_norm: *const f32, k_norm: *const f32, qk_norm_len: usize, n_heads: usize,
                                 n_kv_heads: usize, head_dim: usize, rope_theta: f64, rms_norm_eps: f64,
                                 capacity: usize, block_size: usize, n_seqs: usize, out: *mut *mut QbkBlock) -> c_int;
    pub fn qbk_block_prefill_seq_dev(ctx: *mut QbkCtx, block: *mut QbkBlock, seq: usize, h: *mut f32, n_tokens: usize,
                                     workspace: *mut c_void, workspace_size: usize, stream: *mut c_void) -> c_int;
    pub fn qbk_block_decode_batch_workspace_size(block: *const QbkBlock, n: usize) -> usize;
    pub fn qbk_block_decode_batch_dev(ctx: *mut QbkCtx, block: *mut QbkBlock, h: *mut f32, pos: *const usize,
                                      n: usize, workspace: *mut c_void, workspace_size: usize,
                                      stream: *mut c_void) -> c_int;
    pub fn qbk_block_decode_pos_dev(ctx: *mut QbkCtx, block: *mut QbkBlock, h: *mut f32, pos: *const u32,
                                    stream: *mut c_void) -> c_int;
    pub fn qbk_block_decode_batch_pos_dev(ctx: *mut QbkCtx, block: *mut QbkBlock, h: *mut f32, pos: *const u32,
                                          n: usize, workspace: *mut c_void, workspace_size: usize,
                                          stream: *mut c_void) -> c_int;
    pub fn qbk_block_set_positions(block: *mut QbkBlock, pos: *const usize, n: usize) -> c_int;
    pub fn qbk_block_set_filled(block: *mut QbkBlock, rows: *const usize, n: usize) -> c_int;
    pub fn qbk_block_set_attention_face(block: *mut QbkBlock, face: c_int) -> c_int;
    pub fn qbk_block_set_serving(ctx: *mut QbkCtx, block: *mut QbkBlock, serving: c_int) -> c_int;
    pub fn qbk_embed(ctx: *mut QbkCtx, table: *const f32, vocab: usize, d_model: usize, tokens: *const i32, n: usize,
                     out: *mut f32, stream: *mut c_void) -> c_int;
    pub fn qbk_embed_dev(ctx: *mut QbkCtx, table: *const f32, vocab: usize, d_model: usize, tokens: *const i32,
                         n: usize, out: *mut f32, stream: *mut c_void) -> c_int;
    pub fn qbk_rms_norm_dev(ctx: *mut QbkCtx, x: *const f32, rows: usize, d: usize, w: *const f32, eps: f64,
                            out: *mut f32, stream: *mut c_void) -> c_int;
    pub fn qbk_rms_norm_f32_dev(ctx: *mut QbkCtx, x: *const f32, rows: usize, d: usize, w: *const f32, eps: f64,
                                out: *mut f32, stream: *mut c_void) -> c_int;
    pub fn qbk_argmax_dev(ctx: *mut QbkCtx, logits: *const f32, rows: usize, vocab: usize, out: *mut i32,
                          stream: *mut c_void) -> c_int;
    pub fn qbk_positions_advance_dev(ctx: *mut QbkCtx, pos: *mut u32, n: usize, stream: *mut c_void) -> c_int;
    pub fn qbk_attention_dev(ctx: *mut QbkCtx, shape: *const AttentionShape, q: *const f32, k: *const f32,
                             v: *const f32, causal: c_int, out: *mut f32, stream: *mut c_void) -> c_int;
    pub fn qbk_attention_sage_dev(ctx: *mut QbkCtx, shape: *const AttentionShape, q: *const f32, k: *const f32,
                                  v: *const f32, causal: c_int, block_size: usize, out: *mut f32,
                                  stream: *mut c_void) -> c_int;
    pub fn qbk_sage_decode_workspace_size(shape: *const AttentionShape, block_size: usize) -> usize;
    pub fn qbk_attention_sage_decode_dev(ctx: *mut QbkCtx, shape: *const AttentionShape, q: *const f32, k: *const f32,
                                         v: *const f32, block_size: usize, out: *mut f32, workspace: *mut c_void,
                                         workspace_size: usize, stream: *mut c_void) -> c_int;
    pub fn qbk_attention_sage_decode_step_dev(ctx: *mut QbkCtx, shape: *const AttentionShape, q: *const f32,
                                              k: *const f32, v: *const f32, block_size: usize, out: *mut f32,
                                              state: *mut c_void, state_size: usize, capacity: usize,
                                              cached_tokens: usize, stream: *mut c_void) -> c_int;
    pub fn qbk_sage_blk_workspace_size(shape: *const AttentionShape) -> usize;
    pub fn qbk_attention_sage_blk_dev(ctx: *mut QbkCtx, shape: *const AttentionShape, q: *const u16, k: *const u16,
                                      v: *const u16, causal: c_int, out: *mut u16, workspace: *mut c_void,
                                      workspace_size: usize, stream: *mut c_void) -> c_int;
    pub fn qbk_sage_blk_quantize_dev(ctx: *mut QbkCtx, shape: *const AttentionShape, q: *const u16, k: *const u16,
                                     v: *const u16, qhat: *mut i8, qscale: *mut f32, khat: *mut i8, kscale: *mut f32,
                                     kmean: *mut f32, vh: *mut u16, stream: *mut c_void) -> c_int;
    pub fn qbk_head_create_dev(ctx: *mut QbkCtx, head: *const f32, vocab: usize, d_model: usize,
                               out: *mut *mut QbkHead) -> c_int;
    pub fn qbk_head_info(head: *const QbkHead, vocab: *mut usize, d_model: *mut usize, bf16: *mut c_int) -> c_int;
    pub fn qbk_head_logits_dev(ctx: *mut QbkCtx, head: *const QbkHead, hidden: *const f32, batch: usize,
                               logits: *mut f32, stream: *mut c_void) -> c_int;
}

/// core.rs:31 KernelError: the reference's message text.
#[derive(Debug, Clone, PartialEq, Eq)]
pub struct KernelError(pub String);

impl std::fmt::Display for KernelError {
    fn fmt(&self, f: &mut std::fmt::Formatter<'_>) -> std::fmt::Result {
        f.write_str(&self.0)
    }
}

impl std::error::Error for KernelError {}

fn check(rc: c_int) -> Result<(), KernelError> {
    if rc == QBK_OK {
        return Ok(());
    }
    let msg = unsafe { CStr::from_ptr(qbk_last_error()) }.to_string_lossy().into_owned();
    Err(KernelError(msg))
}

/// lib.rs:94-97 backend_version.
pub fn backend_version() -> String {
    unsafe { CStr::from_ptr(qbk_backend_version()) }.to_string_lossy().into_owned()
}

/// gpu.rs:187-189 gpu_available.
pub fn gpu_available() -> bool {
    unsafe { qbk_gpu_available() != 0 }
}

/// core.rs:129-162 pack_bits.
pub fn pack_bits(factor: &[i8], n_rows: usize, n_cols: usize) -> Result<Vec<u8>, KernelError> {
    let mut out = vec![0u8; n_rows * n_cols.div_ceil(8)];
    check(unsafe { qbk_pack_bits(factor.as_ptr(), factor.len(), n_rows, n_cols, out.as_mut_ptr()) })?;
    Ok(out)
}

/// core.rs:166-189 unpack_bits.
pub fn unpack_bits(packed: &[u8], n_rows: usize, n_bits: usize) -> Result<Vec<i8>, KernelError> {
    let mut out = vec![0i8; n_rows * n_bits];
    check(unsafe { qbk_unpack_bits(packed.as_ptr(), packed.len(), n_rows, n_bits, out.as_mut_ptr()) })?;
    Ok(out)
}

/// core.rs:318-424 joint_itq -> (u_t, v_t, n_iter, converged).
pub fn joint_itq(u_hat: &[f64], v_hat: &[f64], dout: usize, din: usize, rank: usize, max_iter: usize, tol: f64,
                 seed: u64) -> Result<(Vec<i8>, Vec<i8>, usize, bool), KernelError> {
    let mut u_t = vec![0i8; dout * rank];
    let mut v_t = vec![0i8; din * rank];
    let (mut n_iter, mut conv) = (0usize, 0 as c_int);
    check(unsafe {
        qbk_joint_itq(u_hat.as_ptr(), u_hat.len(), v_hat.as_ptr(), v_hat.len(), dout, din, rank, max_iter, tol,
                      seed, u_t.as_mut_ptr(), v_t.as_mut_ptr(), &mut n_iter, &mut conv)
    })?;
    Ok((u_t, v_t, n_iter, conv != 0))
}

/// gpu.rs:76-189 GpuContext: a live context on one device, fail-closed.
pub struct GpuContext {
    raw: *mut QbkCtx,
}

// libqbk's calls on one context are independent (each host call uses its own
// stream and buffers), so the context may be shared across threads.
unsafe impl Send for GpuContext {}
unsafe impl Sync for GpuContext {}

impl GpuContext {
    pub fn init_at(device_index: usize) -> Result<Self, KernelError> {
        let mut raw = std::ptr::null_mut();
        check(unsafe { qbk_ctx_create(device_index as c_int, &mut raw) })?;
        Ok(Self { raw })
    }

    pub fn init() -> Result<Self, KernelError> {
        Self::init_at(0)
    }

    pub fn raw(&self) -> *mut QbkCtx {
        self.raw
    }

    /// gpu.rs:116-185: f64, element order, bit-identical to core::packed_matvec.
    pub fn packed_matvec(&self, packed: &[u8], n_rows: usize, n_bits: usize, vec: &[f64])
                         -> Result<Vec<f64>, KernelError> {
        let mut out = vec![0.0f64; n_rows];
        check(unsafe {
            qbk_packed_matvec(self.raw, QBK_F64, packed.as_ptr(), packed.len(), n_rows, n_bits,
                              vec.as_ptr().cast(), vec.len(), out.as_mut_ptr().cast())
        })?;
        Ok(out)
    }

    /// gpu_attention.rs:451-570: exact f32 attention (Q unscaled, GQA).
    pub fn attention(&self, shape: AttentionShape, query: &[f32], key: &[f32], value: &[f32], causal: bool)
                     -> Result<Vec<f32>, KernelError> {
        let mut out = vec![0.0f32; shape.batch * shape.n_heads * shape.seq_q * shape.val_dim];
        check(unsafe {
            qbk_attention(self.raw, &shape, query.as_ptr(), query.len(), key.as_ptr(), key.len(), value.as_ptr(),
                          value.len(), causal as c_int, out.as_mut_ptr())
        })?;
        Ok(out)
    }

    /// gpu_attention.rs:589-756: the [SA] s4 reference scheme.
    pub fn attention_sage(&self, shape: AttentionShape, query: &[f32], key: &[f32], value: &[f32], causal: bool,
                          block_size: usize) -> Result<Vec<f32>, KernelError> {
        let mut out = vec![0.0f32; shape.batch * shape.n_heads * shape.seq_q * shape.val_dim];
        check(unsafe {
            qbk_attention_sage(self.raw, &shape, query.as_ptr(), query.len(), key.as_ptr(), key.len(),
                               value.as_ptr(), value.len(), causal as c_int, block_size, out.as_mut_ptr())
        })?;
        Ok(out)
    }

    /// Row 0 of engine/mod.rs:984-1030's padded decode call, computed alone
    /// over the row-major cache (seq_kv, n_kv_heads, d): (n_heads, d).
    pub fn attention_sage_decode(&self, shape: AttentionShape, query: &[f32], keys: &[f32], values: &[f32],
                                 block_size: usize) -> Result<Vec<f32>, KernelError> {
        let mut out = vec![0.0f32; shape.n_heads * shape.val_dim];
        check(unsafe {
            qbk_attention_sage_decode(self.raw, &shape, query.as_ptr(), query.len(), keys.as_ptr(), keys.len(),
                                      values.as_ptr(), values.len(), block_size, out.as_mut_ptr(), out.len())
        })?;
        Ok(out)
    }
}

impl Drop for GpuContext {
    fn drop(&mut self) {
        unsafe { qbk_ctx_destroy(self.raw) }
    }
}

/// engine/mod.rs:313-481 PackedLayer, uploaded once from a qpk1 stream.
pub struct FactorLayer {
    raw: *mut QbkFactor,
    pub dout: usize,
    pub din: usize,
    pub r: usize,
}

unsafe impl Send for FactorLayer {}
unsafe impl Sync for FactorLayer {}

impl FactorLayer {
    /// quantibbler-qpk1 lib.rs:229-320 parse + engine/mod.rs:342-381 from_layer.
    pub fn from_qpk1(ctx: &GpuContext, stream: &[u8]) -> Result<Self, KernelError> {
        let mut raw = std::ptr::null_mut();
        check(unsafe { qbk_factor_from_qpk1(ctx.raw, stream.as_ptr(), stream.len(), &mut raw) })?;
        let (mut dout, mut din, mut r) = (0usize, 0usize, 0usize);
        check(unsafe { qbk_factor_dims(raw, &mut dout, &mut din, &mut r) })?;
        Ok(Self { raw, dout, din, r })
    }

    /// engine/mod.rs:393-460 apply (fp32 serving: `bf16 == false`) /
    /// apply_bf16 (`bf16 == true`), `batch` rows of din.
    pub fn apply(&self, ctx: &GpuContext, x: &[f32], bf16: bool) -> Result<Vec<f32>, KernelError> {
        let batch = x.len() / self.din.max(1);
        let mut y = vec![0.0f32; batch * self.dout];
        let serving = if bf16 { QBK_BF16 } else { QBK_F32 };
        check(unsafe { qbk_factor_apply(ctx.raw, self.raw, serving, x.as_ptr(), batch, y.as_mut_ptr()) })?;
        Ok(y)
    }

    pub fn raw(&self) -> *mut QbkFactor {
        self.raw
    }
}

impl Drop for FactorLayer {
    fn drop(&mut self) {
        unsafe { qbk_factor_destroy(self.raw) }
    }
}

/// engine/mod.rs:781-800 Engine::logits on a head uploaded once.
pub struct LmHead {
    raw: *mut QbkHead,
    vocab: usize,
}

unsafe impl Send for LmHead {}
unsafe impl Sync for LmHead {}

impl LmHead {
    pub fn from_rows(ctx: &GpuContext, head: &[f32], vocab: usize, d_model: usize) -> Result<Self, KernelError> {
        let mut raw = std::ptr::null_mut();
        check(unsafe { qbk_head_create(ctx.raw, head.as_ptr(), head.len(), vocab, d_model, &mut raw) })?;
        Ok(Self { raw, vocab })
    }

    pub fn logits(&self, ctx: &GpuContext, hidden: &[f32]) -> Result<Vec<f32>, KernelError> {
        let mut out = vec![0.0f32; self.vocab];
        check(unsafe {
            qbk_head_logits(ctx.raw, self.raw, hidden.as_ptr(), hidden.len(), out.as_mut_ptr(), out.len())
        })?;
        Ok(out)
    }
}

impl Drop for LmHead {
    fn drop(&mut self) {
        unsafe { qbk_head_destroy(self.raw) }
    }
}
