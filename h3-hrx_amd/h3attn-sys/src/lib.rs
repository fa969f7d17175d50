//! Raw FFI to `libh3attn.so`: one `extern "C"` function per entry point of
//! `include/h3attn.h`, with `#[repr(C)]` mirrors of its config structs. Every entry point takes
//! device pointers with their byte lengths (`H3View`), a plain config, scalars and a HIP stream,
//! and returns an `i32` status (`H3_OK` = 0; the message of the last failure on the calling
//! thread is `h3_last_error()`). None synchronises; none allocates except `h3_stack_build` and
//! `h3_vsa_build`.
//!
//! In the reference (h3-hrx) each function replaces one `dispatch::emit` of a Loom kernel
//! (`src/dispatch.rs:254-316`); the header names the kernel each one replaces. The caller supplies
//! the device address of each `hrx::View` and the HIP stream of its `hrx::Stream`.
#![allow(non_camel_case_types)]

use std::ffi::{c_char, c_int, c_void, CStr};

/// `hipStream_t`; null is the default stream.
pub type H3Stream = *mut c_void;

/// A device binding: pointer and the bytes it may address.
#[repr(C)]
#[derive(Clone, Copy, Debug)]
pub struct H3View {
    pub ptr: *mut c_void,
    pub bytes: usize,
}

impl H3View {
    pub const NULL: H3View = H3View { ptr: std::ptr::null_mut(), bytes: 0 };
}

pub const H3_OK: c_int = 0;
pub const H3_ERR_BINDING: c_int = 1;
pub const H3_ERR_CONFIG: c_int = 2;
pub const H3_ERR_ARGUMENT: c_int = 3;
pub const H3_ERR_LAUNCH: c_int = 4;
pub const H3_ERR_NO_DEVICE: c_int = 5;

pub const H3_ELEM_F16: u32 = 0;
pub const H3_ELEM_BF16: u32 = 1;
pub const H3_ELEM_F32: u32 = 2;

#[repr(C)]
#[derive(Clone, Copy, Debug, Default)]
pub struct H3PrepareCfg {
    pub row_stride: u32,
    pub head_offset: u32,
    pub heads: u32,
    pub extra_scale: f32,
    pub token_capacity: u32,
    pub eps: f32,
    pub elem: u32,
}

#[repr(C)]
#[derive(Clone, Copy, Debug, Default)]
pub struct H3RopeCfg {
    pub row_stride: u32,
    pub heads: u32,
    pub kv_heads: u32,
    pub k_offset: u32,
    pub eps: f32,
    pub copy_v: u32,
    pub elem: u32,
}

#[repr(C)]
#[derive(Clone, Copy, Debug, Default)]
pub struct H3TransposeCfg {
    pub width: u32,
    pub row_capacity: u32,
    pub elem: u32,
}

#[repr(C)]
#[derive(Clone, Copy, Debug, Default)]
pub struct H3GemmCfg {
    pub k_size: u32,
    pub n_size: u32,
    pub k_stride: u32,
    pub m_group: u32,
}

#[repr(C)]
#[derive(Clone, Copy, Debug, Default)]
pub struct H3PreparePlainCfg {
    pub width: u32,
    pub lanes: u32,
    pub out_stride: u32,
    pub elem: u32,
}

#[repr(C)]
#[derive(Clone, Copy, Debug, Default)]
pub struct H3AttentionCfg {
    pub q_stride: u32,
    pub kv_stride: u32,
    pub out_stride: u32,
    pub tokens: u32,
    pub token_capacity: u32,
    pub scale: f32,
}

#[repr(C)]
#[derive(Clone, Copy, Debug, Default)]
pub struct H3AttentionSkipCfg {
    pub q_stride: u32,
    pub kv_stride: u32,
    pub out_stride: u32,
    pub tokens: u32,
    pub token_capacity: u32,
    pub scale: f32,
    pub skip_tau: f32,
}

#[repr(C)]
#[derive(Clone, Copy, Debug, Default)]
pub struct H3CrossCfg {
    pub q_heads: u32,
    pub kv_heads: u32,
    pub q_tokens: u32,
    pub q_capacity: u32,
    pub kv_tokens: u32,
    pub kv_capacity: u32,
    pub out_stride: u32,
}

#[repr(C)]
#[derive(Clone, Copy, Debug, Default)]
pub struct H3VsaCfg {
    pub tokens: u32,
    pub padded: u32,
    pub width: u32,
    pub blocks: u32,
    pub heads: u32,
    pub prefix: u32,
    pub topk: u32,
}

#[repr(C)]
#[derive(Clone, Copy, Debug, Default)]
pub struct H3VsaSegment {
    pub row0: u32,
    pub rows: u32,
}

#[repr(C)]
#[derive(Clone, Copy, Debug)]
pub struct H3VsaOptions {
    pub keep_percent: f64,
    pub start: f64,
    pub end: f64,
    pub min_tokens: u32,
    pub dense_blocks: *const u32,
    pub n_dense_blocks: u32,
}

#[repr(C)]
#[derive(Clone, Copy, Debug)]
pub struct H3VsaBuffers {
    pub src: H3View,
    pub inverse: H3View,
    pub lengths: H3View,
    pub q: H3View,
    pub k: H3View,
    pub v: H3View,
    pub qm: H3View,
    pub km: H3View,
    pub scores: H3View,
    pub routes: H3View,
    pub qi: H3View,
    pub ki: H3View,
    pub qs: H3View,
    pub ks: H3View,
    pub vt: H3View,
    pub out: H3View,
    pub kmean: H3View,
    pub cfg: H3VsaCfg,
    pub attention: H3AttentionCfg,
}

#[repr(C)]
#[derive(Clone, Copy, Debug, Default)]
pub struct H3StackDims {
    pub heads: u32,
    pub tokens: u32,
    pub eps: f32,
    pub elem: u32,
    pub ksmooth: c_int,
    pub fused: c_int,
    /// f16 GEMM activations: the attention output at gemm_pitch(inner, 16) (src/stack.rs:751-758).
    pub direct_attn: c_int,
}

#[repr(C)]
#[derive(Clone, Copy, Debug)]
pub struct H3IntQk {
    pub qi: H3View,
    pub ki: H3View,
    pub qs: H3View,
    pub ks: H3View,
    pub kmean: H3View,
    pub zmean: H3View,
    pub vt: H3View,
    pub head_major: c_int,
}

/// Opaque `Stack` mirror (`h3_stack_build`).
#[repr(C)]
pub struct h3_stack {
    _private: [u8; 0],
}

/// Opaque VSA runtime (`h3_vsa_build`).
#[repr(C)]
pub struct h3_vsa {
    _private: [u8; 0],
}

extern "C" {
    pub fn h3_last_error() -> *const c_char;
    pub fn h3_version() -> *const c_char;

    // operand preparation
    pub fn h3_prepare_qk_i8(cfg: *const H3PrepareCfg, tokens: u32, x: H3View, mean: H3View,
                            codes: H3View, scales: H3View, stream: H3Stream) -> c_int;
    pub fn h3_prepare_qk_i8hm(cfg: *const H3PrepareCfg, tokens: u32, x: H3View, mean: H3View,
                              codes: H3View, scales: H3View, stream: H3Stream) -> c_int;
    pub fn h3_prepare_qk_i4(cfg: *const H3PrepareCfg, tokens: u32, x: H3View, mean: H3View,
                            codes: H3View, scales: H3View, stream: H3Stream) -> c_int;
    pub fn h3_prepare_qk_rope_i8hm(cfg: *const H3PrepareCfg, tokens: u32, x: H3View,
                                   weight: H3View, cos_t: H3View, sin_t: H3View, codes: H3View,
                                   scales: H3View, stream: H3Stream) -> c_int;
    pub fn h3_prepare_k_rope_smooth_i8hm(cfg: *const H3PrepareCfg, tokens: u32, x: H3View,
                                         weight: H3View, cos_t: H3View, sin_t: H3View,
                                         mean: H3View, codes: H3View, scales: H3View,
                                         stream: H3Stream) -> c_int;
    pub fn h3_rope_qknorm_f16(cfg: *const H3RopeCfg, tokens: u32, x: H3View, qweight: H3View,
                              kweight: H3View, cos_t: H3View, sin_t: H3View, q_out: H3View,
                              k_out: H3View, v_out: H3View, stream: H3Stream) -> c_int;
    pub fn h3_colmean_f32(width: u32, elem: u32, tokens: u32, x: H3View, mean: H3View,
                          stream: H3Stream) -> c_int;
    pub fn h3_transpose_f16(cfg: *const H3TransposeCfg, launch_rows: u32, rows: u32, x: H3View,
                            out: H3View, stream: H3Stream) -> c_int;
    pub fn h3_transpose_qkv_v_f16(cfg: *const H3TransposeCfg, launch_rows: u32, rows: u32,
                                  x: H3View, out: H3View, stream: H3Stream) -> c_int;

    // producers either side of the path
    pub fn h3_gemm_i8_qkv_256(cfg: *const H3GemmCfg, tokens: u32, a: H3View, w: H3View,
                              w_scale: H3View, a_scale: H3View, out: H3View,
                              stream: H3Stream) -> c_int;
    pub fn h3_prepare_plain_i8(cfg: *const H3PreparePlainCfg, tokens: u32, x: H3View,
                               codes: H3View, scales: H3View, stream: H3Stream) -> c_int;
    pub fn h3_rope_dit_tables(pos: *const f64, rows: usize, inv_freq: *const f32,
                              cos_t: *mut f32, sin_t: *mut f32) -> c_int;

    // attention
    pub fn h3_attention_i8qkhm(cfg: *const H3AttentionCfg, token_count: u32, heads: u32,
                               qi: H3View, qs: H3View, ki: H3View, ks: H3View, vt: H3View,
                               out: H3View, stream: H3Stream) -> c_int;
    pub fn h3_attention_i8qk(cfg: *const H3AttentionCfg, token_count: u32, heads: u32,
                             qi: H3View, qs: H3View, ki: H3View, ks: H3View, vt: H3View,
                             out: H3View, stream: H3Stream) -> c_int;
    pub fn h3_attention_i4qk(cfg: *const H3AttentionCfg, token_count: u32, heads: u32,
                             qi: H3View, qs: H3View, ki: H3View, ks: H3View, vt: H3View,
                             out: H3View, stream: H3Stream) -> c_int;
    pub fn h3_attention_i4qks(cfg: *const H3AttentionSkipCfg, token_count: u32, heads: u32,
                              qi: H3View, qs: H3View, ki: H3View, ks: H3View, vt: H3View,
                              out: H3View, stream: H3Stream) -> c_int;
    pub fn h3_scales_workspace_bytes(cfg: *const H3AttentionCfg) -> usize;
    pub fn h3_attention_i8qk_ws(cfg: *const H3AttentionCfg, token_count: u32, heads: u32,
                                qi: H3View, qs: H3View, ki: H3View, ks: H3View, vt: H3View,
                                out: H3View, workspace: H3View, stream: H3Stream) -> c_int;
    pub fn h3_attention_i4qk_ws(cfg: *const H3AttentionCfg, token_count: u32, heads: u32,
                                qi: H3View, qs: H3View, ki: H3View, ks: H3View, vt: H3View,
                                out: H3View, workspace: H3View, stream: H3Stream) -> c_int;
    pub fn h3_attention_i4qks_ws(cfg: *const H3AttentionSkipCfg, token_count: u32, heads: u32,
                                 qi: H3View, qs: H3View, ki: H3View, ks: H3View, vt: H3View,
                                 out: H3View, workspace: H3View, stream: H3Stream) -> c_int;
    /// `h3_attention_i4qk`'s bindings and results (to the north-star tolerance) on the FP6 MFMA:
    /// the int4 codes are converted into a lent workspace of `h3_fp6_workspace_bytes(cfg)` bytes.
    pub fn h3_attention_i4qk_fp6(cfg: *const H3AttentionCfg, token_count: u32, heads: u32,
                                 qi: H3View, qs: H3View, ki: H3View, ks: H3View, vt: H3View,
                                 out: H3View, workspace: H3View, stream: H3Stream) -> c_int;
    pub fn h3_fp6_workspace_bytes(cfg: *const H3AttentionCfg) -> usize;
    /// `h3_attention_i8qk_ws` with the library's static 8 MiB device array as the workspace:
    /// allocates nothing, for callers that cannot; (kv_stride/128)·tokens ≤ 2,097,152, and
    /// calls that overlap on one GPU race on the array.
    pub fn h3_attention_i8qk_static(cfg: *const H3AttentionCfg, token_count: u32, heads: u32,
                                    qi: H3View, qs: H3View, ki: H3View, ks: H3View, vt: H3View,
                                    out: H3View, stream: H3Stream) -> c_int;
    pub fn h3_attention_i8qkhm_cross(cfg: *const H3CrossCfg, qi: H3View, qs: H3View, ki: H3View,
                                     ks: H3View, vt: H3View, key_mask: H3View, out: H3View,
                                     stream: H3Stream) -> c_int;

    // VSA block-sparse attention
    pub fn h3_vsa_gather(cfg: *const H3VsaCfg, src: H3View, x: H3View, y: H3View,
                         stream: H3Stream) -> c_int;
    pub fn h3_vsa_scatter(cfg: *const H3VsaCfg, inverse: H3View, x: H3View, y: H3View,
                          stream: H3Stream) -> c_int;
    pub fn h3_vsa_pool(cfg: *const H3VsaCfg, lengths: H3View, x: H3View, means: H3View,
                       stream: H3Stream) -> c_int;
    pub fn h3_vsa_scores(cfg: *const H3VsaCfg, qm: H3View, km: H3View, scores: H3View,
                         stream: H3Stream) -> c_int;
    pub fn h3_vsa_route(cfg: *const H3VsaCfg, scores: H3View, routes: H3View,
                        stream: H3Stream) -> c_int;
    pub fn h3_vsa_coarse(cfg: *const H3VsaCfg, scores: H3View, vm: H3View, coarse: H3View,
                         stream: H3Stream) -> c_int;
    pub fn h3_vsa_gated_scatter(cfg: *const H3VsaCfg, inverse: H3View, fine: H3View,
                                gate: H3View, coarse: H3View, out: H3View,
                                stream: H3Stream) -> c_int;
    pub fn h3_vsa_kmean(width: u32, tokens: u32, x: H3View, mean: H3View,
                        stream: H3Stream) -> c_int;
    pub fn h3_vsa_attention_i8(cfg: *const H3AttentionCfg, token_count: u32, heads: u32,
                               qi: H3View, qs: H3View, ki: H3View, ks: H3View, vt: H3View,
                               out: H3View, routes: H3View, lengths: H3View,
                               stream: H3Stream) -> c_int;
    pub fn h3_vsa_attention_i8_ws(cfg: *const H3AttentionCfg, token_count: u32, heads: u32,
                                  qi: H3View, qs: H3View, ki: H3View, ks: H3View, vt: H3View,
                                  out: H3View, routes: H3View, lengths: H3View,
                                  workspace: H3View, stream: H3Stream) -> c_int;
    pub fn h3_vsa_attention_f16(cfg: *const H3AttentionCfg, token_count: u32, heads: u32,
                                q: H3View, k: H3View, v: H3View, out: H3View, routes: H3View,
                                lengths: H3View, stream: H3Stream) -> c_int;
    pub fn h3_vsa_plan_blocks(segments: *const H3VsaSegment, n_segments: u32, nt: u32, nh: u32,
                              nw: u32, blocks: *mut u32) -> c_int;
    pub fn h3_vsa_plan(segments: *const H3VsaSegment, n_segments: u32, seq_len: u32, nt: u32,
                       nh: u32, nw: u32, src: *mut i32, inverse: *mut i32, lengths: *mut i32,
                       prefix_blocks: *mut u32) -> c_int;
    pub fn h3_vsa_validate(options: *const H3VsaOptions, attention_bits: u32) -> c_int;
    pub fn h3_vsa_topk(keep_percent: f64, nonprefix: u32) -> u32;
    pub fn h3_vsa_dense_reason(options: *const H3VsaOptions, tokens: u32, sigma: f32,
                               shift: f64) -> *const c_char;
    pub fn h3_vsa_build(src: *const i32, inverse: *const i32, lengths: *const i32, blocks: u32,
                        seq_len: u32, prefix_blocks: u32, options: *const H3VsaOptions,
                        heads: u32, layers: u32, out: *mut *mut h3_vsa) -> c_int;
    pub fn h3_vsa_build_bits(src: *const i32, inverse: *const i32, lengths: *const i32,
                             blocks: u32, seq_len: u32, prefix_blocks: u32,
                             options: *const H3VsaOptions, heads: u32, bits: u32, layers: u32,
                             out: *mut *mut h3_vsa) -> c_int;
    pub fn h3_vsa_destroy(vsa: *mut h3_vsa);
    pub fn h3_vsa_reset(vsa: *mut h3_vsa, stream: H3Stream) -> c_int;
    pub fn h3_vsa_attend(vsa: *mut h3_vsa, layer: u32, q: H3View, k: H3View, v: H3View,
                         out: H3View, gate: H3View, stream: H3Stream) -> c_int;
    pub fn h3_vsa_inspect(vsa: *const h3_vsa, layer: u32, out: *mut H3VsaBuffers) -> c_int;

    // the Stack mirror
    pub fn h3_capacity(tokens: u32, causal: c_int) -> u32;
    pub fn h3_stack_build(dims: *const H3StackDims, out: *mut *mut h3_stack) -> c_int;
    pub fn h3_stack_destroy(stack: *mut h3_stack);
    pub fn h3_stack_capacity(stack: *const h3_stack) -> u32;
    pub fn h3_stack_attend_fused(stack: *mut h3_stack, t: u32, fused: H3View, qnorm: H3View,
                                 knorm: H3View, cos_t: H3View, sin_t: H3View, out: H3View,
                                 stream: H3Stream) -> c_int;
    pub fn h3_stack_attend_compact(stack: *mut h3_stack, t: u32, compact: H3View, qnorm: H3View,
                                   knorm: H3View, cos_t: H3View, sin_t: H3View, out: H3View,
                                   stream: H3Stream) -> c_int;
    pub fn h3_stack_attend(stack: *mut h3_stack, t: u32, q: H3View, k: H3View, v: H3View,
                           out: H3View, stream: H3Stream) -> c_int;
    pub fn h3_stack_operands(stack: *const h3_stack, out: *mut H3IntQk) -> c_int;
}

/// A failed call: its status and the library's message (binding errors carry the reference's
/// text "{stage}: binding {i} is {n} bytes, the kernel addresses {need}").
#[derive(Clone, Debug, PartialEq, Eq)]
pub struct H3Error {
    pub status: c_int,
    pub message: String,
}

impl std::fmt::Display for H3Error {
    fn fmt(&self, f: &mut std::fmt::Formatter<'_>) -> std::fmt::Result {
        write!(f, "h3attn status {}: {}", self.status, self.message)
    }
}

impl std::error::Error for H3Error {}

/// `Ok(())` for `H3_OK`, else the status with `h3_last_error()`.
pub fn check(status: c_int) -> Result<(), H3Error> {
    if status == H3_OK {
        return Ok(());
    }
    // SAFETY: h3_last_error returns a NUL-terminated thread-local string that stays valid until
    // the next failing call on this thread; it is copied out here.
    let message = unsafe { CStr::from_ptr(h3_last_error()) }.to_string_lossy().into_owned();
    Err(H3Error { status, message })
}

#[cfg(test)]
mod tests {
    use super::*;
    use std::mem::size_of;

    // The struct sizes the header implies (no padding except where the header has it).
    #[test]
    fn layouts_match_the_header() {
        assert_eq!(size_of::<H3View>(), 16);
        assert_eq!(size_of::<H3PrepareCfg>(), 28);
        assert_eq!(size_of::<H3RopeCfg>(), 28);
        assert_eq!(size_of::<H3TransposeCfg>(), 12);
        assert_eq!(size_of::<H3GemmCfg>(), 16);
        assert_eq!(size_of::<H3PreparePlainCfg>(), 16);
        assert_eq!(size_of::<H3AttentionCfg>(), 24);
        assert_eq!(size_of::<H3AttentionSkipCfg>(), 28);
        assert_eq!(size_of::<H3CrossCfg>(), 28);
        assert_eq!(size_of::<H3VsaCfg>(), 28);
        assert_eq!(size_of::<H3StackDims>(), 28);
    }

    #[test]
    fn capacity_follows_the_reference() {
        // src/stack.rs:299-302
        assert_eq!(unsafe { h3_capacity(129_024, 0) }, 129_056);
        assert_eq!(unsafe { h3_capacity(1_024, 0) }, 1_056);
    }
}
