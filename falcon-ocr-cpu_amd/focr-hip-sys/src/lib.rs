//! Raw bindings to `libfocr_hip.so`, declared one for one from
//! `include/focr_hip.h`. This is the crate the Falcon-OCR runner links when
//! its `Backend` gains `Hip` (src/config.rs:19-35): `QuantLinear::from_mapped`
//! uploads each matrix once (`focr_linear_upload`), `QuantLinear::prefill` /
//! `linear` / `linear_glu` and `kernels::attention_with` call the entry points
//! below on device buffers, and every status code passes through [`check`].
//!
//! Pointers named `*_dev` are device (HBM) addresses; the others are host
//! addresses. Every function returns `FOCR_OK` (0) or a negative `FOCR_E_*`
//! code and never unwinds or aborts across the boundary.
#![allow(non_camel_case_types)]

use std::ffi::CStr;
use std::fmt;
use std::os::raw::{c_char, c_int, c_void};

/// Opaque handles.
#[repr(C)]
pub struct focr_ctx {
    _private: [u8; 0],
}
#[repr(C)]
pub struct focr_linear {
    _private: [u8; 0],
}
#[repr(C)]
pub struct focr_screen {
    _private: [u8; 0],
}
#[repr(C)]
pub struct focr_kv_split {
    _private: [u8; 0],
}

// Status codes.
pub const FOCR_OK: c_int = 0;
pub const FOCR_E_ARG: c_int = -1;
pub const FOCR_E_SHAPE: c_int = -2;
pub const FOCR_E_UNSUPPORTED: c_int = -3;
pub const FOCR_E_HIP: c_int = -4;
pub const FOCR_E_VALUE: c_int = -5;
pub const FOCR_E_NONFINITE: c_int = -6;

// Epilogue (src/kernels/panels/panel.rs:26-33).
pub const FOCR_EPI_STORE: c_int = 0;
pub const FOCR_EPI_GLU: c_int = 1;
pub const FOCR_EPI_ADD: c_int = 2;

// Prefill projection kernels, the `hip` kinds of PrefillProjection
// (src/kernels/mod.rs:71-84).
pub const FOCR_PROJ_F32_MFMA: c_int = 0;
pub const FOCR_PROJ_F32_CHAIN: c_int = 1;
pub const FOCR_PROJ_I16: c_int = 2;
pub const FOCR_PROJ_F32_SPLIT: c_int = 3;

// Prefill softmax and exp mode.
pub const FOCR_SOFTMAX_ONLINE: c_int = 0;
pub const FOCR_SOFTMAX_STATIC: c_int = 1;
pub const FOCR_EXP_FAST: c_int = 0;
pub const FOCR_EXP_EXACT: c_int = 1;

extern "C" {
    // ---- context ----------------------------------------------------------
    pub fn focr_ctx_create(device: c_int, out: *mut *mut focr_ctx) -> c_int;
    pub fn focr_ctx_destroy(ctx: *mut focr_ctx) -> c_int;
    pub fn focr_ctx_set_stream(ctx: *mut focr_ctx, hip_stream: *mut c_void) -> c_int;
    pub fn focr_ctx_use_own_stream(ctx: *mut focr_ctx) -> c_int;
    pub fn focr_ctx_stream(ctx: *const focr_ctx) -> *mut c_void;
    pub fn focr_ctx_sync(ctx: *mut focr_ctx) -> c_int;
    pub fn focr_ctx_reserve_scratch(ctx: *mut focr_ctx, bytes: usize) -> c_int;
    pub fn focr_ctx_scratch_bytes(ctx: *const focr_ctx, bytes: *mut usize) -> c_int;
    pub fn focr_last_error() -> *const c_char;
    pub fn focr_malloc(ctx: *mut focr_ctx, bytes: usize, out_dev: *mut *mut c_void) -> c_int;
    pub fn focr_free(ctx: *mut focr_ctx, dev: *mut c_void) -> c_int;
    pub fn focr_memcpy_h2d(ctx: *mut focr_ctx, dst_dev: *mut c_void, src: *const c_void, bytes: usize) -> c_int;
    pub fn focr_memcpy_d2h(ctx: *mut focr_ctx, dst: *mut c_void, src_dev: *const c_void, bytes: usize) -> c_int;

    // ---- A1: quantized linear storage (QuantLinear::from_parts / from_mapped)
    pub fn focr_linear_upload(
        ctx: *mut focr_ctx,
        bits: c_int,
        out_dim: usize,
        in_dim: usize,
        group: usize,
        codes: *const c_void,
        scales: *const f32,
        exc_cols: *const i32,
        exc_vals: *const f32,
        n_exc: usize,
        out: *mut *mut focr_linear,
    ) -> c_int;
    pub fn focr_linear_free(lin: *mut focr_linear) -> c_int;
    pub fn focr_linear_info(
        lin: *const focr_linear,
        bits: *mut c_int,
        out_dim: *mut usize,
        in_dim: *mut usize,
        group: *mut usize,
        n_exc: *mut usize,
        device_bytes: *mut usize,
    ) -> c_int;
    pub fn focr_linear_dequantize(ctx: *mut focr_ctx, lin: *const focr_linear, out_dev: *mut f32) -> c_int;

    // ---- A4 / A5: decode and draft-verify GEMV (QuantLinear::linear / linear_glu)
    pub fn focr_linear_decode(
        ctx: *mut focr_ctx,
        lin: *const focr_linear,
        x_dev: *const f32,
        rows: usize,
        out_dev: *mut f32,
    ) -> c_int;
    pub fn focr_linear_decode_glu(
        ctx: *mut focr_ctx,
        lin: *const focr_linear,
        x_dev: *const f32,
        rows: usize,
        gated_dev: *mut f32,
    ) -> c_int;
    pub fn focr_linear_decode_ex(
        ctx: *mut focr_ctx,
        lin: *const focr_linear,
        x_dev: *const f32,
        rows: usize,
        row_scale_dev: *const f32,
        rms_norm: c_int,
        epilogue: c_int,
        out_dev: *mut f32,
    ) -> c_int;

    // ---- A2 / A3: prefill projection (QuantLinear::prefill)
    pub fn focr_linear_prefill(
        ctx: *mut focr_ctx,
        lin: *const focr_linear,
        x_dev: *const f32,
        rows: usize,
        row_scale_dev: *const f32,
        epilogue: c_int,
        kernel: c_int,
        out_dev: *mut f32,
    ) -> c_int;

    // ---- A6: RMS row scales
    pub fn focr_row_scales(
        ctx: *mut focr_ctx,
        h_dev: *const f32,
        rows: usize,
        width: usize,
        eps: f32,
        out_dev: *mut f32,
    ) -> c_int;

    // ---- A7 / A8: prefill attention (kernels::attention_with)
    pub fn focr_attention_prefill(
        ctx: *mut focr_ctx,
        q_dev: *const f32,
        prefix_k_dev: *const f32,
        generated_k_dev: *const f32,
        v_dev: *const f32,
        query_len: usize,
        prefix_len: usize,
        total_len: usize,
        n_heads: usize,
        n_kv_heads: usize,
        head_dim: usize,
        query_offset: usize,
        image_start: usize,
        image_end: usize,
        sinks_dev: *const f32,
        softmax: c_int,
        exp_mode: c_int,
        out_dev: *mut f32,
    ) -> c_int;
    pub fn focr_attention_prefill_split(
        ctx: *mut focr_ctx,
        q_dev: *const f32,
        prefix_k_dev: *const f32,
        generated_k_dev: *const f32,
        v_dev: *const f32,
        query_len: usize,
        prefix_len: usize,
        total_len: usize,
        n_heads: usize,
        n_kv_heads: usize,
        head_dim: usize,
        query_offset: usize,
        image_start: usize,
        image_end: usize,
        sinks_dev: *const f32,
        softmax: c_int,
        exp_mode: c_int,
        out_dev: *mut f32,
    ) -> c_int;
    pub fn focr_attention_prefill_bf16(
        ctx: *mut focr_ctx,
        q_dev: *const f32,
        k_dev: *const f32,
        v_dev: *const f32,
        query_len: usize,
        n_heads: usize,
        n_kv_heads: usize,
        head_dim: usize,
        image_start: usize,
        image_end: usize,
        sinks_dev: *const f32,
        softmax: c_int,
        exp_mode: c_int,
        out_dev: *mut f32,
    ) -> c_int;

    // ---- the QKV row step and decode attention
    pub fn focr_qkv_rows(
        ctx: *mut focr_ctx,
        qkv_dev: *const f32,
        rows: usize,
        rope_dev: *const f32,
        n_heads: usize,
        n_kv_heads: usize,
        head_dim: usize,
        prefix_rows: usize,
        q_dev: *mut f32,
        prefix_k_dev: *mut f32,
        generated_k_dev: *mut f32,
        v_dev: *mut f32,
    ) -> c_int;
    pub fn focr_attention_decode(
        ctx: *mut focr_ctx,
        q_dev: *const f32,
        prefix_k_dev: *const f32,
        generated_k_dev: *const f32,
        v_dev: *const f32,
        query_len: usize,
        prefix_len: usize,
        total_len: usize,
        n_heads: usize,
        n_kv_heads: usize,
        head_dim: usize,
        query_offset: usize,
        image_start: usize,
        image_end: usize,
        sinks_dev: *const f32,
        out_dev: *mut f32,
    ) -> c_int;
    pub fn focr_attention_decode_row(
        ctx: *mut focr_ctx,
        qkv_dev: *const f32,
        rope_dev: *const f32,
        prefix_k_dev: *const f32,
        generated_k_dev: *mut f32,
        v_dev: *mut f32,
        prefix_len: usize,
        total_len: usize,
        n_heads: usize,
        n_kv_heads: usize,
        head_dim: usize,
        image_start: usize,
        image_end: usize,
        sinks_dev: *const f32,
        q_dev: *mut f32,
        out_dev: *mut f32,
    ) -> c_int;

    // ---- A9: greedy selection
    pub fn focr_argmax(
        ctx: *mut focr_ctx,
        logits_dev: *const f32,
        rows: usize,
        vocab: usize,
        tokens: *mut u32,
    ) -> c_int;

    // ---- sealed split KV cache (Kv::Q8 / Kv::Q16)
    pub fn focr_kv_seal(
        ctx: *mut focr_ctx,
        bits: c_int,
        prefix_k_dev: *const f32,
        v_dev: *const f32,
        prefix_len: usize,
        capacity: usize,
        n_heads: usize,
        n_kv_heads: usize,
        head_dim: usize,
        out: *mut *mut focr_kv_split,
    ) -> c_int;
    pub fn focr_kv_append(
        ctx: *mut focr_ctx,
        kv: *mut focr_kv_split,
        k_dev: *const f32,
        v_dev: *const f32,
        rows: usize,
    ) -> c_int;
    pub fn focr_kv_qkv_rows(
        ctx: *mut focr_ctx,
        kv: *mut focr_kv_split,
        qkv_dev: *const f32,
        rows: usize,
        rope_dev: *const f32,
        q_dev: *mut f32,
    ) -> c_int;
    pub fn focr_kv_decode_row(
        ctx: *mut focr_ctx,
        kv: *mut focr_kv_split,
        qkv_dev: *const f32,
        rope_dev: *const f32,
        sinks_dev: *const f32,
        q_dev: *mut f32,
        out_dev: *mut f32,
    ) -> c_int;
    pub fn focr_kv_attention_decode(
        ctx: *mut focr_ctx,
        kv: *const focr_kv_split,
        q_dev: *const f32,
        rows: usize,
        sinks_dev: *const f32,
        out_dev: *mut f32,
    ) -> c_int;
    pub fn focr_kv_attention_decode_noalloc(
        ctx: *mut focr_ctx,
        kv: *const focr_kv_split,
        q_dev: *const f32,
        rows: usize,
        sinks_dev: *const f32,
        out_dev: *mut f32,
    ) -> c_int;
    pub fn focr_kv_dequantize(
        ctx: *mut focr_ctx,
        kv: *const focr_kv_split,
        prefix_k_dev: *mut f32,
        values_dev: *mut f32,
        generated_k_dev: *mut f32,
    ) -> c_int;
    pub fn focr_kv_truncate_tail(kv: *mut focr_kv_split, tail_len: usize) -> c_int;
    pub fn focr_kv_set_fast_exp(kv: *mut focr_kv_split, fast: c_int) -> c_int;
    pub fn focr_kv_fast_exp(kv: *const focr_kv_split, fast: *mut c_int) -> c_int;
    pub fn focr_kv_info(
        kv: *const focr_kv_split,
        bits: *mut c_int,
        prefix_len: *mut usize,
        tail_len: *mut usize,
        capacity: *mut usize,
        device_bytes: *mut usize,
    ) -> c_int;
    pub fn focr_kv_free(kv: *mut focr_kv_split) -> c_int;

    // ---- INT8 screened vocabulary head (src/head_screen.rs)
    pub fn focr_screen_build(
        ctx: *mut focr_ctx,
        weights_host: *const f32,
        vocab: usize,
        dim: usize,
        out: *mut *mut focr_screen,
    ) -> c_int;
    pub fn focr_screen_upload(
        ctx: *mut focr_ctx,
        codes_host: *const i8,
        scales_host: *const f32,
        vocab: usize,
        dim: usize,
        weight_abs_max: f32,
        kappa: f32,
        out: *mut *mut focr_screen,
    ) -> c_int;
    pub fn focr_screen_free(screen: *mut focr_screen) -> c_int;
    pub fn focr_screen_constants(screen: *const focr_screen, weight_abs_max: *mut f32, kappa: *mut f32) -> c_int;
    pub fn focr_screen_bounds(screen: *const focr_screen, rows: usize, upper_host: *mut f32) -> c_int;
    pub fn focr_screen_select(
        ctx: *mut focr_ctx,
        screen: *const focr_screen,
        fp32_head: *const focr_linear,
        x_dev: *const f32,
        rows: usize,
        tokens: *mut i32,
        candidates: *mut u32,
    ) -> c_int;
}

/// A failed call: the status code and `focr_last_error()`'s message, the
/// counterpart of the reference's `anyhow` errors and shape assertions.
#[derive(Debug, Clone, PartialEq, Eq)]
pub struct Error {
    pub code: c_int,
    pub message: String,
}

impl fmt::Display for Error {
    fn fmt(&self, f: &mut fmt::Formatter<'_>) -> fmt::Result {
        write!(f, "focr_hip error {}: {}", self.code, self.message)
    }
}

impl std::error::Error for Error {}

/// `Ok(())` for FOCR_OK, otherwise the code with the calling thread's last
/// error message.
pub fn check(rc: c_int) -> Result<(), Error> {
    if rc == FOCR_OK {
        return Ok(());
    }
    // SAFETY: focr_last_error returns a NUL-terminated string owned by the
    // library's thread-local state, valid until the thread's next call.
    let message = unsafe { CStr::from_ptr(focr_last_error()) }.to_string_lossy().into_owned();
    Err(Error { code: rc, message })
}
