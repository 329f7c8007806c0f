//! Raw declarations of the C ABI in include/diffrast_hip.h, one item per
//! declaration there, in the same order, with the same parameter names
//! (lower-cased) and `#[repr(C)]` structs with the same fields in the same
//! order. Every function returns a status code (`DRH_OK` or `DRH_ERR_*`); the
//! message of the calling thread's last failure is `drh_last_error()`.
//!
//! Pointers are device pointers unless `DRH_HOST_PTRS` is in `flags`; with
//! device pointers a call only enqueues work on `stream` (a `hipStream_t`, null
//! for the null stream) and returns.

#![allow(non_camel_case_types)]

use std::os::raw::{c_char, c_int, c_void};

pub const DRH_OK: c_int = 0;
pub const DRH_ERR_NO_DEVICE: c_int = 1;
pub const DRH_ERR_TIMEOUT: c_int = 2;
pub const DRH_ERR_DEVICE: c_int = 3;
pub const DRH_ERR_READBACK: c_int = 4;
pub const DRH_ERR_TOO_LARGE: c_int = 5;
pub const DRH_ERR_INVALID_ARG: c_int = 6;

pub const DRH_HOST_PTRS: u32 = 0x1;
pub const DRH_SYNC: u32 = 0x2;
pub const DRH_EXACT_MATH: u32 = 0x4;
pub const DRH_DETERMINISTIC: u32 = 0x8;
pub const DRH_CHANNELS_FIRST: u32 = 0x10;
pub const DRH_PHASES: u32 = 0x20;

pub const DRH_WAIT_TIMEOUT_S: u64 = 60;

pub const DRH_STOP_COMPLETED: i32 = 0;
pub const DRH_STOP_CONVERGED: i32 = 1;
pub const DRH_STOP_DIVERGED: i32 = 2;

pub const DRH_CFG_OK: c_int = 0;
pub const DRH_CFG_NO_TRIANGLES: c_int = 1;
pub const DRH_CFG_NON_POSITIVE_SIGMA: c_int = 2;
pub const DRH_CFG_SIGMA_NOT_DECREASING: c_int = 3;
pub const DRH_CFG_NON_POSITIVE_LEARNING_RATE: c_int = 4;

/// `drh_ctx`: a device, its buffer pool and its timing state.
#[repr(C)]
pub struct drh_ctx {
    _opaque: [u8; 0],
}

/// `drh_fitter`: a fit advanced one iteration at a time.
#[repr(C)]
pub struct drh_fitter {
    _opaque: [u8; 0],
}

#[repr(C)]
#[derive(Clone, Copy, Debug, Default)]
pub struct drh_timings {
    pub setup_ms: f64,
    pub raster_ms: f64,
    pub reduce_ms: f64,
    pub adam_ms: f64,
    pub setup_n: i64,
    pub raster_n: i64,
    pub reduce_n: i64,
    pub adam_n: i64,
    pub backward_ms: f64,
    pub backward_n: i64,
}

#[repr(C)]
#[derive(Clone, Copy, Debug, Default)]
pub struct drh_phase_timings {
    pub pack_ms: f64,
    pub alloc_ms: f64,
    pub dispatch_ms: f64,
    pub readback_ms: f64,
    pub loss_ms: f64,
    pub total_ms: f64,
}

#[repr(C)]
#[derive(Clone, Copy, Debug, Default)]
pub struct drh_fit_config {
    pub iters: i64,
    pub sigma_start: f32,
    pub sigma_end: f32,
    pub lr_pos: f32,
    pub lr_color: f32,
    pub lr_alpha: f32,
    pub patience: i64,
    pub min_delta: f32,
}

#[repr(C)]
#[derive(Clone, Copy, Debug, Default)]
pub struct drh_fit_report {
    pub n_losses: i64,
    pub best_iter: i64,
    pub best_loss: f32,
    pub stop_reason: i32,
}

#[repr(C)]
#[derive(Clone, Copy, Debug, Default)]
pub struct drh_step_info {
    pub iter: i64,
    pub loss: f32,
    pub sigma: f32,
}

#[repr(C)]
#[derive(Clone, Copy, Debug, Default)]
pub struct drh_fit_status {
    pub iter: i64,
    pub best_iter: i64,
    pub best_loss: f32,
    pub sigma: f32,
    pub done: i32,
    pub stop_reason: i32,
}

extern "C" {
    pub fn drh_create(out: *mut *mut drh_ctx) -> c_int;
    pub fn drh_destroy(ctx: *mut drh_ctx) -> c_int;
    pub fn drh_last_error() -> *const c_char;
    pub fn drh_device_info(ctx: *const drh_ctx, buf: *mut c_char, len: usize) -> c_int;
    pub fn drh_is_discrete(ctx: *const drh_ctx) -> c_int;
    pub fn drh_params_per_triangle() -> c_int;
    pub fn drh_pool_stats(ctx: *mut drh_ctx, hits: *mut u64, misses: *mut u64, bytes: *mut u64) -> c_int;
    pub fn drh_clear_pool(ctx: *mut drh_ctx) -> c_int;

    pub fn drh_timing_enable(ctx: *mut drh_ctx, enable: c_int) -> c_int;
    pub fn drh_timing_read(ctx: *mut drh_ctx, out: *mut drh_timings) -> c_int;
    pub fn drh_phases_read(out: *mut drh_phase_timings) -> c_int;

    pub fn drh_render(
        ctx: *mut drh_ctx,
        params: *const f32,
        backgrounds: *const f32,
        b: i64,
        t: i64,
        h: i64,
        w: i64,
        sigma: f32,
        out_images: *mut f32,
        stream: *mut c_void,
        flags: u32,
    ) -> c_int;

    pub fn drh_fused_loss_backward(
        ctx: *mut drh_ctx,
        params: *const f32,
        backgrounds: *const f32,
        targets: *const f32,
        b: i64,
        t: i64,
        h: i64,
        w: i64,
        sigma: f32,
        out_losses: *mut f32,
        out_grads: *mut f32,
        out_images: *mut f32,
        stream: *mut c_void,
        flags: u32,
    ) -> c_int;

    pub fn drh_fused_loss_backward_noalloc(
        ctx: *mut drh_ctx,
        params: *const f32,
        backgrounds: *const f32,
        targets: *const f32,
        b: i64,
        t: i64,
        h: i64,
        w: i64,
        sigma: f32,
        out_losses: *mut f32,
        out_grads: *mut f32,
        out_images: *mut f32,
        stream: *mut c_void,
        flags: u32,
    ) -> c_int;

    pub fn drh_backward_from_grad(
        ctx: *mut drh_ctx,
        params: *const f32,
        backgrounds: *const f32,
        grad_images: *const f32,
        b: i64,
        t: i64,
        h: i64,
        w: i64,
        sigma: f32,
        out_grads: *mut f32,
        stream: *mut c_void,
        flags: u32,
    ) -> c_int;

    pub fn drh_record_bytes(b: i64, t: i64, h: i64, w: i64, out_bytes: *mut u64) -> c_int;

    pub fn drh_render_record(
        ctx: *mut drh_ctx,
        params: *const f32,
        backgrounds: *const f32,
        b: i64,
        t: i64,
        h: i64,
        w: i64,
        sigma: f32,
        out_images: *mut f32,
        record: *mut c_void,
        record_bytes: u64,
        stream: *mut c_void,
        flags: u32,
    ) -> c_int;

    pub fn drh_backward_recorded(
        ctx: *mut drh_ctx,
        record: *const c_void,
        record_bytes: u64,
        grad_images: *const f32,
        b: i64,
        t: i64,
        h: i64,
        w: i64,
        sigma: f32,
        out_grads: *mut f32,
        stream: *mut c_void,
        flags: u32,
    ) -> c_int;

    pub fn drh_adam_project_step(
        ctx: *mut drh_ctx,
        params: *mut f32,
        grads: *const f32,
        m: *mut f32,
        v: *mut f32,
        lr: *const f32,
        n: i64,
        step: u32,
        beta1: f32,
        beta2: f32,
        eps: f32,
        project: c_int,
        stream: *mut c_void,
        flags: u32,
    ) -> c_int;

    pub fn drh_fit_validate(cfg: *const drh_fit_config, t: i64) -> c_int;

    pub fn drh_fit(
        ctx: *mut drh_ctx,
        target: *const f32,
        h: i64,
        w: i64,
        background: *const f32,
        init_params: *const f32,
        t: i64,
        cfg: *const drh_fit_config,
        out_losses: *mut f32,
        out_best_params: *mut f32,
        out_params: *mut f32,
        report: *mut drh_fit_report,
        stream: *mut c_void,
        flags: u32,
    ) -> c_int;

    pub fn drh_fitter_create(
        ctx: *mut drh_ctx,
        target: *const f32,
        h: i64,
        w: i64,
        background: *const f32,
        init_params: *const f32,
        t: i64,
        cfg: *const drh_fit_config,
        stream: *mut c_void,
        flags: u32,
        out: *mut *mut drh_fitter,
    ) -> c_int;
    pub fn drh_fitter_destroy(f: *mut drh_fitter) -> c_int;
    pub fn drh_fitter_step(f: *mut drh_fitter, stepped: *mut c_int, info: *mut drh_step_info) -> c_int;
    pub fn drh_fitter_run(f: *mut drh_fitter, max_steps: i64, ran: *mut i64) -> c_int;
    pub fn drh_fitter_status(f: *const drh_fitter, out: *mut drh_fit_status) -> c_int;
    pub fn drh_fitter_scene(f: *mut drh_fitter, out_params: *mut f32, flags: u32) -> c_int;
    pub fn drh_fitter_losses(f: *mut drh_fitter, out: *mut f32, capacity: i64, n_out: *mut i64, flags: u32) -> c_int;
    pub fn drh_fitter_render_current(f: *mut drh_fitter, out_image: *mut f32, flags: u32) -> c_int;
    pub fn drh_fitter_report(
        f: *mut drh_fitter,
        out_best_params: *mut f32,
        report: *mut drh_fit_report,
        flags: u32,
    ) -> c_int;

    pub fn drh_encode_srgb(
        ctx: *mut drh_ctx,
        values: *const f32,
        n: i64,
        out: *mut u8,
        stream: *mut c_void,
        flags: u32,
    ) -> c_int;
    pub fn drh_decode_srgb(
        ctx: *mut drh_ctx,
        bytes: *const u8,
        n: i64,
        out: *mut f32,
        stream: *mut c_void,
        flags: u32,
    ) -> c_int;

    pub fn drh_resize_lanczos3(
        ctx: *mut drh_ctx,
        src: *const u8,
        h: i64,
        w: i64,
        c: i64,
        dst: *mut u8,
        new_h: i64,
        new_w: i64,
        stream: *mut c_void,
        flags: u32,
    ) -> c_int;
}
