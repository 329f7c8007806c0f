//! diffrast on AMD Instinct MI355X (gfx950) through libdiffrast_hip's C ABI.
//!
//! Two layers, both over [`ffi`]:
//!
//! * [`GpuRasterizer`] has the methods of `diffrast_gpu::GpuRasterizer`
//!   (crates/diffrast-gpu/src/lib.rs:232-910) with the same names, arguments
//!   and error type, so a caller switches backends by changing the import.
//! * The free functions [`render`], [`render_batch`], [`render_with_tape`],
//!   [`backward`], [`backward_batch`] and [`fit`] and the step-wise [`Fitter`]
//!   have the signatures of the `diffrast` crate's (crates/diffrast/src/lib.rs:18-24,
//!   fit.rs:166-335). They run on one rasterizer shared by the process and
//!   panic with the device's message where the CPU versions cannot fail,
//!   since there is no CPU fallback behind them.
//!
//! Results follow the CPU crate's semantics (raster.rs, grad.rs, fit.rs): the
//! library's tests compare every entry point with a CPU restatement of those
//! files at 1e-5 per pixel, 1e-4 relative per loss and 1e-4 of each parameter
//! group's gradient norm.

pub mod ffi;

use std::ffi::CStr;
use std::os::raw::{c_char, c_int};
use std::ptr::{self, NonNull};
use std::sync::OnceLock;
use std::time::{Duration, Instant};

use rand::rngs::StdRng;
use rand::{Rng, SeedableRng};

pub use diffrast::{
    fit_within, scene_to_json, Adam, Canvas, ConfigError, FitConfig, FitProgress, FitReport, RenderParams, Scene,
    StepInfo, StopReason, Triangle,
};

const NP: usize = Triangle::N_PARAMS;

/// Something went wrong talking to the GPU: the variants of
/// `diffrast_gpu::GpuError` (crates/diffrast-gpu/src/lib.rs:42-50), one per
/// status code 1-5 of the C ABI. Code 6, an argument the library rejects
/// (sizes that do not match, a non-positive sigma), is reported as
/// `TooLarge` with the library's message, as the reference reports its own
/// batch-shape mismatches.
#[derive(Debug)]
pub enum GpuError {
    NoAdapter,
    /// A host wait exceeded [`GpuRasterizer::POLL_TIMEOUT`].
    Timeout,
    DeviceRequest(String),
    Readback(String),
    TooLarge(String),
}

impl std::fmt::Display for GpuError {
    fn fmt(&self, f: &mut std::fmt::Formatter<'_>) -> std::fmt::Result {
        match self {
            Self::NoAdapter => write!(f, "no HIP device found: check that the GPU is visible (rocm-smi)"),
            Self::Timeout => write!(
                f,
                "the GPU did not finish within {:?}: another process may hold it, or the batch is too large \
                 for one call",
                GpuRasterizer::POLL_TIMEOUT
            ),
            Self::DeviceRequest(m) => write!(f, "HIP runtime error: {m}"),
            Self::Readback(m) => write!(f, "could not copy results to the host: {m}"),
            Self::TooLarge(m) => write!(f, "{m}"),
        }
    }
}

impl std::error::Error for GpuError {}

fn last_error() -> String {
    // SAFETY: drh_last_error returns a NUL-terminated string owned by the
    // calling thread, valid until that thread's next failing call.
    let p: *const c_char = unsafe { ffi::drh_last_error() };
    if p.is_null() {
        return String::new();
    }
    unsafe { CStr::from_ptr(p) }.to_string_lossy().into_owned()
}

fn check(rc: c_int) -> Result<(), GpuError> {
    match rc {
        ffi::DRH_OK => Ok(()),
        ffi::DRH_ERR_NO_DEVICE => Err(GpuError::NoAdapter),
        ffi::DRH_ERR_TIMEOUT => Err(GpuError::Timeout),
        ffi::DRH_ERR_DEVICE => Err(GpuError::DeviceRequest(last_error())),
        ffi::DRH_ERR_READBACK => Err(GpuError::Readback(last_error())),
        _ => Err(GpuError::TooLarge(last_error())),
    }
}

fn ms_since(t: Instant) -> f32 {
    t.elapsed().as_secs_f32() * 1e3
}

/// How the batched backward pass sums gradients over pixels
/// (`diffrast_gpu::ReduceMode`, crates/diffrast-gpu/src/lib.rs:76-85).
///
/// The kernels reduce each 16x16 block's pixels in local memory first in
/// every mode. `Direct` and `Workgroup` then add one float atomic per triangle
/// parameter per block; `Deterministic` writes per-block partial rows and sums
/// them in a fixed order, so repeated calls give identical bits.
#[derive(Clone, Copy, Debug, PartialEq, Eq, Default)]
pub enum ReduceMode {
    Direct,
    #[default]
    Workgroup,
    Deterministic,
}

impl ReduceMode {
    fn flags(self) -> u32 {
        match self {
            Self::Direct | Self::Workgroup => 0,
            Self::Deterministic => ffi::DRH_DETERMINISTIC,
        }
    }
}

/// How the backward pass recovers the canvas beneath each triangle
/// (`diffrast_gpu::BackwardMode`, crates/diffrast-gpu/src/lib.rs:211-220).
///
/// Both modes run the same kernels: the forward pass keeps, per pixel, the
/// transmittance and colour state the backward pass needs and, per 8x8 tile,
/// the list of triangles that reach it. That is the taped design's O(T)
/// backward at a memory cost of O(pixels + tiles x listed triangles)
/// ([`GpuRasterizer::tape_bytes`]), not O(T x pixels).
#[derive(Clone, Copy, Debug, PartialEq, Eq)]
pub enum BackwardMode {
    Taped,
    Recompute,
}

/// Per-item `(loss, gradients)`, one entry per scene in a batch.
pub type BatchGradients = Vec<(f32, Vec<f32>)>;

/// Where the time went inside one batched backward call
/// (`diffrast_gpu::BackwardTimings`, crates/diffrast-gpu/src/lib.rs:96-114).
///
/// From [`GpuRasterizer::backward_many_timed`] the phases are separated by
/// waiting for the device between them (`DRH_PHASES`), so the total bounds the
/// untimed call from above. `loss_ms` stays 0: the per-item loss is reduced on
/// the device, inside `dispatch_ms`.
#[derive(Clone, Copy, Debug, Default)]
pub struct BackwardTimings {
    /// Flattening the scenes and filling the parameter and background buffers.
    pub pack_ms: f32,
    /// Taking the target, image, gradient and loss buffers (targets filled).
    pub alloc_ms: f32,
    /// Every kernel enqueued and finished.
    pub dispatch_ms: f32,
    /// Copying the results back and splitting them per item.
    pub readback_ms: f32,
    /// Reducing the per-item loss on the host.
    pub loss_ms: f32,
}

impl BackwardTimings {
    pub fn total_ms(&self) -> f32 {
        self.pack_ms + self.alloc_ms + self.dispatch_ms + self.readback_ms + self.loss_ms
    }
}

/// Pool counters (`diffrast_gpu::PoolStats`, crates/diffrast-gpu/src/lib.rs:148-158).
#[derive(Clone, Copy, Debug, Default, PartialEq, Eq)]
pub struct PoolStats {
    pub hits: u64,
    pub misses: u64,
    pub bytes: u64,
}

/// Accumulated device time per kernel since the last read
/// ([`GpuRasterizer::kernel_timings`]).
#[derive(Clone, Copy, Debug, Default)]
pub struct KernelTimings {
    pub setup_ms: f64,
    pub forward_ms: f64,
    pub backward_ms: f64,
    pub reduce_ms: f64,
    pub adam_ms: f64,
    pub launches: i64,
}

/// A batch flattened into the C ABI's layout: params B x T x 10, backgrounds B x 3.
struct Packed {
    b: usize,
    t: usize,
    params: Vec<f32>,
    backgrounds: Vec<f32>,
}

impl Packed {
    /// The reference's check_batch (crates/diffrast-gpu/src/lib.rs:914-929):
    /// `None` for an empty batch, an error for a ragged one.
    fn new(scenes: &[Scene]) -> Result<Option<Self>, GpuError> {
        let Some(first) = scenes.first() else { return Ok(None) };
        let t = first.len();
        if let Some(i) = scenes.iter().position(|s| s.len() != t) {
            return Err(GpuError::TooLarge(format!(
                "every scene in a batch must have the same triangle count: item 0 has {t}, item {i} has {}",
                scenes[i].len()
            )));
        }
        let mut params = Vec::with_capacity(scenes.len() * t * NP);
        let mut backgrounds = Vec::with_capacity(scenes.len() * 3);
        for s in scenes {
            params.extend(s.params());
            backgrounds.extend_from_slice(&s.background);
        }
        Ok(Some(Self { b: scenes.len(), t, params, backgrounds }))
    }
}

fn dims(p: &RenderParams) -> (i64, i64) {
    (p.height as i64, p.width as i64)
}

fn canvases(data: &[f32], p: RenderParams) -> Vec<Canvas> {
    let n = p.width * p.height * 3;
    if n == 0 {
        return Vec::new();
    }
    data.chunks_exact(n).map(|c| Canvas { width: p.width, height: p.height, data: c.to_vec() }).collect()
}

fn check_targets(targets: &[Canvas], p: &RenderParams) -> Result<(), GpuError> {
    for (i, c) in targets.iter().enumerate() {
        if c.width != p.width || c.height != p.height || c.data.len() != p.width * p.height * 3 {
            return Err(GpuError::TooLarge(format!(
                "target {i} is {}x{} ({} values), the render is {}x{}",
                c.width,
                c.height,
                c.data.len(),
                p.width,
                p.height
            )));
        }
    }
    Ok(())
}

/// The device, its buffer pool and compiled kernels.
///
/// Creating one initialises the HIP runtime and the pool; build one and reuse
/// it. It is safe to share between threads: the library locks its pool and
/// orders buffer reuse across streams.
pub struct GpuRasterizer {
    ctx: NonNull<ffi::drh_ctx>,
    info: String,
    discrete: bool,
}

// SAFETY: the C context is internally locked (include/diffrast_hip.h: "A
// context is safe to use from several threads at once").
unsafe impl Send for GpuRasterizer {}
unsafe impl Sync for GpuRasterizer {}

impl Drop for GpuRasterizer {
    fn drop(&mut self) {
        // SAFETY: ctx came from drh_create and is destroyed once.
        unsafe { ffi::drh_destroy(self.ctx.as_ptr()) };
    }
}

impl GpuRasterizer {
    /// How long a host wait lasts before the call fails with
    /// [`GpuError::Timeout`] (crates/diffrast-gpu/src/lib.rs:229).
    pub const POLL_TIMEOUT: Duration = Duration::from_secs(ffi::DRH_WAIT_TIMEOUT_S);

    pub fn new() -> Result<Self, GpuError> {
        let mut raw = ptr::null_mut();
        // SAFETY: drh_create writes a context pointer on success.
        check(unsafe { ffi::drh_create(&mut raw) })?;
        let ctx = NonNull::new(raw).ok_or_else(|| GpuError::DeviceRequest("drh_create returned NULL".into()))?;
        let mut buf = vec![0 as c_char; 256];
        // SAFETY: buf holds len bytes; the library NUL-terminates within them.
        let rc = unsafe { ffi::drh_device_info(ctx.as_ptr(), buf.as_mut_ptr(), buf.len()) };
        let info = if rc == ffi::DRH_OK {
            unsafe { CStr::from_ptr(buf.as_ptr()) }.to_string_lossy().into_owned()
        } else {
            String::new()
        };
        let discrete = unsafe { ffi::drh_is_discrete(ctx.as_ptr()) } != 0;
        Ok(Self { ctx, info, discrete })
    }

    fn raw(&self) -> *mut ffi::drh_ctx {
        self.ctx.as_ptr()
    }

    /// Reuse counters of the buffer pool.
    pub fn pool_stats(&self) -> PoolStats {
        let mut s = PoolStats::default();
        // SAFETY: three valid out-pointers.
        let _ = unsafe { ffi::drh_pool_stats(self.raw(), &mut s.hits, &mut s.misses, &mut s.bytes) };
        s
    }

    /// Free every pooled buffer.
    pub fn clear_pool(&self) {
        // SAFETY: a live context.
        let _ = unsafe { ffi::drh_clear_pool(self.raw()) };
    }

    /// Device name, architecture and compute-unit count.
    pub fn adapter_info(&self) -> &str {
        &self.info
    }

    /// Whether the device has its own memory (an Instinct card does).
    pub fn is_discrete(&self) -> bool {
        self.discrete
    }

    /// Bytes of the record one scene's backward pass reads (per-pixel state,
    /// per-tile triangle lists, triangle records): the counterpart of the
    /// reference's tape size (crates/diffrast-gpu/src/lib.rs:389-393). 0 for
    /// an empty canvas.
    pub fn tape_bytes(n_tris: usize, width: usize, height: usize) -> u64 {
        let mut out = 0u64;
        // SAFETY: host-only sizing with a valid out-pointer.
        let rc = unsafe { ffi::drh_record_bytes(1, n_tris as i64, height as i64, width as i64, &mut out) };
        if rc == ffi::DRH_OK {
            out
        } else {
            0
        }
    }

    /// Render one scene (crates/diffrast-gpu/src/lib.rs:414-418).
    pub fn render(&self, scene: &Scene, p: RenderParams) -> Result<Canvas, GpuError> {
        Ok(self.render_many(std::slice::from_ref(scene), p)?.remove(0))
    }

    /// `(loss, gradients)` of one scene, 10 values per triangle
    /// (crates/diffrast-gpu/src/lib.rs:498-510).
    pub fn backward(&self, scene: &Scene, p: RenderParams, target: &Canvas) -> Result<(f32, Vec<f32>), GpuError> {
        self.backward_with(scene, p, target, BackwardMode::Recompute)
    }

    /// As [`Self::backward`] with an explicit [`BackwardMode`]
    /// (crates/diffrast-gpu/src/lib.rs:512-523); both modes give the same
    /// result here.
    pub fn backward_with(
        &self,
        scene: &Scene,
        p: RenderParams,
        target: &Canvas,
        mode: BackwardMode,
    ) -> Result<(f32, Vec<f32>), GpuError> {
        assert_eq!(target.width, p.width, "target width mismatch");
        assert_eq!(target.height, p.height, "target height mismatch");
        let _ = mode;
        let mut r = self.backward_many(std::slice::from_ref(scene), p, std::slice::from_ref(target))?;
        Ok(r.remove(0))
    }

    /// Render a batch of scenes with one triangle count in one call
    /// (crates/diffrast-gpu/src/lib.rs:606-633).
    pub fn render_many(&self, scenes: &[Scene], p: RenderParams) -> Result<Vec<Canvas>, GpuError> {
        let Some(batch) = Packed::new(scenes)? else { return Ok(Vec::new()) };
        let (h, w) = dims(&p);
        let mut out = vec![0.0f32; batch.b * p.width * p.height * 3];
        // SAFETY: host arrays of the sizes the call reads and writes.
        check(unsafe {
            ffi::drh_render(
                self.raw(),
                batch.params.as_ptr(),
                batch.backgrounds.as_ptr(),
                batch.b as i64,
                batch.t as i64,
                h,
                w,
                p.sigma,
                out.as_mut_ptr(),
                ptr::null_mut(),
                ffi::DRH_HOST_PTRS,
            )
        })?;
        Ok(canvases(&out, p))
    }

    /// Render and differentiate a batch in one call
    /// (crates/diffrast-gpu/src/lib.rs:635-646).
    pub fn backward_many(&self, scenes: &[Scene], p: RenderParams, targets: &[Canvas]) -> Result<BatchGradients, GpuError> {
        self.backward_many_inner(scenes, p, targets, ReduceMode::default(), false).map(|(r, _)| r)
    }

    /// As [`Self::backward_many`], with the time of each phase
    /// (crates/diffrast-gpu/src/lib.rs:648-664).
    pub fn backward_many_timed(
        &self,
        scenes: &[Scene],
        p: RenderParams,
        targets: &[Canvas],
    ) -> Result<(BatchGradients, BackwardTimings), GpuError> {
        self.backward_many_inner(scenes, p, targets, ReduceMode::default(), true)
    }

    /// Choose how gradients are reduced (crates/diffrast-gpu/src/lib.rs:665-675).
    /// The phases are not separated: `pack_ms` is the host flattening and
    /// `dispatch_ms` the whole library call.
    pub fn backward_many_full(
        &self,
        scenes: &[Scene],
        p: RenderParams,
        targets: &[Canvas],
        reduce: ReduceMode,
    ) -> Result<(BatchGradients, BackwardTimings), GpuError> {
        self.backward_many_inner(scenes, p, targets, reduce, false)
    }

    fn backward_many_inner(
        &self,
        scenes: &[Scene],
        p: RenderParams,
        targets: &[Canvas],
        reduce: ReduceMode,
        phases: bool,
    ) -> Result<(BatchGradients, BackwardTimings), GpuError> {
        let mut t = BackwardTimings::default();
        if scenes.len() != targets.len() {
            return Err(GpuError::TooLarge(format!(
                "batch mismatch: {} scenes but {} targets",
                scenes.len(),
                targets.len()
            )));
        }
        let clock = Instant::now();
        let Some(batch) = Packed::new(scenes)? else { return Ok((Vec::new(), t)) };
        check_targets(targets, &p)?;
        let mut packed_targets = Vec::with_capacity(batch.b * p.width * p.height * 3);
        for c in targets {
            packed_targets.extend_from_slice(&c.data);
        }
        t.pack_ms = ms_since(clock);

        let (h, w) = dims(&p);
        let mut losses = vec![0.0f32; batch.b];
        let mut grads = vec![0.0f32; batch.b * batch.t * NP];
        let flags = ffi::DRH_HOST_PTRS | reduce.flags() | if phases { ffi::DRH_PHASES } else { 0 };
        let call = Instant::now();
        // SAFETY: host arrays of the sizes the call reads and writes; no image output.
        check(unsafe {
            ffi::drh_fused_loss_backward(
                self.raw(),
                batch.params.as_ptr(),
                batch.backgrounds.as_ptr(),
                packed_targets.as_ptr(),
                batch.b as i64,
                batch.t as i64,
                h,
                w,
                p.sigma,
                losses.as_mut_ptr(),
                grads.as_mut_ptr(),
                ptr::null_mut(),
                ptr::null_mut(),
                flags,
            )
        })?;
        if phases {
            let mut ph = ffi::drh_phase_timings::default();
            // SAFETY: a valid out-pointer; the phases are this thread's last call's.
            check(unsafe { ffi::drh_phases_read(&mut ph) })?;
            t.pack_ms += ph.pack_ms as f32;
            t.alloc_ms = ph.alloc_ms as f32;
            t.dispatch_ms = ph.dispatch_ms as f32;
            t.readback_ms = ph.readback_ms as f32;
            t.loss_ms = ph.loss_ms as f32;
        } else {
            t.dispatch_ms = ms_since(call);
        }

        let split = Instant::now();
        let per = batch.t * NP;
        let out: BatchGradients = losses
            .into_iter()
            .enumerate()
            .map(|(i, l)| (l, grads[i * per..(i + 1) * per].to_vec()))
            .collect();
        t.readback_ms += ms_since(split);
        Ok((out, t))
    }

    /// Parameter gradients from an upstream image gradient dL/dpixel,
    /// `(batch, height, width, 3)` flattened (crates/diffrast-gpu/src/lib.rs:815-910).
    pub fn backward_many_from_grad(
        &self,
        scenes: &[Scene],
        p: RenderParams,
        grad_images: &[f32],
    ) -> Result<Vec<Vec<f32>>, GpuError> {
        let Some(batch) = Packed::new(scenes)? else { return Ok(Vec::new()) };
        let expected = batch.b * p.width * p.height * 3;
        if grad_images.len() != expected {
            return Err(GpuError::TooLarge(format!(
                "expected {expected} gradient values, got {}",
                grad_images.len()
            )));
        }
        let (h, w) = dims(&p);
        let mut grads = vec![0.0f32; batch.b * batch.t * NP];
        // SAFETY: host arrays of the sizes the call reads and writes.
        check(unsafe {
            ffi::drh_backward_from_grad(
                self.raw(),
                batch.params.as_ptr(),
                batch.backgrounds.as_ptr(),
                grad_images.as_ptr(),
                batch.b as i64,
                batch.t as i64,
                h,
                w,
                p.sigma,
                grads.as_mut_ptr(),
                ptr::null_mut(),
                ffi::DRH_HOST_PTRS,
            )
        })?;
        let per = batch.t * NP;
        Ok((0..batch.b).map(|i| grads[i * per..(i + 1) * per].to_vec()).collect())
    }

    /// Bracket every kernel with device events from now on (`true`) or stop.
    pub fn set_kernel_timing(&self, enable: bool) -> Result<(), GpuError> {
        // SAFETY: a live context.
        check(unsafe { ffi::drh_timing_enable(self.raw(), enable as c_int) })
    }

    /// Device milliseconds per kernel since the last read; resets them.
    pub fn kernel_timings(&self) -> Result<KernelTimings, GpuError> {
        let mut raw = ffi::drh_timings::default();
        // SAFETY: a valid out-pointer.
        check(unsafe { ffi::drh_timing_read(self.raw(), &mut raw) })?;
        Ok(KernelTimings {
            setup_ms: raw.setup_ms,
            forward_ms: raw.raster_ms,
            backward_ms: raw.backward_ms,
            reduce_ms: raw.reduce_ms,
            adam_ms: raw.adam_ms,
            launches: raw.setup_n + raw.raster_n + raw.backward_n + raw.reduce_n + raw.adam_n,
        })
    }

    /// Linear values to sRGB bytes as `Canvas::save_png` encodes them
    /// (crates/diffrast/src/canvas.rs:61-68, 100-105), bit for bit.
    pub fn encode_srgb(&self, values: &[f32]) -> Result<Vec<u8>, GpuError> {
        let mut out = vec![0u8; values.len()];
        // SAFETY: host arrays of n elements each.
        check(unsafe {
            ffi::drh_encode_srgb(
                self.raw(),
                values.as_ptr(),
                values.len() as i64,
                out.as_mut_ptr(),
                ptr::null_mut(),
                ffi::DRH_HOST_PTRS,
            )
        })?;
        Ok(out)
    }

    /// sRGB bytes to linear values as `Canvas::load_image` decodes them
    /// (canvas.rs:70-86, 108-115).
    pub fn decode_srgb(&self, bytes: &[u8]) -> Result<Vec<f32>, GpuError> {
        let mut out = vec![0.0f32; bytes.len()];
        // SAFETY: host arrays of n elements each.
        check(unsafe {
            ffi::drh_decode_srgb(
                self.raw(),
                bytes.as_ptr(),
                bytes.len() as i64,
                out.as_mut_ptr(),
                ptr::null_mut(),
                ffi::DRH_HOST_PTRS,
            )
        })?;
        Ok(out)
    }

    /// The resample of `Canvas::load_image` (canvas.rs:71-79): image 0.25's
    /// `resize_exact(new_width, new_height, FilterType::Lanczos3)` of a
    /// `height x width x channels` byte image (channels 1-4), bit for bit.
    /// Feed the result to [`Self::decode_srgb`] for the linear canvas.
    pub fn resize_lanczos3(
        &self,
        image: &[u8],
        width: usize,
        height: usize,
        channels: usize,
        new_width: usize,
        new_height: usize,
    ) -> Result<Vec<u8>, GpuError> {
        if image.len() != width * height * channels {
            return Err(GpuError::TooLarge(format!(
                "expected {} bytes for {width}x{height}x{channels}, got {}",
                width * height * channels,
                image.len()
            )));
        }
        let mut out = vec![0u8; new_width * new_height * channels];
        // SAFETY: host arrays of the sizes the call reads and writes.
        check(unsafe {
            ffi::drh_resize_lanczos3(
                self.raw(),
                image.as_ptr(),
                height as i64,
                width as i64,
                channels as i64,
                out.as_mut_ptr(),
                new_height as i64,
                new_width as i64,
                ptr::null_mut(),
                ffi::DRH_HOST_PTRS,
            )
        })?;
        Ok(out)
    }

    /// A step-wise fit on this device (`diffrast::Fitter::new`, fit.rs:214-237).
    pub fn fitter(&self, target: Canvas, cfg: FitConfig) -> Result<Fitter<'_>, FitError> {
        Fitter::on(self, target, cfg)
    }

    /// The batch fit with a per-iteration callback (`diffrast::fit`,
    /// fit.rs:166-181): one device iteration per step, the current scene read
    /// back for each callback.
    pub fn fit(
        &self,
        target: &Canvas,
        cfg: &FitConfig,
        mut on_progress: impl FnMut(FitProgress),
    ) -> Result<FitReport, FitError> {
        let mut fitter = Fitter::on(self, target.clone(), cfg.clone())?;
        while let Some(step) = fitter.try_step()? {
            on_progress(FitProgress { iter: step.iter, loss: step.loss, sigma: step.sigma, scene: fitter.scene() });
        }
        Ok(fitter.try_into_report()?)
    }

    /// The batch fit without a callback: the whole loop stays on the device and
    /// its state is read back every 64 iterations (`drh_fit`). Same report as
    /// [`Self::fit`].
    pub fn fit_quiet(&self, target: &Canvas, cfg: &FitConfig) -> Result<FitReport, FitError> {
        cfg.validate()?;
        let (background, init) = seed_scene(target, cfg);
        let c = raw_config(cfg);
        let mut losses = vec![0.0f32; cfg.iters];
        let mut best = vec![0.0f32; cfg.triangles * NP];
        let mut rep = ffi::drh_fit_report::default();
        // SAFETY: host arrays of the sizes drh_fit reads and writes.
        check(unsafe {
            ffi::drh_fit(
                self.raw(),
                target.data.as_ptr(),
                target.height as i64,
                target.width as i64,
                background.as_ptr(),
                init.as_ptr(),
                cfg.triangles as i64,
                &c,
                losses.as_mut_ptr(),
                best.as_mut_ptr(),
                ptr::null_mut(),
                &mut rep,
                ptr::null_mut(),
                ffi::DRH_HOST_PTRS,
            )
        })?;
        losses.truncate(rep.n_losses.max(0) as usize);
        Ok(report_from(background, cfg.triangles, &best, losses, &rep))
    }
}

/// Why a fit did not start or did not finish: an invalid configuration (the
/// CPU crate's only error, fit.rs:26-32) or a device failure.
#[derive(Debug)]
pub enum FitError {
    Config(ConfigError),
    Gpu(GpuError),
}

impl std::fmt::Display for FitError {
    fn fmt(&self, f: &mut std::fmt::Formatter<'_>) -> std::fmt::Result {
        match self {
            Self::Config(e) => write!(f, "{e}"),
            Self::Gpu(e) => write!(f, "{e}"),
        }
    }
}

impl std::error::Error for FitError {}

impl From<ConfigError> for FitError {
    fn from(e: ConfigError) -> Self {
        Self::Config(e)
    }
}

impl From<GpuError> for FitError {
    fn from(e: GpuError) -> Self {
        Self::Gpu(e)
    }
}

fn raw_config(cfg: &FitConfig) -> ffi::drh_fit_config {
    ffi::drh_fit_config {
        iters: cfg.iters as i64,
        sigma_start: cfg.sigma_start,
        sigma_end: cfg.sigma_end,
        lr_pos: cfg.lr_pos,
        lr_color: cfg.lr_color,
        lr_alpha: cfg.lr_alpha,
        patience: cfg.patience.map_or(-1, |p| p as i64),
        min_delta: cfg.min_delta,
    }
}

fn stop_reason(code: i32) -> StopReason {
    match code {
        ffi::DRH_STOP_CONVERGED => StopReason::Converged,
        ffi::DRH_STOP_DIVERGED => StopReason::Diverged,
        _ => StopReason::Completed,
    }
}

fn scene_from(background: [f32; 3], n_tris: usize, params: &[f32]) -> Scene {
    let mut s = Scene::new(background);
    for _ in 0..n_tris {
        s.push(Triangle::new([[0.0; 2]; 3], [0.0; 3], 0.0));
    }
    s.set_params(params);
    s
}

fn report_from(background: [f32; 3], n_tris: usize, best: &[f32], losses: Vec<f32>, rep: &ffi::drh_fit_report) -> FitReport {
    FitReport {
        scene: scene_from(background, n_tris, best),
        losses,
        stop_reason: stop_reason(rep.stop_reason),
        best_iter: rep.best_iter.max(0) as usize,
        best_loss: rep.best_loss,
    }
}

/// Mean colour of a canvas, summed per channel in f64 (fit.rs:369-377).
fn mean_color(c: &Canvas) -> [f32; 3] {
    let n = (c.data.len() / 3) as f32;
    let sums = c.data.chunks_exact(3).fold([0.0f64; 3], |mut acc, px| {
        for (a, v) in acc.iter_mut().zip(px) {
            *a += *v as f64;
        }
        acc
    });
    sums.map(|s| (s / n as f64) as f32)
}

/// The initial scene of `Fitter::new` (fit.rs:214-237 via seed_scene,
/// fit.rs:356-367): `Scene::random` over `StdRng::seed_from_u64(cfg.seed)`,
/// then per triangle, in order, the target's nearest-pixel colour at the
/// centroid (fit.rs:380-385) and an alpha drawn from [0.3, 0.7). The draws
/// come in the reference's order, so the same seed gives the same scene.
/// Returns the background and the flat parameters.
fn seed_scene(target: &Canvas, cfg: &FitConfig) -> ([f32; 3], Vec<f32>) {
    let background = mean_color(target);
    let mut rng = StdRng::seed_from_u64(cfg.seed);
    let mut scene = Scene::random(cfg.triangles, background, 0.18, &mut rng);
    let (w, h) = (target.width as isize, target.height as isize);
    for tri in &mut scene.tris {
        let cx = (tri.verts[0][0] + tri.verts[1][0] + tri.verts[2][0]) / 3.0;
        let cy = (tri.verts[0][1] + tri.verts[1][1] + tri.verts[2][1]) / 3.0;
        let px = ((cx * target.width as f32) as isize).clamp(0, w - 1) as usize;
        let py = ((cy * target.height as f32) as isize).clamp(0, h - 1) as usize;
        let i = (py * target.width + px) * 3;
        tri.color = [target.data[i], target.data[i + 1], target.data[i + 2]];
        tri.alpha = rng.gen_range(0.3..0.7);
    }
    (background, scene.params())
}

/// A fit advanced one iteration at a time (`diffrast::Fitter`, fit.rs:191-335),
/// its state on the device. The methods the CPU `Fitter` has keep their
/// signatures; where a device failure can occur they panic with its message,
/// and a `try_` form returns it instead.
pub struct Fitter<'a> {
    _gpu: &'a GpuRasterizer,
    raw: NonNull<ffi::drh_fitter>,
    target: Canvas,
    cfg: FitConfig,
    scene: Scene,
    params: Vec<f32>,
    losses: Vec<f32>,
    status: ffi::drh_fit_status,
}

impl Drop for Fitter<'_> {
    fn drop(&mut self) {
        // SAFETY: raw came from drh_fitter_create and is destroyed once.
        unsafe { ffi::drh_fitter_destroy(self.raw.as_ptr()) };
    }
}

impl Fitter<'static> {
    /// `Fitter::new` (fit.rs:214-237) on the process-wide rasterizer.
    pub fn new(target: Canvas, cfg: FitConfig) -> Result<Self, FitError> {
        Fitter::on(shared(), target, cfg)
    }
}

impl<'a> Fitter<'a> {
    fn on(gpu: &'a GpuRasterizer, target: Canvas, cfg: FitConfig) -> Result<Self, FitError> {
        cfg.validate()?;
        let (background, init) = seed_scene(&target, &cfg);
        let c = raw_config(&cfg);
        let mut raw = ptr::null_mut();
        // SAFETY: host inputs of the declared sizes; the library copies them.
        check(unsafe {
            ffi::drh_fitter_create(
                gpu.raw(),
                target.data.as_ptr(),
                target.height as i64,
                target.width as i64,
                background.as_ptr(),
                init.as_ptr(),
                cfg.triangles as i64,
                &c,
                ptr::null_mut(),
                ffi::DRH_HOST_PTRS,
                &mut raw,
            )
        })?;
        let raw = NonNull::new(raw).ok_or_else(|| GpuError::DeviceRequest("drh_fitter_create returned NULL".into()))?;
        let scene = scene_from(background, cfg.triangles, &init);
        let mut f = Self {
            _gpu: gpu,
            raw,
            losses: Vec::with_capacity(cfg.iters),
            target,
            cfg,
            scene,
            params: init,
            status: ffi::drh_fit_status::default(),
        };
        f.refresh_status()?;
        Ok(f)
    }

    fn refresh_status(&mut self) -> Result<(), GpuError> {
        // SAFETY: a live fitter and a valid out-pointer.
        check(unsafe { ffi::drh_fitter_status(self.raw.as_ptr(), &mut self.status) })
    }

    /// `Fitter::step` (fit.rs:239-288); `Ok(None)` once the fit has stopped.
    pub fn try_step(&mut self) -> Result<Option<StepInfo>, GpuError> {
        let mut stepped: c_int = 0;
        let mut info = ffi::drh_step_info::default();
        // SAFETY: a live fitter and valid out-pointers.
        check(unsafe { ffi::drh_fitter_step(self.raw.as_ptr(), &mut stepped, &mut info) })?;
        self.refresh_status()?;
        if stepped == 0 {
            return Ok(None);
        }
        self.losses.push(info.loss);
        // SAFETY: params holds T x 10 floats.
        check(unsafe { ffi::drh_fitter_scene(self.raw.as_ptr(), self.params.as_mut_ptr(), ffi::DRH_HOST_PTRS) })?;
        self.scene.set_params(&self.params);
        Ok(Some(StepInfo { iter: info.iter as usize, loss: info.loss, sigma: info.sigma }))
    }

    /// `Fitter::step` (fit.rs:239-288): one iteration, `None` once stopped.
    /// Panics if the device fails.
    pub fn step(&mut self) -> Option<StepInfo> {
        self.try_step().unwrap_or_else(|e| panic!("Fitter::step: {e}"))
    }

    /// The current scene, mid-optimization (fit.rs:290-293).
    pub fn scene(&self) -> &Scene {
        &self.scene
    }

    pub fn target(&self) -> &Canvas {
        &self.target
    }

    /// Iterations recorded so far (fit.rs:299-301).
    pub fn iter(&self) -> usize {
        self.status.iter.max(0) as usize
    }

    pub fn losses(&self) -> &[f32] {
        &self.losses
    }

    pub fn best_loss(&self) -> f32 {
        self.status.best_loss
    }

    pub fn is_done(&self) -> bool {
        self.status.done != 0
    }

    /// Softness of the next iteration (fit.rs:315-318).
    pub fn sigma(&self) -> f32 {
        self.status.sigma
    }

    /// The current scene at `sigma_end` (fit.rs:320-324).
    pub fn try_render_current(&self) -> Result<Canvas, GpuError> {
        let mut out = vec![0.0f32; self.target.width * self.target.height * 3];
        // SAFETY: an H x W x 3 host buffer.
        check(unsafe { ffi::drh_fitter_render_current(self.raw.as_ptr(), out.as_mut_ptr(), ffi::DRH_HOST_PTRS) })?;
        Ok(Canvas { width: self.target.width, height: self.target.height, data: out })
    }

    /// Panics if the device fails.
    pub fn render_current(&self) -> Canvas {
        self.try_render_current().unwrap_or_else(|e| panic!("Fitter::render_current: {e}"))
    }

    /// `Fitter::into_report` (fit.rs:326-334).
    pub fn try_into_report(self) -> Result<FitReport, GpuError> {
        let mut best = vec![0.0f32; self.cfg.triangles * NP];
        let mut rep = ffi::drh_fit_report::default();
        // SAFETY: a T x 10 host buffer and a valid out-pointer.
        check(unsafe { ffi::drh_fitter_report(self.raw.as_ptr(), best.as_mut_ptr(), &mut rep, ffi::DRH_HOST_PTRS) })?;
        Ok(report_from(self.scene.background, self.cfg.triangles, &best, self.losses.clone(), &rep))
    }

    /// Panics if the device fails.
    pub fn into_report(self) -> FitReport {
        self.try_into_report().unwrap_or_else(|e| panic!("Fitter::into_report: {e}"))
    }
}

/// The rasterizer behind the free functions, created on first use. Panics if
/// no device is present: these functions have no CPU fallback.
pub fn shared() -> &'static GpuRasterizer {
    static SHARED: OnceLock<GpuRasterizer> = OnceLock::new();
    SHARED.get_or_init(|| GpuRasterizer::new().unwrap_or_else(|e| panic!("diffrast-hip: {e}")))
}

/// `diffrast::render` (raster.rs:37-45).
pub fn render(scene: &Scene, p: RenderParams) -> Canvas {
    shared().render(scene, p).unwrap_or_else(|e| panic!("render: {e}"))
}

/// `diffrast::render_batch` (grad.rs:209-212).
pub fn render_batch(scenes: &[Scene], p: RenderParams) -> Vec<Canvas> {
    shared().render_many(scenes, p).unwrap_or_else(|e| panic!("render_batch: {e}"))
}

/// What [`backward`] needs from [`render_with_tape`] (`diffrast::Tape`,
/// grad.rs:37-51). The device pass keeps its own record during [`backward`],
/// so this holds only the render's shape.
pub struct Tape {
    n_tris: usize,
    width: usize,
    height: usize,
}

impl Tape {
    /// Bytes of the device record the backward pass reads for this render.
    pub fn memory_bytes(&self) -> usize {
        GpuRasterizer::tape_bytes(self.n_tris, self.width, self.height) as usize
    }
}

/// `diffrast::render_with_tape` (grad.rs:53-96).
pub fn render_with_tape(scene: &Scene, p: RenderParams) -> (Canvas, Tape) {
    (render(scene, p), Tape { n_tris: scene.len(), width: p.width, height: p.height })
}

/// `diffrast::backward` (grad.rs:93-182): `(mse, gradient)` with 10 gradient
/// values per triangle. The loss is reduced on the device in f64 over the
/// same render.
pub fn backward(scene: &Scene, p: RenderParams, tape: &Tape, rendered: &Canvas, target: &Canvas) -> (f32, Vec<f32>) {
    assert_eq!(tape.n_tris, scene.len(), "tape does not match scene");
    assert_eq!(rendered.data.len(), target.data.len(), "target size mismatch");
    shared().backward(scene, p, target).unwrap_or_else(|e| panic!("backward: {e}"))
}

/// `diffrast::backward_batch` (grad.rs:184-207).
pub fn backward_batch(scenes: &[Scene], p: RenderParams, targets: &[Canvas]) -> Vec<(f32, Vec<f32>)> {
    assert_eq!(scenes.len(), targets.len(), "batch size mismatch");
    shared().backward_many(scenes, p, targets).unwrap_or_else(|e| panic!("backward_batch: {e}"))
}

/// `diffrast::fit` (fit.rs:159-181). Device failures panic; an invalid
/// configuration is returned as in the CPU crate.
pub fn fit(target: &Canvas, cfg: &FitConfig, on_progress: impl FnMut(FitProgress)) -> Result<FitReport, ConfigError> {
    match shared().fit(target, cfg, on_progress) {
        Ok(r) => Ok(r),
        Err(FitError::Config(e)) => Err(e),
        Err(FitError::Gpu(e)) => panic!("fit: {e}"),
    }
}
