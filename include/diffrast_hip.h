/*
 * diffrast_hip — C ABI of the MI355X (gfx950) soft-triangle rasterizer.
 *
 * Plain pointers and sizes only. Every function returns a status code; the
 * message for the last failure on the calling thread is drh_last_error().
 *
 * Layouts are the reference's (crates/diffrast-py/src/lib.rs:10-13):
 *   params      B x T x 10 float, [x0,y0,x1,y1,x2,y2,r,g,b,a] per triangle,
 *               vertices in normalized image space, index 0 drawn first
 *   images      B x H x W x 3 float, linear RGB, row-major
 *   backgrounds B x 3 float (per scene, as the GPU crate packs them,
 *               crates/diffrast-gpu/src/lib.rs:936-954)
 *
 * Pointers are device pointers unless DRH_HOST_PTRS is set. With device
 * pointers a call only enqueues work on `stream` (a hipStream_t; NULL is the
 * null stream) and returns; with host pointers it stages through pooled device
 * buffers and returns once the results are back on the host.
 *
 * A context is safe to use from several threads at once: scratch buffers come
 * from a locked pool and a buffer reused on another stream waits for the work
 * that last used it.
 */
#ifndef DIFFRAST_HIP_H
#define DIFFRAST_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes. 1-5 are the reference's GpuError variants
 * (crates/diffrast-gpu/src/lib.rs:42-50); 6 covers the argument checks its
 * Python binding raises ValueError for (crates/diffrast-py/src/lib.rs:85-94,
 * 162-167, 185-195, 261-273). */
enum {
    DRH_OK = 0,
    DRH_ERR_NO_DEVICE = 1,   /* GpuError::NoAdapter */
    DRH_ERR_TIMEOUT = 2,     /* GpuError::Timeout: a host wait exceeded DRH_WAIT_TIMEOUT_S */
    DRH_ERR_DEVICE = 3,      /* GpuError::DeviceRequest: a HIP runtime failure */
    DRH_ERR_READBACK = 4,    /* GpuError::Readback: copying results to the host failed */
    DRH_ERR_TOO_LARGE = 5,   /* GpuError::TooLarge: sizes beyond what one call supports (more
                                than 65535 scenes, 2^23 triangles per scene, 2^20 pixels a side,
                                or B x T of 2^25 or more) */
    DRH_ERR_INVALID_ARG = 6  /* bad sigma, zero height/width, NULL pointer, bad config */
};

/* Flags. */
#define DRH_HOST_PTRS 0x1u  /* array arguments are host memory */
#define DRH_SYNC 0x2u       /* with device pointers: wait for the stream before returning */
#define DRH_EXACT_MATH 0x4u /* IEEE division, sqrt and expf in the per-pixel geometry */
#define DRH_DETERMINISTIC 0x8u /* gradients summed in a fixed order: bit-identical run to run
                                  (default: one float atomic per triangle parameter per block) */
#define DRH_CHANNELS_FIRST 0x10u /* images, targets and grad_images are B x 3 x H x W (the
                                    layout torch_layer.rasterize returns) instead of B x H x W x 3 */
#define DRH_PHASES 0x20u  /* drh_render, drh_fused_loss_backward, drh_backward_from_grad: wait for
                             the stream between phases and keep their host times (drh_phases_read) */

/* Bounded host wait, as GpuRasterizer::POLL_TIMEOUT (crates/diffrast-gpu/src/lib.rs:229). */
#define DRH_WAIT_TIMEOUT_S 60

typedef struct drh_ctx drh_ctx;

/* GpuRasterizer::new (crates/diffrast-gpu/src/lib.rs:238-319): binds the
 * current HIP device. DRH_ERR_NO_DEVICE when there is none. */
int drh_create(drh_ctx **out);

/* shutdown_gpu (crates/diffrast-py/src/lib.rs:435-444): frees the pool and
 * the context. NULL is accepted. */
int drh_destroy(drh_ctx *ctx);

/* Message for the last failure on this thread ("" when none). */
const char *drh_last_error(void);

/* adapter_info (crates/diffrast-gpu/src/lib.rs:370-373). */
int drh_device_info(const drh_ctx *ctx, char *buf, size_t len);

/* is_discrete (crates/diffrast-gpu/src/lib.rs:383-385): 1 or 0. */
int drh_is_discrete(const drh_ctx *ctx);

/* params_per_triangle (crates/diffrast-py/src/lib.rs:452-456): 10. */
int drh_params_per_triangle(void);

/* pool_stats / clear_pool (crates/diffrast-gpu/src/lib.rs:345-356). */
int drh_pool_stats(drh_ctx *ctx, uint64_t *hits, uint64_t *misses, uint64_t *bytes);
int drh_clear_pool(drh_ctx *ctx);

/* Device-side kernel timings, the counterpart of BackwardTimings /
 * backward_many_timed (crates/diffrast-gpu/src/lib.rs:96-114, 649-655). While
 * enabled, every kernel a call launches is bracketed by HIP events on the
 * call's stream; drh_timing_read waits for them, returns the accumulated
 * milliseconds and launch counts since the last read, and resets them. The
 * events do not synchronize the host between kernels. */
typedef struct {
    double setup_ms, raster_ms, reduce_ms, adam_ms;  /* raster: the forward kernel */
    int64_t setup_n, raster_n, reduce_n, adam_n;
    double backward_ms;                              /* the backward kernel */
    int64_t backward_n;
} drh_timings;

int drh_timing_enable(drh_ctx *ctx, int enable);
int drh_timing_read(drh_ctx *ctx, drh_timings *out);

/* Host wall-clock phases of one call made with DRH_PHASES: BackwardTimings
 * (crates/diffrast-gpu/src/lib.rs:96-114) as backward_many_timed
 * (lib.rs:649-664) measures it, by waiting for the stream between phases, so
 * the total is an upper bound on the call without the flag.
 *   pack_ms      pooled device buffers for params and backgrounds taken and
 *                filled (0 with device pointers)
 *   alloc_ms     pooled buffers for targets / upstream gradients (filled),
 *                images, gradients and losses taken
 *   dispatch_ms  every kernel enqueued and finished (all device execution)
 *   readback_ms  results copied back to the host
 *   loss_ms      per-item loss on the host: always 0, the loss is reduced on
 *                the device inside dispatch
 *   total_ms     the sum of the five, BackwardTimings::total_ms */
typedef struct {
    double pack_ms, alloc_ms, dispatch_ms, readback_ms, loss_ms, total_ms;
} drh_phase_timings;

/* The phases of the calling thread's last DRH_PHASES call (zeros before the
 * first). */
int drh_phases_read(drh_phase_timings *out);

/* Batched forward render: render_many (crates/diffrast-gpu/src/lib.rs:615-633)
 * and render_batch (crates/diffrast-py/src/lib.rs:174-231), per-pixel
 * semantics of raster.rs:37-168. out_images is B x H x W x 3. B == 0 is a
 * no-op; T == 0 renders the backgrounds. */
int drh_render(drh_ctx *ctx, const float *params, const float *backgrounds, int64_t B, int64_t T,
               int64_t H, int64_t W, float sigma, float *out_images, void *stream, uint32_t flags);

/* Render, per-item MSE and its parameter gradients in one call:
 * backward_many (crates/diffrast-gpu/src/lib.rs:639-646) and
 * fused_loss_backward (crates/diffrast-py/src/lib.rs:333-412), semantics of
 * grad.rs:56-182 and canvas.rs:45-58. out_losses is B floats, out_grads
 * B x T x 10. out_images (B x H x W x 3) may be NULL. */
int drh_fused_loss_backward(drh_ctx *ctx, const float *params, const float *backgrounds,
                            const float *targets, int64_t B, int64_t T, int64_t H, int64_t W,
                            float sigma, float *out_losses, float *out_grads, float *out_images,
                            void *stream, uint32_t flags);

/* drh_fused_loss_backward for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc). No counterpart in the reference. Device pointers only
 * (DRH_HOST_PTRS is refused: staging would allocate). The call's buffers
 * besides its inputs and outputs live in a 128 MiB array that the library
 * holds on each GPU until the process ends; sizes whose buffers exceed it
 * (far beyond B=16 at 256x256, T=128) return DRH_ERR_TOO_LARGE. The calls
 * on one GPU share that array, so the library runs them one after another:
 * a call on another stream than the previous call's waits on the device for
 * that call to finish (calls from several threads and streams are safe).
 * Under graph capture that ordering is left to the caller: replays of a
 * captured call must not overlap other calls on the same GPU. Results equal
 * drh_fused_loss_backward's; its launches are not counted by drh_timing_*. */
int drh_fused_loss_backward_noalloc(drh_ctx *ctx, const float *params, const float *backgrounds,
                                    const float *targets, int64_t B, int64_t T, int64_t H, int64_t W,
                                    float sigma, float *out_losses, float *out_grads, float *out_images,
                                    void *stream, uint32_t flags);

/* Parameter gradients from an upstream image gradient dL/dpixel
 * (B x H x W x 3): backward_many_from_grad
 * (crates/diffrast-gpu/src/lib.rs:828-910) and backward_batch
 * (crates/diffrast-py/src/lib.rs:245-324). out_grads is B x T x 10. */
int drh_backward_from_grad(drh_ctx *ctx, const float *params, const float *backgrounds,
                           const float *grad_images, int64_t B, int64_t T, int64_t H, int64_t W,
                           float sigma, float *out_grads, void *stream, uint32_t flags);

/* A render kept for its backward pass. The reference has no counterpart: its
 * PyTorch op renders in forward (python/diffrast/torch_layer.py:40-52) and its
 * backward re-renders the batch (torch_layer.py:55-66 via backward_batch,
 * crates/diffrast-py/src/lib.rs:245-324). Here the forward keeps, in device
 * memory the caller owns, what the backward kernel reads (triangle records,
 * backgrounds, per-pixel transmittance, per-tile entry lists), so the backward
 * runs only the backward kernel.
 *
 * drh_record_bytes gives the size of that memory for B x T triangles at H x W
 * (0 when B == 0). */
int drh_record_bytes(int64_t B, int64_t T, int64_t H, int64_t W, uint64_t *out_bytes);

/* drh_render that also fills `record` (device memory, 256-byte aligned, of
 * exactly drh_record_bytes(B, T, H, W) bytes). The image is drh_render's, bit
 * for bit. The record stays valid until the caller frees or overwrites it;
 * params and backgrounds are not needed afterwards. */
int drh_render_record(drh_ctx *ctx, const float *params, const float *backgrounds, int64_t B, int64_t T,
                      int64_t H, int64_t W, float sigma, float *out_images, void *record,
                      uint64_t record_bytes, void *stream, uint32_t flags);

/* drh_backward_from_grad for the scenes of a drh_render_record call, from its
 * record, without rendering again: B, T, H, W, sigma and DRH_EXACT_MATH must be
 * those of that call, else DRH_ERR_INVALID_ARG (the record's head holds them;
 * DRH_CHANNELS_FIRST here describes grad_images). The record is only read, so
 * one record serves any number of backward calls. */
int drh_backward_recorded(drh_ctx *ctx, const void *record, uint64_t record_bytes,
                          const float *grad_images, int64_t B, int64_t T, int64_t H, int64_t W,
                          float sigma, float *out_grads, void *stream, uint32_t flags);

/* One Adam step (optim.rs:40-60) over n parameters with per-parameter
 * learning rates, then fit.rs:399-424 project() when `project` is nonzero
 * (n must then be a multiple of 10). `step` is the step count after the
 * increment (the reference's `t`, starting at 1). */
int drh_adam_project_step(drh_ctx *ctx, float *params, const float *grads, float *m, float *v,
                          const float *lr, int64_t n, uint32_t step, float beta1, float beta2,
                          float eps, int project, void *stream, uint32_t flags);

/* FitConfig (crates/diffrast/src/fit.rs:49-65) minus the scene size and seed,
 * which drh_fit takes as the initial scene. patience < 0 means None. */
typedef struct {
    int64_t iters;
    float sigma_start, sigma_end;
    float lr_pos, lr_color, lr_alpha;
    int64_t patience;
    float min_delta;
} drh_fit_config;

/* StopReason (fit.rs:14-23). */
enum { DRH_STOP_COMPLETED = 0, DRH_STOP_CONVERGED = 1, DRH_STOP_DIVERGED = 2 };

/* ConfigError (fit.rs:26-32) as returned by drh_fit_validate; 0 when valid. */
enum {
    DRH_CFG_OK = 0,
    DRH_CFG_NO_TRIANGLES = 1,
    DRH_CFG_NON_POSITIVE_SIGMA = 2,
    DRH_CFG_SIGMA_NOT_DECREASING = 3,
    DRH_CFG_NON_POSITIVE_LEARNING_RATE = 4
};

/* FitReport (fit.rs:128-140) minus the scene, which drh_fit writes out. */
typedef struct {
    int64_t n_losses;
    int64_t best_iter;
    float best_loss;
    int32_t stop_reason;
} drh_fit_report;

/* FitConfig::validate (fit.rs:98-117) for a scene of T triangles. */
int drh_fit_validate(const drh_fit_config *cfg, int64_t T);

/* The fit loop (fit.rs:166-181, the batch form `fit` without its progress
 * callback) from a given initial scene, with every step on the device: sigma
 * annealing, fused loss and gradients, divergence, best snapshot and patience
 * bookkeeping, Adam and projection. The device state is read back every 64
 * iterations and at the end, not per step; once the fit has stopped, the
 * kernels of iterations already launched return at entry. target is
 * H x W x 3, init_params and out_best_params T x 10, out_losses room for
 * cfg->iters floats, out_params (optional) receives the last iterate.
 * Equivalent to drh_fitter_create + drh_fitter_run(iters) + drh_fitter_losses
 * + drh_fitter_report. */
int drh_fit(drh_ctx *ctx, const float *target, int64_t H, int64_t W, const float *background,
            const float *init_params, int64_t T, const drh_fit_config *cfg, float *out_losses,
            float *out_best_params, float *out_params, drh_fit_report *report, void *stream,
            uint32_t flags);

/* A fit advanced one iteration at a time: Fitter (fit.rs:191-335). Its state
 * (scene, Adam moments, losses, best snapshot, stop reason) lives on the
 * device; the fitter owns copies of the target and background. A fitter is
 * used from one thread at a time and enqueues on the stream it was created
 * with; its context must outlive it. */
typedef struct drh_fitter drh_fitter;

/* StepInfo (fit.rs:183-189). */
typedef struct {
    int64_t iter;
    float loss;
    float sigma;
} drh_step_info;

/* Fitter::{iter, best_loss, sigma, is_done} (fit.rs:299-318) and the stop
 * reason so far (-1 while running, else DRH_STOP_*). best_iter is the
 * iteration of the best snapshot. */
typedef struct {
    int64_t iter;
    int64_t best_iter;
    float best_loss;
    float sigma;
    int32_t done;
    int32_t stop_reason;
} drh_fit_status;

/* Fitter::new (fit.rs:214-237) from a given initial scene (T x 10) instead of
 * seed_scene's random one; DRH_ERR_INVALID_ARG for an invalid configuration
 * (drh_fit_validate names it). flags: DRH_HOST_PTRS for host inputs,
 * DRH_EXACT_MATH. */
int drh_fitter_create(drh_ctx *ctx, const float *target, int64_t H, int64_t W, const float *background,
                      const float *init_params, int64_t T, const drh_fit_config *cfg, void *stream,
                      uint32_t flags, drh_fitter **out);
int drh_fitter_destroy(drh_fitter *f);

/* Fitter::step (fit.rs:239-288): runs one iteration and waits for its loss.
 * *stepped = 1 and *info (optional) filled when it ran (Some), 0 once the fit
 * has stopped, for any reason (None). */
int drh_fitter_step(drh_fitter *f, int *stepped, drh_step_info *info);

/* Up to max_steps iterations without waiting between them (the device state
 * is read back every 64 iterations and at the end); *ran (optional) is the
 * number of iterations recorded. */
int drh_fitter_run(drh_fitter *f, int64_t max_steps, int64_t *ran);

int drh_fitter_status(const drh_fitter *f, drh_fit_status *out);

/* Fitter::scene (fit.rs:290-293): the current parameters, T x 10. */
int drh_fitter_scene(drh_fitter *f, float *out_params, uint32_t flags);

/* Fitter::losses (fit.rs:303-305): *n_out losses into out (capacity floats). */
int drh_fitter_losses(drh_fitter *f, float *out, int64_t capacity, int64_t *n_out, uint32_t flags);

/* Fitter::render_current (fit.rs:320-324): the current scene at sigma_end,
 * H x W x 3. */
int drh_fitter_render_current(drh_fitter *f, float *out_image, uint32_t flags);

/* Fitter::into_report (fit.rs:326-334): the best scene (T x 10) and the report. */
int drh_fitter_report(drh_fitter *f, float *out_best_params, drh_fit_report *report, uint32_t flags);

/* The gamma of Canvas::save_png (crates/diffrast/src/canvas.rs:61-68):
 * encode_srgb (canvas.rs:100-105) of n linear values, in any layout, to sRGB
 * bytes; clamped to [0, 1], NaN to 0. Bit-identical to the reference. */
int drh_encode_srgb(drh_ctx *ctx, const float *values, int64_t n, uint8_t *out, void *stream,
                    uint32_t flags);

/* The gamma of Canvas::load_image (canvas.rs:70-86): decode_srgb
 * (canvas.rs:108-115) of n sRGB bytes to linear values. */
int drh_decode_srgb(drh_ctx *ctx, const uint8_t *bytes, int64_t n, float *out, void *stream,
                    uint32_t flags);

/* The resize of Canvas::load_image (canvas.rs:71-79): `resize_exact(new_W,
 * new_H, FilterType::Lanczos3)` of image 0.25.10 (Cargo.lock:410-411) on an
 * H x W x C byte image (C in 1..4, channels resampled independently) into
 * new_H x new_W x C bytes; the same size is a copy. The weights are built on
 * the host, so the call waits for the stream before returning whenever it
 * resamples. */
int drh_resize_lanczos3(drh_ctx *ctx, const uint8_t *src, int64_t H, int64_t W, int64_t C, uint8_t *dst,
                        int64_t new_H, int64_t new_W, void *stream, uint32_t flags);

#ifdef __cplusplus
}
#endif
#endif /* DIFFRAST_HIP_H */
