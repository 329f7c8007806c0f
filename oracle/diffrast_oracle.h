/*
 * CPU oracle for the soft-triangle rasterizer hot path.
 *
 * TEST INFRASTRUCTURE ONLY. This is a plain-C restatement of the reference's
 * CPU implementation (crates/diffrast/src/{raster,grad,canvas,optim,fit}.rs),
 * used by tests/, __graft_entry__.smoke() and the cpu_baseline leg of bench.py
 * to check the GPU results against. The product (libdiffrast_hip.so and the
 * Python package) never links, loads or calls it.
 *
 * Layouts follow the reference exactly:
 *   params  : T x 10 floats per scene, [x0,y0,x1,y1,x2,y2,r,g,b,a]
 *             (scene.rs:81-92), index 0 composited first (back).
 *   images  : H x W x 3 floats, row-major, (y*W + x)*3 + ch (canvas.rs:27-29).
 * Batched entry points take B consecutive scenes / images and B backgrounds.
 */
#ifndef DIFFRAST_ORACLE_H
#define DIFFRAST_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Work counters for the roofline: pixels inside a live triangle's padded
 * bounding box (n_box) and those whose weight passed MIN_WEIGHT (n_contrib). */
typedef struct {
    uint64_t n_box;
    uint64_t n_contrib;
} orc_counts;

/* raster.rs:37-68 render(). counts may be NULL. */
void orc_render(const float *params, size_t T, const float bg[3], size_t W,
                size_t H, float sigma, float *out, orc_counts *counts);

/* canvas.rs:45-58 Canvas::mse(). */
float orc_mse(const float *a, const float *b, size_t n);

/* grad.rs:56-131: render_with_tape + backward against a target.
 * Returns the loss; writes T*10 grads. out_image (H*W*3) may be NULL. */
float orc_loss_backward(const float *params, size_t T, const float bg[3],
                        size_t W, size_t H, float sigma, const float *target,
                        float *grads, float *out_image, orc_counts *counts);

/* Upstream-gradient backward, the reference's CPU semantics
 * (crates/diffrast-py/src/lib.rs:301-318): rebuild t = r - g*N/2 and run
 * backward() against it. */
void orc_backward_from_grad_inverted(const float *params, size_t T,
                                     const float bg[3], size_t W, size_t H,
                                     float sigma, const float *grad_image,
                                     float *grads);

/* Upstream-gradient backward with dL/dpixel taken as given, the semantics of
 * the reference GPU path (backward_batch_reduced.wgsl:143-156). */
void orc_backward_from_grad(const float *params, size_t T, const float bg[3],
                            size_t W, size_t H, float sigma,
                            const float *grad_image, float *grads);

/* grad.rs:192-212: batch forms, one worker thread per item, results in input
 * order (rayon par_iter). nthreads <= 0 means one per online CPU, capped at B. */
void orc_render_batch(const float *params, size_t B, size_t T,
                      const float *bgs, size_t W, size_t H, float sigma,
                      float *out, int nthreads, orc_counts *counts);
void orc_loss_backward_batch(const float *params, size_t B, size_t T,
                             const float *bgs, size_t W, size_t H, float sigma,
                             const float *targets, float *losses, float *grads,
                             int nthreads, orc_counts *counts);
void orc_backward_from_grad_batch(const float *params, size_t B, size_t T,
                                  const float *bgs, size_t W, size_t H,
                                  float sigma, const float *grad_images,
                                  float *grads, int nthreads);

/* grad.rs:298-323 finite_difference(): central differences of the loss. */
float orc_finite_difference(const float *params, size_t T, const float bg[3],
                            size_t W, size_t H, float sigma,
                            const float *target, float eps, float *grads);

/* optim.rs:40-60 Adam::step(). t is the step count before the call; the
 * function increments it. */
void orc_adam_step(float *params, const float *grads, const float *lr,
                   float *m, float *v, uint32_t *t, size_t n, float beta1,
                   float beta2, float eps);

/* fit.rs:399-424 project(). n must be a multiple of 10. */
void orc_project(float *params, size_t n);

/* fit.rs:343-349 sigma_at(). */
float orc_sigma_at(float sigma_start, float sigma_end, size_t iters, size_t i);

/* fit.rs:49-65 FitConfig (patience < 0 means None). The initial scene is
 * passed in: the reference draws it from rand::StdRng (fit.rs:217, 356-367),
 * whose stream is not restated here. */
typedef struct {
    size_t iters;
    float sigma_start, sigma_end;
    float lr_pos, lr_color, lr_alpha;
    long patience;
    float min_delta;
} orc_fit_config;

enum { ORC_COMPLETED = 0, ORC_CONVERGED = 1, ORC_DIVERGED = 2 };

typedef struct {
    size_t n_losses;
    size_t best_iter;
    float best_loss;
    int stop_reason;
} orc_fit_report;

/* fit.rs:166-288: the Fitter loop from a given initial scene. losses must hold
 * cfg->iters floats; best_params T*10 floats. */
void orc_fit(const float *target, size_t W, size_t H, const float bg[3],
             const float *init_params, size_t T, const orc_fit_config *cfg,
             float *losses, float *best_params, orc_fit_report *report,
             orc_counts *counts);

/* fit.rs:369-385 mean_color() and sample(), used by seed_scene(). */
void orc_mean_color(const float *image, size_t W, size_t H, float out[3]);
void orc_sample(const float *image, size_t W, size_t H, float x, float y,
                float out[3]);

/* Primitives exposed for the reference's unit tests (raster.rs:170-241,
 * grad.rs:231-270). tri points at one 10-float triangle record. */
float orc_signed_distance(const float *tri, float px, float py);
float orc_coverage(const float *tri, float px, float py, float sigma);
float orc_coverage_with_grad(const float *tri, float px, float py, float sigma,
                             float dcov_dverts[6]);
int orc_pixel_bounds(const float *tri, size_t W, size_t H, float sigma,
                     uint64_t out[4]);

/* canvas.rs:100-105 encode_srgb and canvas.rs:108-115 decode_srgb, the gamma of
 * save_png / load_image: linear f32 -> sRGB byte and back. */
uint8_t orc_encode_srgb1(float v);
float orc_decode_srgb1(uint8_t v);
void orc_encode_srgb(const float *v, size_t n, uint8_t *out);
void orc_decode_srgb(const uint8_t *v, size_t n, float *out);
/* Over every f32 in [2^-14, 1] (below it every byte is 0), the number of inputs
 * whose byte is below the byte of the next smaller float (0 when encode_srgb is
 * monotonic there), and the smallest input giving each byte 1..255
 * (thresholds[0] = 0). */
uint64_t orc_srgb_encode_scan(float thresholds[256]);

/* The resize of Canvas::load_image (canvas.rs:71-79): image 0.25.10's
 * imageops::resize with FilterType::Lanczos3 (Cargo.lock:410-411; the crate is
 * not in the reference tree, so this restates its published algorithm).
 * Separable: a vertical pass from bytes to f32 rows, then a horizontal pass
 * that clamps to [0, 255] and rounds half away from zero; the same size is a
 * plain copy. Each output index o of a pass over n_src -> n_dst samples
 * reads the source indices [left, left + count) with weights that sum to 1:
 *   ratio = n_src / n_dst, scale = max(ratio, 1), support = 3 * scale,
 *   centre = (o + 0.5) * ratio,
 *   left = clamp(floor(centre - support), 0, n_src - 1),
 *   right = clamp(ceil(centre + support), left + 1, n_src),
 *   w_i = lanczos3((i - (centre - 0.5)) / scale) / sum, all in f32.
 * orc_lanczos3_taps writes left and at most `cap` weights and returns count
 * (0 if cap is too small). Images are H x W x C bytes, C in 1..4. */
float orc_lanczos3(float x);
size_t orc_lanczos3_taps(size_t n_src, size_t n_dst, size_t o, size_t *left, float *w, size_t cap);
void orc_resize_lanczos3(const uint8_t *src, size_t W, size_t H, size_t C, uint8_t *dst, size_t new_W,
                         size_t new_H);

#ifdef __cplusplus
}
#endif
#endif
