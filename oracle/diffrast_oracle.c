/*
 * CPU oracle for the soft-triangle rasterizer — TEST INFRASTRUCTURE ONLY.
 *
 * A plain-C restatement of the reference's CPU algorithm, kept operation for
 * operation so that it rounds the way the reference does:
 *   - build with -ffp-contract=off and no fast-math (Rust neither contracts
 *     a*b+c into an FMA nor reassociates; Cargo.toml:10-13 release profile);
 *   - f32 arithmetic throughout except where the reference widens to f64;
 *   - glibc expf/powf, the libm that Rust's f32::exp/powf call on Linux.
 * Each function cites the reference lines it follows. Only tests/, the smoke
 * check and bench.py's CPU-baseline leg use this file; the product never does.
 */
#define _GNU_SOURCE
#include "diffrast_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdatomic.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

#define NP 10

/* raster.rs:31-34 */
static const float MIN_WEIGHT = 1e-6f;

/* Rust `f32::clamp` (NaN passes through both comparisons). */
static inline float rclamp(float x, float lo, float hi) {
    if (x < lo) x = lo;
    if (x > hi) x = hi;
    return x;
}

/* Rust `f32 as usize` on a 64-bit target: saturating, NaN -> 0. */
static inline uint64_t sat_usize(float v) {
    if (!(v >= 0.0f)) return 0;
    if (v >= 18446744073709551616.0f) return UINT64_MAX;
    return (uint64_t)v;
}

/* raster.rs:79-87 / grad.rs:286-294 */
static inline float sigmoid(float x) {
    if (x >= 0.0f) {
        return 1.0f / (1.0f + expf(-x));
    }
    float e = expf(x);
    return e / (1.0f + e);
}

/* raster.rs:124-134 point_segment_distance / grad.rs:275-284
 * closest_point_on_segment (identical arithmetic; t returned optionally). */
static inline float seg_dist(const float a[2], const float b[2],
                             const float pt[2], float *t_out) {
    float ab0 = b[0] - a[0], ab1 = b[1] - a[1];
    float ap0 = pt[0] - a[0], ap1 = pt[1] - a[1];
    float len2 = ab0 * ab0 + ab1 * ab1;
    float t = (len2 <= 1e-20f) ? 0.0f : rclamp((ap0 * ab0 + ap1 * ab1) / len2, 0.0f, 1.0f);
    float dx = ap0 - t * ab0;
    float dy = ap1 - t * ab1;
    if (t_out) *t_out = t;
    return sqrtf(dx * dx + dy * dy);
}

/* raster.rs:119-121 */
static inline float cross2(const float a[2], const float b[2], const float pt[2]) {
    return (b[0] - a[0]) * (pt[1] - a[1]) - (b[1] - a[1]) * (pt[0] - a[0]);
}

/* raster.rs:111-116 */
static inline int is_inside(const float v[3][2], const float pt[2]) {
    float c0 = cross2(v[0], v[1], pt);
    float c1 = cross2(v[1], v[2], pt);
    float c2 = cross2(v[2], v[0], pt);
    return (c0 >= 0.0f && c1 >= 0.0f && c2 >= 0.0f) ||
           (c0 <= 0.0f && c1 <= 0.0f && c2 <= 0.0f);
}

/* raster.rs:96-106: min over edges via fold(INFINITY, f32::min). */
static inline float signed_distance(const float v[3][2], const float pt[2]) {
    float d = INFINITY;
    for (int i = 0; i < 3; i++) d = fminf(d, seg_dist(v[i], v[(i + 1) % 3], pt, NULL));
    return is_inside(v, pt) ? d : -d;
}

/* raster.rs:74-76 */
static inline float coverage(const float v[3][2], const float pt[2], float sigma) {
    return sigmoid(signed_distance(v, pt) / fmaxf(sigma, 1e-8f));
}

/* raster.rs:138-140 */
static inline void pixel_center(size_t x, size_t y, size_t W, size_t H, float pt[2]) {
    pt[0] = ((float)x + 0.5f) / (float)W;
    pt[1] = ((float)y + 0.5f) / (float)H;
}

/* raster.rs:144-168 pixel_bounds(): the padded, clipped integer bbox; 0 when
 * a vertex is non-finite or the box is empty. The `+ 1` wraps like a release
 * build's usize addition. */
static int pixel_bounds(const float *tri, size_t W, size_t H, float sigma,
                        size_t *x0, size_t *y0, size_t *x1, size_t *y1) {
    float pad = 6.0f * sigma; /* raster.rs:26-28 cull_radius */
    float lo_x = INFINITY, lo_y = INFINITY, hi_x = -INFINITY, hi_y = -INFINITY;
    for (int v = 0; v < 3; v++) {
        float vx = tri[2 * v], vy = tri[2 * v + 1];
        if (!isfinite(vx) || !isfinite(vy)) return 0;
        lo_x = fminf(lo_x, vx);
        hi_x = fmaxf(hi_x, vx);
        lo_y = fminf(lo_y, vy);
        hi_y = fmaxf(hi_y, vy);
    }
    uint64_t bx0 = sat_usize(fmaxf(floorf((lo_x - pad) * (float)W), 0.0f));
    uint64_t by0 = sat_usize(fmaxf(floorf((lo_y - pad) * (float)H), 0.0f));
    uint64_t bx1 = sat_usize(fmaxf(ceilf((hi_x + pad) * (float)W), 0.0f)) + 1u;
    uint64_t by1 = sat_usize(fmaxf(ceilf((hi_y + pad) * (float)H), 0.0f)) + 1u;
    if (bx1 > W) bx1 = W;
    if (by1 > H) by1 = H;
    if (!(bx0 < bx1 && by0 < by1)) return 0;
    *x0 = (size_t)bx0;
    *y0 = (size_t)by0;
    *x1 = (size_t)bx1;
    *y1 = (size_t)by1;
    return 1;
}

static inline void tri_verts(const float *tri, float v[3][2]) {
    for (int i = 0; i < 3; i++) {
        v[i][0] = tri[2 * i];
        v[i][1] = tri[2 * i + 1];
    }
}

static void fill_bg(float *img, size_t W, size_t H, const float bg[3]) {
    for (size_t i = 0; i < W * H; i++) {
        img[3 * i] = bg[0];
        img[3 * i + 1] = bg[1];
        img[3 * i + 2] = bg[2];
    }
}

/* raster.rs:46-68 composite(): bounds first, then the clamped-alpha test
 * (`alpha <= 0` lets a NaN alpha through, so NaN paints NaN here). */
static void composite(float *img, const float *tri, size_t W, size_t H,
                      float sigma, orc_counts *cnt) {
    size_t x0, y0, x1, y1;
    if (!pixel_bounds(tri, W, H, sigma, &x0, &y0, &x1, &y1)) return;
    float alpha = rclamp(tri[9], 0.0f, 1.0f);
    if (alpha <= 0.0f) return;
    float v[3][2];
    tri_verts(tri, v);
    for (size_t y = y0; y < y1; y++) {
        for (size_t x = x0; x < x1; x++) {
            float pt[2];
            pixel_center(x, y, W, H, pt);
            float w = alpha * coverage(v, pt, sigma);
            if (cnt) cnt->n_box++;
            if (w <= MIN_WEIGHT) continue;
            if (cnt) cnt->n_contrib++;
            float *dst = img + (y * W + x) * 3;
            float out[3];
            for (int ch = 0; ch < 3; ch++) out[ch] = tri[6 + ch] * w + dst[ch] * (1.0f - w);
            dst[0] = out[0];
            dst[1] = out[1];
            dst[2] = out[2];
        }
    }
}

/* raster.rs:37-43 */
void orc_render(const float *params, size_t T, const float bg[3], size_t W,
                size_t H, float sigma, float *out, orc_counts *counts) {
    fill_bg(out, W, H, bg);
    for (size_t k = 0; k < T; k++) composite(out, params + k * NP, W, H, sigma, counts);
}

/* canvas.rs:45-58: f32 difference, squared and summed in f64. */
float orc_mse(const float *a, const float *b, size_t n) {
    double sum = 0.0;
    for (size_t i = 0; i < n; i++) {
        double d = (double)(a[i] - b[i]);
        sum += d * d;
    }
    return (float)(sum / (double)n);
}

/* grad.rs:27-35 Patch */
typedef struct {
    int live;
    size_t x0, y0, x1, y1;
    float *before;
} patch_t;

/* grad.rs:56-90 render_with_tape(): bounds are filtered by `alpha > 0`, so a
 * NaN alpha culls the triangle here (unlike composite()). */
static patch_t *render_with_tape(const float *params, size_t T, const float bg[3],
                                 size_t W, size_t H, float sigma, float *canvas,
                                 orc_counts *cnt) {
    fill_bg(canvas, W, H, bg);
    patch_t *patches = (patch_t *)calloc(T ? T : 1, sizeof(patch_t));
    for (size_t k = 0; k < T; k++) {
        const float *tri = params + k * NP;
        float alpha = rclamp(tri[9], 0.0f, 1.0f);
        size_t x0, y0, x1, y1;
        if (!pixel_bounds(tri, W, H, sigma, &x0, &y0, &x1, &y1) || !(alpha > 0.0f)) continue;
        patch_t *p = &patches[k];
        p->live = 1;
        p->x0 = x0;
        p->y0 = y0;
        p->x1 = x1;
        p->y1 = y1;
        p->before = (float *)malloc((x1 - x0) * (y1 - y0) * 3 * sizeof(float));
        float v[3][2];
        tri_verts(tri, v);
        float *bp = p->before;
        for (size_t y = y0; y < y1; y++) {
            for (size_t x = x0; x < x1; x++) {
                float *dst = canvas + (y * W + x) * 3;
                bp[0] = dst[0];
                bp[1] = dst[1];
                bp[2] = dst[2];
                bp += 3;
                float pt[2];
                pixel_center(x, y, W, H, pt);
                float w = alpha * coverage(v, pt, sigma);
                if (cnt) cnt->n_box++;
                if (w <= MIN_WEIGHT) continue;
                if (cnt) cnt->n_contrib++;
                float out[3];
                for (int ch = 0; ch < 3; ch++) out[ch] = tri[6 + ch] * w + dst[ch] * (1.0f - w);
                dst[0] = out[0];
                dst[1] = out[1];
                dst[2] = out[2];
            }
        }
    }
    return patches;
}

static void free_tape(patch_t *patches, size_t T) {
    for (size_t k = 0; k < T; k++) free(patches[k].before);
    free(patches);
}

/* grad.rs:231-270 coverage_with_grad(). */
static float coverage_with_grad(const float v[3][2], const float pt[2], float sigma,
                                float d[3][2]) {
    sigma = fmaxf(sigma, 1e-8f);
    int edge = 0;
    float bt = 0.0f, bd = INFINITY;
    for (int i = 0; i < 3; i++) {
        float t;
        float dd = seg_dist(v[i], v[(i + 1) % 3], pt, &t);
        if (dd < bd) {
            edge = i;
            bt = t;
            bd = dd;
        }
    }
    float t = bt, dist = bd;
    int inside = signed_distance(v, pt) > 0.0f;
    float sign = inside ? 1.0f : -1.0f;
    float cov = sigmoid(sign * dist / sigma);
    memset(d, 0, sizeof(float) * 6);
    if (dist < 1e-9f) return cov;
    const float *a = v[edge];
    const float *b = v[(edge + 1) % 3];
    float cp0 = a[0] + t * (b[0] - a[0]);
    float cp1 = a[1] + t * (b[1] - a[1]);
    float u[2] = {(pt[0] - cp0) / dist, (pt[1] - cp1) / dist};
    float chain = cov * (1.0f - cov) / sigma * sign;
    int e1 = (edge + 1) % 3;
    for (int ax = 0; ax < 2; ax++) {
        d[edge][ax] = chain * -(1.0f - t) * u[ax];
        d[e1][ax] += chain * -t * u[ax];
    }
    return cov;
}

/* grad.rs:135-182 backward_one(): accumulate one triangle and attenuate
 * d_canvas for the layers beneath it. */
static void backward_one(const float *tri, size_t W, size_t H, float sigma,
                         const patch_t *patch, float *d_canvas, float *g) {
    float alpha = rclamp(tri[9], 0.0f, 1.0f);
    int alpha_active = tri[9] > 0.0f && tri[9] < 1.0f;
    float v[3][2];
    tri_verts(tri, v);
    size_t row_len = (patch->x1 - patch->x0) * 3;
    for (size_t y = patch->y0; y < patch->y1; y++) {
        for (size_t x = patch->x0; x < patch->x1; x++) {
            float pt[2];
            pixel_center(x, y, W, H, pt);
            float dcdv[3][2];
            float cov = coverage_with_grad(v, pt, sigma, dcdv);
            float w = alpha * cov;
            if (w <= MIN_WEIGHT) continue;
            size_t off = (y - patch->y0) * row_len + (x - patch->x0) * 3;
            const float *dst = patch->before + off;
            size_t di = (y * W + x) * 3;
            float d_out[3] = {d_canvas[di], d_canvas[di + 1], d_canvas[di + 2]};
            float d_w = 0.0f;
            for (int ch = 0; ch < 3; ch++) {
                g[6 + ch] += d_out[ch] * w;
                d_w += d_out[ch] * (tri[6 + ch] - dst[ch]);
                d_canvas[di + ch] = d_out[ch] * (1.0f - w);
            }
            if (alpha_active) g[9] += d_w * cov;
            float d_cov = d_w * alpha;
            for (int vv = 0; vv < 3; vv++) {
                g[vv * 2] += d_cov * dcdv[vv][0];
                g[vv * 2 + 1] += d_cov * dcdv[vv][1];
            }
        }
    }
}

/* grad.rs:124-128: the front-to-back sweep over the tape. */
static void sweep_back(const float *params, size_t T, size_t W, size_t H, float sigma,
                       const patch_t *tape, float *d_canvas, float *grads) {
    memset(grads, 0, sizeof(float) * T * NP);
    for (size_t kk = T; kk-- > 0;) {
        if (!tape[kk].live) continue;
        backward_one(params + kk * NP, W, H, sigma, &tape[kk], d_canvas, grads + kk * NP);
    }
}

/* grad.rs:98-131 backward() after render_with_tape(). */
float orc_loss_backward(const float *params, size_t T, const float bg[3],
                        size_t W, size_t H, float sigma, const float *target,
                        float *grads, float *out_image, orc_counts *counts) {
    size_t n = W * H * 3;
    float *rendered = (float *)malloc(n * sizeof(float));
    patch_t *tape = render_with_tape(params, T, bg, W, H, sigma, rendered, counts);
    float loss = orc_mse(rendered, target, n);
    float scale = 2.0f / (float)n;
    float *d_canvas = (float *)malloc(n * sizeof(float));
    for (size_t i = 0; i < n; i++) d_canvas[i] = scale * (rendered[i] - target[i]);
    sweep_back(params, T, W, H, sigma, tape, d_canvas, grads);
    if (out_image) memcpy(out_image, rendered, n * sizeof(float));
    free(d_canvas);
    free(rendered);
    free_tape(tape, T);
    return loss;
}

/* crates/diffrast-py/src/lib.rs:301-318: rebuild the target the upstream
 * gradient implies (t = r - g*N/2), then run backward() against it. */
void orc_backward_from_grad_inverted(const float *params, size_t T,
                                     const float bg[3], size_t W, size_t H,
                                     float sigma, const float *grad_image,
                                     float *grads) {
    size_t n = W * H * 3;
    float n_pixels = (float)n;
    float *rendered = (float *)malloc(n * sizeof(float));
    float *target = (float *)malloc(n * sizeof(float));
    patch_t *tape = render_with_tape(params, T, bg, W, H, sigma, rendered, NULL);
    for (size_t i = 0; i < n; i++) target[i] = rendered[i] - grad_image[i] * n_pixels / 2.0f;
    float scale = 2.0f / (float)n;
    float *d_canvas = (float *)malloc(n * sizeof(float));
    for (size_t i = 0; i < n; i++) d_canvas[i] = scale * (rendered[i] - target[i]);
    sweep_back(params, T, W, H, sigma, tape, d_canvas, grads);
    free(d_canvas);
    free(target);
    free(rendered);
    free_tape(tape, T);
}

/* backward_batch_reduced.wgsl:143-156 (grad_input != 0): dL/dpixel is used as
 * given; the sweep is grad.rs:124-182 unchanged. */
void orc_backward_from_grad(const float *params, size_t T, const float bg[3],
                            size_t W, size_t H, float sigma,
                            const float *grad_image, float *grads) {
    size_t n = W * H * 3;
    float *rendered = (float *)malloc(n * sizeof(float));
    patch_t *tape = render_with_tape(params, T, bg, W, H, sigma, rendered, NULL);
    float *d_canvas = (float *)malloc(n * sizeof(float));
    memcpy(d_canvas, grad_image, n * sizeof(float));
    sweep_back(params, T, W, H, sigma, tape, d_canvas, grads);
    free(d_canvas);
    free(rendered);
    free_tape(tape, T);
}

/* ---- batch forms: grad.rs:192-212, one item per worker, input order ---- */

typedef struct {
    int kind; /* 0 render, 1 loss+backward, 2 from-grad */
    const float *params;
    size_t B, T, W, H;
    const float *bgs;
    float sigma;
    const float *in_images; /* targets or grad images */
    float *out_images;
    float *losses;
    float *grads;
    orc_counts *item_counts;
    atomic_size_t next;
} batch_job;

static void *batch_worker(void *arg) {
    batch_job *j = (batch_job *)arg;
    size_t n = j->W * j->H * 3;
    for (;;) {
        size_t b = atomic_fetch_add(&j->next, 1);
        if (b >= j->B) break;
        const float *p = j->params + b * j->T * NP;
        const float *bg = j->bgs + 3 * b;
        orc_counts *c = j->item_counts ? &j->item_counts[b] : NULL;
        if (j->kind == 0) {
            orc_render(p, j->T, bg, j->W, j->H, j->sigma, j->out_images + b * n, c);
        } else if (j->kind == 1) {
            j->losses[b] = orc_loss_backward(p, j->T, bg, j->W, j->H, j->sigma,
                                             j->in_images + b * n, j->grads + b * j->T * NP,
                                             NULL, c);
        } else {
            orc_backward_from_grad(p, j->T, bg, j->W, j->H, j->sigma, j->in_images + b * n,
                                   j->grads + b * j->T * NP);
        }
    }
    return NULL;
}

static void run_batch(batch_job *j, int nthreads, orc_counts *counts) {
    if (j->B == 0) return;
    if (nthreads <= 0) nthreads = (int)sysconf(_SC_NPROCESSORS_ONLN);
    if (nthreads < 1) nthreads = 1;
    if ((size_t)nthreads > j->B) nthreads = (int)j->B;
    j->item_counts = counts ? (orc_counts *)calloc(j->B, sizeof(orc_counts)) : NULL;
    atomic_init(&j->next, 0);
    pthread_t *th = (pthread_t *)malloc(sizeof(pthread_t) * (size_t)nthreads);
    for (int i = 1; i < nthreads; i++) pthread_create(&th[i], NULL, batch_worker, j);
    batch_worker(j);
    for (int i = 1; i < nthreads; i++) pthread_join(th[i], NULL);
    free(th);
    if (counts) {
        for (size_t b = 0; b < j->B; b++) {
            counts->n_box += j->item_counts[b].n_box;
            counts->n_contrib += j->item_counts[b].n_contrib;
        }
        free(j->item_counts);
    }
}

void orc_render_batch(const float *params, size_t B, size_t T, const float *bgs,
                      size_t W, size_t H, float sigma, float *out, int nthreads,
                      orc_counts *counts) {
    batch_job j = {0};
    j.kind = 0;
    j.params = params;
    j.B = B;
    j.T = T;
    j.W = W;
    j.H = H;
    j.bgs = bgs;
    j.sigma = sigma;
    j.out_images = out;
    run_batch(&j, nthreads, counts);
}

void orc_loss_backward_batch(const float *params, size_t B, size_t T,
                             const float *bgs, size_t W, size_t H, float sigma,
                             const float *targets, float *losses, float *grads,
                             int nthreads, orc_counts *counts) {
    batch_job j = {0};
    j.kind = 1;
    j.params = params;
    j.B = B;
    j.T = T;
    j.W = W;
    j.H = H;
    j.bgs = bgs;
    j.sigma = sigma;
    j.in_images = targets;
    j.losses = losses;
    j.grads = grads;
    run_batch(&j, nthreads, counts);
}

void orc_backward_from_grad_batch(const float *params, size_t B, size_t T,
                                  const float *bgs, size_t W, size_t H,
                                  float sigma, const float *grad_images,
                                  float *grads, int nthreads) {
    batch_job j = {0};
    j.kind = 2;
    j.params = params;
    j.B = B;
    j.T = T;
    j.W = W;
    j.H = H;
    j.bgs = bgs;
    j.sigma = sigma;
    j.in_images = grad_images;
    j.grads = grads;
    run_batch(&j, nthreads, NULL);
}

/* grad.rs:298-323 */
float orc_finite_difference(const float *params, size_t T, const float bg[3],
                            size_t W, size_t H, float sigma,
                            const float *target, float eps, float *grads) {
    size_t n = W * H * 3, np = T * NP;
    float *img = (float *)malloc(n * sizeof(float));
    float *shifted = (float *)malloc((np ? np : 1) * sizeof(float));
    orc_render(params, T, bg, W, H, sigma, img, NULL);
    float loss = orc_mse(img, target, n);
    for (size_t i = 0; i < np; i++) {
        memcpy(shifted, params, np * sizeof(float));
        shifted[i] = params[i] + eps;
        orc_render(shifted, T, bg, W, H, sigma, img, NULL);
        float hi = orc_mse(img, target, n);
        shifted[i] = params[i] - eps;
        orc_render(shifted, T, bg, W, H, sigma, img, NULL);
        float lo = orc_mse(img, target, n);
        grads[i] = (hi - lo) / (2.0f * eps);
    }
    free(shifted);
    free(img);
    return loss;
}

/* f32::powi with a runtime exponent lowers to the compiler-builtins
 * `__powisf2`: square-and-multiply in f32, reciprocal for negative powers. */
static float powi_f32(float a, int32_t b) {
    int recip = b < 0;
    float r = 1.0f;
    for (;;) {
        if (b & 1) r *= a;
        b /= 2;
        if (b == 0) break;
        a *= a;
    }
    return recip ? 1.0f / r : r;
}

/* optim.rs:40-60 */
void orc_adam_step(float *params, const float *grads, const float *lr,
                   float *m, float *v, uint32_t *t, size_t n, float beta1,
                   float beta2, float eps) {
    *t += 1;
    float bc1 = 1.0f - powi_f32(beta1, (int32_t)*t);
    float bc2 = 1.0f - powi_f32(beta2, (int32_t)*t);
    for (size_t i = 0; i < n; i++) {
        float g = grads[i];
        m[i] = beta1 * m[i] + (1.0f - beta1) * g;
        v[i] = beta2 * v[i] + (1.0f - beta2) * g * g;
        float m_hat = m[i] / bc1;
        float v_hat = v[i] / bc2;
        params[i] -= lr[i] * m_hat / (sqrtf(v_hat) + eps);
    }
}

/* fit.rs:399-424 */
void orc_project(float *params, size_t n) {
    for (size_t base = 0; base + NP <= n; base += NP) {
        float *tri = params + base;
        for (int i = 0; i < NP; i++)
            if (isnan(tri[i])) tri[i] = 0.5f;
        for (int i = 0; i < 6; i++) tri[i] = rclamp(tri[i], -0.25f, 1.25f);
        for (int i = 6; i < 9; i++) tri[i] = rclamp(tri[i], 0.0f, 1.0f);
        tri[9] = rclamp(tri[9], 1e-3f, 0.999f);
    }
}

/* fit.rs:343-349 */
float orc_sigma_at(float sigma_start, float sigma_end, size_t iters, size_t i) {
    if (iters <= 1) return sigma_end;
    float t = (float)i / (float)(iters - 1);
    return sigma_start * powf(sigma_end / sigma_start, t);
}

/* fit.rs:369-378 */
void orc_mean_color(const float *image, size_t W, size_t H, float out[3]) {
    float n = (float)(W * H);
    double sum[3] = {0.0, 0.0, 0.0};
    for (size_t i = 0; i < W * H; i++)
        for (int ch = 0; ch < 3; ch++) sum[ch] += (double)image[3 * i + ch];
    for (int ch = 0; ch < 3; ch++) out[ch] = (float)(sum[ch] / (double)n);
}

/* fit.rs:381-385: `as isize` truncates toward zero and saturates. */
static int64_t sat_isize(float v) {
    if (v != v) return 0;
    if (v >= 9223372036854775808.0f) return INT64_MAX;
    if (v < -9223372036854775808.0f) return INT64_MIN;
    return (int64_t)v;
}

void orc_sample(const float *image, size_t W, size_t H, float x, float y, float out[3]) {
    int64_t px = sat_isize(x * (float)W), py = sat_isize(y * (float)H);
    if (px < 0) px = 0;
    if (px > (int64_t)W - 1) px = (int64_t)W - 1;
    if (py < 0) py = 0;
    if (py > (int64_t)H - 1) py = (int64_t)H - 1;
    const float *c = image + ((size_t)py * W + (size_t)px) * 3;
    out[0] = c[0];
    out[1] = c[1];
    out[2] = c[2];
}

/* fit.rs:214-288 Fitter::new + Fitter::step, driven to completion as fit()
 * does (fit.rs:166-181), from a caller-supplied initial scene. counts (may be
 * NULL) sums every iteration's box and contributing pairs. */
void orc_fit(const float *target, size_t W, size_t H, const float bg[3],
             const float *init_params, size_t T, const orc_fit_config *cfg,
             float *losses, float *best_params, orc_fit_report *report,
             orc_counts *counts) {
    size_t np = T * NP;
    float *params = (float *)malloc((np ? np : 1) * sizeof(float));
    float *grads = (float *)malloc((np ? np : 1) * sizeof(float));
    float *lr = (float *)malloc((np ? np : 1) * sizeof(float));
    float *m = (float *)calloc(np ? np : 1, sizeof(float));
    float *v = (float *)calloc(np ? np : 1, sizeof(float));
    uint32_t t = 0;
    memcpy(params, init_params, np * sizeof(float));
    memcpy(best_params, init_params, np * sizeof(float));
    /* fit.rs:388-396 learning_rates() */
    for (size_t k = 0; k < T; k++) {
        for (int i = 0; i < 6; i++) lr[k * NP + i] = cfg->lr_pos;
        for (int i = 6; i < 9; i++) lr[k * NP + i] = cfg->lr_color;
        lr[k * NP + 9] = cfg->lr_alpha;
    }
    size_t iter = 0, since = 0, best_iter = 0, n_losses = 0;
    float best_loss = INFINITY;
    int stop = -1;
    for (;;) {
        if (stop >= 0) break;
        if (iter >= cfg->iters) {
            stop = ORC_COMPLETED;
            break;
        }
        size_t i = iter;
        float sigma = orc_sigma_at(cfg->sigma_start, cfg->sigma_end, cfg->iters, i);
        float loss = orc_loss_backward(params, T, bg, W, H, sigma, target, grads, NULL, counts);
        if (!isfinite(loss)) {
            stop = ORC_DIVERGED;
            break;
        }
        losses[n_losses++] = loss;
        if (loss + cfg->min_delta < best_loss) {
            best_loss = loss;
            best_iter = i;
            memcpy(best_params, params, np * sizeof(float));
            since = 0;
        } else {
            since += 1;
        }
        iter += 1;
        if (cfg->patience >= 0 && since >= (size_t)cfg->patience) {
            stop = ORC_CONVERGED;
            continue;
        }
        orc_adam_step(params, grads, lr, m, v, &t, np, 0.9f, 0.999f, 1e-8f);
        orc_project(params, np);
    }
    report->n_losses = n_losses;
    report->best_iter = best_iter;
    report->best_loss = best_loss;
    report->stop_reason = stop;
    free(params);
    free(grads);
    free(lr);
    free(m);
    free(v);
}

/* ---- primitives for the reference's unit tests ---- */

float orc_signed_distance(const float *tri, float px, float py) {
    float v[3][2], pt[2] = {px, py};
    tri_verts(tri, v);
    return signed_distance(v, pt);
}

float orc_coverage(const float *tri, float px, float py, float sigma) {
    float v[3][2], pt[2] = {px, py};
    tri_verts(tri, v);
    return coverage(v, pt, sigma);
}

float orc_coverage_with_grad(const float *tri, float px, float py, float sigma,
                             float dcov_dverts[6]) {
    float v[3][2], pt[2] = {px, py}, d[3][2];
    tri_verts(tri, v);
    float cov = coverage_with_grad(v, pt, sigma, d);
    memcpy(dcov_dverts, d, sizeof(d));
    return cov;
}

int orc_pixel_bounds(const float *tri, size_t W, size_t H, float sigma, uint64_t out[4]) {
    size_t x0, y0, x1, y1;
    if (!pixel_bounds(tri, W, H, sigma, &x0, &y0, &x1, &y1)) return 0;
    out[0] = x0;
    out[1] = y0;
    out[2] = x1;
    out[3] = y1;
    return 1;
}

/* ---------------------------------------------------------------- sRGB */

/* Rust `f32 as u8`: saturating, NaN -> 0. */
static inline uint8_t sat_u8(float v) {
    if (!(v >= 0.0f)) return 0;
    if (v >= 255.0f) return 255;
    return (uint8_t)v;
}

/* canvas.rs:100-105 */
uint8_t orc_encode_srgb1(float v) {
    v = rclamp(v, 0.0f, 1.0f);
    float s = v <= 0.0031308f ? 12.92f * v : 1.055f * powf(v, 1.0f / 2.4f) - 0.055f;
    return sat_u8(s * 255.0f + 0.5f);
}

/* canvas.rs:108-115 */
float orc_decode_srgb1(uint8_t b) {
    float v = (float)b / 255.0f;
    if (v <= 0.04045f) return v / 12.92f;
    return powf((v + 0.055f) / 1.055f, 2.4f);
}

void orc_encode_srgb(const float *v, size_t n, uint8_t *out) {
    for (size_t i = 0; i < n; i++) out[i] = orc_encode_srgb1(v[i]);
}

void orc_decode_srgb(const uint8_t *v, size_t n, float *out) {
    for (size_t i = 0; i < n; i++) out[i] = orc_decode_srgb1(v[i]);
}

uint64_t orc_srgb_encode_scan(float thresholds[256]) {
    uint64_t drops = 0;
    int prev = 0;
    for (int k = 0; k < 256; k++) thresholds[k] = k == 0 ? 0.0f : INFINITY;
    /* Below 2^-14 the linear branch gives 12.92 v 255 + 0.5 < 0.71: byte 0,
     * monotonic by construction (each step is a monotone rounding). From there,
     * every float up to 1.0f in increasing order of value. */
    if (orc_encode_srgb1(0x1p-14f) != 0) return UINT64_MAX;
    for (uint32_t bits = 0x38800000u; bits <= 0x3F800000u; bits++) {
        float v;
        memcpy(&v, &bits, sizeof v);
        int b = orc_encode_srgb1(v);
        if (b < prev) drops++;
        for (int k = prev + 1; k <= b; k++) thresholds[k] = v;
        if (b > prev) prev = b;
    }
    return drops;
}

/* ------------------------------------------------------------------------
 * Lanczos3 resize: image 0.25.10 imageops::resize (sample.rs: resize,
 * vertical_sample, horizontal_sample, lanczos3_kernel), the resample of
 * Canvas::load_image (canvas.rs:71-79). The crate is not in the reference
 * tree; this follows its published source. f32 throughout, glibc sinf (the
 * libm behind Rust's f32::sin on Linux), products and sums unfused.
 * ------------------------------------------------------------------------ */

/* sinc with f32::consts::PI; 1 at 0. */
static float sinc_f32(float t) {
    const float a = t * 3.14159265358979323846f;
    return t == 0.0f ? 1.0f : sinf(a) / a;
}

float orc_lanczos3(float x) {
    return fabsf(x) < 3.0f ? sinc_f32(x) * sinc_f32(x / 3.0f) : 0.0f;
}

size_t orc_lanczos3_taps(size_t n_src, size_t n_dst, size_t o, size_t *left, float *w, size_t cap) {
    const float ratio = (float)n_src / (float)n_dst;
    const float scale = ratio < 1.0f ? 1.0f : ratio;
    const float support = 3.0f * scale;
    const float centre = ((float)o + 0.5f) * ratio;
    int64_t lo = (int64_t)floorf(centre - support);
    if (lo < 0) lo = 0;
    if (lo > (int64_t)n_src - 1) lo = (int64_t)n_src - 1;
    int64_t hi = (int64_t)ceilf(centre + support);
    if (hi < lo + 1) hi = lo + 1;
    if (hi > (int64_t)n_src) hi = (int64_t)n_src;
    const size_t count = (size_t)(hi - lo);
    if (count > cap) return 0;
    const float c = centre - 0.5f;
    float sum = 0.0f;
    for (size_t k = 0; k < count; k++) {
        w[k] = orc_lanczos3(((float)(lo + (int64_t)k) - c) / scale);
        sum += w[k];
    }
    for (size_t k = 0; k < count; k++) w[k] /= sum;
    *left = (size_t)lo;
    return count;
}

void orc_resize_lanczos3(const uint8_t *src, size_t W, size_t H, size_t C, uint8_t *dst, size_t new_W,
                         size_t new_H) {
    if (W == 0 || H == 0 || new_W == 0 || new_H == 0) return;
    if (W == new_W && H == new_H) {
        memcpy(dst, src, W * H * C);
        return;
    }
    const size_t vcap = (size_t)(6.0f * ((float)H / (float)new_H < 1.0f ? 1.0f : (float)H / (float)new_H)) + 3;
    const size_t hcap = (size_t)(6.0f * ((float)W / (float)new_W < 1.0f ? 1.0f : (float)W / (float)new_W)) + 3;
    float *tmp = malloc(sizeof(float) * new_H * W * C);
    float *w = malloc(sizeof(float) * (vcap > hcap ? vcap : hcap));
    if (!tmp || !w) {
        free(tmp);
        free(w);
        return;
    }
    /* vertical: bytes -> f32 rows, new_H x W x C */
    for (size_t oy = 0; oy < new_H; oy++) {
        size_t lo = 0;
        const size_t n = orc_lanczos3_taps(H, new_H, oy, &lo, w, vcap);
        for (size_t e = 0; e < W * C; e++) {
            float t = 0.0f;
            for (size_t k = 0; k < n; k++) t += (float)src[(lo + k) * W * C + e] * w[k];
            tmp[oy * W * C + e] = t;
        }
    }
    /* horizontal: f32 rows -> bytes, clamped to [0, 255], rounded half away from zero */
    for (size_t ox = 0; ox < new_W; ox++) {
        size_t lo = 0;
        const size_t n = orc_lanczos3_taps(W, new_W, ox, &lo, w, hcap);
        for (size_t y = 0; y < new_H; y++) {
            for (size_t c = 0; c < C; c++) {
                float t = 0.0f;
                for (size_t k = 0; k < n; k++) t += tmp[(y * W + lo + k) * C + c] * w[k];
                if (t < 0.0f) t = 0.0f;
                if (t > 255.0f) t = 255.0f;
                dst[(y * new_W + ox) * C + c] = (uint8_t)roundf(t);
            }
        }
    }
    free(tmp);
    free(w);
}
