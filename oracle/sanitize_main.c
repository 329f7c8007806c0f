/*
 * Driver for the oracle's sanitizer builds (test infrastructure only): runs
 * every oracle entry point over ordinary and edge-case inputs so that
 * AddressSanitizer + UndefinedBehaviorSanitizer (and, in a second build,
 * ThreadSanitizer for the batch threads) check its memory accesses, integer
 * arithmetic and thread use. Prints "ok" and exits 0 when nothing fired; the
 * sanitizers abort with a report otherwise.
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "diffrast_oracle.h"

static uint64_t rng_state = 0x9E3779B97F4A7C15ull;

static float urand(void) {
    rng_state ^= rng_state << 13;
    rng_state ^= rng_state >> 7;
    rng_state ^= rng_state << 17;
    return (float)(rng_state >> 40) * (1.0f / 16777216.0f);
}

static void random_scene(float *p, size_t T, float spread) {
    for (size_t k = 0; k < T; k++) {
        const float cx = urand(), cy = urand();
        for (int v = 0; v < 3; v++) {
            p[k * 10 + 2 * v] = spread > 0 ? cx + spread * (2 * urand() - 1) : urand();
            p[k * 10 + 2 * v + 1] = spread > 0 ? cy + spread * (2 * urand() - 1) : urand();
        }
        for (int c = 6; c < 9; c++) p[k * 10 + c] = urand();
        p[k * 10 + 9] = 0.3f + 0.6f * urand();
    }
}

static void *xmalloc(size_t n) {
    void *p = malloc(n ? n : 1);
    if (!p) {
        fprintf(stderr, "out of memory\n");
        exit(2);
    }
    return p;
}

/* One scene through render, loss/backward, both upstream-gradient forms and
 * finite differences, at the given size. */
static void one_scene(float *p, size_t T, size_t W, size_t H, float sigma) {
    const float bg[3] = {0.1f, 0.2f, 0.3f};
    float *img = xmalloc(sizeof(float) * W * H * 3), *tgt = xmalloc(sizeof(float) * W * H * 3);
    float *g = xmalloc(sizeof(float) * T * 10), *gi = xmalloc(sizeof(float) * W * H * 3);
    orc_counts counts = {0, 0};
    orc_render(p, T, bg, W, H, sigma, img, &counts);
    for (size_t i = 0; i < W * H * 3; i++) {
        tgt[i] = urand();
        gi[i] = (urand() - 0.5f) * 1e-3f;
    }
    (void)orc_mse(img, tgt, W * H * 3);
    (void)orc_loss_backward(p, T, bg, W, H, sigma, tgt, g, img, &counts);
    orc_backward_from_grad(p, T, bg, W, H, sigma, gi, g);
    orc_backward_from_grad_inverted(p, T, bg, W, H, sigma, gi, g);
    if (T <= 8 && W * H <= 256) (void)orc_finite_difference(p, T, bg, W, H, sigma, tgt, 1e-3f, g);
    free(img);
    free(tgt);
    free(g);
    free(gi);
}

int main(void) {
    /* ordinary scenes, odd sizes, 1x1 / 1xW / Hx1 canvases, empty scenes */
    const size_t sizes[][3] = {{32, 24, 20}, {8, 37, 11}, {40, 1, 1}, {6, 64, 1}, {6, 1, 64}, {0, 16, 16}, {300, 40, 48}};
    for (size_t s = 0; s < sizeof sizes / sizeof sizes[0]; s++) {
        const size_t T = sizes[s][0], W = sizes[s][1], H = sizes[s][2];
        float *p = xmalloc(sizeof(float) * (T ? T : 1) * 10);
        random_scene(p, T, s == 6 ? 0.05f : 0.0f);
        one_scene(p, T, W, H, s % 2 ? 0.01f : 0.0015f);
        free(p);
    }
    /* special triangles: point, collinear, off-canvas, non-finite, transparent,
     * negative and NaN alpha, a box that saturates and wraps, huge coordinates */
    {
        float p[10 * 10];
        random_scene(p, 10, 0.0f);
        const float nan = nanf("");
        for (int v = 0; v < 6; v++) p[0 * 10 + v] = 0.5f;
        p[1 * 10 + 0] = 0.1f, p[1 * 10 + 1] = 0.1f, p[1 * 10 + 2] = 0.5f, p[1 * 10 + 3] = 0.5f;
        p[1 * 10 + 4] = 0.9f, p[1 * 10 + 5] = 0.9f;
        for (int v = 0; v < 6; v++) p[2 * 10 + v] = 5.0f + (float)v;
        p[3 * 10 + 0] = nan;
        p[4 * 10 + 9] = 0.0f;
        p[5 * 10 + 9] = -0.5f;
        p[6 * 10 + 2] = 1e20f;
        p[7 * 10 + 9] = nan;
        p[8 * 10 + 0] = -1e30f, p[8 * 10 + 3] = 1e30f;
        p[9 * 10 + 6] = INFINITY;
        one_scene(p, 10, 30, 34, 0.01f);
        one_scene(p, 10, 30, 34, 0.002f);
        uint64_t box[4];
        for (int k = 0; k < 10; k++) (void)orc_pixel_bounds(p + 10 * k, 30, 34, 0.01f, box);
        float d[6];
        for (int k = 0; k < 10; k++) (void)orc_coverage_with_grad(p + 10 * k, 0.4f, 0.6f, 0.01f, d);
    }
    /* batches on several threads */
    {
        const size_t B = 6, T = 40, W = 33, H = 27;
        float *p = xmalloc(sizeof(float) * B * T * 10), *bgs = xmalloc(sizeof(float) * B * 3);
        float *img = xmalloc(sizeof(float) * B * W * H * 3), *tgt = xmalloc(sizeof(float) * B * W * H * 3);
        float *g = xmalloc(sizeof(float) * B * T * 10), *losses = xmalloc(sizeof(float) * B);
        random_scene(p, B * T, 0.0f);
        for (size_t i = 0; i < B * 3; i++) bgs[i] = urand();
        for (size_t i = 0; i < B * W * H * 3; i++) tgt[i] = urand();
        orc_counts counts = {0, 0};
        orc_render_batch(p, B, T, bgs, W, H, 0.004f, img, 4, &counts);
        orc_loss_backward_batch(p, B, T, bgs, W, H, 0.004f, tgt, losses, g, 4, &counts);
        orc_backward_from_grad_batch(p, B, T, bgs, W, H, 0.004f, tgt, g, 3);
        orc_loss_backward_batch(p, 0, T, bgs, W, H, 0.004f, tgt, losses, g, 4, NULL);
        free(p), free(bgs), free(img), free(tgt), free(g), free(losses);
    }
    /* Adam, projection, the fit loop (completed, converged, diverged, no iterations) */
    {
        const size_t T = 12, W = 24, H = 20, n = T * 10;
        float *p = xmalloc(sizeof(float) * n), *grads = xmalloc(sizeof(float) * n), *lr = xmalloc(sizeof(float) * n);
        float *m = xmalloc(sizeof(float) * n), *v = xmalloc(sizeof(float) * n);
        random_scene(p, T, 0.18f);
        for (size_t i = 0; i < n; i++) grads[i] = urand() - 0.5f, lr[i] = 0.01f, m[i] = v[i] = 0.0f;
        uint32_t t = 0;
        for (int s = 0; s < 5; s++) orc_adam_step(p, grads, lr, m, v, &t, n, 0.9f, 0.999f, 1e-8f);
        orc_project(p, n);
        (void)orc_sigma_at(0.02f, 0.0015f, 100, 50);
        (void)orc_sigma_at(0.02f, 0.0015f, 1, 0);
        float *target = xmalloc(sizeof(float) * W * H * 3);
        for (size_t i = 0; i < W * H * 3; i++) target[i] = urand();
        float bg[3], col[3];
        orc_mean_color(target, W, H, bg);
        orc_sample(target, W, H, 1.5f, -0.5f, col);
        orc_fit_config cfg = {30, 0.02f, 0.0015f, 0.004f, 0.02f, 0.01f, -1, 1e-7f};
        float *losses = xmalloc(sizeof(float) * 30), *best = xmalloc(sizeof(float) * n);
        orc_fit_report rep;
        orc_fit(target, W, H, bg, p, T, &cfg, losses, best, &rep, NULL);
        cfg.patience = 3;
        orc_fit(target, W, H, bg, p, T, &cfg, losses, best, &rep, NULL);
        cfg.iters = 0;
        orc_fit(target, W, H, bg, p, T, &cfg, losses, best, &rep, NULL);
        cfg.iters = 10;
        target[5] = nanf("");
        orc_fit(target, W, H, bg, p, T, &cfg, losses, best, &rep, NULL);
        free(p), free(grads), free(lr), free(m), free(v), free(target), free(losses), free(best);
    }
    /* sRGB both ways, every byte and a scan of the encoding */
    {
        float vals[1000], thr[256];
        uint8_t bytes[1000];
        for (int i = 0; i < 1000; i++) vals[i] = 1.2f * urand() - 0.1f;
        vals[0] = nanf("");
        vals[1] = INFINITY;
        orc_encode_srgb(vals, 1000, bytes);
        for (int i = 0; i < 256; i++) bytes[i] = (uint8_t)i;
        orc_decode_srgb(bytes, 256, vals);
        (void)orc_srgb_encode_scan(thr);
    }
    /* Lanczos3 resize: shrink, grow, one axis, 1x1, same size, every channel count */
    {
        const size_t cases[][4] = {{40, 30, 15, 20}, {7, 9, 64, 5}, {1, 1, 3, 4}, {33, 47, 33, 47}, {300, 2, 1, 3}};
        for (size_t k = 0; k < sizeof cases / sizeof cases[0]; k++) {
            for (size_t C = 1; C <= 4; C++) {
                const size_t W = cases[k][0], H = cases[k][1], nW = cases[k][2], nH = cases[k][3];
                uint8_t *src = xmalloc(W * H * C), *dst = xmalloc(nW * nH * C);
                for (size_t i = 0; i < W * H * C; i++) src[i] = (uint8_t)(urand() * 255.0f);
                orc_resize_lanczos3(src, W, H, C, dst, nW, nH);
                free(src);
                free(dst);
            }
        }
        size_t left = 0;
        float w[64];
        if (orc_lanczos3_taps(100, 3, 1, &left, w, 4) != 0) return 1; /* too small a buffer is refused */
    }
    printf("ok\n");
    return 0;
}
