// The fit loop (crates/diffrast/src/fit.rs:166-335) behind the C ABI: a
// step-wise fitter whose state lives on the device, and drh_fit on top of it.
//
// Every iteration is the deterministic raster kernels -> fit_step, which sums
// the partial rows in a fixed order (so a fit with a given start is
// reproducible like the reference's, fit.rs:487-496) and does the bookkeeping
// of fit.rs:243-288 on the device: divergence stop before the optimizer sees
// the loss, loss record, best snapshot taken before the update, patience, then
// Adam and the projection, and makes the next iteration's triangle records
// (the first iteration's come from setup_records). The device state is
// double-buffered by iteration parity (iteration i reads state i & 1 and
// writes the other).
// Once fit_step has stopped the fit, every kernel of a later iteration returns
// at entry (the `halt` flag mirrors the stop code) and fit_step only carries
// the state forward, so iterations launched ahead of a host check do no work.

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <string>
#include <vector>

#include "runtime.h"

using drh::NP;
using namespace drh_rt;

struct drh_fitter {
    drh_ctx* ctx = nullptr;
    hipStream_t s = nullptr;
    uint32_t math = 0;  // DRH_EXACT_MATH or 0
    int T = 0, H = 0, W = 0;
    drh_fit_config cfg{};
    Lease work, state, images, recs;
    // work: params, m, v, lr, grads, best (T x 10 each), losses (iters), loss (1)
    float *params = nullptr, *m = nullptr, *v = nullptr, *lr = nullptr, *grads = nullptr, *best = nullptr;
    float *losses = nullptr, *loss = nullptr;
    // images: the target (H x W x 3) and the background (3)
    float *target = nullptr, *bg = nullptr;
    float* rec = nullptr;         // the triangle records (T x REC; null when T = 0)
    int64_t rec_iter = -1;        // the iteration whose records `rec` holds (fit_step makes the next one's)
    drh::FitState* st = nullptr;  // two states, by iteration parity
    int* halt = nullptr;          // the stop code once stopped, else -1
    drh::FitState last{};   // the device state as last read back
    int64_t next = 0;       // index of the next iteration to launch
    int64_t launched = 0;   // iterations launched (the latest state is st[launched & 1])
    bool stopped = false;   // Fitter::stop_reason.is_some()
    int stop_reason = DRH_STOP_COMPLETED;
};

namespace {

constexpr float BETA1 = 0.9f, BETA2 = 0.999f, EPS = 1e-8f;  // optim.rs:29-31

// The fitter's device state: the bookkeeping by iteration parity and the halt flag.
struct FitDevState {
    drh::FitState st[2];
    int halt;
};
constexpr int64_t POLL_EVERY = 64;  // drh_fitter_run reads the device state this often

// fit.rs:343-349
float sigma_at(const drh_fit_config& c, int64_t i) {
    if (c.iters <= 1) return c.sigma_end;
    const float t = (float)i / (float)(c.iters - 1);
    return c.sigma_start * std::pow(c.sigma_end / c.sigma_start, t);
}

// Launches iteration i (nothing waits for it).
int launch_iteration(drh_fitter* f, int64_t i) {
    const float sigma = sigma_at(f->cfg, i);
    const uint32_t flags = f->math | DRH_DETERMINISTIC;
    const int32_t t = (int32_t)(i + 1);  // Adam's step count after its increment (optim.rs:41)
    drh::FitTail tail{};
    tail.iter = (int)i;
    tail.loss = f->loss;
    tail.params = f->params;
    tail.grads = f->grads;
    tail.m = f->m;
    tail.v = f->v;
    tail.lr = f->lr;
    tail.beta1 = BETA1;
    tail.beta2 = BETA2;
    tail.eps = EPS;
    tail.bc1 = 1.0f - powi_f32(BETA1, t);
    tail.bc2 = 1.0f - powi_f32(BETA2, t);
    tail.min_delta = f->cfg.min_delta;
    tail.patience = f->cfg.patience;
    tail.st = f->st;
    tail.halt = f->halt;
    tail.losses_out = f->losses;
    tail.best = f->best;
    // the records: made by the previous iteration's fit_step when that was i - 1
    tail.rec = f->rec;
    tail.rec_ready = f->rec && f->rec_iter == i ? 1 : 0;
    tail.sigma_next = sigma_at(f->cfg, i + 1);
    tail.W = f->W;
    tail.H = f->H;
    f->rec_iter = -1;
    int rc = run_raster(f->ctx, drh::MODE_LOSS, f->params, f->bg, f->target, 1, f->T, f->H, f->W, sigma, nullptr,
                        f->grads, f->loss, flags, f->s, f->halt, &tail);
    if (rc) return rc;
    f->rec_iter = f->rec ? i + 1 : -1;
    f->launched = i + 1;
    return DRH_OK;
}

// Reads the device state (and, when `loss` is given, the last loss) back.
int read_state(drh_fitter* f, float* loss = nullptr) {
    HIP_TRY(hipMemcpyAsync(&f->last, f->st + (f->launched & 1), sizeof f->last, hipMemcpyDeviceToHost, f->s),
            "read fit state");
    if (loss) HIP_TRY(hipMemcpyAsync(loss, f->loss, sizeof(float), hipMemcpyDeviceToHost, f->s), "read loss");
    int rc = wait_stream(f->s);
    if (rc) return rc;
    if (f->last.stop >= 0) {
        f->stopped = true;
        f->stop_reason = f->last.stop;
    }
    // the device has recorded n_losses iterations; the next one is n_losses
    // unless it stopped (a diverged iteration records nothing)
    if (!f->stopped) f->next = f->last.n_losses;
    return DRH_OK;
}

int copy_out(drh_fitter* f, float* dst, const float* src, size_t n, uint32_t flags) {
    if (n == 0) return DRH_OK;
    if (!dst) return fail(DRH_ERR_INVALID_ARG, "output pointer is NULL");
    const hipMemcpyKind k = (flags & DRH_HOST_PTRS) ? hipMemcpyDeviceToHost : hipMemcpyDeviceToDevice;
    hipError_t e = hipMemcpyAsync(dst, src, n * sizeof(float), k, f->s);
    if (e != hipSuccess) return fail(DRH_ERR_READBACK, std::string("hipMemcpyAsync: ") + hipGetErrorString(e));
    return finish(flags, f->s);
}

}  // namespace

extern "C" {

int drh_fit_validate(const drh_fit_config* c, int64_t T) {
    if (!c) return fail(DRH_ERR_INVALID_ARG, "config is NULL");
    // fit.rs:98-117, in the reference's order, with its messages (fit.rs:34-44).
    if (T <= 0) return (void)fail(DRH_ERR_INVALID_ARG, "triangles must be greater than zero"), DRH_CFG_NO_TRIANGLES;
    if (!(std::isfinite(c->sigma_start) && std::isfinite(c->sigma_end)) || c->sigma_start <= 0.0f ||
        c->sigma_end <= 0.0f)
        return (void)fail(DRH_ERR_INVALID_ARG, "sigma_start and sigma_end must be positive and finite"),
               DRH_CFG_NON_POSITIVE_SIGMA;
    if (c->sigma_start < c->sigma_end)
        return (void)fail(DRH_ERR_INVALID_ARG, "sigma_start must be greater than or equal to sigma_end"),
               DRH_CFG_SIGMA_NOT_DECREASING;
    for (float lr : {c->lr_pos, c->lr_color, c->lr_alpha})
        if (!std::isfinite(lr) || lr <= 0.0f)
            return (void)fail(DRH_ERR_INVALID_ARG, "learning rates must be positive and finite"),
                   DRH_CFG_NON_POSITIVE_LEARNING_RATE;
    return DRH_CFG_OK;
}

int drh_fitter_create(drh_ctx* ctx, const float* target, int64_t H, int64_t W, const float* background,
                      const float* init_params, int64_t T, const drh_fit_config* cfg, void* stream, uint32_t flags,
                      drh_fitter** out) {
    if (!out) return fail(DRH_ERR_INVALID_ARG, "out is NULL");
    *out = nullptr;
    if (!ctx) return fail(DRH_ERR_INVALID_ARG, "context is NULL");
    if (drh_fit_validate(cfg, T) != DRH_CFG_OK) return DRH_ERR_INVALID_ARG;
    int rc = check_shape(ctx, 1, T, H, W, cfg->sigma_end);
    if (rc) return rc;
    if (cfg->iters < 0 || cfg->iters > INT32_MAX) return fail(DRH_ERR_INVALID_ARG, "bad iteration count");
    if (!background || !target || !init_params) return fail(DRH_ERR_INVALID_ARG, "NULL argument");
    DeviceGuard dg(ctx->device);
    auto* f = new drh_fitter();
    f->ctx = ctx;
    f->s = (hipStream_t)stream;
    f->math = flags & DRH_EXACT_MATH;
    f->T = (int)T;
    f->H = (int)H;
    f->W = (int)W;
    f->cfg = *cfg;
    const bool host = flags & DRH_HOST_PTRS;
    const size_t n = (size_t)T * NP, iters = (size_t)cfg->iters, npix3 = (size_t)H * W * 3;
    auto bail = [&](int code) {
        delete f;
        return code;
    };
    if ((rc = f->work.acquire(ctx, K_FIT_F32, (n * 6 + iters + 1) * sizeof(float), f->s))) return bail(rc);
    if ((rc = f->state.acquire(ctx, K_FIT_STATE, sizeof(FitDevState), f->s))) return bail(rc);
    if ((rc = f->images.acquire(ctx, K_FIT_TARGET, (npix3 + 3) * sizeof(float), f->s))) return bail(rc);
    if ((rc = f->recs.acquire(ctx, K_REC, (size_t)T * drh::REC * sizeof(float), f->s))) return bail(rc);
    f->rec = f->recs.get<float>();
    f->params = f->work.get<float>();
    f->m = f->params + n;
    f->v = f->m + n;
    f->lr = f->v + n;
    f->grads = f->lr + n;
    f->best = f->grads + n;
    f->losses = f->best + n;
    f->loss = f->losses + iters;
    f->target = f->images.get<float>();
    f->bg = f->target + npix3;
    f->st = f->state.get<FitDevState>()->st;
    f->halt = &f->state.get<FitDevState>()->halt;

    // fit.rs:388-396 learning_rates()
    std::vector<float> lr(n);
    for (int64_t k = 0; k < T; k++) {
        for (int j = 0; j < 6; j++) lr[k * NP + j] = cfg->lr_pos;
        for (int j = 6; j < 9; j++) lr[k * NP + j] = cfg->lr_color;
        lr[k * NP + 9] = cfg->lr_alpha;
    }
    const drh::FitState st0{INFINITY, 0, 0, 0, -1};
    const FitDevState dev0{{st0, st0}, -1};
    const hipMemcpyKind in = host ? hipMemcpyHostToDevice : hipMemcpyDeviceToDevice;
    auto copy = [&](void* dst, const void* src, size_t bytes, hipMemcpyKind k) {
        return hipMemcpyAsync(dst, src, bytes, k, f->s);
    };
    hipError_t e = copy(f->params, init_params, n * sizeof(float), in);
    if (e == hipSuccess) e = copy(f->best, init_params, n * sizeof(float), in);
    if (e == hipSuccess) e = copy(f->target, target, npix3 * sizeof(float), in);
    if (e == hipSuccess) e = copy(f->bg, background, 3 * sizeof(float), in);
    if (e == hipSuccess) e = copy(f->lr, lr.data(), n * sizeof(float), hipMemcpyHostToDevice);
    if (e == hipSuccess) e = copy(f->state.get<FitDevState>(), &dev0, sizeof dev0, hipMemcpyHostToDevice);
    if (e != hipSuccess) return bail(hip_fail(e, "fitter set-up copies"));
    if ((e = drh::launch_zero(f->m, 2 * n, f->s)) != hipSuccess) return bail(hip_fail(e, "zero moments"));
    // lr and dev0 are host stack memory: wait before they go
    if ((rc = wait_stream(f->s))) return bail(rc);
    f->last = st0;
    *out = f;
    return DRH_OK;
}

int drh_fitter_destroy(drh_fitter* f) {
    if (!f) return DRH_OK;
    DeviceGuard dg(f->ctx->device);
    delete f;  // the leases go back to the context's pool, ordered by the fitter's stream
    return DRH_OK;
}

int drh_fitter_step(drh_fitter* f, int* stepped, drh_step_info* info) {
    if (!f || !stepped) return fail(DRH_ERR_INVALID_ARG, "NULL argument");
    *stepped = 0;
    if (f->stopped) return DRH_OK;
    if (f->next >= f->cfg.iters) {  // fit.rs:243-246
        f->stopped = true;
        f->stop_reason = DRH_STOP_COMPLETED;
        return DRH_OK;
    }
    DeviceGuard dg(f->ctx->device);
    const int64_t i = f->next;
    int rc = launch_iteration(f, i);
    if (rc) return rc;
    float loss = NAN;
    if ((rc = read_state(f, &loss))) return rc;
    if (f->stopped && f->stop_reason == DRH_STOP_DIVERGED) return DRH_OK;  // fit.rs:259-265: None
    *stepped = 1;
    if (info) {
        info->iter = i;
        info->loss = loss;
        info->sigma = sigma_at(f->cfg, i);
    }
    return DRH_OK;
}

int drh_fitter_run(drh_fitter* f, int64_t max_steps, int64_t* ran) {
    if (!f) return fail(DRH_ERR_INVALID_ARG, "fitter is NULL");
    if (ran) *ran = 0;
    if (max_steps < 0) return fail(DRH_ERR_INVALID_ARG, "negative step count");
    if (f->stopped) return DRH_OK;
    DeviceGuard dg(f->ctx->device);
    const int64_t before = f->last.n_losses;
    const int64_t end = std::min<int64_t>(f->cfg.iters, f->next + max_steps);
    int rc;
    for (int64_t i = f->next; i < end; i++) {
        if ((rc = launch_iteration(f, i))) return rc;
        // stop launching once the device has stopped; checked now and then
        // rather than per step, so the loop has no per-step host round trip
        if ((i + 1) % POLL_EVERY == 0 && i + 1 < end) {
            if ((rc = read_state(f))) return rc;
            if (f->stopped) break;
        }
    }
    if ((rc = read_state(f))) return rc;
    if (!f->stopped) f->next = f->last.n_losses;
    if (ran) *ran = f->last.n_losses - before;
    return DRH_OK;
}

int drh_fitter_status(const drh_fitter* f, drh_fit_status* out) {
    if (!f || !out) return fail(DRH_ERR_INVALID_ARG, "NULL argument");
    const int64_t iter = f->last.n_losses;  // Fitter::iter counts recorded iterations
    out->iter = iter;
    out->best_iter = f->last.best_iter;
    out->best_loss = f->last.best_loss;
    // Fitter::sigma (fit.rs:315-318): the softness of the next iteration
    const int64_t last_i = f->cfg.iters > 0 ? f->cfg.iters - 1 : 0;
    out->sigma = sigma_at(f->cfg, std::min(iter, last_i));
    out->done = (f->stopped || iter >= f->cfg.iters) ? 1 : 0;
    out->stop_reason = f->stopped ? f->stop_reason : -1;
    return DRH_OK;
}

int drh_fitter_scene(drh_fitter* f, float* out_params, uint32_t flags) {
    if (!f) return fail(DRH_ERR_INVALID_ARG, "fitter is NULL");
    DeviceGuard dg(f->ctx->device);
    return copy_out(f, out_params, f->params, (size_t)f->T * NP, flags);
}

int drh_fitter_losses(drh_fitter* f, float* out, int64_t capacity, int64_t* n_out, uint32_t flags) {
    if (!f || !n_out) return fail(DRH_ERR_INVALID_ARG, "NULL argument");
    const int64_t n = f->last.n_losses;
    *n_out = n;
    if (capacity < n) return fail(DRH_ERR_INVALID_ARG, "losses need room for " + std::to_string(n) + " floats");
    DeviceGuard dg(f->ctx->device);
    return copy_out(f, out, f->losses, (size_t)n, flags);
}

int drh_fitter_render_current(drh_fitter* f, float* out_image, uint32_t flags) {
    if (!f) return fail(DRH_ERR_INVALID_ARG, "fitter is NULL");
    if (!out_image) return fail(DRH_ERR_INVALID_ARG, "output pointer is NULL");
    DeviceGuard dg(f->ctx->device);
    // fit.rs:320-324: the current scene at its sharpest setting
    Out img;
    int rc = stage_out(f->ctx, img, K_OUT_IMAGES, out_image, (size_t)f->H * f->W * 3, flags & DRH_HOST_PTRS, f->s);
    if (rc) return rc;
    if ((rc = run_raster(f->ctx, drh::MODE_RENDER, f->params, f->bg, nullptr, 1, f->T, f->H, f->W, f->cfg.sigma_end,
                         img.dev, nullptr, nullptr, f->math, f->s)))
        return rc;
    if ((rc = copy_back(img, f->s))) return rc;
    return finish(flags, f->s);
}

int drh_fitter_report(drh_fitter* f, float* out_best_params, drh_fit_report* report, uint32_t flags) {
    if (!f || !report) return fail(DRH_ERR_INVALID_ARG, "NULL argument");
    DeviceGuard dg(f->ctx->device);
    int rc = copy_out(f, out_best_params, f->best, (size_t)f->T * NP, flags | DRH_SYNC);
    if (rc) return rc;
    // Fitter::into_report (fit.rs:326-334): stop_reason.unwrap_or(Completed)
    report->n_losses = f->last.n_losses;
    report->best_iter = f->last.best_iter;
    report->best_loss = f->last.best_loss;
    report->stop_reason = f->stopped ? f->stop_reason : DRH_STOP_COMPLETED;
    return DRH_OK;
}

int drh_fit(drh_ctx* ctx, const float* target, int64_t H, int64_t W, const float* background,
            const float* init_params, int64_t T, const drh_fit_config* cfg, float* out_losses,
            float* out_best_params, float* out_params, drh_fit_report* report, void* stream, uint32_t flags) {
    if (!ctx) return fail(DRH_ERR_INVALID_ARG, "context is NULL");
    if (!report || !out_best_params || (cfg && cfg->iters > 0 && !out_losses))
        return fail(DRH_ERR_INVALID_ARG, "NULL argument");
    drh_fitter* f = nullptr;
    int rc = drh_fitter_create(ctx, target, H, W, background, init_params, T, cfg, stream, flags, &f);
    if (rc) return rc;
    const uint32_t out_flags = flags & DRH_HOST_PTRS;
    int64_t n = 0;
    if (!(rc = drh_fitter_run(f, cfg->iters, nullptr)) &&
        !(rc = drh_fitter_losses(f, out_losses, cfg->iters, &n, out_flags)) &&
        !(rc = out_params ? drh_fitter_scene(f, out_params, out_flags) : DRH_OK))
        rc = drh_fitter_report(f, out_best_params, report, out_flags);
    drh_fitter_destroy(f);
    return rc;
}

}  // extern "C"
