// Lanczos3 resize of 8-bit images: the resample that Canvas::load_image
// applies to a target before a fit (crates/diffrast/src/canvas.rs:71-79,
// `resize_exact(w, h, FilterType::Lanczos3)` of image 0.25.10, Cargo.lock:410-411).
//
// The image crate's algorithm (imageops::resize): two separable passes, rows
// first into f32 (new_H x W x C), then columns back to bytes, clamped to
// [0, 255] and rounded half away from zero; the same size is a plain copy.
// Output index o of a pass over n_src -> n_dst samples reads source indices
// [left, left + count) with normalised Lanczos3 weights:
//   ratio = n_src / n_dst, scale = max(ratio, 1), support = 3 * scale,
//   centre = (o + 0.5) * ratio,
//   left = clamp(floor(centre - support), 0, n_src - 1),
//   right = clamp(ceil(centre + support), left + 1, n_src),
//   w_i = lanczos3((i - (centre - 0.5)) / scale) / sum_i.
// The weight tables are built on the host in f32 with the host libm's sinf,
// as the reference computes them, so the device applies the same weights; the
// device sums in the same order without fusing (built with -ffp-contract=off).
//
// Memory traffic per pass is one read of its input rows per tap that covers
// them and one write; this is a load-time helper (a few milliseconds for a
// photograph), not part of the fit's hot path.

#include <hip/hip_runtime.h>

#include <climits>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <vector>

#include "runtime.h"

namespace drh_rt {
namespace {

struct Tap {
    int left, offset, count;
};

// sinc with f32::consts::PI, 1 at 0; the Lanczos3 window (image 0.25 sample.rs).
float sinc_f32(float t) {
    const float a = t * 3.14159265358979323846f;
    return t == 0.0f ? 1.0f : sinf(a) / a;
}

float lanczos3(float x) { return fabsf(x) < 3.0f ? sinc_f32(x) * sinc_f32(x / 3.0f) : 0.0f; }

// Appends one pass's table: a Tap per output index, into `weights`.
void build_taps(int64_t n_src, int64_t n_dst, std::vector<Tap>& taps, std::vector<float>& weights) {
    const float ratio = (float)n_src / (float)n_dst;
    const float scale = ratio < 1.0f ? 1.0f : ratio;
    const float support = 3.0f * scale;
    for (int64_t o = 0; o < n_dst; o++) {
        const float centre = ((float)o + 0.5f) * ratio;
        int64_t lo = (int64_t)floorf(centre - support);
        lo = lo < 0 ? 0 : (lo > n_src - 1 ? n_src - 1 : lo);
        int64_t hi = (int64_t)ceilf(centre + support);
        hi = hi < lo + 1 ? lo + 1 : (hi > n_src ? n_src : hi);
        const float c = centre - 0.5f;
        const size_t first = weights.size();
        float sum = 0.0f;
        for (int64_t i = lo; i < hi; i++) {
            const float w = lanczos3(((float)i - c) / scale);
            weights.push_back(w);
            sum += w;
        }
        for (size_t k = first; k < weights.size(); k++) weights[k] /= sum;
        taps.push_back(Tap{(int)lo, (int)first, (int)(hi - lo)});
    }
}

constexpr int RS_THREADS = 256;
constexpr int RS_MAX_GRID_Y = 65535;

// Rows: tmp[oy][e] = sum_k w[k] * src[left + k][e], e over the W * C bytes of a row.
__global__ __launch_bounds__(RS_THREADS) void resize_rows(const uint8_t* __restrict__ src, int row_elems,
                                                          int new_h, const Tap* __restrict__ taps,
                                                          const float* __restrict__ weights,
                                                          float* __restrict__ tmp) {
    const int e = blockIdx.x * RS_THREADS + threadIdx.x;
    if (e >= row_elems) return;
    for (int oy = blockIdx.y; oy < new_h; oy += gridDim.y) {
        const Tap tp = taps[oy];
        const float* w = weights + tp.offset;
        const uint8_t* col = src + (size_t)tp.left * row_elems + e;
        float t = 0.0f;
        for (int k = 0; k < tp.count; k++) t += (float)col[(size_t)k * row_elems] * w[k];
        tmp[(size_t)oy * row_elems + e] = t;
    }
}

// Columns: dst[y][ox][c] = round(clamp(sum_k w[k] * tmp[y][left + k][c], 0, 255)).
__global__ __launch_bounds__(RS_THREADS) void resize_cols(const float* __restrict__ tmp, int w_src, int C,
                                                          int new_w, int new_h, const Tap* __restrict__ taps,
                                                          const float* __restrict__ weights,
                                                          uint8_t* __restrict__ dst) {
    const int e = blockIdx.x * RS_THREADS + threadIdx.x;
    if (e >= new_w * C) return;
    const int ox = e / C, c = e - ox * C;
    const Tap tp = taps[ox];
    const float* w = weights + tp.offset;
    for (int y = blockIdx.y; y < new_h; y += gridDim.y) {
        const float* row = tmp + ((size_t)y * w_src + tp.left) * C + c;
        float t = 0.0f;
        for (int k = 0; k < tp.count; k++) t += row[(size_t)k * C] * w[k];
        t = t < 0.0f ? 0.0f : (t > 255.0f ? 255.0f : t);
        dst[((size_t)y * new_w) * C + e] = (uint8_t)roundf(t);
    }
}

}  // namespace
}  // namespace drh_rt

using namespace drh_rt;

extern "C" int drh_resize_lanczos3(drh_ctx* ctx, const uint8_t* src, int64_t H, int64_t W, int64_t C, uint8_t* dst,
                                   int64_t new_H, int64_t new_W, void* stream, uint32_t flags) {
    if (!ctx) return fail(DRH_ERR_INVALID_ARG, "context is NULL");
    if (!src || !dst) return fail(DRH_ERR_INVALID_ARG, "NULL image");
    if (C < 1 || C > 4) return fail(DRH_ERR_INVALID_ARG, "channels must be 1 to 4");
    if (H <= 0 || W <= 0 || new_H <= 0 || new_W <= 0)
        return fail(DRH_ERR_INVALID_ARG, "image sizes must be positive");
    if (W * C > INT_MAX || new_W * C > INT_MAX || H > INT_MAX || new_H > INT_MAX)
        return fail(DRH_ERR_TOO_LARGE, "an image row is too long");
    DeviceGuard dg(ctx->device);
    hipStream_t s = (hipStream_t)stream;
    const bool host = flags & DRH_HOST_PTRS;
    const size_t in_bytes = (size_t)(H * W * C), out_bytes = (size_t)(new_H * new_W * C);
    int rc;

    Lease in_l, out_l;
    const uint8_t* din = src;
    uint8_t* dout = dst;
    if (host) {
        if ((rc = in_l.acquire(ctx, K_SRGB_U8, in_bytes, s)) || (rc = out_l.acquire(ctx, K_RESIZE_U8, out_bytes, s)))
            return rc;
        HIP_TRY(hipMemcpyAsync(in_l.get<uint8_t>(), src, in_bytes, hipMemcpyHostToDevice, s), "hipMemcpyAsync H2D");
        din = in_l.get<uint8_t>();
        dout = out_l.get<uint8_t>();
    }

    if (H == new_H && W == new_W) {  // imageops::resize: the same size is a copy
        HIP_TRY(hipMemcpyAsync(dout, din, in_bytes, hipMemcpyDeviceToDevice, s), "hipMemcpyAsync D2D");
    } else {
        // rows' taps first, then columns'; both index the one weight array
        std::vector<Tap> taps;
        std::vector<float> weights;
        build_taps(H, new_H, taps, weights);
        build_taps(W, new_W, taps, weights);
        const size_t tap_bytes = taps.size() * sizeof(Tap), w_bytes = weights.size() * sizeof(float);
        const size_t tmp_bytes = (size_t)new_H * (size_t)(W * C) * sizeof(float);
        Lease tap_l, w_l, tmp_l;
        if ((rc = tap_l.acquire(ctx, K_RESIZE_TAB, tap_bytes, s)) || (rc = w_l.acquire(ctx, K_RESIZE_TAB, w_bytes, s)) ||
            (rc = tmp_l.acquire(ctx, K_RESIZE_TMP, tmp_bytes, s)))
            return rc;
        // Copied from host vectors: the stream is waited for below, before
        // they go out of scope.
        HIP_TRY(hipMemcpyAsync(tap_l.get<Tap>(), taps.data(), tap_bytes, hipMemcpyHostToDevice, s), "hipMemcpyAsync H2D");
        HIP_TRY(hipMemcpyAsync(w_l.get<float>(), weights.data(), w_bytes, hipMemcpyHostToDevice, s),
                "hipMemcpyAsync H2D");
        const Tap* dv = tap_l.get<Tap>();
        const Tap* dh = dv + new_H;
        const float* dw = w_l.get<float>();
        const int row_elems = (int)(W * C), out_elems = (int)(new_W * C);
        const unsigned gy = (unsigned)(new_H < RS_MAX_GRID_Y ? new_H : RS_MAX_GRID_Y);
        hipLaunchKernelGGL(resize_rows, dim3((unsigned)((row_elems + RS_THREADS - 1) / RS_THREADS), gy),
                           dim3(RS_THREADS), 0, s, din, row_elems, (int)new_H, dv, dw, tmp_l.get<float>());
        HIP_TRY(hipGetLastError(), "resize_rows launch");
        hipLaunchKernelGGL(resize_cols, dim3((unsigned)((out_elems + RS_THREADS - 1) / RS_THREADS), gy),
                           dim3(RS_THREADS), 0, s, tmp_l.get<float>(), (int)W, (int)C, (int)new_W, (int)new_H, dh,
                           dw, dout);
        HIP_TRY(hipGetLastError(), "resize_cols launch");
        if ((rc = wait_stream(s))) return rc;
    }
    if (host) {
        hipError_t e = hipMemcpyAsync(dst, dout, out_bytes, hipMemcpyDeviceToHost, s);
        if (e != hipSuccess) return fail(DRH_ERR_READBACK, std::string("hipMemcpyAsync D2H: ") + hipGetErrorString(e));
    }
    return finish(flags, s);
}
