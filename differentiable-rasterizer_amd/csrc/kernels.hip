// Soft-triangle rasterizer kernels for gfx950 (MI355X).
//
// Semantics follow the reference CPU path (crates/diffrast/src/raster.rs,
// grad.rs, optim.rs, fit.rs); the work decomposition is this file's own:
//
//   setup_records : one thread per (scene, triangle). Computes the padded
//                   integer bounding box exactly as raster.rs:144-168 does,
//                   the edge vectors and the data for a conservative
//                   far-outside / deep-inside classification.
//   forward_kernel : one wave64 per 8x8 pixel tile, four tiles per block.
//                   Each wave compacts the triangles touching its tile into an
//                   ordered LDS list (ballot + mbcnt), then walks it with the
//                   triangle record in SGPRs (scalar loads), compositing in
//                   scene order (raster.rs:46-68); in the gradient modes it
//                   records the contributing entries with their lane masks
//                   and each pixel's total transmittance.
//   backward_kernel : the same tiles, walking the recorded entries again in
//                   scene order: the gradient reaching layer k,
//                   d_canvas * prod_{j>k}(1 - w_j) (grad.rs:162-169), is formed
//                   as a ratio of transmittance products instead of being
//                   peeled off a tape. Per-triangle gradients are summed over
//                   the wave by a transposition through LDS, accumulated in
//                   LDS rows and added to the output once per block (or
//                   written as one partial row per block).
//   reduce_partials : fixed-order sum of the partial rows, so gradients and
//                   losses are bit-reproducible run to run.
//   adam_project  : optim.rs:40-60 followed by fit.rs:399-424, elementwise.
//
// The whole file is compiled with -ffp-contract=off: every a*b+c below that is
// written without an explicit fmaf rounds twice, as the reference does. FMAs
// appear only where the reference's rounding cannot change a result beyond
// the stated tolerance (gradient assembly, conservative classification).

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <climits>
#include <stdint.h>
#include <type_traits>

#include "kernels.h"

namespace drh {

namespace {
thread_local LaunchEvents t_launch_events;
}  // namespace
LaunchEvents& launch_events() { return t_launch_events; }

// Every launch of this file: hipExtLaunchKernel, with the calling thread's
// timing events when it has some (launch_events), which then go to this
// launch alone.
template <typename F, typename... Args>
static void launch_k(F kernel, const dim3& grid, const dim3& block, size_t lds, hipStream_t s, Args... args) {
    LaunchEvents& ev = t_launch_events;
    hipExtLaunchKernelGGL(kernel, grid, block, (uint32_t)lds, s, ev.start, ev.stop, 0u, args...);
    if (ev.start) {
        ev.used = true;
        ev.start = ev.stop = nullptr;
    }
}

constexpr float MIN_WEIGHT = 1e-6f;  // raster.rs:31-34

// ---------------------------------------------------------------- records

__device__ inline float rust_clamp(float x, float lo, float hi) {
    if (x < lo) x = lo;
    if (x > hi) x = hi;
    return x;
}

// raster.rs:144-168 for one bound: floor/ceil of (coord -/+ pad) * n in f32,
// `.max(0.0) as usize`, and for the upper bound `+ 1` (wrapping) then `.min(n)`.
__device__ inline int lower_bound_px(float lo, float pad, int n) {
    float f = fmaxf(floorf((lo - pad) * (float)n), 0.0f);
    return (f >= (float)n) ? n : (int)f;
}
__device__ inline int upper_bound_px(float hi, float pad, int n) {
    float c = fmaxf(ceilf((hi + pad) * (float)n), 0.0f);
    if (c >= 18446744073709551616.0f) return 0;  // saturates, then `+ 1` wraps to 0
    return (c >= (float)n) ? n : (int)c + 1;
}

// A triangle's cull box in order cells (inclusive; x0 > x1 when empty).
struct BlockBox {
    int x0, y0, x1, y1;
};

// The cull box of triangle p (raster.rs:26-28, 144-168) in cells of 2^shift
// pixels, for the block-order estimate (a taped forward's liveness: alpha > 0).
__device__ inline BlockBox block_box(const float* __restrict__ p, int W, int H, float sigma, int shift) {
    float v[6];
    bool finite = true;
    for (int j = 0; j < 6; j++) {
        v[j] = p[j];
        finite = finite && isfinite(v[j]);
    }
    BlockBox bb = {1, 1, 0, 0};
    if (!finite || !(p[9] > 0.0f)) return bb;
    const float pad = 6.0f * sigma;
    const int bx0 = lower_bound_px(fminf(fminf(v[0], v[2]), v[4]), pad, W);
    const int by0 = lower_bound_px(fminf(fminf(v[1], v[3]), v[5]), pad, H);
    const int bx1 = upper_bound_px(fmaxf(fmaxf(v[0], v[2]), v[4]), pad, W);
    const int by1 = upper_bound_px(fmaxf(fmaxf(v[1], v[3]), v[5]), pad, H);
    if (bx0 < bx1 && by0 < by1) bb = {bx0 >> shift, by0 >> shift, (bx1 - 1) >> shift, (by1 - 1) >> shift};
    return bb;
}

// The order estimate of one triangle: which cells it can reach. Its cull box
// in cells, `far` (the distance beyond which its weight is below MIN_WEIGHT:
// alpha sigmoid(-d / sigma) < alpha e^(-d / sigma)), and its vertices sorted
// by y (top t, middle m, bottom b) with the slopes dx/dy of the long edge tb
// and the short edges tm and mb. Made once per triangle and kept in LDS for
// the threads that walk its cell rows. The arithmetic is approximate: the
// estimate only orders the cells.
struct Reach {
    float xt, yt, xm, ym, xb, yb, s_tb, s_tm, s_mb, far;
    uint32_t lo, hi;  // cull box in cells: x0 | y0 << 16, x1 | y1 << 16 (x0 > x1 when culled)
    __device__ int x0() const { return (int)(lo & 0xFFFFu); }
    __device__ int y0() const { return (int)(lo >> 16); }
    __device__ int x1() const { return (int)(hi & 0xFFFFu); }
    __device__ int y1() const { return (int)(hi >> 16); }
};
static_assert(ORD_MAX_CELLS <= 0xFFFF, "cell indices fit 16 bits");

__device__ inline float slope(float dx, float dy) { return dy > 0.0f ? __fdividef(dx, dy) : 0.0f; }

__device__ inline Reach make_reach(const float (&p)[NP], int W, int H, float sigma, int shift) {
    Reach r{};
    const BlockBox bb = block_box(p, W, H, sigma, shift);  // finite vertices, alpha > 0
    r.lo = 1u | 1u << 16;  // culled
    r.hi = 0u;
    if (bb.x0 > bb.x1 || bb.y0 > bb.y1) return r;
    r.lo = (uint32_t)bb.x0 | (uint32_t)bb.y0 << 16;
    r.hi = (uint32_t)bb.x1 | (uint32_t)bb.y1 << 16;
    r.far = fmaxf(__logf(fminf(p[9], 1.0f) * (1.0f / MIN_WEIGHT)) + 0.05f, 0.0f) * fmaxf(sigma, 1e-8f);
    float ax = p[0], ay = p[1], bx = p[2], by = p[3], cx = p[4], cy = p[5];
    auto order = [](float& ux, float& uy, float& vx, float& vy) {
        if (vy < uy) {
            const float tx = ux, ty = uy;
            ux = vx;
            uy = vy;
            vx = tx;
            vy = ty;
        }
    };
    order(ax, ay, bx, by);
    order(bx, by, cx, cy);
    order(ax, ay, bx, by);
    r.xt = ax;
    r.yt = ay;
    r.xm = bx;
    r.ym = by;
    r.xb = cx;
    r.yb = cy;
    r.s_tb = slope(cx - ax, cy - ay);
    r.s_tm = slope(bx - ax, by - ay);
    r.s_mb = slope(cx - bx, cy - by);
    return r;
}

constexpr int REACH_PAIR_ROWS = 8;  // cell rows of a box from which reach_rows walks pairs

// Counts the cells the triangle can reach into the difference rows `cells`
// (pitch ints per cell row), for cell rows j, j + m, ... of its cull box: in
// each row, the run of cells whose pixel centres come within `far` of the
// triangle. The run is the triangle's x extent inside the cell row's band of
// pixel centres widened by `far` (the edges' x at the band's clipped ends, and
// the vertices inside it), widened by `far` in x and clipped to the cull box.
// It over-counts cells near the triangle's corners a little; a count of the
// cull box alone also counts the cells between a thin or slanted triangle's
// edges and its box, which are often most of them. r is taken by value: its
// fields stay in registers over the rows.
// With `rowmask` it also sets the triangle's bit k in the masks of every row of
// its cull box (words 32-bit words per row). Without (no row lists: fewer than
// 256 triangles, which are large), a triangle whose box spans REACH_PAIR_ROWS
// or more cell rows takes them in pairs, each pair's run that of the two rows'
// joint band, added to both: half the walk, which is the order workgroup's
// longest phase for such triangles.
template <bool MASKS>
__device__ inline void reach_rows(const Reach r, const OrderArgs& o, int j, int m, int* cells, int pitch,
                                  uint32_t* rowmask, int words, int k) {
    const float cs = (float)(1 << o.shift), rH = o.r_h, cell_h = o.cell_h, wc = o.w_cells;
    const float band = (cs - 1.0f) * rH + 2.0f * r.far, y_first = 0.5f * rH - r.far;
    const float c0_off = o.c0_off, c1_off = o.c1_off;
    auto short_x = [&](float y) { return y <= r.ym ? fmaf(y - r.yt, r.s_tm, r.xt) : fmaf(y - r.ym, r.s_mb, r.xm); };
    const int x0 = r.x0(), x1 = r.x1(), y1 = r.y1();
    const int rows = !MASKS && y1 - r.y0() + 1 >= REACH_PAIR_ROWS ? 2 : 1;
    const float bandr = band + (float)(rows - 1) * cell_h;
    for (int y = r.y0() + rows * j; y <= y1; y += rows * m) {
        if (MASKS) atomicOr(&rowmask[y * words + (k >> 5)], 1u << (k & 31));
        const float ya = fmaf((float)y, cell_h, y_first);
        const float ca = fmaxf(ya, r.yt), cb = fminf(ya + bandr, r.yb);
        if (!(ca <= cb)) continue;
        const float la = fmaf(ca - r.yt, r.s_tb, r.xt), lb = fmaf(cb - r.yt, r.s_tb, r.xt);
        const float sa = short_x(ca), sb = short_x(cb);
        float lo = fminf(fminf(la, lb), fminf(sa, sb)), hi = fmaxf(fmaxf(la, lb), fmaxf(sa, sb));
        const bool mid = ca <= r.ym && r.ym <= cb, bot = ca <= r.yb && r.yb <= cb;
        lo = fminf(lo, fminf(mid ? r.xm : lo, bot ? r.xb : lo));
        hi = fmaxf(hi, fmaxf(mid ? r.xm : hi, bot ? r.xb : hi));
        // cells c whose centres (c cs + 0.5) / W .. (c cs + cs - 0.5) / W meet [lo - far, hi + far]
        const float c0f = ceilf(fmaf(lo - r.far, wc, c0_off)), c1f = floorf(fmaf(hi + r.far, wc, c1_off));
        const int c0 = (int)fminf(fmaxf(c0f, (float)x0), (float)(x1 + 1));
        const int c1 = (int)fmaxf(fminf(c1f, (float)x1), (float)(x0 - 1));
        if (c0 > c1) continue;
        atomicAdd(&cells[y * pitch + c0], 1);
        atomicAdd(&cells[y * pitch + c1 + 1], -1);
        if (!MASKS && rows == 2 && y + 1 <= y1) {
            atomicAdd(&cells[(y + 1) * pitch + c0], 1);
            atomicAdd(&cells[(y + 1) * pitch + c1 + 1], -1);
        }
    }
}

// The record of triangle i (scene-major index) from its parameters p.
__device__ inline void setup_from(const float* __restrict__ p, size_t i, int W, int H, float sigma, int setup_mode,
                                  float* __restrict__ rec) {
    float* r = rec + i * REC;

    float v[6];
    for (int j = 0; j < 6; j++) v[j] = p[j];
    float alpha = rust_clamp(p[9], 0.0f, 1.0f);

    bool finite = true;
    for (int j = 0; j < 6; j++) finite = finite && isfinite(v[j]);
    int bx0 = 0, by0 = 0, bx1 = 0, by1 = 0;
    if (finite) {
        float pad = 6.0f * sigma;  // raster.rs:26-28
        float lo_x = fminf(fminf(fminf(INFINITY, v[0]), v[2]), v[4]);
        float hi_x = fmaxf(fmaxf(fmaxf(-INFINITY, v[0]), v[2]), v[4]);
        float lo_y = fminf(fminf(fminf(INFINITY, v[1]), v[3]), v[5]);
        float hi_y = fmaxf(fmaxf(fmaxf(-INFINITY, v[1]), v[3]), v[5]);
        bx0 = lower_bound_px(lo_x, pad, W);
        by0 = lower_bound_px(lo_y, pad, H);
        bx1 = upper_bound_px(hi_x, pad, W);
        by1 = upper_bound_px(hi_y, pad, H);
    }
    bool box_ok = finite && bx0 < bx1 && by0 < by1;
    // render (raster.rs:48-51) rejects `alpha <= 0`, which lets NaN through;
    // the taped forward (grad.rs:61-62) keeps only `alpha > 0`.
    const bool taped = box_ok && alpha > 0.0f;
    bool live = setup_mode == SETUP_TAPE ? taped : box_ok && !(alpha <= 0.0f);

    // Edges in the reference's order: (v0,v1), (v1,v2), (v2,v0); e = b - a.
    float e[6];
    for (int j = 0; j < 3; j++) {
        int a = j, b = (j + 1) % 3;
        e[2 * j] = v[2 * b] - v[2 * a];
        e[2 * j + 1] = v[2 * b + 1] - v[2 * a + 1];
    }
    float len2[3], rlen2[3];
    for (int j = 0; j < 3; j++) {
        len2[j] = e[2 * j] * e[2 * j] + e[2 * j + 1] * e[2 * j + 1];
        rlen2[j] = (len2[j] <= 1e-20f) ? 0.0f : 1.0f / len2[j];
    }

    // Conservative classification data. With s the orientation sign, the
    // outward distance of a point to edge line j is l_j = pt.n_j - off_j, and
    // max_j l_j bounds the true distance from the triangle from below (outside)
    // or the distance to the boundary from above (inside). It is only trusted
    // for a triangle whose area is large against the rounding of the
    // reference's cross products, so that its inside test cannot flip.
    float m = 0.0f;
    for (int j = 0; j < 6; j++) m = fmaxf(m, fabsf(v[j]));
    float area2 = e[0] * (v[5] - v[1]) - e[1] * (v[4] - v[0]);
    float slack = 1e-5f * (1.0f + m);
    bool fast = finite && (alpha == alpha) && m <= 1e4f &&
                fabsf(area2) >= 1e-4f * (1.0f + m) * (1.0f + m);
    float s = area2 >= 0.0f ? 1.0f : -1.0f;
    float n[6], off[3];
    for (int j = 0; j < 3; j++) {
        float len = sqrtf(len2[j]);
        float inv = (fast && len > 0.0f) ? s / len : 0.0f;
        n[2 * j] = e[2 * j + 1] * inv;
        n[2 * j + 1] = -e[2 * j] * inv;
        off[j] = v[2 * j] * n[2 * j] + v[2 * j + 1] * n[2 * j + 1];
    }
    float sig = fmaxf(sigma, 1e-8f);

    for (int j = 0; j < 6; j++) r[R_V + j] = v[j];
    for (int j = 0; j < 3; j++) r[R_C + j] = p[6 + j];
    r[R_A] = alpha;
    int* ri = reinterpret_cast<int*>(r);
    ri[R_BOX + 0] = live ? bx0 : 0;
    ri[R_BOX + 1] = live ? by0 : 0;
    ri[R_BOX + 2] = live ? bx1 : 0;
    ri[R_BOX + 3] = live ? by1 : 0;
    bool active = p[9] > 0.0f && p[9] < 1.0f;  // grad.rs:145
    ri[R_FLAGS] = (live ? F_LIVE : 0) | (active ? F_ACTIVE : 0) | (fast && live ? F_FAST : 0) |
                  (area2 >= 0.0f ? F_CCW : 0) | (taped ? F_TAPE : 0);
    r[R_SPARE] = 0.0f;
    for (int j = 0; j < 6; j++) r[R_E + j] = e[j];
    for (int j = 0; j < 3; j++) r[R_LEN2 + j] = len2[j];
    for (int j = 0; j < 3; j++) r[R_RLEN2 + j] = rlen2[j];
    for (int j = 0; j < 6; j++) r[R_N + j] = n[j];
    for (int j = 0; j < 3; j++) r[R_OFF + j] = off[j];
    // Far outside: at a true distance d >= sigma (ln(alpha / MIN_WEIGHT) + 0.05)
    // the weight is alpha * sigmoid(-d / sigma) < alpha e^(-d / sigma)
    // <= 0.951 MIN_WEIGHT, which the f32 rounding of the reference's sigmoid
    // and product (a few ulp) cannot lift to MIN_WEIGHT: it skips the pair too.
    // Deep inside: at a distance to the edge above 17 sigma, exp(-x) < 4.2e-8
    // < 2^-24, so the reference's 1 / (1 + exp(-x)) rounds to exactly 1.0f.
    float xfar = fmaxf(logf(alpha * (1.0f / MIN_WEIGHT)) + 0.05f, 0.0f);
    r[R_FAR] = (xfar == xfar ? xfar : 0.0f) * sig + slack;
    r[R_DEEP] = -(17.0f * sig + slack);
    r[R_SLACK] = slack;
    // Along-edge coordinate s_j = p . d_j - a_j . d_j, with d_j the unit edge
    // direction: with the edge-line distance it bounds the distance of a whole
    // tile to each edge segment when the tile's list is built.
    for (int j = 0; j < 3; j++) {
        float len = sqrtf(len2[j]);
        float inv = (fast && len > 0.0f) ? 1.0f / len : 0.0f;
        float dx = e[2 * j] * inv, dy = e[2 * j + 1] * inv;
        r[R_D + 2 * j] = dx;
        r[R_D + 2 * j + 1] = dy;
        r[R_SOFF + j] = v[2 * j] * dx + v[2 * j + 1] * dy;
        r[R_LEN + j] = len;
        float* eb = r + R_EB + 8 * j;
        eb[0] = v[2 * j];
        eb[1] = v[2 * j + 1];
        eb[2] = e[2 * j];
        eb[3] = e[2 * j + 1];
        eb[4] = len2[j];
        eb[5] = rlen2[j];
        eb[6] = area2 >= 0.0f ? 1.0f : -1.0f;  // F_CCW as a factor: c eb[6] >= 0 inside
        eb[7] = 0.0f;
    }
}

// Setup of triangle i: its record from params[i * NP ...].
__device__ inline void setup_one(const float* __restrict__ params, size_t i, int W, int H, float sigma,
                                 int setup_mode, float* __restrict__ rec, float* __restrict__ zero_grads) {
    // The backward kernel adds into the gradients: they start at zero.
    if (zero_grads)
        for (int j = 0; j < NP; j++) zero_grads[i * NP + j] = 0.0f;
    setup_from(params + i * NP, i, W, H, sigma, setup_mode, rec);
}

// The raster kernels' block order, heaviest first. A block's time follows its
// tiles' lists; the longest blocks, started late in a grid of several rounds,
// run on while most of the device has nothing left, and heavy blocks that land
// on one CU finish last. A block's cost is estimated by the number of
// triangles that can reach it (reach_rows) plus a share for building its lists
// (which reads every triangle). Each scene's workgroup counts them in LDS (a
// difference array per cell row: two adds per triangle and row, then prefix
// sums along the rows), counting-sorts the scene's blocks by the estimate,
// heaviest first, and writes their scene-local indices to perm[b * nb ...]. The raster kernels take launch
// slot i to rank i / B of scene i % B, so the heaviest blocks of every scene go
// first. Nothing crosses workgroups: a device-wide hand-off would cost more
// than the order saves. The records then come from workgroups of
// SETUP_REC_PER triangles: a wave stores each record as 19 16-byte pieces at a
// 304-byte stride, a cache line per lane and store, and one CU issues about one
// line per cycle, so 512 records on one CU took ~6 us and on four ~1.5.
constexpr int SETUP_THREADS = 1024, ORD_BUCKETS = 1024, ORD_REACH = 512, SETUP_REC_PER = 128;
static_assert(ORD_BUCKETS == 16 * 64 && SETUP_THREADS % 64 == 0 && ORD_REACH <= SETUP_THREADS,
              "order workgroup shape: 16 buckets per lane of one wave");

// Inclusive prefix sum within each row of 16 lanes (every lane active): DPP
// row shifts (lanes with no source read the `old` operand, 0).
__device__ inline int row_scan_incl(int v) {
    v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xF, 0xF, false);  // row_shr:1
    v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xF, 0xF, false);  // row_shr:2
    v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xF, 0xF, false);  // row_shr:4
    v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xF, 0xF, false);  // row_shr:8
    return v;
}

// Inclusive prefix sum over the wave's lanes (every lane active).
// DPP row shifts within each row of 16 lanes (lanes with no source read the
// `old` operand, 0), then the last lane of rows 0 and 2 broadcast into rows 1
// and 3, then lane 31 into rows 2 and 3 (gfx9 row_bcast).
__device__ inline int wave_scan_incl(int v, int) {
    v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xF, 0xF, false);  // row_shr:1
    v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xF, 0xF, false);  // row_shr:2
    v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xF, 0xF, false);  // row_shr:4
    v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xF, 0xF, false);  // row_shr:8
    v += __builtin_amdgcn_update_dpp(0, v, 0x142, 0xA, 0xF, false);  // row_bcast:15
    v += __builtin_amdgcn_update_dpp(0, v, 0x143, 0xC, 0xF, false);  // row_bcast:31
    return v;
}

// hist: ORD_BUCKETS zeroes (cleared before the caller's first barrier).
__device__ inline void order_scene(const OrderArgs& o, int* cells, int* hist, int b, int T) {
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6, gx = o.gx, gy = o.gy, pitch = gx + 1, nb = gx * gy;
    const int base = 6 * ((T + 63) / 64);  // list building, against one reaching triangle
    auto key_of = [&](int count) { return ORD_BUCKETS - 1 - min(count + base, ORD_BUCKETS - 1); };
    // prefix sums along the cell rows, one wave per row at a time: 64 cells per
    // step, a wave scan plus the carry of the row's earlier cells; each cell's
    // count goes into the histogram as soon as it is known
    for (int y = wave; y < gy; y += SETUP_THREADS / 64) {
        int carry = 0;
        for (int x0 = 0; x0 <= gx; x0 += 64) {
            const int x = x0 + lane;
            const int v = wave_scan_incl(x <= gx ? cells[y * pitch + x] : 0, lane);
            if (x <= gx) cells[y * pitch + x] = v + carry;
            if (x < gx) atomicAdd(&hist[key_of(v + carry)], 1);
            carry += __shfl(v, 63, 64);
        }
    }
    __syncthreads();
    // exclusive prefix of the histogram in one wave: lane l sums buckets
    // 16 l .. 16 l + 15, a wave scan places the lanes' runs
    if (wave == 0) {
        typedef int i4v __attribute__((ext_vector_type(4)));
        i4v* const h4 = reinterpret_cast<i4v*>(hist + 16 * lane);
        i4v q[4];
        int sum = 0;
        for (int j = 0; j < 4; j++) {
            q[j] = h4[j];
            sum += (q[j].x + q[j].y) + (q[j].z + q[j].w);
        }
        int run = wave_scan_incl(sum, lane) - sum;
        for (int j = 0; j < 4; j++) {
            i4v e;
            e.x = run;
            e.y = e.x + q[j].x;
            e.z = e.y + q[j].y;
            e.w = e.z + q[j].z;
            run = e.w + q[j].w;
            h4[j] = e;
        }
    }
    __syncthreads();
    auto key = [&](int blk) { return key_of(cells[(blk / gx) * pitch + blk % gx]); };
    for (int blk = t; blk < nb; blk += SETUP_THREADS) {
        const int pos = atomicAdd(&hist[key(blk)], 1);  // < nb: the offsets partition [0, nb)
        if (pos < nb) o.perm[(size_t)b * nb + pos] = blk;
    }
}

// Workgroup (b, y): the records of scene b's triangles [x per, x per + per)
// (and every nx per after, nx the records workgroups per scene), per the
// records per workgroup and x = y. With o.perm (then the workgroup
// size is SETUP_THREADS and per SETUP_REC_PER), workgroup (b, 0) makes the
// scene's block order from the triangles' boxes, computed again from the
// parameters, concurrently with the records of workgroups (b, x + 1). The
// order workgroups, the longest, come first in the grid, so that they are
// dispatched before any records.
__global__ __launch_bounds__(SETUP_THREADS) void setup_records(const float* __restrict__ params, int T, int W,
                                                               int H, float sigma, int setup_mode,
                                                               float* __restrict__ rec, float* __restrict__ zero_grads,
                                                               const float* __restrict__ bg_src,
                                                               float* __restrict__ bg_dst, OrderArgs o,
                                                               const int* __restrict__ halt,
                                                               RecordHead* __restrict__ head, RecordHead head_val,
                                                               double* __restrict__ pending, int npending) {
    __shared__ int cells[ORD_MAX_CELLS];
    __shared__ __attribute__((aligned(16))) int hist[ORD_BUCKETS];
    if (halt && *halt >= 0) return;
    const int b = blockIdx.x, part = blockIdx.y, pitch = o.gx + 1;
    const int per = o.perm ? SETUP_REC_PER : (int)blockDim.x;  // records per workgroup
    if (head && b == 0 && part == 0 && threadIdx.x == 0) *head = head_val;
    // A record kept for a later backward holds its own copy of the backgrounds.
    if (bg_dst && part == 0 && threadIdx.x < 3) bg_dst[b * 3 + threadIdx.x] = bg_src[b * 3 + threadIdx.x];
    // the scene's loss slots, pending until the fused kernel's tiles store
    // theirs: from the last workgroup of the scene down, so that the records
    // workgroups' idle threads take them before the order workgroup does
    if (pending)
        for (int i = ((int)gridDim.y - 1 - part) * (int)blockDim.x + (int)threadIdx.x; i < npending;
             i += (int)(gridDim.y * blockDim.x))
            pending[(size_t)b * npending + i] = __longlong_as_double((long long)LOSS_PENDING);
    if (!o.perm || part > 0) {
        // grid rows are capped at 65535: a records workgroup strides over the rest
        const int nparts = (int)gridDim.y - (o.perm ? 1 : 0);
        if ((int)threadIdx.x < per)
            for (int k = (o.perm ? part - 1 : part) * per + (int)threadIdx.x; k < T; k += nparts * per)
                setup_one(params, (size_t)b * T + k, W, H, sigma, setup_mode, rec, zero_grads);
        return;
    }
    // Triangles in batches of up to ORD_REACH: each one's Reach made by one
    // thread into LDS, then its cell rows walked by m threads (when the batch
    // leaves threads over), each taking every m-th row. A batch's parameters
    // are loaded before the work that precedes its Reach (the first batch's
    // before the cells are cleared).
    __shared__ Reach reach[ORD_REACH];
    __shared__ uint32_t rowmask_s[ORD_ROW_WORDS];
    const int words = (T + 31) / 32;
    uint32_t* const rowmask = o.rows && o.gy * words <= ORD_ROW_WORDS ? rowmask_s : nullptr;
    if (rowmask)
        for (int c = threadIdx.x; c < o.gy * words; c += SETUP_THREADS) rowmask[c] = 0u;
    float pk[NP];
    auto load_batch = [&](int k0) {
        const int k = k0 + (int)threadIdx.x;
        if ((int)threadIdx.x < ORD_REACH && k < T)
            for (int q = 0; q < NP; q++) pk[q] = params[((size_t)b * T + k) * NP + q];
    };
    load_batch(0);
    for (int c = threadIdx.x; c < (o.gy + 1) * pitch; c += SETUP_THREADS) cells[c] = 0;
    for (int c = threadIdx.x; c < ORD_BUCKETS; c += SETUP_THREADS) hist[c] = 0;
    for (int k0 = 0; k0 < T; k0 += ORD_REACH) {
        const int nt = min(ORD_REACH, T - k0);
        if ((int)threadIdx.x < nt) reach[threadIdx.x] = make_reach(pk, W, H, sigma, o.shift);
        load_batch(k0 + ORD_REACH);
        __syncthreads();
        // a power of two, so that the thread's triangle and row are a shift and a mask
        const int lg = 31 - __clz(min(SETUP_THREADS / nt, 16)), m = 1 << lg;
        for (int w = threadIdx.x; w < nt * m; w += SETUP_THREADS) {
            if (rowmask)
                reach_rows<true>(reach[w >> lg], o, w & (m - 1), m, cells, pitch, rowmask, words, k0 + (w >> lg));
            else
                reach_rows<false>(reach[w >> lg], o, w & (m - 1), m, cells, pitch, nullptr, 0, 0);
        }
        __syncthreads();
    }
    order_scene(o, cells, hist, b, T);
    if (!rowmask) return;
    // Each row's set bits in index order: a scan of the words' bit counts
    // places each word's indices. Up to 16 words (512 triangles) a row takes
    // one 16-lane row of a wave (four rows per wave, DPP row scans), so that
    // every row is expanded in one pass instead of one row after another.
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (words <= 16) {
        const int sub = lane >> 4, wl = lane & 15;
        for (int y0 = 4 * wave; y0 < o.gy; y0 += 4 * (SETUP_THREADS / 64)) {
            const int y = y0 + sub;
            uint32_t bits = y < o.gy && wl < words ? rowmask[y * words + wl] : 0u;
            const int cnt = __popc(bits), incl = row_scan_incl(cnt);
            const int total = __shfl(incl, lane | 15, 64);
            if (y < o.gy) {
                int* out = o.rows + ((size_t)b * o.gy + y) * T;
                int pos = incl - cnt;
                for (; bits; bits &= bits - 1) out[pos++] = 32 * wl + __ffs((int)bits) - 1;
                if (wl == 0) o.row_n[(size_t)b * o.gy + y] = total;
            }
        }
        return;
    }
    for (int y = wave; y < o.gy; y += SETUP_THREADS / 64) {
        int* out = o.rows + ((size_t)b * o.gy + y) * T;
        int carry = 0;
        for (int w0 = 0; w0 < words; w0 += 64) {
            const int w = w0 + lane;
            uint32_t bits = w < words ? rowmask[y * words + w] : 0u;
            const int cnt = __popc(bits), incl = wave_scan_incl(cnt, lane);
            int pos = carry + incl - cnt;
            for (; bits; bits &= bits - 1) out[pos++] = 32 * w + __ffs((int)bits) - 1;
            carry += __shfl(incl, 63, 64);
        }
        if (lane == 0) o.row_n[(size_t)b * o.gy + y] = carry;
    }
}

// ---------------------------------------------------------------- per-pair math

// One triangle record held in registers. The three vector loads (16 + 16 + 8 floats)
// of a wave-uniform address become s_load_dwordx16/x16/x8 issued together, so a list
// entry costs one scalar-memory round trip instead of one per field.
typedef float f16v __attribute__((ext_vector_type(16)));
typedef float f8v __attribute__((ext_vector_type(8)));
static_assert(REC_HOT == 40 && REC >= REC_HOT, "load_rec reads 16 + 16 + 8 floats");
struct Rec {
    f16v a, b;
    f8v c;
    __device__ float f(int i) const { return i < 16 ? a[i] : (i < 32 ? b[i - 16] : c[i - 32]); }
    __device__ int i(int k) const { return __float_as_int(f(k)); }
};
__device__ inline Rec load_rec(const float* __restrict__ r) {
    const f16v* v = reinterpret_cast<const f16v*>(r);
    return Rec{v[0], v[1], *reinterpret_cast<const f8v*>(r + 32)};
}

// Triangle k's record by a 32-bit byte offset from its scene's records (a
// scene holds at most 2^23 triangles, so T x REC x 4 bytes < 2^32): the scalar
// loads take the offset as their SGPR offset, where a 64-bit index costs a
// multiply-high and a carry add per entry. Entries of a tile's region likewise.
__device__ inline uint32_t rec_off(uint32_t k) { return k * (uint32_t)(REC * sizeof(float)); }
__device__ inline const float* rec_at(const float* __restrict__ rec, uint32_t off) {
    return reinterpret_cast<const float*>(reinterpret_cast<const char*>(rec) + off);
}
__device__ inline TileEnt ent_at(const TileEnt* __restrict__ te, int i) {
    return *reinterpret_cast<const TileEnt*>(reinterpret_cast<const char*>(te) +
                                             (uint32_t)i * (uint32_t)sizeof(TileEnt));
}

// Field i0, i1 or i2 of the record for a per-lane e in {0, 1, 2}: the bits of
// f_e as f0 ^ ((f0 ^ f1) & m1) ^ ((f0 ^ f2) & m2), m1 and m2 the lane masks of
// e == 1 and e == 2 (its two bits, sign-extended). The two xors of scalar
// fields are scalar; per lane it is two ands and a three-way xor, where a
// select among scalar fields needs each field copied into a vector register
// first (a vector instruction reads one scalar register at most): -0.8 us of
// ~88 against the selects at B=16 256x256 T=128.
__device__ inline float pick3_lane(const Rec& r, int e, int i0, int i1, int i2) {
    const uint32_t b0 = __float_as_uint(r.f(i0));
    const uint32_t x1 = b0 ^ __float_as_uint(r.f(i1)), x2 = b0 ^ __float_as_uint(r.f(i2));
    const uint32_t m1 = (uint32_t)__builtin_amdgcn_sbfe(e, 0, 1), m2 = (uint32_t)__builtin_amdgcn_sbfe(e, 1, 1);
    return __uint_as_float(b0 ^ (x1 & m1) ^ (x2 & m2));
}

struct Pix {
    float px, py;
};

// raster.rs:79-87; both branches are formed and the sign picks one.
template <bool FAST>
__device__ inline float sigmoid_f(float x) {
    if (FAST) {
        float e = __expf(-fabsf(x));
        float s = __builtin_amdgcn_rcpf(1.0f + e);
        return x >= 0.0f ? s : e * s;
    } else {
        if (x >= 0.0f) return 1.0f / (1.0f + expf(-x));
        float e = expf(x);
        return e / (1.0f + e);
    }
}

// The exact-path geometry of one (pixel, triangle) pair: raster.rs:96-134 and
// grad.rs:235-247. The cross products, the inside test and the nearest-point
// arithmetic round exactly as the reference does (no FMA), because near an
// edge an error of 1e-7 in position is magnified by 1/sigma in the coverage.
// QUICK (a triangle of moderate coordinates in a fast-math build) forms the
// projection quotient from a refined reciprocal and takes the hardware square
// root; otherwise both are IEEE operations. The choice is made per triangle,
// outside this function, by a wave-uniform branch.
struct Geo {
    float sd;      // signed distance, positive inside
    float dist;    // |nearest segment distance|
    float t;       // clamped projection parameter on the nearest edge
    float ax, ay;  // first vertex of the nearest edge
    float ex, ey;  // its edge vector b - a
    int edge;      // nearest edge index, first minimum wins (grad.rs:236-242)
};

// The reference compares square-rooted distances (grad.rs:236-242): an earlier
// edge whose d2 is an ulp or two above the minimum can round to the same
// distance and then wins. That is routine for the overlapping edges of a
// collinear triangle. Kept out of line of the common path: the empty volatile
// asm stops the compiler from speculating the IEEE square roots into every
// evaluation.
__device__ inline bool same_sqrt(float a, float b) {
    asm volatile("");
    return sqrtf(a) == sqrtf(b);
}

template <bool QUICK>
__device__ inline Geo geometry(const Rec& r, Pix p) {
    float apx[3], apy[3];
    for (int j = 0; j < 3; j++) {
        apx[j] = p.px - r.f(R_V + 2 * j);
        apy[j] = p.py - r.f(R_V + 2 * j + 1);
    }
    float c[3];
    for (int j = 0; j < 3; j++) c[j] = r.f(R_E + 2 * j) * apy[j] - r.f(R_E + 2 * j + 1) * apx[j];
    bool inside = (c[0] >= 0.0f && c[1] >= 0.0f && c[2] >= 0.0f) ||
                  (c[0] <= 0.0f && c[1] <= 0.0f && c[2] <= 0.0f);
    Geo g;
    float best = INFINITY;
    float d2v[3], tv[3];
    g.edge = 0;
    g.t = 0.0f;
    for (int j = 0; j < 3; j++) {
        float ex = r.f(R_E + 2 * j), ey = r.f(R_E + 2 * j + 1);
        float dot = apx[j] * ex + apy[j] * ey;
        float t;
        if (QUICK) {
            // dot / len2 as the reference rounds it: with rlen2 the correctly
            // rounded 1/len2, one residual step q0 + (dot - q0*len2)*rlen2
            // gives the correctly rounded quotient (Markstein). The nearest
            // point then matches the reference bit for bit; an ulp off in t
            // moves the distance of an on-edge pixel by ~|e|*6e-8, which 1/sigma
            // magnifies into visible coverage error at small sigma.
            float rl = r.f(R_RLEN2 + j);
            float q0 = dot * rl;
            float res = fmaf(-q0, r.f(R_LEN2 + j), dot);
            t = __builtin_amdgcn_fmed3f(fmaf(res, rl, q0), 0.0f, 1.0f);
        } else {
            float len2 = r.f(R_LEN2 + j);
            t = (len2 <= 1e-20f) ? 0.0f : rust_clamp(dot / len2, 0.0f, 1.0f);
        }
        float dx = apx[j] - t * ex;
        float dy = apy[j] - t * ey;
        float d2 = dx * dx + dy * dy;
        d2v[j] = d2;
        tv[j] = t;
        if (d2 < best) {  // strict: the first minimum wins, NaN never does
            best = d2;
            g.edge = j;
            g.t = t;
        }
    }
    // Near ties are rare; the wave takes the square roots at every lane when
    // any lane has one (a wave-uniform branch, so no divergent control flow
    // for the compiler to thread path flags through), and the others keep
    // their edge. Edge 0 wins over edge 1, as the first minimum.
    const float near = best * 1.0000005f;
    const bool tie0 = g.edge > 0 && d2v[0] <= near, tie1 = g.edge > 1 && d2v[1] <= near;
    if (__builtin_amdgcn_ballot_w64(tie0 || tie1) != 0) {
        const bool eq0 = same_sqrt(d2v[0], best), eq1 = same_sqrt(d2v[1], best);
        const bool s0 = tie0 && eq0, s1 = !s0 && tie1 && eq1;
        g.t = s0 ? tv[0] : (s1 ? tv[1] : g.t);
        g.edge = s0 ? 0 : (s1 ? 1 : g.edge);
    }
    const int ed = g.edge;
    g.ax = pick3_lane(r, ed, R_V + 0, R_V + 2, R_V + 4);
    g.ay = pick3_lane(r, ed, R_V + 1, R_V + 3, R_V + 5);
    g.ex = pick3_lane(r, ed, R_E + 0, R_E + 2, R_E + 4);
    g.ey = pick3_lane(r, ed, R_E + 1, R_E + 3, R_E + 5);
    // sqrt is monotone, so sqrt(min d2) == min sqrt(d2) (raster.rs:97-99).
    g.dist = QUICK ? __builtin_amdgcn_sqrtf(best) : sqrtf(best);
    g.sd = inside ? g.dist : -g.dist;
    return g;
}

// Entry plans. Built per (tile, triangle) with the tile's list: PLAN_GENERAL,
// or edge j (0-2) when j is provably the nearest edge for every pixel of the
// tile and the other two edge lines stay clear of it, so the signs of their
// cross products are the same at every pixel (inner side when PLAN_INNER).
enum : uint32_t { PLAN_GENERAL = 3, PLAN_INNER = 4 };
// Entry bits 0-1: a single-edge plan (ENT_SINGLE: plan & 3 != PLAN_GENERAL),
// or whole coverage (ENT_FULL), one bit each so that a sweep tests either with
// one scalar bit test; neither: the general path. Bits 2-4: the plan. Bits
// 5-6: the byte offset, within the record's edge blocks, of the plan's block
// (32 min(plan & 3, 2)), so that a sweep addresses it with one bitwise and.
// Bit 7: the tile lies inside the triangle's box (no per-pixel box test).
enum : uint32_t { ENT_SINGLE = 0x1, ENT_FULL = 0x2, ENT_EB = 0x60, ENT_INBOX = 0x80 };

// geometry<true> for a single-edge plan: the reference's distance to edge j
// and its cross product, with the other edges' results known. The excluded
// edges are strictly farther (by a margin well above rounding) at every pixel,
// so the reference's first-minimum selection picks j with the same distance,
// and the inside test reduces to the sign of c_j.
// An entry's record (at byte offset `off`) and, for the fast-path sweeps, the
// record's block of the plan's edge (R_EB + 8 j, j = plan & 3; the general
// plan's 3 reads edge 2's block, unused; `code` is the entry's low byte, whose
// ENT_EB bits hold the block's byte offset), which the asm keeps where it is
// issued: its scalar round trip is the record's instead of a second one inside
// the exact path. WHOLE: the record's second half too, so that all of an
// entry's loads issue together and it costs one scalar round trip; left to
// itself the compiler sinks that load into the branch that first reads it, a
// second round trip (and a 64-bit address add) for most entries. The sweeps
// of the gradient kernels take WHOLE; forward_kernel's forward sweep does
// not (its fast-path entries do not read the second half; +3.6 us at B=16
// 128x128 T=128 with it). In bounds for every record: R_EB + 24 == REC.
static_assert(R_EB + 24 == REC, "three 8-float edge blocks end the record");
template <bool FAST, bool WHOLE>
__device__ inline void load_entry(const float* __restrict__ rec, uint32_t off, uint32_t code, Rec& r, f8v& eb) {
    r = load_rec(rec_at(rec, off));
    eb = f8v{};
    if (FAST) eb = *reinterpret_cast<const f8v*>(rec_at(rec, off + (code & ENT_EB)) + R_EB);
    if (FAST && WHOLE)
        asm volatile("" : "+s"(r.b), "+s"(eb));
    else if (FAST)
        asm volatile("" : "+s"(eb));
    else if (WHOLE)
        asm volatile("" : "+s"(r.b));
}

// The edge's fields come from its block of the record (load_entry).
__device__ inline Geo geometry1(const Rec& r, const f8v& eb, Pix p, uint32_t plan) {
    const int j = (int)(plan & 3u);
    const float ax = eb[0], ay = eb[1], ex = eb[2], ey = eb[3], len2 = eb[4], rl = eb[5];
    const float apx = p.px - ax, apy = p.py - ay;
    const float c = ex * apy - ey * apx;
    const float dot = apx * ex + apy * ey;
    const float q0 = dot * rl;
    const float res = fmaf(-q0, len2, dot);
    Geo g;
    g.t = __builtin_amdgcn_fmed3f(fmaf(res, rl, q0), 0.0f, 1.0f);
    const float dx = apx - g.t * ex;
    const float dy = apy - g.t * ey;
    g.dist = __builtin_amdgcn_sqrtf(dx * dx + dy * dy);
    // c <= 0 is -c >= 0, also for c = +-0
    const float cs = c * eb[6];  // the orientation flag as an exact factor of +-1
    const bool inside = (plan & PLAN_INNER) && cs >= 0.0f;
    g.sd = inside ? g.dist : -g.dist;
    g.edge = j;
    g.ax = ax;
    g.ay = ay;
    g.ex = ex;
    g.ey = ey;
    return g;
}

// Exact-path coverage of one pair. The branches on the triangle's F_FAST flag
// and on the plan are wave-uniform; the empty volatile asm keeps the compiler
// from if-converting them, which would evaluate every variant every time.
template <bool FAST>
__device__ inline void exact_cov(const Rec& r, const f8v& eb, Pix p, uint32_t code, float rsig, float sig, Geo& g,
                                 float& cov) {
    // single-edge plans are given to F_FAST triangles only (build_list)
    if (FAST && (code & ENT_SINGLE)) {
        g = geometry1(r, eb, p, (code >> 2) & 7u);
        cov = sigmoid_f<true>(g.sd * rsig);
    } else if (FAST && (r.i(R_FLAGS) & F_FAST)) {
        asm volatile("");
        g = geometry<true>(r, p);
        cov = sigmoid_f<true>(g.sd * rsig);
    } else {
        asm volatile("");
        g = geometry<false>(r, p);
        cov = sigmoid_f<FAST>(FAST ? g.sd * rsig : g.sd / sig);
    }
}

// The exact coverage at the lanes of `bandm` (`band`: this lane's bit), 1.0f
// at the others. Every lane evaluates it, under a wave-uniform branch on
// `bandm`, and the others discard theirs: a divergent branch would cost the
// same vector issue (masked lanes issue alike) plus the exec-mask saves and
// restores, and makes the compiler carry flags through the branches around it.
template <bool FAST>
__device__ inline void band_cov(const Rec& r, const f8v& eb, Pix p, uint32_t code, uint64_t bandm, bool band,
                                float rsig, float sig, Geo& g, float& cov) {
    cov = 1.0f;
    if (bandm != 0) {
        float c;
        exact_cov<FAST>(r, eb, p, code, rsig, sig, g, c);
        cov = band ? c : 1.0f;
    }
}

// ---------------------------------------------------------------- wave reductions

// DPP controls (gfx9 encoding) used below; every source lane is inside the quad.
constexpr int DPP_XOR1 = 0xB1;  // quad_perm [1,0,3,2]
constexpr int DPP_XOR2 = 0x4E;  // quad_perm [2,3,0,1]

template <int ctrl>
__device__ inline float dpp(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), ctrl, 0xF, 0xF, false));
}

// The wave's lanes for which `c` holds (inactive lanes 0). HIP's __ballot widens
// the condition to an integer and compares it again, two vector instructions
// more per call than the builtin, which takes the compare's lane mask as is.
__device__ inline uint64_t lane_mask(bool c) { return __builtin_amdgcn_ballot_w64(c); }

// Wave-uniform copies of values every lane holds (loaded from one address).
// The builtin returns int: widen through uint32_t, never by sign extension.
__device__ inline uint32_t uniform_u32(uint32_t v) { return (uint32_t)__builtin_amdgcn_readfirstlane((int)v); }
__device__ inline uint64_t uniform_u64(uint64_t v) {
    return ((uint64_t)uniform_u32((uint32_t)(v >> 32)) << 32) | (uint64_t)uniform_u32((uint32_t)v);
}

// A pointer into LDS: 32-bit addresses (a generic pointer is 64-bit).
typedef __attribute__((address_space(3))) float lds_float;

__device__ inline void lds_add(lds_float* p, float v) {
    __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WAVEFRONT);
}

// Sum over the wave (every lane active) by the butterfly v += v[lane ^ off]
// for off = 32, 16, ..., 1, so every lane ends with the same, fixed-order sum.
// The exchanges within 32 lanes are ds_swizzle (xor 16, 8, 4) and DPP quad
// permutes (xor 2, 1) on the two halves of the double, which skip the
// address computation and LDS round trip of a bpermute; xor 32 stays a
// bpermute.
template <int pattern>
__device__ inline double swizzle_f64(double v) {
    const int lo = __builtin_amdgcn_ds_swizzle((int)(uint32_t)__double_as_longlong(v), pattern);
    const int hi = __builtin_amdgcn_ds_swizzle((int)(uint32_t)(__double_as_longlong(v) >> 32), pattern);
    return __longlong_as_double((long long)(((uint64_t)(uint32_t)hi << 32) | (uint32_t)lo));
}
template <int ctrl>
__device__ inline double dpp_f64(double v) {
    const int lo = __builtin_amdgcn_update_dpp(0, (int)(uint32_t)__double_as_longlong(v), ctrl, 0xF, 0xF, false);
    const int hi = __builtin_amdgcn_update_dpp(0, (int)(uint32_t)(__double_as_longlong(v) >> 32), ctrl, 0xF, 0xF, false);
    return __longlong_as_double((long long)(((uint64_t)(uint32_t)hi << 32) | (uint32_t)lo));
}
__device__ inline double wave_sum_f64(double v) {
    v += __shfl_xor(v, 32, 64);
    v += swizzle_f64<(16 << 10) | 0x1F>(v);  // bit mode: and 0x1F, or 0, xor 16
    v += swizzle_f64<(8 << 10) | 0x1F>(v);
    v += swizzle_f64<(4 << 10) | 0x1F>(v);
    v += dpp_f64<DPP_XOR2>(v);
    v += dpp_f64<DPP_XOR1>(v);
    return v;
}

// ---------------------------------------------------------------- forward and backward kernels

enum : uint32_t { CLS_PARTIAL = 1, CLS_FULL = 2 };

// Builds this wave's ordered list of the triangles in [k0, k1) with flag
// `live` (F_LIVE, or F_TAPE for a backward pass) that can touch its tile. Entry: (k_local << 8) | (plan << 2) | class, with class FULL when every
// tile pixel is inside the triangle's box and deep inside the triangle, else
// PARTIAL, and the plan of the exact path (PLAN_* or a single edge).
//
// Plans use bounds over the tile's pixel-centre rectangle: with l the outward
// edge-line distance and s the along-edge coordinate (both affine, so extreme
// at the corners), the distance to segment j is sqrt(l^2 + ex^2) with
// ex = max(0, -s, s - |e|). An edge whose lower bound exceeds the smallest
// upper bound by more than the margin is never nearest.
//
// Two passes: the box test over the chunk compacts the candidates (in order)
// into `list`, then the classification runs over the candidates only, 64 at a
// time, and compacts the entries over them in place. Every branch of the
// classification is taken by some lane of almost any 64 triangles, so the
// wave's cost is per pass of 64, and the candidates are usually one pass.
// The box tests load two passes of 64 triangles at a time (one round trip
// for both).
//
// MERGE (merged chunks): the box tests run on past the first CH triangles
// until the candidates exceed 64 (so at most 128 = CH, the list's size) or
// [k0, k1) ends, and *kend is where they stopped: the sparse candidates of
// many chunks (small triangles) then share one classification pass and one
// entry loop. Entries then hold their triangles' indices (below 2^23, so
// k << 8 fits the entry word) rather than offsets from k0, so only a caller
// that takes every triangle index from the entries (not from a per-chunk
// accumulator row) may merge. The
// classification then also loads every field any of its branches reads up
// front (one round trip instead of one per branch level; the other callers
// keep the lazy loads, whose registers their occupancy needs).
//
// With `ilist` (merged lists only) [k0, k1) are positions in ilist, a list of
// triangle indices in order.
template <bool MERGE = false>
__device__ inline int build_list(const float* __restrict__ rec, int k0, int k1, int tx0, int ty0,
                                 int tx1, int ty1, float cx0, float cy0, float cx1, float cy1,
                                 uint32_t* list, int lane, int live, int* kend = nullptr,
                                 const int* __restrict__ ilist = nullptr) {
    static_assert(CH >= 128, "a merged list holds two passes of candidates");
    static_assert(R_FLAGS == R_BOX + 4, "the box tests read x0 y0 x1 y1 flags as five consecutive ints");
    const int kbase = MERGE ? 0 : k0;
    int nc = 0;
    if (MERGE) *kend = k1;
    for (int base2 = k0; base2 < k1; base2 += 128) {
        int bf[2][5];  // x0 y0 x1 y1 flags of the triangle k of each pass
        int kk[2];     // its index
        for (int h = 0; h < 2; h++) {
            // Lanes past the chunk read its last record (in bounds) and are
            // masked out.
            const int pos = min(base2 + 64 * h + lane, k1 - 1);
            kk[h] = ilist ? ilist[pos] : pos;
            const int* ri = reinterpret_cast<const int*>(rec + (size_t)kk[h] * REC);
            for (int f = 0; f < 5; f++) bf[h][f] = ri[R_BOX + f];
        }
        for (int h = 0; h < 2; h++) {
        const int base = base2 + 64 * h, k = base + lane;
        if (base >= k1) break;
        const int bx0 = bf[h][0], by0 = bf[h][1], bx1 = bf[h][2], by1 = bf[h][3], flags = bf[h][4];
        // the tests are single-compare lane masks, ANDed as scalars
        const uint64_t mask = lane_mask(k < k1) & lane_mask((flags & live) != 0) & lane_mask(tx0 < bx1) &
                              lane_mask(bx0 < tx1) & lane_mask(ty0 < by1) & lane_mask(by0 < ty1);
        const bool cand = __builtin_amdgcn_inverse_ballot_w64(mask);
        const bool in_box = __builtin_amdgcn_inverse_ballot_w64(lane_mask(bx0 <= tx0) & lane_mask(tx1 <= bx1) &
                                                                lane_mask(by0 <= ty0) & lane_mask(ty1 <= by1));
        if (cand) {
            const int pos = nc + (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(mask >> 32),
                                                                 __builtin_amdgcn_mbcnt_lo((uint32_t)mask, 0));
            list[pos] = ((uint32_t)(kk[h] - kbase) << 1) | (in_box ? 1u : 0u);
        }
        nc += (int)__popcll(mask);
        if (MERGE && nc > 64) {
            *kend = min(base + 64, k1);
            goto classify;
        }
        }
    }
classify:
    // Entry i is written at count + rank <= i, a slot this or an earlier pass
    // has read: the wave's LDS accesses complete in program order.
    int count = 0;
    for (int c0 = 0; c0 < nc; c0 += 64) {
        uint32_t cls = 0, plan = PLAN_GENERAL, extra = 0;
        uint32_t kl = 0;
        if (c0 + lane < nc) {
            const uint32_t cd = list[c0 + lane];
            kl = cd >> 1;
            const float* r = rec_at(rec, rec_off((uint32_t)kbase + kl));
            const int flags = reinterpret_cast<const int*>(r)[R_FLAGS];
            // With MERGE the classification's fields, [R_N, R_EB), are loaded
            // together: the empty asm uses them all here, so that the compiler
            // does not sink each load into the branch that reads it.
            static_assert(R_OFF == R_N + 6 && R_FAR == R_N + 9 && R_DEEP == R_N + 10 && R_SLACK == R_N + 11 &&
                              R_D == R_N + 12 && R_SOFF == R_D + 6 && R_LEN == R_D + 9 && R_EB == R_D + 12,
                          "classification fields: 24 consecutive floats");
            float cf[24];
            if (MERGE) {
                for (int q = 0; q < 24; q++) cf[q] = r[R_N + q];
                asm volatile("" ::"v"(cf[0]), "v"(cf[1]), "v"(cf[2]), "v"(cf[3]), "v"(cf[4]), "v"(cf[5]),
                             "v"(cf[6]), "v"(cf[7]), "v"(cf[8]), "v"(cf[9]), "v"(cf[10]), "v"(cf[11]), "v"(flags));
                asm volatile("" ::"v"(cf[12]), "v"(cf[13]), "v"(cf[14]), "v"(cf[15]), "v"(cf[16]), "v"(cf[17]),
                             "v"(cf[18]), "v"(cf[19]), "v"(cf[20]), "v"(cf[21]), "v"(cf[22]), "v"(cf[23]));
            }
            auto fld = [&](int i) { return MERGE ? cf[i - R_N] : r[i]; };
            {
                cls = CLS_PARTIAL;
                const bool in_box = cd & 1u;
                if (in_box) extra |= ENT_INBOX;
                if (flags & F_FAST) {
                    float far = fld(R_FAR), deep = fld(R_DEEP);
                    float lmin[3], lmax[3];
                    bool culled = false, all_deep = true;
                    for (int j = 0; j < 3; j++) {
                        float nx = fld(R_N + 2 * j), ny = fld(R_N + 2 * j + 1), o = fld(R_OFF + j);
                        float l00 = fmaf(cx0, nx, fmaf(cy0, ny, -o));
                        float l10 = fmaf(cx1, nx, fmaf(cy0, ny, -o));
                        float l01 = fmaf(cx0, nx, fmaf(cy1, ny, -o));
                        float l11 = fmaf(cx1, nx, fmaf(cy1, ny, -o));
                        lmin[j] = fminf(fminf(l00, l10), fminf(l01, l11));
                        lmax[j] = fmaxf(fmaxf(l00, l10), fmaxf(l01, l11));
                        culled = culled || (lmin[j] > far);
                        all_deep = all_deep && (lmax[j] < deep);
                    }
                    if (culled) {
                        cls = 0;
                    } else if (all_deep && in_box) {
                        cls = CLS_FULL;
                    } else {
                        const float slack = fld(R_SLACK);
                        float lb[3], ubmin = INFINITY;
                        for (int j = 0; j < 3; j++) {
                            float dx = fld(R_D + 2 * j), dy = fld(R_D + 2 * j + 1), so = fld(R_SOFF + j);
                            float len = fld(R_LEN + j);
                            float s00 = fmaf(cx0, dx, fmaf(cy0, dy, -so));
                            float s10 = fmaf(cx1, dx, fmaf(cy0, dy, -so));
                            float s01 = fmaf(cx0, dx, fmaf(cy1, dy, -so));
                            float s11 = fmaf(cx1, dx, fmaf(cy1, dy, -so));
                            float smin = fminf(fminf(s00, s10), fminf(s01, s11));
                            float smax = fmaxf(fmaxf(s00, s10), fmaxf(s01, s11));
                            float exmin = fmaxf(fmaxf(-smax, smin - len), 0.0f);
                            float exmax = fmaxf(fmaxf(-smin, smax - len), 0.0f);
                            float la = (lmin[j] <= 0.0f && lmax[j] >= 0.0f)
                                           ? 0.0f
                                           : fminf(fabsf(lmin[j]), fabsf(lmax[j]));
                            float lz = fmaxf(fabsf(lmin[j]), fabsf(lmax[j]));
                            lb[j] = sqrtf(la * la + exmin * exmin);
                            ubmin = fminf(ubmin, sqrtf(lz * lz + exmax * exmax));
                        }
                        // The reference's rounded distances are within ~1e-7 (1 + max |v|)
                        // of these bounds' exact values; 0.1 slack is ten times that.
                        const float lim = ubmin + 0.1f * slack;
                        // An edge farther than `sat` from every pixel is nearest only
                        // where the pair saturates (coverage exactly 1 inside, w below
                        // MIN_WEIGHT outside: deep and far include the slack), and there
                        // the plan's edge, no nearer, saturates alike. It is no candidate
                        // unless it is the closest.
                        const float sat = fmaxf(far, -deep);
                        const float lbmin = fminf(fminf(lb[0], lb[1]), lb[2]);
                        int ncand = 0, jc = 0;
                        for (int j = 0; j < 3; j++)
                            if (!(lb[j] > lim) && (lb[j] <= sat || lb[j] == lbmin)) {
                                ncand++;
                                jc = j;
                            }
                        if (ncand == 1) {
                            bool clear = true, inner = true;
                            for (int j = 0; j < 3; j++) {
                                if (j == jc) continue;
                                clear = clear && (lmin[j] > slack || lmax[j] < -slack);
                                inner = inner && (lmax[j] < -slack);
                            }
                            if (clear) plan = (uint32_t)jc | (inner ? PLAN_INNER : 0u);
                        }
                    }
                }
            }
        }
        const uint64_t mask = lane_mask(cls != 0);
        if (cls != 0) {
            const int pos = count + (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(mask >> 32),
                                                                    __builtin_amdgcn_mbcnt_lo((uint32_t)mask, 0));
            const uint32_t kind = cls == CLS_FULL ? ENT_FULL : ((plan & 3u) != PLAN_GENERAL ? ENT_SINGLE : 0u);
            list[pos] = (kl << 8) | extra | (min(plan & 3u, 2u) << 5) | (plan << 2) | kind;
        }
        count += (int)__popcll(mask);
    }
    return count;
}

// Per-pixel weight of one triangle: returns the mask of the lanes where the
// pair contributes (not outside the box, not classified far outside, and
// w > MIN_WEIGHT). `bandm` holds the lanes where the exact path ran with a
// coverage below 1.0f, and there `g` holds its geometry. The tests are
// predicates rather than branches; only the exact path is a (divergent)
// branch, so the wave runs it once for the lanes that need it.
template <bool FAST>
__device__ inline uint64_t pair_weight(const Rec& r, const f8v& eb, uint32_t ent, int x, int y,
                                       Pix p, uint64_t validm, float& w, float& cov, uint64_t& bandm, Geo& g,
                                       float rsig, float sig) {
    const float alpha = r.f(R_A);
    cov = 1.0f;
    // The lane sets are wave masks (`validm`: the lanes whose pixel is in the
    // image), each test one compare's mask ANDed in: kept as scalar mask
    // operations instead of per-lane 0/1 values, which the compiler widens a
    // combined condition into before taking its mask.
    uint64_t actm = validm;
    if (ent & ENT_FULL) {
        bandm = 0;
        w = alpha;
        return actm & lane_mask(!(w <= MIN_WEIGHT));
    }
    if (!(ent & ENT_INBOX))
        actm &= lane_mask((unsigned)(x - r.i(R_BOX)) < (unsigned)(r.i(R_BOX + 2) - r.i(R_BOX))) &
                lane_mask((unsigned)(y - r.i(R_BOX + 1)) < (unsigned)(r.i(R_BOX + 3) - r.i(R_BOX + 1)));
    // build_list gives a single-edge plan to fast-path triangles (F_FAST) only
    if (FAST && (ent & ENT_SINGLE)) {
        // A single-edge plan holds for every pixel of the tile, so every lane
        // evaluates its edge: no classification and no divergent branch. A deep
        // pixel (more than 17 sigma + slack inside every edge line) gets
        // exp(-x) < 2^-24 and coverage exactly 1.0f, as classified; a far one
        // (beyond `far`) a weight below MIN_WEIGHT, skipped as classified.
        g = geometry1(r, eb, p, (ent >> 2) & 7u);
        cov = sigmoid_f<true>(g.sd * rsig);
        w = alpha * cov;
        bandm = actm & lane_mask(cov != 1.0f);
        return actm & lane_mask(!(w <= MIN_WEIGHT));
    }
    bandm = actm;
    if (FAST && (r.i(R_FLAGS) & F_FAST)) {
        // The three-edge path at every lane, for the same reasons as a single
        // edge: a pixel that the edge-line distances would class deep gets
        // coverage exactly 1.0f, a far one a weight below MIN_WEIGHT.
        asm volatile("");
        g = geometry<true>(r, p);
        cov = sigmoid_f<true>(g.sd * rsig);
    } else {
        band_cov<FAST>(r, eb, p, ent, bandm, __builtin_amdgcn_inverse_ballot_w64(bandm), rsig, sig, g, cov);
    }
    w = alpha * cov;
    // `bandm` hands the backward pass the lanes whose coverage it must evaluate:
    // where the exact coverage is 1.0f it takes 1.0f without evaluating, and
    // the vertex terms, proportional to cov (1 - cov), are zero.
    bandm &= lane_mask(cov != 1.0f);
    return actm & lane_mask(!(w <= MIN_WEIGHT));
}

struct Trans {
    float q;  // product of the nonzero (1 - w) factors, kept in [2^-64, 1]
    int z;    // number of zero factors (w == 1 exactly)
    int e;    // number of 2^64 rescalings applied to q
};

__device__ inline void trans_rescale(Trans& t) {
    const bool small = t.q < 5.421010862427522e-20f;  // 2^-64
    t.q = small ? t.q * 1.8446744073709552e19f : t.q;  // 2^64
    t.e += small ? 1 : 0;
}

__device__ inline void trans_mul(Trans& t, float f) {
    const bool zero = f == 0.0f;
    t.q = zero ? t.q : t.q * f;
    t.z += zero ? 1 : 0;
    trans_rescale(t);
}

// prod_{j>k} (1 - w_j) from the totals and the prefix through k.
__device__ inline float trans_suffix(const Trans& total, const Trans& prefix) {
    float ratio = ldexpf(total.q * __builtin_amdgcn_rcpf(prefix.q), -64 * (total.e - prefix.e));
    return total.z != prefix.z ? 0.0f : ratio;
}

// Index of channel ch of this lane's pixel in an image array: B x H x W x 3, or
// B x 3 x H x W when a.chw.
__device__ inline size_t img_index(const RasterArgs& a, size_t pix, int b, int ch) {
    const size_t hw = (size_t)a.H * a.W;
    return a.chw ? ((size_t)b * 3 + ch) * hw + (pix - (size_t)b * hw) : pix * 3 + ch;
}

// Tile geometry shared by both kernels: one wave per 8x8 tile, four tiles
// (2x2) per block, one pixel per lane. `rank`: the block's place in the block
// order (-1 without one); `seg` of `nseg`: the backward segment.
struct TileGeo {
    int lane, wave, b, rank, seg, nseg, bx, by, x, y, tx0, ty0, tx1, ty1;
    bool valid, live;
    Pix p;
    float cx0, cy0, cx1, cy1;
    size_t pix, tile;
};

// The tile of this wave in block (bx, by) of scene b, gx x gy blocks per scene.
// wave: the tile of the block (-1: this wave's place in a block of WAVES waves).
__device__ inline TileGeo tile_at(int W, int H, int gx, int gy, int b, int bx, int by, int rank, int seg,
                                  int nseg, int wave = -1) {
    TileGeo t;
    t.lane = threadIdx.x & 63;
    // uniform: scalar tile indices
    t.wave = wave >= 0 ? wave : __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    t.b = b;
    t.rank = rank;
    t.seg = seg;
    t.nseg = nseg;
    t.bx = bx;
    t.by = by;
    t.tx0 = (t.bx * 2 + (t.wave & 1)) * TILE;
    t.ty0 = (t.by * 2 + (t.wave >> 1)) * TILE;
    t.x = t.tx0 + (t.lane & 7);
    t.y = t.ty0 + (t.lane >> 3);
    t.valid = t.x < W && t.y < H;
    t.tx1 = min(t.tx0 + TILE, W);
    t.ty1 = min(t.ty0 + TILE, H);
    t.live = t.tx0 < W && t.ty0 < H;
    // raster.rs:138-140 pixel centre, correctly rounded division.
    t.p.px = ((float)t.x + 0.5f) / (float)W;
    t.p.py = ((float)t.y + 0.5f) / (float)H;
    // Corners of the tile's pixel-centre rectangle, for the list classification:
    // the centres of the lanes at pixels (tx0, ty0) and (tx1 - 1, ty1 - 1), read
    // across the wave (every lane is active here) instead of divided again. A
    // tile that is not live reads in-range lanes and never uses them. The
    // moves keep the corners in VGPRs: as scalar operands the classification's
    // FMAs with them would issue at the slower rate.
    const int lx = min(max(t.tx1 - 1 - t.tx0, 0), TILE - 1), ly = min(max(t.ty1 - 1 - t.ty0, 0), TILE - 1);
    auto lane_value = [](float v, int l) {
        const int s = __builtin_amdgcn_readlane(__float_as_int(v), l);
        int r;
        asm("v_mov_b32 %0, %1" : "=v"(r) : "s"(s));
        return __int_as_float(r);
    };
    t.cx0 = lane_value(t.p.px, 0);
    t.cy0 = lane_value(t.p.py, 0);
    t.cx1 = lane_value(t.p.px, lx);
    t.cy1 = lane_value(t.p.py, ly * TILE);
    t.pix = ((size_t)t.b * H + (t.valid ? t.y : 0)) * W + (t.valid ? t.x : 0);
    t.tile = (((size_t)t.b * gy + t.by) * gx + t.bx) * WAVES + t.wave;
    return t;
}

// Grid (gx, gy, B). With `perm` (setup_records' block order of B scenes)
// launch slot i (the linear block index) works on block perm[s * nb + i / B]
// of scene s = i % B.
__device__ inline TileGeo tile_geo(int W, int H, const int* perm = nullptr, int B = 1) {
    const int gx = (int)gridDim.x, gy = (int)gridDim.y;
    int b = (int)blockIdx.z, bx = (int)blockIdx.x, by = (int)blockIdx.y, rank = -1;
    if (perm) {
        const int nb = gx * gy;
        const int i = (blockIdx.z * gridDim.y + blockIdx.y) * gridDim.x + blockIdx.x;
        b = i % B;
        rank = i / B;
        const int local = min(max(perm[(size_t)b * nb + rank], 0), nb - 1);
        bx = local % gx;
        by = local / gx;
    }
    return tile_at(W, H, gx, gy, b, bx, by, rank, 0, 1);
}

// One wave per workgroup, B nb WAVES slots in one dimension: slot i is tile
// i % WAVES of the block at rank i / (WAVES B) of scene (i / WAVES) % B, so the
// four tiles of each block by setup_records' block order (perm, heaviest
// first) run in consecutive slots; without perm, block order.
// With perm_tiles, perm orders the scene's 2gx x 2gy tiles: slot i is tile
// rank i / B of scene i % B.
__device__ inline TileGeo tile_geo_wave(int W, int H, int gx, int gy, const int* perm, int B, bool perm_tiles,
                                        uint32_t tdiv_m = 0) {
    const int nb = gx * gy, i = (int)blockIdx.x;
    if (perm && perm_tiles) {
        // A two-dimensional grid (the one-wave fused kernel) has the scene in x
        // and the rank in y, the same dispatch order as slot i = rank B + b.
        const bool xy = gridDim.y > 1;
        const int nt = nb * WAVES, b = xy ? (int)blockIdx.x : i % B, rank = xy ? (int)blockIdx.y : i / B;
        const int t = min(max(perm[(size_t)b * nt + rank], 0), nt - 1);
        // t / (2 gx) by tdiv_m: exact while t 2 gx < 2^32 (the order's cells fit in LDS)
        const int ty = tdiv_m ? (int)__umulhi((uint32_t)t, tdiv_m) : t / (2 * gx), tx = t - ty * (2 * gx);
        return tile_at(W, H, gx, gy, b, tx >> 1, ty >> 1, rank, 0, 1, (ty & 1) * 2 + (tx & 1));
    }
    const int wave = i % WAVES;
    int b, rank, local;
    if (perm) {
        b = (i / WAVES) % B;
        rank = i / (WAVES * B);
        local = min(max(perm[(size_t)b * nb + rank], 0), nb - 1);
    } else {
        b = i / (WAVES * nb);
        rank = -1;
        local = (i / WAVES) % nb;
    }
    return tile_at(W, H, gx, gy, b, local % gx, local / gx, rank, 0, 1, wave);
}

// The split backward's grid: B (nb + K (S - 1)) slots in one dimension. The
// first B K S slots are the S segments of each scene's K heaviest blocks (by
// setup_records' order), heaviest first, the rest one slot per remaining
// block: slot i < B K S is segment (i / B) % S of rank i / (B S), later slots
// segment 0 of rank K + (i - B K S) / B, of scene i % B.
__device__ inline TileGeo tile_geo_split(int W, int H, int gx, int gy, const int* perm, int B, int S, int K) {
    const int nb = gx * gy, i = (int)blockIdx.x, b = i % B;
    int rank, seg = 0;
    if (i < B * K * S) {
        rank = i / (B * S);
        seg = (i / B) % S;
    } else {
        rank = K + (i - B * K * S) / B;
    }
    const int local = min(max(perm[(size_t)b * nb + min(rank, nb - 1)], 0), nb - 1);
    return tile_at(W, H, gx, gy, b, local % gx, local / gx, rank, seg, rank < K ? S : 1);
}

// Forward: composite in scene order (raster.rs:37-68). In the gradient modes it
// also keeps each pixel's total transmittance and records, per tile, the
// entries that contribute at any of its pixels with their lane masks (on,
// and exact-path), so the backward kernel neither rebuilds nor reclassifies.
// MODE_LOSS adds the loss (canvas.rs:45-58) and dL/dpixel (grad.rs:111-114).
// The waves-per-SIMD floors (8 here, 6 for the backward kernel) cap the
// register allocation; both kernels wait on scalar loads of the triangle
// records once per list entry, and the extra waves hide that latency better
// than the registers they cost would have saved (measured on B=16 256x256).
// CKPT: with the split backward's checkpoints (MODE_LOSS, MODE_GRAD_IN).
// The forward sweep of one tile (raster.rs:37-68): composites its pixels over
// every chunk of triangles into col (which comes in as the background) and, in
// the gradient modes, multiplies the taped transmittance into tot (which comes
// in as an empty product) and records the tile's contributing entries: n2 of
// them seen, those of the first rec_chunks chunks all recorded. With CKPT, the
// split backward's checkpoints too. lw: the wave's LDS list. MERGE: lists of
// merged chunks (build_list), for a caller that takes every triangle index from
// the recorded entries; rec_chunks is then meaningless.
// [kbeg, kend) (merged lists without ROWS only; default all of them): the
// triangles swept, and ent_off: where in the tile's region the entries go (a
// segment of fused_seg_kernel).
template <int MODE, bool FAST, bool CKPT, bool MERGE = false, bool ROWS = false>
__device__ __forceinline__ void forward_sweep(const RasterArgs& a, const float* __restrict__ rec, const TileGeo& tg,
                                              uint64_t validm, float rsig, float sig, uint32_t* lw,
                                              float (&col)[3], Trans& tot, int& n2, int& rec_chunks,
                                              int kbeg = 0, int kend = -1, int ent_off = 0) {
    const int T = a.T, lane = tg.lane;
    const int n_chunks = (T + CH - 1) / CH;
    n2 = 0;                 // contributing entries seen (recorded while n2 < cap2)
    rec_chunks = n_chunks;  // chunks whose contributing entries are all recorded
    const int cap2 = a.cap2;
    // wave-uniform: the entry stores address from a scalar base
    TileEnt* te = a.tl_ent + (size_t)uniform_u32((uint32_t)tg.tile) * cap2 + ent_off;
    const TileEnt* const te0 = te;
    // Split backward: before recorded entry (c + 1) seg_m the pixel state goes to
    // checkpoint c of this tile, the start of the backward's segment c + 1 (of
    // the blocks the backward splits: those ranked below nsplit, or all
    // without a block order here).
    const bool split = CKPT && (tg.rank < 0 || tg.rank < a.nsplit);
    const int nck = split ? max(a.nseg, 1) - 1 : 0;
    int ck = 0, ck_at = nck > 0 ? a.seg_m : INT_MAX;
    float* ckw = nck > 0 ? a.ckpt + (size_t)uniform_u32((uint32_t)tg.tile) * nck * (CKPT_WORDS * 64) : nullptr;

    static_assert(!(MERGE && CKPT), "checkpoints count entries per chunk");
    static_assert(MERGE || !ROWS, "row lists are merged lists");
    // ROWS: merged lists over the tile row's triangles, which setup_records listed
    const int* ilist = nullptr;
    int nlist = kend < 0 ? T : kend;
    if (ROWS) {
        const size_t row = (size_t)tg.b * a.row_gy + (tg.ty0 >> 3);
        ilist = a.rows + row * T;
        nlist = a.row_n[row];
    }
    int k1 = MERGE ? kbeg : 0;
    for (int c = 0; MERGE ? k1 < nlist : c < n_chunks; c++) {
        const int k0 = MERGE ? k1 : c * CH;
        k1 = MERGE ? nlist : min(T, k0 + CH);
        int count = tg.live ? build_list<MERGE>(rec, k0, k1, tg.tx0, tg.ty0, tg.tx1, tg.ty1, tg.cx0, tg.cy0,
                                                tg.cx1, tg.cy1, lw, lane, F_LIVE, &k1, ilist)
                            : 0;
        const int kbase = MERGE ? 0 : k0;
        // the list one half (64 entries) at a time, one entry per lane: each
        // iteration takes its entry from its lane (v_readlane) instead of an LDS
        // read, its address arithmetic and its wait
        for (int h = 0; h < count; h += 64) {
            const uint32_t held = lw[min(h + lane, CH - 1)];
            const int nh = (int)uniform_u32((uint32_t)min(count - h, 64));
            for (int i = 0; i < nh; i++) {
                const uint32_t ent = (uint32_t)__builtin_amdgcn_readlane((int)held, i);
                const int k = kbase + (int)(ent >> 8);
                Rec r;
                f8v eb;
                load_entry<FAST, MERGE>(rec, rec_off((uint32_t)k), ent, r, eb);
                float w = 0.0f, cov;
                uint64_t bandm;
                Geo g;
                const uint64_t onm =
                    pair_weight<FAST>(r, eb, ent, tg.x, tg.y, tg.p, validm, w, cov, bandm, g, rsig, sig);
                const bool on = __builtin_amdgcn_inverse_ballot_w64(onm);
                // MODE_RECORD draws what a render draws but hands over what the
                // taped forward keeps (F_TAPE); in the other modes the two agree.
                const uint64_t tapedm = (MODE != MODE_RECORD || (r.i(R_FLAGS) & F_TAPE)) ? onm : 0;
                const bool taped = __builtin_amdgcn_inverse_ballot_w64(tapedm);
                if (CKPT && tapedm != 0 && n2 == ck_at) {
                    // the colour and transmittance with which the backward sweep reaches this entry
                    float* c = ckw + (size_t)ck * (CKPT_WORDS * 64) + lane;
                    c[0] = col[0];
                    c[64] = col[1];
                    c[128] = col[2];
                    c[192] = tot.q;
                    c[256] = __int_as_float(tot.z);
                    c[320] = __int_as_float(tot.e);
                    ck++;
                    ck_at = ck < nck ? ck_at + a.seg_m : INT_MAX;
                }
                {
                    // raster.rs:60-66, kept only where the pair contributes, as
                    // col + w (c - col): one rounding fewer than c w + col (1 - w),
                    // and the form the backward kernel rebuilds the colour with
                    const float omw = 1.0f - w;
                    for (int ch = 0; ch < 3; ch++) {
                        const float o = fmaf(w, r.f(R_C + ch) - col[ch], col[ch]);
                        col[ch] = on ? o : col[ch];
                    }
                    if (MODE != MODE_RENDER) {
                        // trans_mul, by a plain product while it needs neither a zero
                        // count nor a rescaling: a factor (in [0, 1], raster.rs:48)
                        // that is zero, or a product below 2^-64 (or NaN), fails the
                        // test, and only then does the wave take the counting step.
                        const float f = taped ? omw : 1.0f;
                        const float qn = tot.q * f;
                        if (lane_mask(!(qn >= 5.421010862427522e-20f)) == 0)
                            tot.q = qn;
                        else
                            trans_mul(tot, f);
                    }
                }
                if (MODE != MODE_RENDER) {
                    if (tapedm != 0) {
                        // With merged lists (fused_tile_kernel) the region holds every
                        // entry (cap2 >= T: the fused path's condition), and every lane
                        // stores the same (wave-uniform) entry: no lane mask to set up
                        if (MERGE || (n2 < cap2 && lane == 0)) {
                            TileEnt e;
                            e.k = MERGE ? ent : ent + ((uint32_t)kbase << 8);  // (k << 8) | the entry's low byte
                            // the merged lists' consumer reads no row
                            e.row = MERGE ? 0u : (ent >> 8) * (uint32_t)(NP * sizeof(float));
                            e.on = tapedm;
                            e.band = tapedm & bandm;
                            *te = e;
                        }
                        // entry n2 + 1, stored only while n2 < cap2: a running pointer
                        // instead of an index's 64-bit multiply-add. With the constant row
                        // -1.4 us of ~88 at B=16 256x256 T=128, with the rest -1.3 more
                        te++;
                        if (!MERGE) n2++;  // merged lists: from the pointer at the end
                    }
                }
            }
        }
        if (!MERGE && n2 > cap2 && rec_chunks == n_chunks) rec_chunks = c;
    }
    if (MERGE) n2 = (int)(te - te0);
}

template <int MODE, bool FAST, bool CKPT>
__global__ __launch_bounds__(WAVES * 64) __attribute__((amdgpu_waves_per_eu(8))) void forward_kernel(RasterArgs a, const float* __restrict__ records) {
    __shared__ uint32_t list[WAVES][CH];
    __shared__ double loss[WAVES];
    if (a.halt && *a.halt >= 0) return;
    const int W = a.W, H = a.H, T = a.T;
    const TileGeo tg = tile_geo(W, H, a.perm_fwd, a.B);
    const uint64_t validm = lane_mask(tg.valid);  // lanes whose pixel is in the image
    const int lane = tg.lane, wave = tg.wave, b = tg.b;
    const float sig = fmaxf(a.sigma, 1e-8f);
    const float rsig = a.rsig;
    const float* __restrict__ rec = records + (size_t)b * T * REC;

    float col[3];
    col[0] = a.bg[b * 3 + 0];
    col[1] = a.bg[b * 3 + 1];
    col[2] = a.bg[b * 3 + 2];
    Trans tot = {1.0f, 0, 0};
    int n2, rec_chunks;
    forward_sweep<MODE, FAST, CKPT>(a, rec, tg, validm, rsig, sig, list[wave], col, tot, n2, rec_chunks);
    const int cap2 = a.cap2;

    if (MODE == MODE_RENDER || MODE == MODE_RECORD || (MODE == MODE_LOSS && a.out_img)) {
        if (tg.valid) {
            a.out_img[img_index(a, tg.pix, b, 0)] = col[0];
            a.out_img[img_index(a, tg.pix, b, 1)] = col[1];
            a.out_img[img_index(a, tg.pix, b, 2)] = col[2];
        }
    }
    if (MODE == MODE_RENDER) return;

    // the counts only where some lane of the tile has any (TN_IRREGULAR)
    const bool irregular = lane_mask(tot.z != 0 || tot.e != 0) != 0;
    if (lane == 0) {
        a.tl_n[2 * tg.tile] = min(n2, cap2);
        a.tl_n[2 * tg.tile + 1] = rec_chunks | (irregular ? TN_IRREGULAR : 0);
    }
    if (irregular) a.pze[tg.tile * 64 + lane] = make_int2(tot.z, tot.e);
    if (tg.valid) a.pq[tg.pix] = tot.q;
    if (MODE == MODE_LOSS) {
        double l = 0.0;
        if (tg.valid) {
            const float scale = a.lscale;
            for (int ch = 0; ch < 3; ch++) {
                float t = a.target[img_index(a, tg.pix, b, ch)];
                float d = col[ch] - t;
                l += (double)d * (double)d;
                a.pg0[tg.pix * 3 + ch] = scale * (col[ch] - t);
            }
        }
        l = wave_sum_f64(l);
        if (lane == 0) loss[wave] = l;
        __syncthreads();
        if (threadIdx.x == 0) {
            double lb = loss[0];
            for (int q = 1; q < WAVES; q++) lb += loss[q];
            a.partial_loss[tg.tile / WAVES] = lb;
        }
    }
}

// Per-pixel state of the backward sweep.
struct Back {
    float g0[3];   // dL/dpixel
    float col[3];  // canvas before the current layer
    Trans pre;     // transmittance through the current layer
    Trans tot;     // transmittance of the whole stack
};

// The backward of one triangle at this lane's pixel (grad.rs:148-181) into the
// lane's partial gradient `a`, zero where the lane does not contribute. The
// chain is predicated rather than branched: in the backward every entry has
// contributing lanes, so a branch would never skip. `any_band` (wave-uniform)
// skips the vertex terms when no lane took the exact path.
// PLAIN: no pixel of the wave met a zero factor or a rescaling in the forward
// pass (its totals have z == e == 0). The prefixes of a pixel's product are at
// least its total, so none of them needs either, and the transmittance is a
// plain product: trans_mul and trans_suffix then give these same values.
template <bool PLAIN>
__device__ inline void grad_pixel(const Rec& r, bool on, bool band, bool any_band, float w, float cov,
                                  const Geo& g, Pix p, float rsig, Back& st, float (&a)[NP]) {
    const float omw = 1.0f - w;
    // d_canvas as the reference holds it at layer k: g0 prod_{j>k} (1 - w_j)
    float tk;
    if (PLAIN) {
        st.pre.q = on ? st.pre.q * omw : st.pre.q;
        tk = on ? st.tot.q * __builtin_amdgcn_rcpf(st.pre.q) : 0.0f;
    } else {
        trans_mul(st.pre, on ? omw : 1.0f);
        tk = on ? trans_suffix(st.tot, st.pre) : 0.0f;
    }
    const float tw = tk * w;
    float sw = 0.0f;
    for (int ch = 0; ch < 3; ch++) {
        a[6 + ch] = st.g0[ch] * tw;
        const float d = r.f(R_C + ch) - st.col[ch];
        sw = fmaf(st.g0[ch], d, sw);
        const float o = fmaf(w, d, st.col[ch]);  // col + w (c - col)
        st.col[ch] = on ? o : st.col[ch];
    }
    const float d_w = tk * sw;
    a[9] = (r.i(R_FLAGS) & F_ACTIVE) ? d_w * cov : 0.0f;
    for (int j = 0; j < 6; j++) a[j] = 0.0f;
    if (!any_band) return;
    const float d_cov = d_w * r.f(R_A);
    // grad.rs:252-268: vertex terms, zero exactly on the boundary.
    // Every lane evaluates them (no divergent branch: the wave runs this block
    // only for entries with band lanes, where the masked lanes would issue
    // alike) and the lanes off the band or on the boundary take zeros.
    const bool vt = band && g.dist >= 1e-9f;
    // u = (pt - cp) / dist with cp = a + t (b - a), rounded as
    // grad.rs:256-259 does: for a pixel within ~1e-7 of an edge the
    // direction is set by these roundings, and the reference's gradient
    // inherits them.
    float inv = __builtin_amdgcn_rcpf(g.dist);
    float cpx = g.ax + g.t * g.ex, cpy = g.ay + g.t * g.ey;
    float ux = (p.px - cpx) * inv, uy = (p.py - cpy) * inv;
    float chain = d_cov * cov * (1.0f - cov) * rsig;
    chain = g.sd > 0.0f ? chain : -chain;
    float A = -(1.0f - g.t) * chain;  // onto the edge's first vertex
    float Bc = -g.t * chain;           // onto its second vertex
    float s0 = g.edge == 0 ? A : (g.edge == 2 ? Bc : 0.0f);
    float s1 = g.edge == 1 ? A : (g.edge == 0 ? Bc : 0.0f);
    float s2 = g.edge == 2 ? A : (g.edge == 1 ? Bc : 0.0f);
    a[0] = vt ? s0 * ux : 0.0f;
    a[1] = vt ? s0 * uy : 0.0f;
    a[2] = vt ? s1 * ux : 0.0f;
    a[3] = vt ? s1 * uy : 0.0f;
    a[4] = vt ? s2 * ux : 0.0f;
    a[5] = vt ? s2 * uy : 0.0f;
}

// Wave sum of the lanes' partial gradients of one triangle, added to its row
// of an LDS accumulator, by transposition through LDS instead of a shuffle
// tree: cross-row lane permutes (v_permlane32/16_swap) occupy the SIMD ~8
// cycles each and DPP ops ~4, plain FP32 adds ~2. Each lane stores its ten
// values in its column of the wave's area `tw` (ten rows of TP floats); then
// lane 4p + g (p < 10) sums pixels 16g..16g+15 of parameter p (four 16-byte
// reads, fifteen adds), a quad DPP sum combines the four partials and lane 4p
// adds the total into the row. Lanes 40-63 repeat parameter 9's sums (their
// reads stay in the area) and add nothing. The wave's LDS accesses complete
// in program order; the fences only keep the compiler from moving them
// across each other. The sums are in a fixed order, so with a per-wave row
// (deterministic mode) they are reproducible run to run.
constexpr int TP = 68;  // row pitch: the reads of the 40 summing lanes fall on all 32 banks
__device__ inline void reduce_entry(const float (&a)[NP], lds_float* tw, lds_float* row, int lane) {
    for (int q = 0; q < NP; q++) tw[q * TP + lane] = a[q];
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const int prm = min(lane >> 2, NP - 1), g = lane & 3;
    typedef float f4v __attribute__((ext_vector_type(4)));
    typedef __attribute__((address_space(3))) f4v lds_f4v;
    const lds_f4v* src = reinterpret_cast<const lds_f4v*>(tw + prm * TP + 16 * g);
    const f4v x0 = src[0], x1 = src[1], x2 = src[2], x3 = src[3];
    float sum = (((x0.x + x0.y) + (x0.z + x0.w)) + ((x1.x + x1.y) + (x1.z + x1.w))) +
                (((x2.x + x2.y) + (x2.z + x2.w)) + ((x3.x + x3.y) + (x3.z + x3.w)));
    sum += dpp<DPP_XOR1>(sum);
    sum += dpp<DPP_XOR2>(sum);
    if (g == 0 && lane < 4 * NP) lds_add(row + prm, sum);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// The backward sweep of one tile (grad.rs:135-182) over its recorded entries
// [i_begin, i_end) and, with REBUILD, the chunks from rec_chunks on rebuilt and
// classified again; the block's sums go out per chunk (atomics, or partial rows
// with DET). st: the pixel state at entry i_begin; plain: no lane of the tile
// met a zero factor or a rescaling in the forward pass. lw: the wave's LDS
// list; acc: ROWS x CH x NP accumulators; trans: WAVES x NP x TP.
template <int MODE, bool FAST, bool REBUILD, bool DET>
__device__ __forceinline__ void backward_sweep(const RasterArgs& a, const float* __restrict__ rec,
                                               const TileEnt* __restrict__ ents, const TileGeo& tg,
                                               uint64_t validm, float rsig, float sig, Back& st, int i_begin,
                                               int i_end, int rec_chunks, bool plain, uint32_t* lw, float* acc,
                                               float* trans) {
    constexpr int ROWS = DET ? WAVES : 1;  // accumulator row sets
    const int T = a.T, lane = tg.lane, wave = tg.wave, b = tg.b;
    const int n_chunks = (T + CH - 1) / CH;
    // wave-uniform, so the recorded entries are read with scalar loads
    const int cap2 = a.cap2;
    const TileEnt* __restrict__ te = ents + (size_t)uniform_u32((uint32_t)tg.tile) * cap2;
    const size_t blk = tg.tile / WAVES;
    float* accw = acc + (DET ? wave : 0) * (CH * NP);
    lds_float* const tw = (lds_float*)(trans + wave * (NP * TP));
    typedef __attribute__((address_space(3))) char lds_char;
    int i2 = i_begin;

    // The entries the forward kernel recorded: which lanes contribute and
    // which of them took the exact path are known; only w is recomputed. The
    // next entry is read one iteration ahead.
    auto recorded = [&](auto plain_c, int k0, int k1) {
        constexpr bool PLAIN = decltype(plain_c)::value;
        TileEnt nx = ent_at(te, min(i2, cap2 - 1));
        for (; i2 < i_end; i2++) {
            const TileEnt cur = nx;
            const int k = (int)(cur.k >> 8);
            if (k >= k1) break;
            nx = ent_at(te, min(i2 + 1, cap2 - 1));
            const bool on = __builtin_amdgcn_inverse_ballot_w64(cur.on);
            const bool band = __builtin_amdgcn_inverse_ballot_w64(cur.band);
            Rec r;
            f8v eb;
            load_entry<FAST, true>(rec, rec_off((uint32_t)k), cur.k, r, eb);
            float cov;
            Geo g;
            band_cov<FAST>(r, eb, tg.p, cur.k, cur.band, band, rsig, sig, g, cov);
            const float w = r.f(R_A) * cov;
            float part[NP];
            grad_pixel<PLAIN>(r, on, band, cur.band != 0, w, cov, g, tg.p, rsig, st, part);
            // the recorded byte offset of the triangle's row (the product
            // (k - k0) * NP would become a 64-bit multiply-add on the vector unit)
            reduce_entry(part, tw, (lds_float*)((lds_char*)accw + cur.row), lane);
        }
    };

    for (int c = 0; c < n_chunks; c++) {
        int k0 = c * CH, k1 = min(T, k0 + CH);
        int nk = k1 - k0;
        if (DET) {
            // the wave's own accumulator rows (CH * NP floats, 16-byte aligned),
            // four floats per store
            float4* acc4 = reinterpret_cast<float4*>(accw);
            for (int j = lane; j < CH * NP / 4; j += 64) acc4[j] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
        } else {
            // the block's shared rows, cleared by all its threads
            float4* acc4 = reinterpret_cast<float4*>(accw);
            for (int j = threadIdx.x; j < CH * NP / 4; j += WAVES * 64) acc4[j] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            __syncthreads();
        }

        if (c < rec_chunks) {
            if (plain)
                recorded(std::true_type{}, k0, k1);
            else
                recorded(std::false_type{}, k0, k1);
        } else if (REBUILD) {
            // Fallback when the forward kernel ran out of record space: rebuild
            // the chunk's list and classify every pair again.
            int count = tg.live ? build_list(rec, k0, k1, tg.tx0, tg.ty0, tg.tx1, tg.ty1, tg.cx0, tg.cy0,
                                             tg.cx1, tg.cy1, lw, lane, F_TAPE)
                                : 0;
            for (int i = 0; i < count; i++) {
                const uint32_t ent = uniform_u32(lw[i]);
                const int kl = (int)(ent >> 8);
                Rec r;
                f8v eb;
                load_entry<FAST, true>(rec, rec_off((uint32_t)(k0 + kl)), ent, r, eb);
                float w = 0.0f, cov = 0.0f;
                uint64_t bandm;
                Geo g;
                const uint64_t onm =
                    pair_weight<FAST>(r, eb, ent, tg.x, tg.y, tg.p, validm, w, cov, bandm, g, rsig, sig);
                if (onm == 0) continue;
                bandm &= onm;
                const bool any_band = bandm != 0;
                const bool on = __builtin_amdgcn_inverse_ballot_w64(onm);
                const bool band = __builtin_amdgcn_inverse_ballot_w64(bandm);
                float part[NP];
                grad_pixel<false>(r, on, band, any_band, w, cov, g, tg.p, rsig, st, part);
                reduce_entry(part, tw, (lds_float*)accw + kl * NP, lane);
            }
        }
        __syncthreads();
        // The block's sums: the four waves' accumulators added in wave order.
        // Deterministic mode writes them as the block's partial row for
        // reduce_partials; otherwise each nonzero sum is one native float
        // atomic add into the output (one per triangle parameter per block).
        if (DET) {
            float* prow = a.partials + (blk * T + k0) * NP;
            for (int j = threadIdx.x; j < nk * NP; j += WAVES * 64) {
                float v = acc[j];
                for (int q = 1; q < ROWS; q++) v += acc[q * (CH * NP) + j];
                prow[j] = v;
            }
        } else {
            float* grow = a.grads + ((size_t)b * T + k0) * NP;
            for (int j = threadIdx.x; j < nk * NP; j += WAVES * 64) {
                const float v = acc[j];
                if (v != 0.0f) unsafeAtomicAdd(grow + j, v);
            }
        }
        __syncthreads();
    }
}

// reduce_entry's wave sum, added by lane 4p straight into parameter p of the
// triangle's gradient row `grow` in global memory (one float atomic each).
__device__ inline void reduce_entry_global(const float (&a)[NP], lds_float* tw, float* grow, int lane) {
    for (int q = 0; q < NP; q++) tw[q * TP + lane] = a[q];
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const int prm = min(lane >> 2, NP - 1), g = lane & 3;
    typedef float f4v __attribute__((ext_vector_type(4)));
    typedef __attribute__((address_space(3))) f4v lds_f4v;
    const lds_f4v* src = reinterpret_cast<const lds_f4v*>(tw + prm * TP + 16 * g);
    const f4v x0 = src[0], x1 = src[1], x2 = src[2], x3 = src[3];
    float sum = (((x0.x + x0.y) + (x0.z + x0.w)) + ((x1.x + x1.y) + (x1.z + x1.w))) +
                (((x2.x + x2.y) + (x2.z + x2.w)) + ((x3.x + x3.y) + (x3.z + x3.w)));
    sum += dpp<DPP_XOR1>(sum);
    sum += dpp<DPP_XOR2>(sum);
    if (g == 0 && lane < 4 * NP && sum != 0.0f) unsafeAtomicAdd(grow + prm, sum);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// reduce_entry_global for an entry with no band lane, whose vertex terms are
// all zero (grad_pixel): only parameters 6-9 are summed. Lane 16p + g sums
// pixels 4g..4g+3 of parameter 6 + p (one 16-byte read, three adds), the row
// of sixteen partials is combined across its lanes (two quad steps, the
// half-row and the row mirror) and lane 16p adds the total. About half of the
// entries of B=16 256x256 T=128 have no band lane: -1.0 us of ~88.
constexpr int DPP_ROW_MIRROR = 0x140, DPP_ROW_HALF_MIRROR = 0x141;
__device__ inline void reduce_entry_global_cw(const float (&a)[NP], lds_float* tw, float* grow, int lane) {
    for (int q = 0; q < 4; q++) tw[q * TP + lane] = a[6 + q];
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const int prm = lane >> 4, g = lane & 15;
    typedef float f4v __attribute__((ext_vector_type(4)));
    typedef __attribute__((address_space(3))) f4v lds_f4v;
    const f4v x = *reinterpret_cast<const lds_f4v*>(tw + prm * TP + 4 * g);
    float sum = (x.x + x.y) + (x.z + x.w);
    sum += dpp<DPP_XOR1>(sum);
    sum += dpp<DPP_XOR2>(sum);
    sum += dpp<DPP_ROW_HALF_MIRROR>(sum);
    sum += dpp<DPP_ROW_MIRROR>(sum);
    if (g == 0 && sum != 0.0f) unsafeAtomicAdd(grow + 6 + prm, sum);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Backward: the reverse-mode sweep (grad.rs:135-182) over the entries the
// forward kernel recorded, again in scene order. The gradient reaching layer
// k, d_canvas * prod_{j>k} (1 - w_j) (grad.rs:162-169), is formed as a ratio
// of transmittance products instead of being peeled off a tape. Per-triangle
// gradients are wave-reduced, accumulated per wave in LDS and written as one
// partial row per block and chunk.
// REBUILD: with the rebuild path for tiles past the recorded entries. Without
// it (the entries cover T, the usual case) the kernel needs ~55 VGPRs instead
// of ~95, so it runs uncapped.
// DET: deterministic mode. Each wave adds into its own accumulator rows and the
// block sums them in wave order; otherwise the four waves share one set of
// rows (adds from different waves land in any order, as the float atomics
// into the output do anyway) and the block needs a quarter of the LDS.
template <int MODE, bool FAST, bool REBUILD, bool DET>
__global__ __launch_bounds__(WAVES * 64) __attribute__((amdgpu_waves_per_eu(REBUILD ? (DET ? 4 : 6) : (DET ? 5 : 7)))) void backward_kernel(RasterArgs a, const float* __restrict__ records,
                                                               const TileEnt* __restrict__ ents) {
    constexpr int ROWS = DET ? WAVES : 1;  // accumulator row sets
    __shared__ uint32_t list[WAVES][CH];
    __shared__ __attribute__((aligned(16))) float acc[ROWS][CH * NP];
    __shared__ __attribute__((aligned(16))) float trans[WAVES][NP * TP];
    if (a.halt && *a.halt >= 0) return;
    const int W = a.W, H = a.H, T = a.T;
    // segments per tile: only the variant with neither rebuild nor fixed-order sums splits
    const int S = (!REBUILD && !DET && a.perm_bwd) ? max(a.nseg, 1) : 1;
    const TileGeo tg = S > 1 ? tile_geo_split(W, H, a.gx, a.gy, a.perm_bwd, a.B, S, a.nsplit)
                             : tile_geo(W, H, a.perm_bwd, a.B);
    const uint64_t validm = lane_mask(tg.valid);  // lanes whose pixel is in the image
    const int lane = tg.lane, wave = tg.wave, b = tg.b;
    const float sig = fmaxf(a.sigma, 1e-8f);
    const float rsig = a.rsig;
    const float* __restrict__ rec = records + (size_t)b * T * REC;

    const int n2r = (int)uniform_u32((uint32_t)a.tl_n[2 * tg.tile]);
    const int rec_chunks = (int)uniform_u32((uint32_t)a.tl_n[2 * tg.tile + 1]) & ~TN_IRREGULAR;
    // This wave's entries: [i_begin, i_end) of the tile's recorded list.
    int i_begin = 0, i_end = n2r;
    if (tg.nseg > 1) {
        i_begin = tg.seg * a.seg_m;
        i_end = tg.seg == tg.nseg - 1 ? n2r : min(n2r, i_begin + a.seg_m);
        if (tg.seg > 0) {
            // the block (all of it, before any barrier) leaves when none of its
            // four tiles has entries in this segment
            const size_t t0 = tg.tile - (size_t)wave;
            int most = 0;
            for (int q = 0; q < WAVES; q++) most = max(most, (int)uniform_u32((uint32_t)a.tl_n[2 * (t0 + q)]));
            if (most <= i_begin) return;
        }
    }

    Back st;
    const bool irregular = (a.tl_n[2 * tg.tile + 1] & TN_IRREGULAR) != 0;  // wave-uniform
    {
        int2 ze = make_int2(0, 0);
        if (irregular) ze = a.pze[tg.tile * 64 + lane];
        st.tot = {a.pq[tg.pix], ze.x, ze.y};
        for (int ch = 0; ch < 3; ch++) {
            st.g0[ch] = !tg.valid ? 0.0f
                                  : (MODE == MODE_LOSS ? a.pg0[tg.pix * 3 + ch] : a.grad_in[img_index(a, tg.pix, b, ch)]);
        }
    }
    if (i_begin > 0 && i_begin < n2r) {
        // the forward kernel's checkpoint before entry i_begin
        const float* c = a.ckpt + ((size_t)tg.tile * (a.nseg - 1) + (tg.seg - 1)) * (CKPT_WORDS * 64) + lane;
        st.col[0] = c[0];
        st.col[1] = c[64];
        st.col[2] = c[128];
        st.pre = {c[192], __float_as_int(c[256]), __float_as_int(c[320])};
    } else {
        st.col[0] = a.bg[b * 3 + 0];
        st.col[1] = a.bg[b * 3 + 1];
        st.col[2] = a.bg[b * 3 + 2];
        st.pre = {1.0f, 0, 0};
    }
    // no lane of the tile met a zero factor or a rescaling in the forward pass
    backward_sweep<MODE, FAST, REBUILD, DET>(a, rec, ents, tg, validm, rsig, sig, st, i_begin, i_end, rec_chunks,
                                             !irregular, list[wave], &acc[0][0], &trans[0][0]);
    // The per-item loss (canvas.rs:45-58) from the forward kernel's per-block
    // sums, by the scene's first block, in a fixed order.
    if (MODE == MODE_LOSS && !DET && tg.bx == 0 && tg.by == 0 && tg.seg == 0 && wave == 0) {
        // blocks per scene from the image size: the split grid is one-dimensional
        const int nblk = ((W + 2 * TILE - 1) / (2 * TILE)) * ((H + 2 * TILE - 1) / (2 * TILE));
        const double* pl = a.partial_loss + (size_t)b * nblk;
        double l = 0.0;
        for (int r = lane; r < nblk; r += 64) l += pl[r];
        l = wave_sum_f64(l);
        if (lane == 0) a.losses[b] = (float)(l / (3.0 * (double)W * (double)H));
    }
}

// The gradient paths' forward and backward in one kernel: each block
// composites its four tiles (forward_sweep), forms dL/dpixel (MODE_LOSS: with
// the loss partial; MODE_GRAD_IN: the caller's), then sweeps the same tiles'
// recorded entries backward (backward_sweep) with the per-pixel state still in
// registers, so nothing goes through HBM between the two sweeps but the entry
// lists, and the device drains once instead of twice. Without the split
// backward, when every tile's list is recorded whole in regions of whole
// 64-byte lines (cap2 >= T, cap2 % 8 == 0); both sweeps take the backward
// kernel's block order. Then reduce_partials (DET) or, in MODE_LOSS,
// sum_losses forms the results from the per-block sums.
// DET: per-wave accumulator rows and partial rows per block, as backward_kernel.
template <int MODE, bool FAST, bool DET>
__global__ __launch_bounds__(WAVES * 64) __attribute__((amdgpu_waves_per_eu(DET ? 4 : 7))) void fused_kernel(RasterArgs a, const float* __restrict__ records,
                                                                            const TileEnt* __restrict__ ents) {
    static_assert(MODE == MODE_LOSS || MODE == MODE_GRAD_IN, "gradient modes only");
    constexpr int ROWS = DET ? WAVES : 1;  // accumulator row sets
    __shared__ uint32_t list[WAVES][CH];
    __shared__ double loss[WAVES];
    __shared__ __attribute__((aligned(16))) float acc[ROWS * CH * NP];
    __shared__ __attribute__((aligned(16))) float trans[WAVES][NP * TP];
    if (a.halt && *a.halt >= 0) return;
    const int W = a.W, H = a.H, T = a.T;
    const TileGeo tg = tile_geo(W, H, a.perm_bwd, a.B);
    const uint64_t validm = lane_mask(tg.valid);  // lanes whose pixel is in the image
    const int lane = tg.lane, wave = tg.wave, b = tg.b;
    const float sig = fmaxf(a.sigma, 1e-8f);
    const float rsig = a.rsig;
    const float* __restrict__ rec = records + (size_t)b * T * REC;

    Back st;
    float col[3];
    for (int ch = 0; ch < 3; ch++) col[ch] = st.col[ch] = a.bg[b * 3 + ch];
    Trans tot = {1.0f, 0, 0};
    int n2, rec_chunks;
    forward_sweep<MODE, FAST, false>(a, rec, tg, validm, rsig, sig, list[wave], col, tot, n2, rec_chunks);
    if (MODE == MODE_LOSS && a.out_img && tg.valid)
        for (int ch = 0; ch < 3; ch++) a.out_img[img_index(a, tg.pix, b, ch)] = col[ch];
    for (int ch = 0; ch < 3; ch++) st.g0[ch] = 0.0f;
    double l = 0.0;
    if (tg.valid) {
        if (MODE == MODE_LOSS) {
            // the loss (canvas.rs:45-58) and dL/dpixel (grad.rs:111-114) as forward_kernel forms them
            const float scale = a.lscale;
            for (int ch = 0; ch < 3; ch++) {
                float t = a.target[img_index(a, tg.pix, b, ch)];
                float d = col[ch] - t;
                l += (double)d * (double)d;
                st.g0[ch] = scale * (col[ch] - t);
            }
        } else {
            for (int ch = 0; ch < 3; ch++) st.g0[ch] = a.grad_in[img_index(a, tg.pix, b, ch)];
        }
    }
    if (MODE == MODE_LOSS) {
        l = wave_sum_f64(l);
        if (lane == 0) loss[wave] = l;
    }
    // The entries this wave recorded with vector stores are read back below with
    // scalar loads: the stores are complete (in L2, which the scalar cache reads
    // from) before any of those loads issue. A tile's region holds whole cache
    // lines, so no scalar-cache line of it was loaded before its entries were.
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (MODE == MODE_LOSS && threadIdx.x == 0) {
        double lb = loss[0];
        for (int q = 1; q < WAVES; q++) lb += loss[q];
        a.partial_loss[tg.tile / WAVES] = lb;
    }
    st.tot = tot;
    st.pre = {1.0f, 0, 0};
    const bool irregular = lane_mask(tot.z != 0 || tot.e != 0) != 0;
    backward_sweep<MODE, FAST, false, DET>(a, rec, ents, tg, validm, rsig, sig, st, 0, n2, rec_chunks, !irregular,
                                           list[wave], acc, &trans[0][0]);
}

// fused_kernel with one tile per workgroup (one wave) and no block-level
// state: each recorded entry's wave sum goes straight into the gradients with
// float atomics, so a wave needs no accumulator rows, block sums or barriers,
// and its slot frees as soon as its own tile is done (a block of four waves
// holds all four until its slowest tile finishes). Slots follow setup_records'
// order, of tiles (perm_tiles) or of blocks four tiles at a time
// (tile_geo_wave). Its loss partials are per tile, summed
// per block in wave order by sum_losses, as the four-wave blocks sum them.
// Used where fused_kernel would be, outside the deterministic mode. ROWS: its
// lists scan the tile row's triangles (RasterArgs::rows), else all of them.
// The fused kernels' last B workgroups (RasterArgs::loss_tail): scene
// b's loss from its tiles' partials once every slot holds one, in sum_losses'
// order (per lane, blocks lane, lane + 64, ... each as its four tiles in wave
// order; then the lanes summed), so the same bits as sum_losses. Every poll
// loads the slots with device-scope atomic loads, which see the tiles'
// device-scope atomic stores from any XCD. The wait is bounded: a scene whose
// slots are still pending after TAIL_SPIN polls gets a NaN loss.
constexpr int TAIL_U = 4;           // blocks per lane held in registers (scenes of up to 256 blocks)
constexpr int TAIL_SPIN = 1 << 22;  // polls, each at least one round trip to memory
__device__ inline double tail_load(const double* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ inline bool tail_pending(double v) { return (uint64_t)__double_as_longlong(v) == LOSS_PENDING; }

__device__ inline void loss_tail(const RasterArgs& a, int b) {
    const int lane = threadIdx.x & 63, nblk = a.gx * a.gy;
    const double* pl = a.partial_loss + (size_t)b * nblk * WAVES;
    const bool held = nblk <= 64 * TAIL_U;
    double v[TAIL_U][WAVES];
    bool ok = false;
    for (int spin = 0; spin < TAIL_SPIN; spin++) {
        bool pending = false;
        if (held) {
            for (int u = 0; u < TAIL_U; u++) {
                const int r = lane + 64 * u;
                for (int q = 0; q < WAVES; q++) {
                    v[u][q] = r < nblk ? tail_load(pl + (size_t)r * WAVES + q) : 0.0;
                    pending = pending || (r < nblk && tail_pending(v[u][q]));
                }
            }
        } else {
            for (int r = lane; r < nblk; r += 64)
                for (int q = 0; q < WAVES; q++)
                    pending = pending || tail_pending(tail_load(pl + (size_t)r * WAVES + q));
        }
        if (lane_mask(pending) == 0) {
            ok = true;
            break;
        }
        __builtin_amdgcn_s_sleep(2);
    }
    double l = 0.0;
    if (held) {
        for (int u = 0; u < TAIL_U; u++) {
            double lb = v[u][0];
            for (int q = 1; q < WAVES; q++) lb += v[u][q];
            l = lane + 64 * u < nblk ? l + lb : l;
        }
    } else {
        for (int r = lane; r < nblk; r += 64) {
            double lb = tail_load(pl + (size_t)r * WAVES);
            for (int q = 1; q < WAVES; q++) lb += tail_load(pl + (size_t)r * WAVES + q);
            l += lb;
        }
    }
    l = wave_sum_f64(l);
    if (lane == 0) a.losses[b] = ok ? (float)(l / (3.0 * (double)a.H * (double)a.W)) : __builtin_nanf("");
}

template <int MODE, bool FAST, bool ROWS>
__global__ __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(7))) void fused_tile_kernel(RasterArgs a, const float* __restrict__ records,
                                                                                const TileEnt* __restrict__ ents) {
    static_assert(MODE == MODE_LOSS || MODE == MODE_GRAD_IN, "gradient modes only");
    __shared__ uint32_t list[CH];
    __shared__ __attribute__((aligned(16))) float trans[NP * TP];
    if (a.halt && *a.halt >= 0) return;
    if (MODE == MODE_LOSS && a.loss_tail) {
        // the last B workgroups: the last row of a two-dimensional grid
        if (gridDim.y > 1 ? blockIdx.y == gridDim.y - 1 : (int)blockIdx.x >= (int)gridDim.x - a.B) {
            loss_tail(a, gridDim.y > 1 ? (int)blockIdx.x : (int)blockIdx.x - ((int)gridDim.x - a.B));
            return;
        }
    }
    const int W = a.W, H = a.H, T = a.T;
    const TileGeo tg = tile_geo_wave(W, H, a.gx, a.gy, a.perm_bwd, a.B, a.perm_tiles != 0, a.tdiv_m);
    const uint64_t validm = lane_mask(tg.valid);  // lanes whose pixel is in the image
    const int lane = tg.lane, b = tg.b;
    const float sig = fmaxf(a.sigma, 1e-8f);
    const float rsig = a.rsig;
    const float* __restrict__ rec = records + (size_t)b * T * REC;

    Back st;
    float col[3];
    for (int ch = 0; ch < 3; ch++) col[ch] = st.col[ch] = a.bg[b * 3 + ch];
    Trans tot = {1.0f, 0, 0};
    int n2, rec_chunks;
    // merged chunks: the sweep below reads each entry's triangle index
    forward_sweep<MODE, FAST, false, true, ROWS>(a, rec, tg, validm, rsig, sig, list, col, tot, n2, rec_chunks);
    if (MODE == MODE_LOSS && a.out_img && tg.valid)
        for (int ch = 0; ch < 3; ch++) a.out_img[img_index(a, tg.pix, b, ch)] = col[ch];
    for (int ch = 0; ch < 3; ch++) st.g0[ch] = 0.0f;
    double l = 0.0;
    if (tg.valid) {
        if (MODE == MODE_LOSS) {
            // the loss (canvas.rs:45-58) and dL/dpixel (grad.rs:111-114) as forward_kernel forms them
            const float scale = a.lscale;
            for (int ch = 0; ch < 3; ch++) {
                float t = a.target[img_index(a, tg.pix, b, ch)];
                float d = col[ch] - t;
                l += (double)d * (double)d;
                st.g0[ch] = scale * (col[ch] - t);
            }
        } else {
            for (int ch = 0; ch < 3; ch++) st.g0[ch] = a.grad_in[img_index(a, tg.pix, b, ch)];
        }
    }
    if (MODE == MODE_LOSS) {
        l = wave_sum_f64(l);
        if (lane == 0) {
            if (a.loss_tail)
                __hip_atomic_store(&a.partial_loss[tg.tile], l, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            else
                a.partial_loss[tg.tile] = l;
        }
    }
    // The entries this wave recorded with vector stores are read back below with
    // scalar loads: the stores are complete (in L2, which the scalar cache reads
    // from) before any of those loads issue. A tile's region holds whole cache
    // lines, so no scalar-cache line of it was loaded before its entries were.
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    st.tot = tot;
    st.pre = {1.0f, 0, 0};
    const bool plain = lane_mask(tot.z != 0 || tot.e != 0) == 0;
    const TileEnt* __restrict__ te = ents + (size_t)uniform_u32((uint32_t)tg.tile) * a.cap2;
    float* const grads = a.grads + (size_t)b * T * NP;
    lds_float* const tw = (lds_float*)trans;
    // The entry after the last one read is at byte offset `end`, inside the
    // tile's region (cap2 > T >= n2 for this kernel): the loop prefetches it
    // unclamped, and its byte offset is the loop's only counter.
    const uint32_t end = (uint32_t)n2 * (uint32_t)sizeof(TileEnt);
    // The recorded entries in scene order (backward_sweep's recorded loop, with
    // every chunk at once: the gradient rows are global).
    auto sweep = [&](auto plain_c) {
        constexpr bool PLAIN = decltype(plain_c)::value;
        TileEnt nx = te[0];
        for (uint32_t off = 0; off < end;) {
            const TileEnt cur = nx;
            const int k = (int)(cur.k >> 8);
            off += (uint32_t)sizeof(TileEnt);
            nx = *reinterpret_cast<const TileEnt*>(reinterpret_cast<const char*>(te) + off);
            const bool on = __builtin_amdgcn_inverse_ballot_w64(cur.on);
            const bool band = __builtin_amdgcn_inverse_ballot_w64(cur.band);
            Rec r;
            f8v eb;
            load_entry<FAST, true>(rec, rec_off((uint32_t)k), cur.k, r, eb);
            float cov;
            Geo g;
            band_cov<FAST>(r, eb, tg.p, cur.k, cur.band, band, rsig, sig, g, cov);
            const float w = r.f(R_A) * cov;
            float part[NP];
            grad_pixel<PLAIN>(r, on, band, cur.band != 0, w, cov, g, tg.p, rsig, st, part);
            if (cur.band != 0)
                reduce_entry_global(part, tw, grads + (size_t)k * NP, lane);
            else
                reduce_entry_global_cw(part, tw, grads + (size_t)k * NP, lane);
        }
    };
    if (plain)
        sweep(std::true_type{});
    else
        sweep(std::false_type{});
}

// Grids of few tiles (a single scene of a few hundred 8x8 tiles, the fit):
// one tile per workgroup of S waves. Where the one-wave kernel runs about one
// wave per SIMD and is bound by the chain of dependent waits per entry of its
// tile (scalar record loads, LDS round trips), this one splits the tile's
// triangles over the waves, wave s taking [s T / S, (s + 1) T / S):
//  A. each wave lists its triangles and evaluates their weights at the tile's
//     pixels (pair_weight: the exact path, the classification), records its
//     entries for the backward, and leaves each entry's weights, colour and
//     contributing lanes in LDS;
//  B. every wave composites all the tile's entries from LDS in scene order
//     (raster.rs:37-68), exactly as the one-wave kernel's forward sweep does,
//     so the image, the transmittance and the loss are the same bits; a wave
//     keeps the canvas and the transmittance at the start of its segment;
//  C. each wave sweeps its own entries backward from that state, as the
//     one-wave kernel sweeps all of them.
// The tile's entry region (cap2 = S x capS entries) holds segment s's entries
// at s capS. DET: each wave sums its entries' gradients into LDS rows of its
// segment's triangles and the tile writes its partial rows (B x tiles x T x
// NP) for reduce_partials / fit_step; otherwise each entry's wave sum goes to
// the gradients as float atomics. The loss partial is per tile either way,
// summed four to a 16x16 block first, as sum_losses sums the one-wave
// kernel's.
//
// Dynamic LDS: phases A and B hold SEG_WAVES x seg_tris(T) SegEnt records;
// phase C reuses the same area for the waves' transposition areas (and DET
// accumulator rows).
struct SegEnt {
    float w[64];       // weight at each lane's pixel
    float c[3];        // colour
    uint32_t on[2];    // lanes it contributes at (low, high word)
    uint32_t pad[3];
};
static_assert(sizeof(SegEnt) == 288 && sizeof(SegEnt) % 16 == 0, "SegEnt keeps 16-byte alignment");

// Triangles per segment (at most), the pitch of the segments' SegEnt records
// in LDS; phase C's LDS bytes; and the workgroup's dynamic LDS.
__host__ __device__ constexpr int seg_tris(int T) { return (T + SEG_WAVES - 1) / SEG_WAVES; }
__host__ __device__ constexpr size_t seg_lds_c(bool det, int T) {
    return (size_t)SEG_WAVES * NP * TP * sizeof(float) +
           (det ? (size_t)SEG_WAVES * seg_tris(T) * NP * sizeof(float) : 0);
}
__host__ __device__ constexpr size_t seg_lds_bytes(bool det, int T) {
    return (size_t)SEG_WAVES * seg_tris(T) * sizeof(SegEnt) > seg_lds_c(det, T)
               ? (size_t)SEG_WAVES * seg_tris(T) * sizeof(SegEnt)
               : seg_lds_c(det, T);
}

template <int MODE, bool FAST, bool DET, int S>
__global__ __launch_bounds__(S * 64) void fused_seg_kernel(RasterArgs a, const float* __restrict__ records,
                                                          const TileEnt* __restrict__ ents) {
    static_assert(MODE == MODE_LOSS || MODE == MODE_GRAD_IN, "gradient modes only");
    static_assert(S == SEG_WAVES, "seg_lds_bytes sizes the LDS for SEG_WAVES waves");
    __shared__ uint32_t list[S][CH];
    __shared__ int nent[S];
    extern __shared__ __attribute__((aligned(16))) float seg_lds[];
    SegEnt* const sent = reinterpret_cast<SegEnt*>(seg_lds);
    if (a.halt && *a.halt >= 0) return;
    if (MODE == MODE_LOSS && !DET && a.loss_tail && (int)blockIdx.x >= (int)gridDim.x - a.B) {
        if (threadIdx.x < 64) loss_tail(a, (int)blockIdx.x - ((int)gridDim.x - a.B));
        return;
    }
    const int W = a.W, H = a.H, T = a.T;
    const int s = (int)uniform_u32(threadIdx.x >> 6);  // this wave's segment
    const TileGeo tg = tile_geo_wave(W, H, a.gx, a.gy, a.perm_bwd, a.B, a.perm_tiles != 0);
    const uint64_t validm = lane_mask(tg.valid);  // lanes whose pixel is in the image
    const int lane = tg.lane, b = tg.b;
    const float sig = fmaxf(a.sigma, 1e-8f);
    const float rsig = a.rsig;
    const float* __restrict__ rec = records + (size_t)b * T * REC;
    const int k0 = (int)(((long long)s * T) / S), k1 = (int)(((long long)(s + 1) * T) / S);
    const int capS = a.cap2 / S;     // entry slots per segment in the tile's region
    const int lcap = seg_tris(T);    // SegEnt slots per segment in LDS (>= k1 - k0)
    // wave-uniform: the entry stores and loads address from a scalar base
    TileEnt* const te = a.tl_ent + (size_t)uniform_u32((uint32_t)tg.tile) * a.cap2 + s * capS;

    // A. the segment's entries and their weights
    int n2 = 0;
    for (int kb = k0; kb < k1;) {
        int kend;
        const int count = tg.live ? build_list<true>(rec, kb, k1, tg.tx0, tg.ty0, tg.tx1, tg.ty1, tg.cx0, tg.cy0,
                                                     tg.cx1, tg.cy1, list[s], lane, F_LIVE, &kend)
                                  : 0;
        kb = tg.live ? kend : k1;
        // the list one half at a time, one entry per lane (as forward_sweep)
        for (int h = 0; h < count; h += 64) {
            const uint32_t held = list[s][min(h + lane, CH - 1)];
            const int nh = (int)uniform_u32((uint32_t)min(count - h, 64));
            for (int i = 0; i < nh; i++) {
                const uint32_t ent = (uint32_t)__builtin_amdgcn_readlane((int)held, i);
                const int k = (int)(ent >> 8);  // merged lists hold the triangle index
                Rec r;
                f8v eb;
                load_entry<FAST, true>(rec, rec_off((uint32_t)k), ent, r, eb);
                float w = 0.0f, cov;
                uint64_t bandm;
                Geo g;
                const uint64_t onm =
                    pair_weight<FAST>(r, eb, ent, tg.x, tg.y, tg.p, validm, w, cov, bandm, g, rsig, sig);
                if (onm == 0) continue;  // wave-uniform
                SegEnt& e = sent[s * lcap + n2];
                e.w[lane] = w;
                if (lane == 0) {
                    e.c[0] = r.f(R_C);
                    e.c[1] = r.f(R_C + 1);
                    e.c[2] = r.f(R_C + 2);
                    e.on[0] = (uint32_t)onm;
                    e.on[1] = (uint32_t)(onm >> 32);
                    TileEnt t;
                    t.k = ent;
                    t.row = 0;
                    t.on = onm;
                    t.band = onm & bandm;
                    te[n2] = t;
                }
                n2++;
            }
        }
    }
    if (lane == 0) nent[s] = n2;
    // The entries were recorded with vector stores and are read back below with
    // scalar loads: the stores are complete (in L2, which the scalar cache reads
    // from) before any of those loads issue (the regions are whole cache lines).
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();

    // B. the tile's composite in scene order, forward_sweep's arithmetic
    Back st;
    float col[3];
    Trans tot = {1.0f, 0, 0};
    for (int ch = 0; ch < 3; ch++) col[ch] = a.bg[b * 3 + ch];
    for (int q = 0; q < S; q++) {
        if (q == s) {
            for (int ch = 0; ch < 3; ch++) st.col[ch] = col[ch];
            st.pre = tot;
        }
        const int n = nent[q];
        for (int i = 0; i < n; i++) {
            const SegEnt& e = sent[q * lcap + i];
            const float w = e.w[lane];
            const bool on = ((lane < 32 ? e.on[0] >> lane : e.on[1] >> (lane - 32)) & 1u) != 0;
            const float omw = 1.0f - w;
            for (int ch = 0; ch < 3; ch++) {
                const float o = fmaf(w, e.c[ch] - col[ch], col[ch]);
                col[ch] = on ? o : col[ch];
            }
            const float f = on ? omw : 1.0f;
            const float qn = tot.q * f;
            if (lane_mask(!(qn >= 5.421010862427522e-20f)) == 0)
                tot.q = qn;
            else
                trans_mul(tot, f);
        }
    }
    st.tot = tot;
    if (MODE == MODE_LOSS && a.out_img && tg.valid && s == 0)
        for (int ch = 0; ch < 3; ch++) a.out_img[img_index(a, tg.pix, b, ch)] = col[ch];
    for (int ch = 0; ch < 3; ch++) st.g0[ch] = 0.0f;
    double l = 0.0;
    if (tg.valid) {
        if (MODE == MODE_LOSS) {
            // the loss (canvas.rs:45-58) and dL/dpixel (grad.rs:111-114) as forward_kernel forms them
            const float scale = a.lscale;
            for (int ch = 0; ch < 3; ch++) {
                float t = a.target[img_index(a, tg.pix, b, ch)];
                float d = col[ch] - t;
                l += (double)d * (double)d;
                st.g0[ch] = scale * (col[ch] - t);
            }
        } else {
            for (int ch = 0; ch < 3; ch++) st.g0[ch] = a.grad_in[img_index(a, tg.pix, b, ch)];
        }
    }
    if (MODE == MODE_LOSS && s == 0) {
        l = wave_sum_f64(l);
        if (lane == 0) {
            if (!DET && a.loss_tail)
                __hip_atomic_store(&a.partial_loss[tg.tile], l, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            else
                a.partial_loss[tg.tile] = l;
        }
    }
    const bool plain = lane_mask(tot.z != 0 || tot.e != 0) == 0;  // the same in every wave
    __syncthreads();  // phase C reuses the SegEnt area

    // C. this segment's entries backward
    lds_float* const tw = (lds_float*)(seg_lds + s * (NP * TP));
    lds_float* const accs = (lds_float*)(seg_lds + S * (NP * TP) + s * (lcap * NP));
    if (DET) {
        for (int j = lane; j < lcap * NP; j += 64) accs[j] = 0.0f;
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
    }
    const TileEnt* __restrict__ tr = te;
    float* const grads = DET ? nullptr : a.grads + (size_t)b * T * NP;
    auto sweep = [&](auto plain_c) {
        constexpr bool PLAIN = decltype(plain_c)::value;
        TileEnt nx = tr[0];
        for (int i2 = 0; i2 < n2; i2++) {
            const TileEnt cur = nx;
            const int k = (int)(cur.k >> 8);
            nx = ent_at(tr, min(i2 + 1, capS - 1));
            const bool on = __builtin_amdgcn_inverse_ballot_w64(cur.on);
            const bool band = __builtin_amdgcn_inverse_ballot_w64(cur.band);
            Rec r;
            f8v eb;
            load_entry<FAST, true>(rec, rec_off((uint32_t)k), cur.k, r, eb);
            float cov;
            Geo g;
            band_cov<FAST>(r, eb, tg.p, cur.k, cur.band, band, rsig, sig, g, cov);
            const float w = r.f(R_A) * cov;
            float part[NP];
            grad_pixel<PLAIN>(r, on, band, cur.band != 0, w, cov, g, tg.p, rsig, st, part);
            if (DET)
                reduce_entry(part, tw, accs + (k - k0) * NP, lane);
            else if (cur.band != 0)
                reduce_entry_global(part, tw, grads + (size_t)k * NP, lane);
            else
                reduce_entry_global_cw(part, tw, grads + (size_t)k * NP, lane);
        }
    };
    if (plain)
        sweep(std::true_type{});
    else
        sweep(std::false_type{});
    if (DET) {
        // the tile's partial rows of this segment's triangles
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
        float* prow = a.partials + ((size_t)tg.tile * T + k0) * NP;
        for (int j = lane; j < (k1 - k0) * NP; j += 64) prow[j] = accs[j];
    }
}

// Lane `lane`'s share of a scene's block loss sums: blocks lane, lane + 64, ...
// added in turn to a double, each block's PER partials summed in order first.
// The loads of SUM_UNROLL blocks are issued before any of them is added, so up
// to 64 SUM_UNROLL blocks take one round of loads.
constexpr int SUM_UNROLL = 8;
template <int PER>
__device__ inline double lane_block_losses(const double* __restrict__ pl, int nblk, int lane) {
    double l = 0.0;
    for (int r0 = lane; r0 < nblk; r0 += 64 * SUM_UNROLL) {
        double part[SUM_UNROLL][PER];
#pragma unroll
        for (int u = 0; u < SUM_UNROLL; u++) {
            const int r = min(r0 + 64 * u, nblk - 1);
#pragma unroll
            for (int q = 0; q < PER; q++) part[u][q] = pl[(size_t)r * PER + q];
        }
#pragma unroll
        for (int u = 0; u < SUM_UNROLL; u++) {
            double lb = part[u][0];
#pragma unroll
            for (int q = 1; q < PER; q++) lb += part[u][q];
            // A select, not a branch, so that every load above is issued first.
            l = r0 + 64 * u < nblk ? l + lb : l;
        }
    }
    return l;
}

// base[r * stride] for r in [r0, r1) added in order to 0, BATCH loads (ROW_BATCH, or FIT_ROW_BATCH in fit_step)
// issued before they are added.
constexpr int ROW_BATCH = 8, FIT_ROW_BATCH = 32;
template <int BATCH = ROW_BATCH>
__device__ inline float sum_rows_in_order(const float* __restrict__ base, size_t stride, int r0, int r1) {
    float acc = 0.0f;
    for (int rr = r0; rr < r1; rr += BATCH) {
        float v[BATCH];
#pragma unroll
        for (int u = 0; u < BATCH; u++) v[u] = base[(size_t)min(rr + u, r1 - 1) * stride];
#pragma unroll
        for (int u = 0; u < BATCH; u++) acc = rr + u < r1 ? acc + v[u] : acc;
    }
    return acc;
}

// The per-item loss (canvas.rs:45-58) from the fused kernel's per-block sums,
// one wave per scene, in the order of backward_kernel's sum (the lanes' shares,
// then the lanes summed).
// PER: partials per block, 1 or WAVES (per tile, summed in wave order first).
template <int PER>
__global__ __launch_bounds__(64) void sum_losses(const double* __restrict__ partial_loss, int nblk, double npix3,
                                                 float* __restrict__ losses, const int* __restrict__ halt) {
    if (halt && *halt >= 0) return;
    const int b = (int)blockIdx.x, lane = (int)threadIdx.x;
    const double l = wave_sum_f64(lane_block_losses<PER>(partial_loss + (size_t)b * nblk * PER, nblk, lane));
    if (lane == 0) losses[b] = (float)(l / npix3);
}

// Sum the per-block partial rows of each scene in block order. One block per
// (scene, 64 columns); its 16 waves each sum a contiguous range of rows
// (sum_rows_in_order), and the ranges are combined in row order.
constexpr int RED_WAVES = 16;
// loss_per: loss partials per block (1, or WAVES when the rows and partials
// are per tile: fused_seg_kernel), summed per block first as sum_losses does.
__device__ inline double scene_loss(const double* __restrict__ pl, int nrows, int loss_per, int lane) {
    return loss_per == WAVES ? lane_block_losses<WAVES>(pl, nrows / WAVES, lane)
                             : lane_block_losses<1>(pl, nrows, lane);
}
__global__ __launch_bounds__(RED_WAVES * 64) void reduce_partials(const float* __restrict__ partials,
                                                                  const double* __restrict__ partial_loss,
                                                                  int nblk, int loss_per, int T, double npix3,
                                                                  float* __restrict__ grads,
                                                                  float* __restrict__ losses,
                                                                  const int* __restrict__ halt) {
    __shared__ float part[RED_WAVES][64];
    if (halt && *halt >= 0) return;
    const int b = blockIdx.y;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int cols = T * NP;
    const int col = blockIdx.x * 64 + lane;
    float acc = 0.0f;
    if (col < cols)
        acc = sum_rows_in_order(partials + (size_t)b * nblk * cols + col, cols, (nblk * wave) / RED_WAVES,
                                (nblk * (wave + 1)) / RED_WAVES);
    part[wave][lane] = acc;
    __syncthreads();
    if (wave == 0 && col < cols) {
        float v = part[0][lane];
        for (int q = 1; q < RED_WAVES; q++) v += part[q][lane];
        grads[(size_t)b * cols + col] = v;
    }
    if (losses && blockIdx.x == 0 && wave == 0) {
        const double s = wave_sum_f64(scene_loss(partial_loss + (size_t)b * nblk, nblk, loss_per, lane));
        if (lane == 0) losses[b] = (float)(s / npix3);
    }
}

// optim.rs:40-60 then (optionally) fit.rs:399-424, one thread per parameter.
// bc1 / bc2 are the bias corrections 1 - beta^t, formed on the host with the
// reference's powi.
__global__ void adam_project(float* __restrict__ params, const float* __restrict__ grads,
                             float* __restrict__ m, float* __restrict__ v, const float* __restrict__ lr,
                             int n, float beta1, float beta2, float eps, float bc1, float bc2, int project) {
    int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    float g = grads[i];
    float mi = beta1 * m[i] + (1.0f - beta1) * g;
    float vi = beta2 * v[i] + (1.0f - beta2) * g * g;
    m[i] = mi;
    v[i] = vi;
    float m_hat = mi / bc1;
    float v_hat = vi / bc2;
    float pv = params[i] - lr[i] * m_hat / (sqrtf(v_hat) + eps);
    if (project) {
        int j = i % NP;
        if (pv != pv) pv = 0.5f;
        if (j < 6) pv = rust_clamp(pv, -0.25f, 1.25f);
        else if (j < 9) pv = rust_clamp(pv, 0.0f, 1.0f);
        else pv = rust_clamp(pv, 1e-3f, 0.999f);
    }
    params[i] = pv;
}

// The fit loop's iteration tail in one kernel (B = 1): reduce_partials' sums,
// then the iteration's bookkeeping (fit.rs:243-288: divergence, loss record,
// best, patience), the best snapshot before the update, and Adam
// (optim.rs:40-60) with the projection (fit.rs:399-424), for the parameters
// of triangles [FIT_TRIS x, FIT_TRIS x + FIT_TRIS) of block x; with ft.rec,
// then those triangles' records for the next iteration. Every block sums the
// loss partials in reduce_partials' order and decides from st[iter & 1], so
// all take the same decision; block 0 records it in st[(iter + 1) & 1] (and
// the loss, the loss history and `halt`). An iteration launched after the
// stop only carries the state forward (its raster kernels returned at entry).
__global__ __launch_bounds__(RED_WAVES * 64) void fit_step(const float* __restrict__ partials,
                                                           const double* __restrict__ partial_loss, int nblk,
                                                           int loss_per, int T, double npix3, FitTail ft) {
    __shared__ float part[RED_WAVES][64];
    __shared__ float newp[FIT_TRIS * NP];  // the block's parameters after the update
    __shared__ int decision;
    const FitState cur = ft.st[ft.iter & 1];
    FitState* const nxt = ft.st + ((ft.iter + 1) & 1);
    // The stop is read from the state, not from `halt`, which block 0 of this
    // kernel may already have set while another block starts.
    if (cur.stop >= 0) {
        if (blockIdx.x == 0 && threadIdx.x == 0) *nxt = cur;
        return;
    }
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int cols = T * NP;
    // FIT_TRIS whole triangles per block (lanes 60-63 idle)
    const int col = blockIdx.x * (FIT_TRIS * NP) + lane;
    const bool mine = lane < FIT_TRIS * NP && col < cols;
    // Wave 0's Adam operands, loaded here so that they arrive with the sums
    // (only this thread writes column col in this kernel).
    float p0 = 0.0f, m0 = 0.0f, v0 = 0.0f, lr0 = 0.0f;
    if (wave == 0 && mine) {
        p0 = ft.params[col];
        m0 = ft.m[col];
        v0 = ft.v[col];
        lr0 = ft.lr[col];
    }
    float acc = 0.0f;
    if (mine)
        // the fit's rows (a few hundred tiles) in one round of loads per wave
        acc = sum_rows_in_order<FIT_ROW_BATCH>(partials + col, cols, (nblk * wave) / RED_WAVES,
                                               (nblk * (wave + 1)) / RED_WAVES);
    part[wave][lane] = acc;
    if (wave == 1) {
        const double s = wave_sum_f64(scene_loss(partial_loss, nblk, loss_per, lane));
        if (lane == 0) {
            // fit.rs:243-288
            const float L = (float)(s / npix3);
            FitState n = cur;
            int d = -1;
            if (!isfinite(L)) {
                n.stop = STOP_DIVERGED;
            } else {
                const bool improved = L + ft.min_delta < cur.best_loss;
                if (improved) {
                    n.best_loss = L;
                    n.best_iter = ft.iter;
                    n.since = 0;
                } else {
                    n.since = cur.since + 1;
                }
                n.n_losses = cur.n_losses + 1;
                const bool converged = ft.patience >= 0 && (long long)n.since >= ft.patience;
                if (converged) n.stop = STOP_CONVERGED;
                d = (improved ? 1 : 0) | (converged ? 2 : 0);
            }
            decision = d;
            if (blockIdx.x == 0) {
                *ft.loss = L;
                if (d >= 0) ft.losses_out[cur.n_losses] = L;
                *nxt = n;
                if (n.stop >= 0) *ft.halt = n.stop;
            }
        }
    }
    __syncthreads();
    const int d = decision;
    if (wave == 0 && mine) {
        float g = part[0][lane];
        for (int q = 1; q < RED_WAVES; q++) g += part[q][lane];
        ft.grads[col] = g;
        float pn = p0;  // the parameter after this iteration
        if (d >= 0) {
            if (d & 1) ft.best[col] = p0;
            if (!(d & 2)) {
                const float mi = ft.beta1 * m0 + (1.0f - ft.beta1) * g;
                const float vi = ft.beta2 * v0 + (1.0f - ft.beta2) * g * g;
                ft.m[col] = mi;
                ft.v[col] = vi;
                float pv = p0 - lr0 * (mi / ft.bc1) / (sqrtf(vi / ft.bc2) + ft.eps);
                const int j = col % NP;
                if (pv != pv) pv = 0.5f;
                if (j < 6) pv = rust_clamp(pv, -0.25f, 1.25f);
                else if (j < 9) pv = rust_clamp(pv, 0.0f, 1.0f);
                else pv = rust_clamp(pv, 1e-3f, 0.999f);
                ft.params[col] = pv;
                pn = pv;
            }
        }
        newp[lane] = pn;
    }
    if (ft.rec) {
        // the next iteration's records of the block's triangles, as
        // setup_records would make them from the updated parameters (handed
        // over in LDS instead of read back)
        __syncthreads();
        const int k = blockIdx.x * FIT_TRIS + (int)threadIdx.x;
        if ((int)threadIdx.x < FIT_TRIS && k < T)
            setup_from(newp + threadIdx.x * NP, (size_t)k, ft.W, ft.H, ft.sigma_next, SETUP_TAPE, ft.rec);
    }
}

// Grid-stride fill with zeros.
__global__ __launch_bounds__(256) void zero_floats(float* __restrict__ p, size_t n) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
        p[i] = 0.0f;
}

// ---------------------------------------------------------------- sRGB bytes

// canvas.rs:100-105 encode_srgb, one value per thread: the byte is the number
// of thresholds t_1 < ... < t_255 at or below v (t_k the smallest linear value
// the reference encodes to k), found by an 8-step binary search in LDS. The
// reference's encoding is monotonic in v on [0, 1] (checked over every float
// there) and constant outside it after its clamp, so the count is its byte;
// NaN compares false everywhere and gives 0, as its saturating cast does.
__global__ __launch_bounds__(256) void encode_srgb_kernel(const float* __restrict__ in, int64_t n,
                                                          uint8_t* __restrict__ out, SrgbTable thr) {
    __shared__ float t[256];
    t[threadIdx.x] = thr.v[threadIdx.x];
    __syncthreads();
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
        const float v = in[i];
        int b = 0;
#pragma unroll
        for (int step = 128; step >= 1; step >>= 1) b += (t[b + step] <= v) ? step : 0;
        out[i] = (uint8_t)b;
    }
}

// canvas.rs:108-115 decode_srgb: a lookup in the table of all 256 values.
__global__ __launch_bounds__(256) void decode_srgb_kernel(const uint8_t* __restrict__ in, int64_t n,
                                                          float* __restrict__ out, SrgbTable val) {
    __shared__ float t[256];
    t[threadIdx.x] = val.v[threadIdx.x];
    __syncthreads();
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) out[i] = t[in[i]];
}

static dim3 stream_grid(int64_t n) {
    // enough blocks to fill the chip a few times over; the loops stride the rest
    const int64_t blocks = (n + 255) / 256;
    return dim3((unsigned)(blocks < 8192 ? (blocks > 0 ? blocks : 1) : 8192));
}

hipError_t launch_encode_srgb(const float* in, int64_t n, uint8_t* out, const SrgbTable& thresholds, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    launch_k(encode_srgb_kernel, stream_grid(n), dim3(256), 0, s, in, n, out, thresholds);
    return hipGetLastError();
}

hipError_t launch_decode_srgb(const uint8_t* in, int64_t n, float* out, const SrgbTable& values, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    launch_k(decode_srgb_kernel, stream_grid(n), dim3(256), 0, s, in, n, out, values);
    return hipGetLastError();
}

// ---------------------------------------------------------------- launchers

hipError_t launch_fit_step(const float* partials, const double* partial_loss, int nblk, int loss_per, int T,
                           double npix3, const FitTail& ft, hipStream_t s) {
    if (loss_per != 1 && (loss_per != WAVES || nblk % WAVES != 0)) return hipErrorInvalidValue;
    const dim3 grid((unsigned)((T + FIT_TRIS - 1) / FIT_TRIS));
    launch_k(fit_step, grid, dim3(RED_WAVES * 64), 0, s, partials, partial_loss, nblk, loss_per, T, npix3, ft);
    return hipGetLastError();
}

hipError_t launch_setup(const float* params, int B, int T, int W, int H, float sigma, int setup_mode,
                        float* rec, float* zero_grads, hipStream_t s, const float* bg_src, float* bg_dst,
                        const OrderArgs& o, const int* halt, RecordHead* head, const RecordHead& head_val,
                        double* pending, int npending) {
    if (B == 0 || (T == 0 && !bg_dst && !o.perm && !head && !pending)) return hipSuccess;
    if (o.perm && (o.gy + 1) * (o.gx + 1) > ORD_MAX_CELLS) return hipErrorInvalidValue;
    // without an order, small workgroups spread the triangles over more CUs;
    // with one, a last workgroup per scene makes it
    const int n = o.perm ? SETUP_THREADS : 64;
    const int per = o.perm ? SETUP_REC_PER : n;  // records per workgroup (setup_records' `per`)
    const int gx = min((T + per - 1) / per, 65534) + (o.perm || T == 0 ? 1 : 0);
    OrderArgs oa = o;
    const float cs = (float)(1 << o.shift);
    oa.r_h = 1.0f / (float)H;
    oa.cell_h = cs * oa.r_h;
    oa.w_cells = (float)W / cs;
    oa.c0_off = (0.5f - cs) / cs;
    oa.c1_off = -0.5f / cs;
    launch_k(setup_records, dim3(B, gx), dim3(n), 0, s, params, T, W, H, sigma, setup_mode, rec,
                       zero_grads, bg_src, bg_dst, oa, halt, head, head_val, pending, npending);
    return hipGetLastError();
}

hipError_t launch_zero(float* p, size_t n, hipStream_t s) {
    if (n == 0) return hipSuccess;
    const size_t blocks = (n + 255) / 256;
    launch_k(zero_floats, dim3((unsigned)(blocks < 4096 ? blocks : 4096)), dim3(256), 0, s, p, n);
    return hipGetLastError();
}

dim3 raster_grid(int B, int W, int H) {
    return dim3((W + 2 * TILE - 1) / (2 * TILE), (H + 2 * TILE - 1) / (2 * TILE), B);
}

template <int MODE, bool FAST, bool CKPT = false>
static hipError_t launch_forward_t(const RasterArgs& a, hipStream_t s) {
    launch_k((forward_kernel<MODE, FAST, CKPT>), raster_grid(a.B, a.W, a.H), dim3(WAVES * 64), 0, s, a,
                       a.rec);
    return hipGetLastError();
}

template <int MODE, bool FAST>
static hipError_t launch_forward_c(const RasterArgs& a, hipStream_t s) {
    return (a.ckpt && a.nseg > 1) ? launch_forward_t<MODE, FAST, true>(a, s) : launch_forward_t<MODE, FAST, false>(a, s);
}

hipError_t launch_forward(int mode, bool fast, const RasterArgs& a, hipStream_t s) {
    if (mode == MODE_RENDER)
        return fast ? launch_forward_t<MODE_RENDER, true>(a, s) : launch_forward_t<MODE_RENDER, false>(a, s);
    if (mode == MODE_LOSS)
        return fast ? launch_forward_c<MODE_LOSS, true>(a, s) : launch_forward_c<MODE_LOSS, false>(a, s);
    if (mode == MODE_RECORD)
        return fast ? launch_forward_t<MODE_RECORD, true>(a, s) : launch_forward_t<MODE_RECORD, false>(a, s);
    return fast ? launch_forward_c<MODE_GRAD_IN, true>(a, s) : launch_forward_c<MODE_GRAD_IN, false>(a, s);
}

template <int MODE, bool FAST, bool REBUILD, bool DET>
static hipError_t launch_backward_t(const RasterArgs& a, hipStream_t s) {
    const bool split = !REBUILD && !DET && a.perm_bwd && a.nseg > 1;
    const dim3 grid = split ? dim3((unsigned)(a.B * (a.gx * a.gy + a.nsplit * (a.nseg - 1)))) : raster_grid(a.B, a.W, a.H);
    launch_k((backward_kernel<MODE, FAST, REBUILD, DET>), grid, dim3(WAVES * 64), 0, s, a, a.rec, a.tl_ent);
    return hipGetLastError();
}

template <int MODE, bool FAST, bool REBUILD>
static hipError_t launch_backward_d(const RasterArgs& a, hipStream_t s) {
    return a.deterministic ? launch_backward_t<MODE, FAST, REBUILD, true>(a, s)
                           : launch_backward_t<MODE, FAST, REBUILD, false>(a, s);
}

template <int MODE, bool FAST>
static hipError_t launch_backward_r(bool rebuild, const RasterArgs& a, hipStream_t s) {
    return rebuild ? launch_backward_d<MODE, FAST, true>(a, s) : launch_backward_d<MODE, FAST, false>(a, s);
}

hipError_t launch_backward(int mode, bool fast, bool rebuild, const RasterArgs& a, hipStream_t s) {
    if (mode == MODE_LOSS)
        return fast ? launch_backward_r<MODE_LOSS, true>(rebuild, a, s)
                    : launch_backward_r<MODE_LOSS, false>(rebuild, a, s);
    return fast ? launch_backward_r<MODE_GRAD_IN, true>(rebuild, a, s)
                : launch_backward_r<MODE_GRAD_IN, false>(rebuild, a, s);
}

template <int MODE, bool DET>
static void launch_fused_d(bool fast, const RasterArgs& a, dim3 grid, hipStream_t s) {
    if (fast)
        launch_k((fused_kernel<MODE, true, DET>), grid, dim3(WAVES * 64), 0, s, a, a.rec, a.tl_ent);
    else
        launch_k((fused_kernel<MODE, false, DET>), grid, dim3(WAVES * 64), 0, s, a, a.rec, a.tl_ent);
}

template <int MODE>
static void launch_fused_m(bool fast, const RasterArgs& a, dim3 grid, hipStream_t s) {
    if (a.segw) {
        // with the loss tail (not in the fixed-order mode), B more workgroups after the tiles
        const dim3 tiles(grid.x * grid.y * grid.z * WAVES +
                         (MODE == MODE_LOSS && !a.deterministic && a.loss_tail ? a.B : 0)),
            threads(SEG_WAVES * 64);
        const size_t lds = seg_lds_bytes(a.deterministic != 0, a.T);
        if (a.deterministic && fast)
            launch_k((fused_seg_kernel<MODE, true, true, SEG_WAVES>), tiles, threads, lds, s, a, a.rec, a.tl_ent);
        else if (a.deterministic)
            launch_k((fused_seg_kernel<MODE, false, true, SEG_WAVES>), tiles, threads, lds, s, a, a.rec, a.tl_ent);
        else if (fast)
            launch_k((fused_seg_kernel<MODE, true, false, SEG_WAVES>), tiles, threads, lds, s, a, a.rec, a.tl_ent);
        else
            launch_k((fused_seg_kernel<MODE, false, false, SEG_WAVES>), tiles, threads, lds, s, a, a.rec, a.tl_ent);
        return;
    }
    if (a.deterministic) {
        launch_fused_d<MODE, true>(fast, a, grid, s);
        return;
    }
    // with the loss tail, B more workgroups after the tiles. With an order of
    // tiles: scenes in x and ranks in y (no division in the kernel), the loss
    // tail the last row.
    const bool tail = MODE == MODE_LOSS && a.loss_tail;
    const unsigned nt = grid.x * grid.y * WAVES;  // tiles per scene
    const bool xy = a.perm_bwd && a.perm_tiles && nt + 1 <= 65535u;
    const dim3 tiles = xy ? dim3((unsigned)a.B, nt + (tail ? 1u : 0u)) : dim3(nt * grid.z + (tail ? a.B : 0));
    RasterArgs b = a;
    b.tdiv_m = xy ? (uint32_t)((0xFFFFFFFFull + 2ull * a.gx) / (2ull * a.gx)) : 0u;
    const bool rows = a.rows && a.row_n;
    if (fast && rows)
        launch_k((fused_tile_kernel<MODE, true, true>), tiles, dim3(64), 0, s, b, b.rec, b.tl_ent);
    else if (fast)
        launch_k((fused_tile_kernel<MODE, true, false>), tiles, dim3(64), 0, s, b, b.rec, b.tl_ent);
    else if (rows)
        launch_k((fused_tile_kernel<MODE, false, true>), tiles, dim3(64), 0, s, b, b.rec, b.tl_ent);
    else
        launch_k((fused_tile_kernel<MODE, false, false>), tiles, dim3(64), 0, s, b, b.rec, b.tl_ent);
}

hipError_t launch_fused(int mode, bool fast, const RasterArgs& a, hipStream_t s) {
    if ((size_t)a.B * a.H * a.W == 0) return hipSuccess;
    if ((mode != MODE_LOSS && mode != MODE_GRAD_IN) || a.cap2 < a.T || a.cap2 % 8 != 0 || a.nseg > 1)
        return hipErrorInvalidValue;
    if (a.segw && (a.segw != SEG_WAVES || a.T > SEG_MAX_T || a.cap2 % (8 * SEG_WAVES) != 0 ||
                   a.cap2 / SEG_WAVES < (a.T + SEG_WAVES - 1) / SEG_WAVES))
        return hipErrorInvalidValue;
    const dim3 grid = raster_grid(a.B, a.W, a.H);
    if (mode == MODE_LOSS)
        launch_fused_m<MODE_LOSS>(fast, a, grid, s);
    else
        launch_fused_m<MODE_GRAD_IN>(fast, a, grid, s);
    return hipGetLastError();
}

hipError_t launch_sum_losses(const double* partial_loss, int B, int nblk, int per, double npix3, float* losses,
                             hipStream_t s, const int* halt) {
    if (B == 0) return hipSuccess;
    if (nblk <= 0) return hipErrorInvalidValue;
    if (per == WAVES)
        launch_k(sum_losses<WAVES>, dim3(B), dim3(64), 0, s, partial_loss, nblk, npix3, losses, halt);
    else if (per == 1)
        launch_k(sum_losses<1>, dim3(B), dim3(64), 0, s, partial_loss, nblk, npix3, losses, halt);
    else
        return hipErrorInvalidValue;
    return hipGetLastError();
}

hipError_t launch_reduce(const float* partials, const double* partial_loss, int B, int nblk, int loss_per, int T,
                         double npix3, float* grads, float* losses, hipStream_t s, const int* halt) {
    if (loss_per != 1 && (loss_per != WAVES || nblk % WAVES != 0)) return hipErrorInvalidValue;
    int cols = T * NP;
    dim3 grid((cols + 63) / 64 > 0 ? (cols + 63) / 64 : 1, B);
    launch_k(reduce_partials, grid, dim3(RED_WAVES * 64), 0, s, partials, partial_loss, nblk, loss_per, T,
                       npix3, grads, losses, halt);
    return hipGetLastError();
}

hipError_t launch_adam(float* params, const float* grads, float* m, float* v, const float* lr, int n,
                       float beta1, float beta2, float eps, float bc1, float bc2, int project,
                       hipStream_t s) {
    if (n == 0) return hipSuccess;
    launch_k(adam_project, dim3((n + 255) / 256), dim3(256), 0, s, params, grads, m, v, lr, n, beta1,
                       beta2, eps, bc1, bc2, project);
    return hipGetLastError();
}

}  // namespace drh
