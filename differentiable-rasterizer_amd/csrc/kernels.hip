// Soft-triangle rasterizer kernels for gfx950 (MI355X).
//
// Semantics follow the reference CPU path (crates/diffrast/src/raster.rs,
// grad.rs, optim.rs, fit.rs); the work decomposition is this file's own:
//
//   setup_records : one thread per (scene, triangle). Computes the padded
//                   integer bounding box exactly as raster.rs:144-168 does,
//                   the edge vectors and the data for a conservative
//                   far-outside / deep-inside classification.
//   raster_kernel : one wave64 per 8x8 pixel tile, four tiles per block.
//                   Each wave compacts the triangles touching its tile into an
//                   ordered LDS list (ballot + mbcnt), then walks it with the
//                   triangle record in SGPRs (scalar loads). Sweep 1 composites
//                   in scene order (raster.rs:46-68). The backward is a second
//                   sweep in the same order: the gradient reaching layer k,
//                   d_canvas * prod_{j>k}(1 - w_j) (grad.rs:162-169), is formed
//                   as a ratio of transmittance products instead of being
//                   peeled off a tape. Per-triangle gradients are wave-reduced
//                   with DPP, accumulated per wave in LDS and written as one
//                   partial row per block.
//   reduce_partials : fixed-order sum of the partial rows, so gradients and
//                   losses are bit-reproducible run to run.
//   adam_project  : optim.rs:40-60 followed by fit.rs:399-424, elementwise.
//
// The whole file is compiled with -ffp-contract=off: every a*b+c below that is
// written without an explicit fmaf rounds twice, as the reference does. FMAs
// appear only where the reference's rounding cannot change a result beyond
// the stated tolerance (gradient assembly, conservative classification).

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "kernels.h"

namespace drh {

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

__global__ void setup_records(const float* __restrict__ params, int n_tri, int W, int H,
                              float sigma, int tape_mode, float* __restrict__ rec) {
    int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n_tri) return;
    const float* p = params + (size_t)i * NP;
    float* r = rec + (size_t)i * REC;

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
    bool live = box_ok && (tape_mode ? (alpha > 0.0f) : !(alpha <= 0.0f));

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
    ri[R_FLAGS] = (live ? F_LIVE : 0) | (active ? F_ACTIVE : 0) | (fast && live ? F_FAST : 0);
    r[R_SPARE] = 0.0f;
    for (int j = 0; j < 6; j++) r[R_E + j] = e[j];
    for (int j = 0; j < 3; j++) r[R_LEN2 + j] = len2[j];
    for (int j = 0; j < 3; j++) r[R_RLEN2 + j] = rlen2[j];
    for (int j = 0; j < 6; j++) r[R_N + j] = n[j];
    for (int j = 0; j < 3; j++) r[R_OFF + j] = off[j];
    // far outside: true distance > 20 sigma  =>  w <= alpha * sigmoid(-19.99) < MIN_WEIGHT
    // deep inside: distance to the edge > 18 sigma  =>  sigmoid rounds to exactly 1.0f
    r[R_FAR] = 20.0f * sig + slack;
    r[R_DEEP] = -(18.0f * sig + slack);
    for (int j = R_DEEP + 1; j < REC; j++) r[j] = 0.0f;
}

// ---------------------------------------------------------------- per-pair math

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
// With `fast` (a triangle of moderate coordinates in a FAST build) the
// projection quotient comes from a refined reciprocal and the square root from
// the hardware instruction; otherwise both are IEEE operations.
struct Geo {
    float sd;      // signed distance, positive inside
    float dist;    // |nearest segment distance|
    float t;       // clamped projection parameter on the nearest edge
    float ax, ay;  // first vertex of the nearest edge
    float ex, ey;  // its edge vector b - a
    int edge;      // nearest edge index, first minimum wins (grad.rs:236-242)
};

__device__ inline Geo geometry(const float* __restrict__ r, Pix p, bool fast) {
    float apx[3], apy[3];
    for (int j = 0; j < 3; j++) {
        apx[j] = p.px - r[R_V + 2 * j];
        apy[j] = p.py - r[R_V + 2 * j + 1];
    }
    float c[3];
    for (int j = 0; j < 3; j++) c[j] = r[R_E + 2 * j] * apy[j] - r[R_E + 2 * j + 1] * apx[j];
    bool inside = (c[0] >= 0.0f && c[1] >= 0.0f && c[2] >= 0.0f) ||
                  (c[0] <= 0.0f && c[1] <= 0.0f && c[2] <= 0.0f);
    Geo g;
    float best = INFINITY;
    float d2v[3], tv[3];
    g.edge = 0;
    g.t = 0.0f;
    for (int j = 0; j < 3; j++) {
        float ex = r[R_E + 2 * j], ey = r[R_E + 2 * j + 1];
        float dot = apx[j] * ex + apy[j] * ey;
        float t;
        if (fast) {
            // dot / len2 as the reference rounds it: with rlen2 the correctly
            // rounded 1/len2, one residual step q0 + (dot - q0*len2)*rlen2
            // gives the correctly rounded quotient (Markstein). The nearest
            // point then matches the reference bit for bit; an ulp off in t
            // moves the distance of an on-edge pixel by ~|e|*6e-8, which 1/sigma
            // magnifies into visible coverage error at small sigma.
            float rl = r[R_RLEN2 + j];
            float q0 = dot * rl;
            float res = fmaf(-q0, r[R_LEN2 + j], dot);
            t = __builtin_amdgcn_fmed3f(fmaf(res, rl, q0), 0.0f, 1.0f);
        } else {
            float len2 = r[R_LEN2 + j];
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
    // The reference compares the square-rooted distances (grad.rs:236-242):
    // an earlier edge whose d2 is an ulp or two above the minimum can round to
    // the same distance and then wins. That is routine for overlapping edges
    // of a collinear triangle, so such near ties are re-checked with the
    // correctly rounded sqrt the reference uses.
    for (int j = 0; j < 2; j++) {
        if (j < g.edge && d2v[j] <= best * 1.0000005f && sqrtf(d2v[j]) == sqrtf(best)) {
            g.edge = j;
            g.t = tv[j];
            break;
        }
    }
    // selects rather than a lane-varying index into the (scalar) record
    const int ed = g.edge;
    g.ax = ed == 0 ? r[R_V + 0] : (ed == 1 ? r[R_V + 2] : r[R_V + 4]);
    g.ay = ed == 0 ? r[R_V + 1] : (ed == 1 ? r[R_V + 3] : r[R_V + 5]);
    g.ex = ed == 0 ? r[R_E + 0] : (ed == 1 ? r[R_E + 2] : r[R_E + 4]);
    g.ey = ed == 0 ? r[R_E + 1] : (ed == 1 ? r[R_E + 3] : r[R_E + 5]);
    // sqrt is monotone, so sqrt(min d2) == min sqrt(d2) (raster.rs:97-99).
    g.dist = fast ? __builtin_amdgcn_sqrtf(best) : sqrtf(best);
    g.sd = inside ? g.dist : -g.dist;
    return g;
}

// ---------------------------------------------------------------- wave reduction

// Full wave64 sum, valid in lane 63: xor1, xor2 (quad_perm), half-row and row
// mirrors give every lane its row sum; row_bcast15 / row_bcast31 fold the rows.
template <int ctrl, int rmask>
__device__ inline float dpp_add(float v) {
    return v + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), ctrl, rmask, 0xF, false));
}
__device__ inline float wave_sum_to_lane63(float v) {
    v = dpp_add<0xB1, 0xF>(v);   // quad_perm [1,0,3,2]
    v = dpp_add<0x4E, 0xF>(v);   // quad_perm [2,3,0,1]
    v = dpp_add<0x141, 0xF>(v);  // row_half_mirror
    v = dpp_add<0x140, 0xF>(v);  // row_mirror
    v = dpp_add<0x142, 0xA>(v);  // row_bcast15 into rows 1 and 3
    v = dpp_add<0x143, 0xC>(v);  // row_bcast31 into rows 2 and 3
    return v;
}
__device__ inline double wave_sum_f64(double v) {
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

// ---------------------------------------------------------------- main kernel

// LDS layout per block.
template <int MODE>
struct Smem {
    uint32_t list[WAVES][CH];                  // (k_local << 2) | class
    float acc[MODE == MODE_RENDER ? 1 : WAVES][MODE == MODE_RENDER ? 1 : CH * NP];
    double loss[WAVES];
};

enum : uint32_t { CLS_PARTIAL = 1, CLS_FULL = 2 };

// Builds this wave's ordered list of triangles in [k0, k1) that can touch its
// tile, with a class per entry: FULL when every tile pixel is inside the
// triangle's box and deep inside the triangle, else PARTIAL.
__device__ inline int build_list(const float* __restrict__ rec, int k0, int k1, int tx0, int ty0,
                                 int tx1, int ty1, float cx0, float cy0, float cx1, float cy1,
                                 uint32_t* list, int lane) {
    int count = 0;
    for (int base = k0; base < k1; base += 64) {
        int k = base + lane;
        uint32_t cls = 0;
        if (k < k1) {
            const float* r = rec + (size_t)k * REC;
            const int* ri = reinterpret_cast<const int*>(r);
            int flags = ri[R_FLAGS];
            int bx0 = ri[R_BOX], by0 = ri[R_BOX + 1], bx1 = ri[R_BOX + 2], by1 = ri[R_BOX + 3];
            if ((flags & F_LIVE) && tx0 < bx1 && bx0 < tx1 && ty0 < by1 && by0 < ty1) {
                cls = CLS_PARTIAL;
                if (flags & F_FAST) {
                    float far = r[R_FAR], deep = r[R_DEEP];
                    bool culled = false, all_deep = true;
                    for (int j = 0; j < 3; j++) {
                        float nx = r[R_N + 2 * j], ny = r[R_N + 2 * j + 1], o = r[R_OFF + j];
                        float l00 = fmaf(cx0, nx, fmaf(cy0, ny, -o));
                        float l10 = fmaf(cx1, nx, fmaf(cy0, ny, -o));
                        float l01 = fmaf(cx0, nx, fmaf(cy1, ny, -o));
                        float l11 = fmaf(cx1, nx, fmaf(cy1, ny, -o));
                        float lmin = fminf(fminf(l00, l10), fminf(l01, l11));
                        float lmax = fmaxf(fmaxf(l00, l10), fmaxf(l01, l11));
                        culled = culled || (lmin > far);
                        all_deep = all_deep && (lmax < deep);
                    }
                    bool in_box = bx0 <= tx0 && tx1 <= bx1 && by0 <= ty0 && ty1 <= by1;
                    if (culled) cls = 0;
                    else if (all_deep && in_box) cls = CLS_FULL;
                }
            }
        }
        uint64_t mask = __ballot(cls != 0);
        if (cls != 0) {
            int pos = count + (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(mask >> 32),
                                                              __builtin_amdgcn_mbcnt_lo((uint32_t)mask, 0));
            list[pos] = ((uint32_t)(k - k0) << 2) | cls;
        }
        count += (int)__popcll(mask);
    }
    return count;
}

// Per-pixel weight of one triangle: returns false when the pair is skipped
// (outside the box, classified far outside, or w <= MIN_WEIGHT). For the band
// pairs it also returns the geometry the backward needs.
template <bool FAST, bool NEED_GEO>
__device__ inline bool pair_weight(const float* __restrict__ r, uint32_t cls, int x, int y, Pix p,
                                   bool valid, float& w, float& cov, bool& band, Geo& g, float rsig,
                                   float sig) {
    band = false;
    if (!valid) return false;
    float alpha = r[R_A];
    if (cls == CLS_FULL) {
        cov = 1.0f;
        w = alpha;
    } else {
        const int* ri = reinterpret_cast<const int*>(r);
        if (!(x >= ri[R_BOX] && x < ri[R_BOX + 2] && y >= ri[R_BOX + 1] && y < ri[R_BOX + 3]))
            return false;
        bool exact = true;
        if (ri[R_FLAGS] & F_FAST) {
            float l0 = fmaf(p.px, r[R_N + 0], fmaf(p.py, r[R_N + 1], -r[R_OFF + 0]));
            float l1 = fmaf(p.px, r[R_N + 2], fmaf(p.py, r[R_N + 3], -r[R_OFF + 1]));
            float l2 = fmaf(p.px, r[R_N + 4], fmaf(p.py, r[R_N + 5], -r[R_OFF + 2]));
            float lm = fmaxf(fmaxf(l0, l1), l2);
            if (lm > r[R_FAR]) return false;
            if (lm < r[R_DEEP]) {
                cov = 1.0f;
                w = alpha;
                exact = false;
            }
        }
        if (exact) {
            g = geometry(r, p, FAST && (ri[R_FLAGS] & F_FAST));
            float x_ = FAST ? g.sd * rsig : g.sd / sig;
            cov = sigmoid_f<FAST>(x_);
            w = alpha * cov;
            band = true;
        }
    }
    return !(w <= MIN_WEIGHT);
}

struct Trans {
    float q;  // product of the nonzero (1 - w) factors, kept in [2^-64, 1]
    int z;    // number of zero factors (w == 1 exactly)
    int e;    // number of 2^64 rescalings applied to q
};

__device__ inline void trans_mul(Trans& t, float f) {
    if (f == 0.0f) {
        t.z += 1;
    } else {
        t.q *= f;
        if (t.q < 5.421010862427522e-20f) {  // 2^-64
            t.q *= 1.8446744073709552e19f;   // 2^64
            t.e += 1;
        }
    }
}

// prod_{j>k} (1 - w_j) from the totals and the prefix through k.
__device__ inline float trans_suffix(const Trans& total, const Trans& prefix) {
    if (total.z != prefix.z) return 0.0f;
    float ratio = total.q * __builtin_amdgcn_rcpf(prefix.q);
    return ldexpf(ratio, -64 * (total.e - prefix.e));
}

template <int MODE, bool FAST>
__global__ __launch_bounds__(WAVES * 64) void raster_kernel(RasterArgs a) {
    __shared__ Smem<MODE> sm;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int b = blockIdx.z;
    const int W = a.W, H = a.H, T = a.T;
    const int tx0 = (blockIdx.x * 2 + (wave & 1)) * TILE;
    const int ty0 = (blockIdx.y * 2 + (wave >> 1)) * TILE;
    const int x = tx0 + (lane & 7), y = ty0 + (lane >> 3);
    const bool valid = x < W && y < H;
    const int tx1 = min(tx0 + TILE, W), ty1 = min(ty0 + TILE, H);
    const bool tile_live = tx0 < W && ty0 < H;

    // raster.rs:138-140 pixel centre, correctly rounded division.
    Pix p;
    p.px = ((float)x + 0.5f) / (float)W;
    p.py = ((float)y + 0.5f) / (float)H;
    // Corners of the tile's pixel-centre rectangle, for the list classification.
    float cx0 = ((float)tx0 + 0.5f) / (float)W, cy0 = ((float)ty0 + 0.5f) / (float)H;
    float cx1 = ((float)(tx1 - 1) + 0.5f) / (float)W, cy1 = ((float)(ty1 - 1) + 0.5f) / (float)H;

    const float sig = fmaxf(a.sigma, 1e-8f);
    const float rsig = 1.0f / sig;
    const float* __restrict__ rec = a.rec + (size_t)b * T * REC;
    const size_t pix = ((size_t)b * H + (valid ? y : 0)) * W + (valid ? x : 0);

    float col[3];
    col[0] = a.bg[b * 3 + 0];
    col[1] = a.bg[b * 3 + 1];
    col[2] = a.bg[b * 3 + 2];
    Trans tot = {1.0f, 0, 0};

    const int n_chunks = (T + CH - 1) / CH;
    int count = 0;

    // ---- sweep 1: composite in scene order (raster.rs:37-68)
    for (int c = 0; c < n_chunks; c++) {
        int k0 = c * CH, k1 = min(T, k0 + CH);
        if (tile_live)
            count = build_list(rec, k0, k1, tx0, ty0, tx1, ty1, cx0, cy0, cx1, cy1, sm.list[wave], lane);
        else
            count = 0;
        for (int i = 0; i < count; i++) {
            uint32_t ent = __builtin_amdgcn_readfirstlane(sm.list[wave][i]);
            int k = k0 + (int)(ent >> 2);
            const float* r = rec + (size_t)k * REC;
            float w, cov;
            bool band;
            Geo g;
            if (pair_weight<FAST, false>(r, ent & 3u, x, y, p, valid, w, cov, band, g, rsig, sig)) {
                float omw = 1.0f - w;
                for (int ch = 0; ch < 3; ch++) col[ch] = r[R_C + ch] * w + col[ch] * omw;
                if (MODE != MODE_RENDER) trans_mul(tot, omw);
            }
        }
    }

    if (MODE == MODE_RENDER) {
        if (valid) {
            a.out_img[pix * 3 + 0] = col[0];
            a.out_img[pix * 3 + 1] = col[1];
            a.out_img[pix * 3 + 2] = col[2];
        }
        return;
    }

    // ---- dL/dpixel (grad.rs:111-114) and the loss (canvas.rs:45-58)
    float g0[3] = {0.0f, 0.0f, 0.0f};
    if (MODE == MODE_LOSS) {
        double l = 0.0;
        if (valid) {
            float scale = 2.0f / (float)(3 * (size_t)W * H);
            for (int ch = 0; ch < 3; ch++) {
                float t = a.target[pix * 3 + ch];
                float d = col[ch] - t;
                l += (double)d * (double)d;
                g0[ch] = scale * (col[ch] - t);
            }
        }
        l = wave_sum_f64(l);
        if (lane == 0) sm.loss[wave] = l;
        if (a.out_img && valid) {
            a.out_img[pix * 3 + 0] = col[0];
            a.out_img[pix * 3 + 1] = col[1];
            a.out_img[pix * 3 + 2] = col[2];
        }
    } else {
        if (valid)
            for (int ch = 0; ch < 3; ch++) g0[ch] = a.grad_in[pix * 3 + ch];
    }

    // ---- sweep 2: gradients, again in scene order
    const size_t blk = ((size_t)b * gridDim.y + blockIdx.y) * gridDim.x + blockIdx.x;
    col[0] = a.bg[b * 3 + 0];
    col[1] = a.bg[b * 3 + 1];
    col[2] = a.bg[b * 3 + 2];
    Trans pre = {1.0f, 0, 0};
    float* accw = sm.acc[wave];

    for (int c = 0; c < n_chunks; c++) {
        int k0 = c * CH, k1 = min(T, k0 + CH);
        int nk = k1 - k0;
        for (int j = lane; j < nk * NP; j += 64) accw[j] = 0.0f;
        if (n_chunks > 1) {
            if (tile_live)
                count = build_list(rec, k0, k1, tx0, ty0, tx1, ty1, cx0, cy0, cx1, cy1, sm.list[wave], lane);
            else
                count = 0;
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");

        for (int i = 0; i < count; i++) {
            uint32_t ent = __builtin_amdgcn_readfirstlane(sm.list[wave][i]);
            int kl = (int)(ent >> 2);
            const float* r = rec + (size_t)(k0 + kl) * REC;
            float w = 0.0f, cov = 0.0f;
            bool band = false;
            Geo g;
            bool on = pair_weight<FAST, true>(r, ent & 3u, x, y, p, valid, w, cov, band, g, rsig, sig);
            float gc[3] = {0.0f, 0.0f, 0.0f}, ga = 0.0f;
            float gv[6] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
            if (on) {
                float omw = 1.0f - w;
                trans_mul(pre, omw);
                float tk = trans_suffix(tot, pre);
                float d_w = 0.0f;
                for (int ch = 0; ch < 3; ch++) {
                    float gk = g0[ch] * tk;  // d_canvas as the reference holds it at layer k
                    gc[ch] = gk * w;
                    d_w = fmaf(gk, r[R_C + ch] - col[ch], d_w);
                    col[ch] = r[R_C + ch] * w + col[ch] * omw;
                }
                const int* ri = reinterpret_cast<const int*>(r);
                if (ri[R_FLAGS] & F_ACTIVE) ga = d_w * cov;
                float d_cov = d_w * r[R_A];
                // grad.rs:252-268: vertex terms, zero exactly on the boundary.
                if (band && g.dist >= 1e-9f) {
                    // u = (pt - cp) / dist with cp = a + t (b - a), rounded as
                    // grad.rs:256-259 does: for a pixel within ~1e-7 of an edge
                    // the direction is set by these roundings, and the
                    // reference's gradient inherits them.
                    float inv = __builtin_amdgcn_rcpf(g.dist);
                    float cpx = g.ax + g.t * g.ex, cpy = g.ay + g.t * g.ey;
                    float ux = (p.px - cpx) * inv, uy = (p.py - cpy) * inv;
                    float sgn = g.sd > 0.0f ? 1.0f : -1.0f;
                    float chain = d_cov * cov * (1.0f - cov) * rsig * sgn;
                    float A = -(1.0f - g.t) * chain;  // onto the edge's first vertex
                    float Bc = -g.t * chain;           // onto its second vertex
                    float s0 = g.edge == 0 ? A : (g.edge == 2 ? Bc : 0.0f);
                    float s1 = g.edge == 1 ? A : (g.edge == 0 ? Bc : 0.0f);
                    float s2 = g.edge == 2 ? A : (g.edge == 1 ? Bc : 0.0f);
                    gv[0] = s0 * ux;
                    gv[1] = s0 * uy;
                    gv[2] = s1 * ux;
                    gv[3] = s1 * uy;
                    gv[4] = s2 * ux;
                    gv[5] = s2 * uy;
                }
            }
            // Uniform branches: skip the reduction when no lane contributed,
            // and the six vertex sums when no lane was in the band.
            if (__ballot(on) == 0) continue;
            float s[NP];
            s[6] = wave_sum_to_lane63(gc[0]);
            s[7] = wave_sum_to_lane63(gc[1]);
            s[8] = wave_sum_to_lane63(gc[2]);
            s[9] = wave_sum_to_lane63(ga);
            bool any_band = __ballot(band) != 0;
            if (any_band) {
                for (int j = 0; j < 6; j++) s[j] = wave_sum_to_lane63(gv[j]);
            }
            if (lane == 63) {
                float* dst = accw + kl * NP;
                if (any_band)
                    for (int j = 0; j < 6; j++) dst[j] += s[j];
                for (int j = 6; j < NP; j++) dst[j] += s[j];
            }
        }
        __syncthreads();
        // One partial row per block: the four waves' accumulators summed in
        // wave order, so the result does not depend on scheduling.
        float* prow = a.partials + (blk * T + k0) * NP;
        for (int j = threadIdx.x; j < nk * NP; j += WAVES * 64) {
            float v = sm.acc[0][j];
            for (int q = 1; q < WAVES; q++) v += sm.acc[q][j];
            prow[j] = v;
        }
        __syncthreads();
    }
    __syncthreads();  // also orders sm.loss when there are no chunks (T == 0)
    if (MODE == MODE_LOSS && threadIdx.x == 0) {
        double l = sm.loss[0];
        for (int q = 1; q < WAVES; q++) l += sm.loss[q];
        a.partial_loss[blk] = l;
    }
}

// Sum the per-block partial rows of each scene in block order. One block per
// (scene, 64 columns); its four waves split the rows and are combined in order.
__global__ __launch_bounds__(256) void reduce_partials(const float* __restrict__ partials,
                                                       const double* __restrict__ partial_loss,
                                                       int nblk, int T, int npix3, float* __restrict__ grads,
                                                       float* __restrict__ losses) {
    __shared__ float part[4][64];
    const int b = blockIdx.y;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int cols = T * NP;
    const int col = blockIdx.x * 64 + lane;
    float acc = 0.0f;
    if (col < cols) {
        const float* base = partials + (size_t)b * nblk * cols + col;
        int r0 = (nblk * wave) / 4, r1 = (nblk * (wave + 1)) / 4;
        for (int rr = r0; rr < r1; rr++) acc += base[(size_t)rr * cols];
    }
    part[wave][lane] = acc;
    __syncthreads();
    if (wave == 0 && col < cols) {
        float v = ((part[0][lane] + part[1][lane]) + part[2][lane]) + part[3][lane];
        grads[(size_t)b * cols + col] = v;
    }
    if (losses && blockIdx.x == 0 && threadIdx.x == 0) {
        double s = 0.0;
        for (int rr = 0; rr < nblk; rr++) s += partial_loss[(size_t)b * nblk + rr];
        losses[b] = (float)(s / (double)npix3);
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

// One fit iteration's bookkeeping and update (fit.rs:243-288), after the loss
// of iteration `iter` has been reduced into loss[0]. One block: thread 0
// decides (divergence, record, best, patience), then all threads snapshot the
// best scene before the update and apply Adam + projection.
__global__ __launch_bounds__(256) void fit_tail(int iter, const float* __restrict__ loss,
                                                float* __restrict__ params, const float* __restrict__ grads,
                                                float* __restrict__ m, float* __restrict__ v,
                                                const float* __restrict__ lr, int n, float beta1, float beta2,
                                                float eps, float bc1, float bc2, float min_delta,
                                                long long patience, FitState* __restrict__ st,
                                                float* __restrict__ losses_out, float* __restrict__ best_params) {
    __shared__ int decision;
    if (threadIdx.x == 0) {
        int d = -1;
        if (st->stop < 0) {
            float L = loss[0];
            if (!isfinite(L)) {
                st->stop = STOP_DIVERGED;  // before the optimizer sees it (fit.rs:259-265)
            } else {
                losses_out[st->n_losses++] = L;
                bool improved = L + min_delta < st->best_loss;
                if (improved) {
                    st->best_loss = L;
                    st->best_iter = iter;
                    st->since = 0;
                } else {
                    st->since += 1;
                }
                bool converged = patience >= 0 && (long long)st->since >= patience;
                if (converged) st->stop = STOP_CONVERGED;
                d = (improved ? 1 : 0) | (converged ? 2 : 0);
            }
        }
        decision = d;
    }
    __syncthreads();
    int d = decision;
    if (d < 0) return;
    if (d & 1)
        for (int i = threadIdx.x; i < n; i += blockDim.x) best_params[i] = params[i];
    if (d & 2) return;
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
        float g = grads[i];
        float mi = beta1 * m[i] + (1.0f - beta1) * g;
        float vi = beta2 * v[i] + (1.0f - beta2) * g * g;
        m[i] = mi;
        v[i] = vi;
        float pv = params[i] - lr[i] * (mi / bc1) / (sqrtf(vi / bc2) + eps);
        int j = i % NP;
        if (pv != pv) pv = 0.5f;
        if (j < 6) pv = rust_clamp(pv, -0.25f, 1.25f);
        else if (j < 9) pv = rust_clamp(pv, 0.0f, 1.0f);
        else pv = rust_clamp(pv, 1e-3f, 0.999f);
        params[i] = pv;
    }
}

// ---------------------------------------------------------------- launchers

hipError_t launch_fit_tail(int iter, const float* loss, float* params, const float* grads, float* m, float* v,
                           const float* lr, int n, float beta1, float beta2, float eps, float bc1, float bc2,
                           float min_delta, long long patience, FitState* st, float* losses_out,
                           float* best_params, hipStream_t s) {
    hipLaunchKernelGGL(fit_tail, dim3(1), dim3(256), 0, s, iter, loss, params, grads, m, v, lr, n, beta1, beta2,
                       eps, bc1, bc2, min_delta, patience, st, losses_out, best_params);
    return hipGetLastError();
}

hipError_t launch_setup(const float* params, int B, int T, int W, int H, float sigma, int tape_mode,
                        float* rec, hipStream_t s) {
    int n = B * T;
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(setup_records, dim3((n + 255) / 256), dim3(256), 0, s, params, n, W, H, sigma,
                       tape_mode, rec);
    return hipGetLastError();
}

dim3 raster_grid(int B, int W, int H) {
    return dim3((W + 2 * TILE - 1) / (2 * TILE), (H + 2 * TILE - 1) / (2 * TILE), B);
}

template <int MODE, bool FAST>
static hipError_t launch_raster_t(const RasterArgs& a, hipStream_t s) {
    hipLaunchKernelGGL((raster_kernel<MODE, FAST>), raster_grid(a.B, a.W, a.H), dim3(WAVES * 64), 0, s, a);
    return hipGetLastError();
}

hipError_t launch_raster(int mode, bool fast, const RasterArgs& a, hipStream_t s) {
    if (mode == MODE_RENDER) return fast ? launch_raster_t<MODE_RENDER, true>(a, s) : launch_raster_t<MODE_RENDER, false>(a, s);
    if (mode == MODE_LOSS) return fast ? launch_raster_t<MODE_LOSS, true>(a, s) : launch_raster_t<MODE_LOSS, false>(a, s);
    return fast ? launch_raster_t<MODE_GRAD_IN, true>(a, s) : launch_raster_t<MODE_GRAD_IN, false>(a, s);
}

hipError_t launch_reduce(const float* partials, const double* partial_loss, int B, int nblk, int T,
                         int npix3, float* grads, float* losses, hipStream_t s) {
    int cols = T * NP;
    dim3 grid((cols + 63) / 64 > 0 ? (cols + 63) / 64 : 1, B);
    hipLaunchKernelGGL(reduce_partials, grid, dim3(256), 0, s, partials, partial_loss, nblk, T, npix3, grads,
                       losses);
    return hipGetLastError();
}

hipError_t launch_adam(float* params, const float* grads, float* m, float* v, const float* lr, int n,
                       float beta1, float beta2, float eps, float bc1, float bc2, int project,
                       hipStream_t s) {
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(adam_project, dim3((n + 255) / 256), dim3(256), 0, s, params, grads, m, v, lr, n, beta1,
                       beta2, eps, bc1, bc2, project);
    return hipGetLastError();
}

}  // namespace drh
