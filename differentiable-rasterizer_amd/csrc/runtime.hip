// Host runtime behind the C ABI in include/diffrast_hip.h: argument checks,
// the device-buffer pool, host/device pointer staging, kernel sequencing and
// the raster, record, Adam and sRGB entry points. The fit loop is in fit.hip,
// the entry point that allocates nothing in scratch.hip.

#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <string>
#include <thread>
#include <unordered_map>
#include <vector>

#include "runtime.h"

using drh::NP;

namespace drh_rt {

namespace {
thread_local std::string g_err;
}  // namespace

const char* last_error_text() { return g_err.c_str(); }

int fail(int code, const std::string& msg) {
    g_err = msg;
    return code;
}

int hip_fail(hipError_t e, const char* what) {
    return fail(DRH_ERR_DEVICE, std::string(what) + ": " + hipGetErrorString(e));
}

int Lease::acquire(drh_ctx* ctx, uint64_t kind, size_t bytes, hipStream_t s) {
    ctx_ = ctx;
    kind_ = kind;
    stream_ = s;
    if (bytes == 0) return DRH_OK;
    {
        std::lock_guard<std::mutex> g(ctx->mu);
        auto it = ctx->free_bufs.find(pool_key(kind, bytes));
        if (it != ctx->free_bufs.end() && !it->second.empty()) {
            buf_ = it->second.back();
            it->second.pop_back();
            ctx->bytes -= bytes;
            ctx->hits += 1;
        }
    }
    if (buf_.ptr) {
        if (buf_.used && buf_.stream != s) {
            if (buf_.ev_recorded) {
                hipError_t e = hipStreamWaitEvent(s, buf_.ev, 0);
                if (e != hipSuccess) return hip_fail(e, "hipStreamWaitEvent");
            } else {
                hipError_t e = hipDeviceSynchronize();
                if (e != hipSuccess) return hip_fail(e, "hipDeviceSynchronize");
            }
            std::lock_guard<std::mutex> g(ctx->mu);
            ctx->multi_stream = true;
        }
        return DRH_OK;
    }
    {
        std::lock_guard<std::mutex> g(ctx->mu);
        ctx->misses += 1;
    }
    hipError_t e = hipMalloc(&buf_.ptr, bytes);
    if (e != hipSuccess) {
        buf_.ptr = nullptr;
        return fail(e == hipErrorOutOfMemory ? DRH_ERR_TOO_LARGE : DRH_ERR_DEVICE,
                    std::string("hipMalloc of ") + std::to_string(bytes) + " bytes: " + hipGetErrorString(e));
    }
    buf_.bytes = bytes;
    e = hipEventCreateWithFlags(&buf_.ev, hipEventDisableTiming);
    if (e != hipSuccess) return hip_fail(e, "hipEventCreate");
    return DRH_OK;
}

void Lease::release() {
    if (!buf_.ptr) return;
    bool multi;
    {
        std::lock_guard<std::mutex> g(ctx_->mu);
        multi = ctx_->multi_stream;
    }
    buf_.ev_recorded = multi && hipEventRecord(buf_.ev, stream_) == hipSuccess;
    buf_.stream = stream_;
    buf_.used = true;
    bool keep = false;
    {
        std::lock_guard<std::mutex> g(ctx_->mu);
        if (ctx_->bytes + buf_.bytes <= ctx_->pool_limit) {
            ctx_->bytes += buf_.bytes;
            ctx_->free_bufs[pool_key(kind_, buf_.bytes)].push_back(buf_);
            keep = true;
        }
    }
    if (!keep) {
        // the queued work that uses the buffer finishes before it is freed
        if (buf_.ev_recorded)
            (void)hipEventSynchronize(buf_.ev);
        else
            (void)hipStreamSynchronize(stream_);
        (void)hipEventDestroy(buf_.ev);
        (void)hipFree(buf_.ptr);
    }
    buf_ = PoolBuf{};
}

int wait_stream(hipStream_t s) {
    hipEvent_t ev;
    hipError_t e = hipEventCreateWithFlags(&ev, hipEventDisableTiming);
    if (e != hipSuccess) return hip_fail(e, "hipEventCreate");
    e = hipEventRecord(ev, s);
    if (e != hipSuccess) {
        (void)hipEventDestroy(ev);
        return hip_fail(e, "hipEventRecord");
    }
    auto deadline = std::chrono::steady_clock::now() + std::chrono::seconds(DRH_WAIT_TIMEOUT_S);
    int spins = 0;
    for (;;) {
        e = hipEventQuery(ev);
        if (e == hipSuccess) break;
        if (e != hipErrorNotReady) {
            (void)hipEventDestroy(ev);
            return hip_fail(e, "device execution");
        }
        if (std::chrono::steady_clock::now() > deadline) {
            (void)hipEventDestroy(ev);
            return fail(DRH_ERR_TIMEOUT, "the GPU did not finish within " + std::to_string(DRH_WAIT_TIMEOUT_S) +
                                             " s; it may be busy with another process (check rocm-smi)");
        }
        if (++spins > 64) std::this_thread::sleep_for(std::chrono::microseconds(50));
    }
    (void)hipEventDestroy(ev);
    return DRH_OK;
}

int check_sizes(int64_t B, int64_t T, int64_t H, int64_t W) {
    if (B < 0 || T < 0 || H < 0 || W < 0) return fail(DRH_ERR_INVALID_ARG, "sizes must be non-negative");
    if (H == 0 || W == 0) return fail(DRH_ERR_INVALID_ARG, "height and width must be non-zero");
    if (B > 65535) return fail(DRH_ERR_TOO_LARGE, "batch of " + std::to_string(B) + " exceeds 65535 scenes per call");
    if (H > (1 << 20) || W > (1 << 20)) return fail(DRH_ERR_TOO_LARGE, "height and width are limited to 2^20");
    if (T > (1 << 23)) return fail(DRH_ERR_TOO_LARGE, "more than 2^23 triangles per scene");
    if (B * T > (int64_t)INT32_MAX / 64) return fail(DRH_ERR_TOO_LARGE, "batch x triangles too large for one call");
    return DRH_OK;
}

int check_shape(drh_ctx* ctx, int64_t B, int64_t T, int64_t H, int64_t W, float sigma) {
    if (!ctx) return fail(DRH_ERR_INVALID_ARG, "context is NULL");
    if (!(std::isfinite(sigma) && sigma > 0.0f)) return fail(DRH_ERR_INVALID_ARG, "sigma must be positive and finite");
    return check_sizes(B, T, H, W);
}

int stage_in(drh_ctx* ctx, Staged& st, uint64_t kind, const float* src, size_t n, bool host, hipStream_t s) {
    if (n == 0) {
        st.dev = src;
        return DRH_OK;
    }
    if (!src) return fail(DRH_ERR_INVALID_ARG, "input pointer is NULL");
    if (!host) {
        st.dev = src;
        return DRH_OK;
    }
    int rc = st.lease.acquire(ctx, kind, n * sizeof(float), s);
    if (rc) return rc;
    HIP_TRY(hipMemcpyAsync(st.lease.get<float>(), src, n * sizeof(float), hipMemcpyHostToDevice, s), "hipMemcpyAsync H2D");
    st.dev = st.lease.get<float>();
    return DRH_OK;
}

int stage_out(drh_ctx* ctx, Out& o, uint64_t kind, float* dst, size_t n, bool host, hipStream_t s) {
    o.n = n;
    if (n == 0 || !dst) {
        o.dev = nullptr;
        return DRH_OK;
    }
    if (!host) {
        o.dev = dst;
        return DRH_OK;
    }
    int rc = o.lease.acquire(ctx, kind, n * sizeof(float), s);
    if (rc) return rc;
    o.dev = o.lease.get<float>();
    o.host_dst = dst;
    return DRH_OK;
}

int copy_back(Out& o, hipStream_t s) {
    if (!o.host_dst || o.n == 0) return DRH_OK;
    hipError_t e = hipMemcpyAsync(o.host_dst, o.dev, o.n * sizeof(float), hipMemcpyDeviceToHost, s);
    if (e != hipSuccess) return fail(DRH_ERR_READBACK, std::string("hipMemcpyAsync D2H: ") + hipGetErrorString(e));
    return DRH_OK;
}

int finish(uint32_t flags, hipStream_t s) {
    if (flags & (DRH_HOST_PTRS | DRH_SYNC | DRH_PHASES)) return wait_stream(s);
    return DRH_OK;
}

namespace {
thread_local drh_phase_timings g_phases{};

double now_ms() {
    return std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now().time_since_epoch()).count();
}
}  // namespace

PhaseClock::PhaseClock(uint32_t flags, hipStream_t s) : on_((flags & DRH_PHASES) != 0), s_(s) {
    if (on_) t_ = now_ms();
}

int PhaseClock::lap(int phase) {
    if (!on_) return DRH_OK;
    int rc = wait_stream(s_);
    double t = now_ms();
    ms_[phase] += t - t_;
    t_ = t;
    return rc;
}

void PhaseClock::publish() const {
    if (!on_) return;
    g_phases.pack_ms = ms_[PH_PACK];
    g_phases.alloc_ms = ms_[PH_ALLOC];
    g_phases.dispatch_ms = ms_[PH_DISPATCH];
    g_phases.readback_ms = ms_[PH_READBACK];
    g_phases.loss_ms = 0.0;
    g_phases.total_ms = ms_[PH_PACK] + ms_[PH_ALLOC] + ms_[PH_DISPATCH] + ms_[PH_READBACK];
}

float powi_f32(float a, int32_t b) {
    bool recip = b < 0;
    float r = 1.0f;
    for (;;) {
        if (b & 1) r *= a;
        b /= 2;
        if (b == 0) break;
        a *= a;
    }
    return recip ? 1.0f / r : r;
}

KernelTimer::KernelTimer(drh_ctx* ctx, int kernel, bool enabled) : ctx_(ctx) {
    if (!enabled || !ctx->timing) return;
    l_.kernel = kernel;
    if (hipEventCreate(&l_.start) != hipSuccess) return;
    if (hipEventCreate(&l_.stop) != hipSuccess) {
        (void)hipEventDestroy(l_.start);
        return;
    }
    // the scope's launch takes them as its own start and end (hipExtLaunchKernel)
    drh::launch_events() = drh::LaunchEvents{l_.start, l_.stop, false};
    on_ = true;
}

KernelTimer::~KernelTimer() {
    if (!on_) return;
    drh::LaunchEvents& ev = drh::launch_events();
    const bool used = ev.used;
    ev = drh::LaunchEvents{};
    if (!used) {  // nothing was launched in the scope
        (void)hipEventDestroy(l_.start);
        (void)hipEventDestroy(l_.stop);
        return;
    }
    std::lock_guard<std::mutex> g(ctx_->mu);
    ctx_->pending.push_back(l_);
}

// All T entries per tile (the backward kernel then needs no rebuild path)
// while that fits the budget, else as many as fit, at least min_cap.
int tile_entries(size_t ntiles, int T, size_t budget, size_t min_cap) {
    size_t cap = (size_t)(T > 0 ? T : 1);
    const size_t fit = budget / (ntiles * sizeof(drh::TileEnt));
    if (cap > fit) cap = fit > min_cap ? fit : min_cap;
    if (const char* e = std::getenv("DRH_MAX_TILE_ENTRIES")) {
        const long v = std::strtol(e, nullptr, 10);
        if (v >= 1 && (size_t)v < cap) cap = (size_t)v;
    }
    return (int)cap;
}

// The raster kernels' block order (OrderArgs) is made for a batch (B > 1)
// whose grid has more blocks than the device has CUs (with fewer, every block
// has a CU to itself) and whose scenes' difference grids fit in LDS. A single
// scene is left in launch order: one workgroup would make its whole order,
// which costs about what it saves on one scene's kernels. The forward kernel
// follows it when its lists are short (T <= FWD_ORDER_MAX_T), so that the
// overlap count sets its cost; with longer lists every block spends about the
// same building them, and the order only costs it locality. The backward
// kernel always follows it.
bool use_order(const drh_ctx* ctx, int B, int gx, int gy) {
    return B > 1 && (size_t)B * gx * gy > (size_t)ctx->cus &&
           (size_t)(gx + 1) * (gy + 1) <= (size_t)drh::ORD_MAX_CELLS;
}

bool fused_gradients(int mode, int nseg, int cap2, int T) {
    // cap2 > T: the one-wave kernel's backward loop reads the slot after a
    // tile's last entry (at most T of them); the segmented kernel's regions
    // are sized alike
    if ((mode != drh::MODE_LOSS && mode != drh::MODE_GRAD_IN) || nseg > 1 || cap2 <= T || cap2 % 8 != 0)
        return false;
    const char* e = std::getenv("DRH_UNFUSED");
    return !(e && e[0] == '1');
}

bool use_segments(int mode, size_t ntiles, int T) {
    if ((mode != drh::MODE_LOSS && mode != drh::MODE_GRAD_IN) || T < SEG_MIN_T || T > drh::SEG_MAX_T ||
        ntiles > SEG_MAX_TILES)
        return false;
    const char* e = std::getenv("DRH_NO_SEGMENTS");
    return !(e && e[0] == '1');
}

int run_raster_bufs(drh_ctx* ctx, int mode, const float* params, const float* bgs, const float* img_in, int B,
                    int T, int H, int W, float sigma, float* out_img, float* out_grads, float* out_losses,
                    uint32_t flags, const RasterBufs& bufs, hipStream_t s, const int* halt, bool timed,
                    const drh::FitTail* tail) {
    const bool fast = !(flags & DRH_EXACT_MATH);
    const bool det = (flags & DRH_DETERMINISTIC) != 0;
    const dim3 grid = drh::raster_grid(B, W, H);
    const int nblk = (int)(grid.x * grid.y);
    // fixed-order partial rows (and loss partials) per scene: per block, or per tile in fused_seg_kernel
    const int nrows = bufs.segw ? nblk * drh::WAVES : nblk;
    drh::OrderArgs ord{};
    if (bufs.order)
        ord = bufs.order_tiles ? drh::OrderArgs{bufs.order, 2 * (int)grid.x, 2 * (int)grid.y, 3, bufs.rows, bufs.row_n}
                               : drh::OrderArgs{bufs.order, (int)grid.x, (int)grid.y, 4};
    // the fused kernels sum the losses themselves outside the fixed-order mode
    // (RasterArgs::loss_tail): setup_records marks the loss slots pending
    const bool loss_tail = bufs.fused && !det && mode == drh::MODE_LOSS && !(tail && tail->rec_ready);
    if (!(tail && tail->rec_ready)) {  // else the previous fit_step made this iteration's records
        KernelTimer kt(ctx, TK_SETUP, timed);
        HIP_TRY(drh::launch_setup(params, B, T, W, H, sigma,
                                  mode == drh::MODE_RENDER ? drh::SETUP_RENDER : drh::SETUP_TAPE, bufs.rec,
                                  mode != drh::MODE_RENDER && !det ? out_grads : nullptr, s, nullptr, nullptr,
                                  ord, halt, nullptr, drh::RecordHead{}, loss_tail ? bufs.ploss : nullptr,
                                  nblk * drh::WAVES),
                "setup_records launch");
    }
    drh::RasterArgs a{};
    drh::set_sizes(a, B, T, H, W, sigma);
    a.rec = bufs.rec;
    a.bg = bgs;
    a.target = mode == drh::MODE_LOSS ? img_in : nullptr;
    a.grad_in = mode == drh::MODE_GRAD_IN ? img_in : nullptr;
    a.out_img = out_img;
    a.partials = bufs.partials;
    a.partial_loss = bufs.ploss;
    a.pq = bufs.pq;
    a.pg0 = bufs.pg0;
    a.pze = bufs.pze;
    a.tl_ent = bufs.tent;
    a.cap2 = bufs.cap2;
    a.segw = bufs.fused ? bufs.segw : 0;
    a.tl_n = bufs.tn;
    a.grads = out_grads;
    a.losses = out_losses;
    a.loss_tail = loss_tail ? 1 : 0;
    a.deterministic = det ? 1 : 0;
    a.chw = (flags & DRH_CHANNELS_FIRST) ? 1 : 0;
    a.perm_fwd = T <= FWD_ORDER_MAX_T ? ord.perm : nullptr;
    a.perm_bwd = ord.perm;
    a.perm_tiles = bufs.order_tiles ? 1 : 0;
    a.rows = bufs.order_tiles ? bufs.rows : nullptr;
    a.row_n = bufs.order_tiles ? bufs.row_n : nullptr;
    a.row_gy = 2 * (int)grid.y;
    a.halt = halt;
    a.nseg = bufs.ckpt && ord.perm ? bufs.nseg : 1;
    a.seg_m = bufs.seg_m;
    a.nsplit = bufs.nsplit;
    a.gx = (int)grid.x;
    a.gy = (int)grid.y;
    a.ckpt = bufs.ckpt;
    if (bufs.fused) {
        KernelTimer kt(ctx, TK_RASTER, timed);
        HIP_TRY(drh::launch_fused(mode, fast, a, s), "fused_kernel launch");
    } else {
        {
            KernelTimer kt(ctx, TK_RASTER, timed);
            HIP_TRY(drh::launch_forward(mode, fast, a, s), "forward_kernel launch");
        }
        if (mode == drh::MODE_RENDER) return DRH_OK;
        KernelTimer kt(ctx, TK_BACKWARD, timed);
        HIP_TRY(drh::launch_backward(mode, fast, bufs.cap2 < T, a, s), "backward_kernel launch");
    }
    if (det && tail) {
        KernelTimer kt(ctx, TK_ADAM, timed);
        HIP_TRY(drh::launch_fit_step(a.partials, a.partial_loss, nrows, nrows / nblk, T, 3.0 * (double)H * (double)W,
                                     *tail, s),
                "fit_step launch");
    } else if (det) {
        KernelTimer kt(ctx, TK_REDUCE, timed);
        HIP_TRY(drh::launch_reduce(a.partials, a.partial_loss, B, nrows, nrows / nblk, T, 3.0 * (double)H * (double)W,
                                   out_grads,
                                   mode == drh::MODE_LOSS ? out_losses : nullptr, s, halt),
                "reduce_partials launch");
    } else if (bufs.fused && mode == drh::MODE_LOSS && !loss_tail) {
        KernelTimer kt(ctx, TK_REDUCE, timed);
        HIP_TRY(drh::launch_sum_losses(a.partial_loss, B, nblk, drh::loss_partials_per_block(true, false),
                                       3.0 * (double)H * (double)W, out_losses, s, halt),
                "sum_losses launch");
    }
    return DRH_OK;
}

int backward_segments(int T, int cap2, bool det, size_t blocks, int cus) {
    if (det || cap2 < T || T < SPLIT_MIN_T || blocks >= (size_t)SPLIT_MAX_BLOCKS_PER_CU * (size_t)cus) return 1;
    return SPLIT_SEGMENTS;
}

int run_raster(drh_ctx* ctx, int mode, const float* params, const float* bgs, const float* img_in, int B, int T,
               int H, int W, float sigma, float* out_img, float* out_grads, float* out_losses, uint32_t flags,
               hipStream_t s, const int* halt, const drh::FitTail* tail) {
    const bool det = (flags & DRH_DETERMINISTIC) != 0;
    const dim3 grid = drh::raster_grid(B, W, H);
    const int nblk = (int)(grid.x * grid.y);
    const size_t ntiles = (size_t)B * nblk * drh::WAVES;
    Lease rec, partials, ploss, pq, pg0, pze, tent, tn, order, ckpt, rows;
    RasterBufs bufs;
    // whole 64-byte lines per tile (8 entries) and one slot past T entries, as
    // the fused kernel needs
    bufs.cap2 = tile_entries(ntiles, (T + 8) & ~7);
    // the records: the fit's own (FitTail::rec), else pooled
    int rc = tail && tail->rec ? DRH_OK : rec.acquire(ctx, K_REC, (size_t)B * T * drh::REC * sizeof(float), s);
    if (rc) return rc;
    const bool ordered =
        use_order(ctx, B, (int)grid.x, (int)grid.y) && (mode != drh::MODE_RENDER || T <= FWD_ORDER_MAX_T);
    if (ordered) {
        const int nseg = mode == drh::MODE_RENDER ? 1 : backward_segments(T, bufs.cap2, det, (size_t)B * nblk, ctx->cus);
        if (nseg > 1) {
            const size_t words = ntiles * (size_t)(nseg - 1) * drh::CKPT_WORDS * 64;
            if ((rc = ckpt.acquire(ctx, K_CKPT, words * sizeof(float), s))) return rc;
            bufs.ckpt = ckpt.get<float>();
            bufs.nseg = nseg;
            bufs.seg_m = (T + SPLIT_DIVISOR - 1) / SPLIT_DIVISOR;
            bufs.nsplit = std::max(1, nblk / SPLIT_BLOCK_SHARE);
        }
    }
    bufs.fused = fused_gradients(mode, bufs.nseg, bufs.cap2, T);
    if (bufs.fused && use_segments(mode, ntiles, T)) {
        // each wave's region whole 64-byte lines
        bufs.segw = drh::SEG_WAVES;
        bufs.cap2 = drh::seg_cap2(T);
    }
    if (ordered) {
        // the one-wave fused kernel takes an order of tiles where its cells fit
        bufs.order_tiles = bufs.fused && !det &&
                           (size_t)(2 * grid.x + 1) * (2 * grid.y + 1) <= (size_t)drh::ORD_MAX_CELLS;
        const size_t cells = (size_t)B * nblk * (bufs.order_tiles ? drh::WAVES : 1);
        if ((rc = order.acquire(ctx, K_ORDER, cells * sizeof(int), s))) return rc;
        bufs.order = order.get<int>();
        // the tile rows' triangle lists, where their bit masks fit setup_records' LDS
        const size_t trows = (size_t)B * 2 * grid.y;
        if (bufs.order_tiles && !bufs.segw && T >= ROW_LISTS_MIN_T &&
            (size_t)2 * grid.y * ((T + 31) / 32) <= (size_t)drh::ORD_ROW_WORDS) {
            if ((rc = rows.acquire(ctx, K_ROWS, (trows * T + trows) * sizeof(int), s))) return rc;
            bufs.rows = rows.get<int>();
            bufs.row_n = bufs.rows + trows * T;
        }
    }
    if (mode != drh::MODE_RENDER) {
        const size_t prows = (size_t)B * nblk * (bufs.segw ? drh::WAVES : 1);  // per block, or per tile
        if (det && (rc = partials.acquire(ctx, K_PARTIALS, prows * T * NP * sizeof(float), s))) return rc;
        if ((rc = ploss.acquire(ctx, K_PLOSS, (size_t)B * nblk * drh::WAVES * sizeof(double), s))) return rc;  // per tile
        if ((rc = tent.acquire(ctx, K_TILE_ENT, ntiles * bufs.cap2 * sizeof(drh::TileEnt), s))) return rc;
        // the hand-over between the two kernels (the fused kernel keeps it in registers)
        if (!bufs.fused) {
            if ((rc = pq.acquire(ctx, K_PIXSTATE, (size_t)B * H * W * sizeof(float), s))) return rc;
            if (mode == drh::MODE_LOSS &&
                (rc = pg0.acquire(ctx, K_PIX_G0, (size_t)B * H * W * 3 * sizeof(float), s)))
                return rc;
            if ((rc = pze.acquire(ctx, K_PIX_ZE, ntiles * 64 * sizeof(int2), s))) return rc;
            if ((rc = tn.acquire(ctx, K_TILE_N, ntiles * 2 * sizeof(int), s))) return rc;
        }
    }
    bufs.rec = tail && tail->rec ? tail->rec : rec.get<float>();
    bufs.partials = partials.get<float>();
    bufs.ploss = ploss.get<double>();
    bufs.pq = pq.get<float>();
    bufs.pg0 = pg0.get<float>();
    bufs.pze = pze.get<int2>();
    bufs.tent = tent.get<drh::TileEnt>();
    bufs.tn = tn.get<int>();
    return run_raster_bufs(ctx, mode, params, bgs, img_in, B, T, H, W, sigma, out_img, out_grads, out_losses, flags,
                           bufs, s, halt, true, tail);
}

}  // namespace drh_rt

namespace {

using namespace drh_rt;

// The forward record that drh_render_record leaves for drh_backward_recorded,
// in device memory the caller owns: a head (sizes, sigma, math mode), the
// triangle records, a copy of the backgrounds, the per-pixel hand-over (total
// transmittance, and the zero and rescaling counts of the tiles that have
// any), the per-tile entries (with their counts) and the backward kernel's
// block order, each starting at a 256-byte boundary.
struct RecordLayout {
    size_t head = 0, rec = 0, bg = 0, pq = 0, pze = 0, tl_n = 0, tl_ent = 0, ord = 0, total = 0;
    int cap2 = 0;
};

RecordLayout record_layout(int64_t B, int64_t T, int64_t H, int64_t W) {
    RecordLayout L;
    if (B == 0) return L;
    const dim3 grid = drh::raster_grid((int)B, (int)W, (int)H);
    const size_t ntiles = (size_t)B * grid.x * grid.y * drh::WAVES;
    L.cap2 = tile_entries(ntiles, (int)T);
    auto up = [](size_t x) { return (x + 255) & ~(size_t)255; };
    size_t off = 0;
    L.head = off;
    off = up(off + sizeof(drh::RecordHead));
    L.rec = off;
    off = up(off + (size_t)B * T * drh::REC * sizeof(float));
    L.bg = off;
    off = up(off + (size_t)B * 3 * sizeof(float));
    L.pq = off;
    off = up(off + (size_t)B * H * W * sizeof(float));
    L.pze = off;
    off = up(off + ntiles * 64 * sizeof(int2));
    L.tl_n = off;
    off = up(off + ntiles * 2 * sizeof(int));
    L.tl_ent = off;
    off = up(off + ntiles * (size_t)L.cap2 * sizeof(drh::TileEnt));
    L.ord = off;
    off = up(off + ntiles / drh::WAVES * sizeof(int));
    L.total = off;
    return L;
}

int check_record(const void* record, uint64_t record_bytes, const RecordLayout& L) {
    if (!record) return fail(DRH_ERR_INVALID_ARG, "record is NULL");
    if (record_bytes != L.total)
        return fail(DRH_ERR_INVALID_ARG, "record of " + std::to_string(record_bytes) + " bytes; these sizes need " +
                                             std::to_string(L.total) + " (drh_record_bytes)");
    if (reinterpret_cast<uintptr_t>(record) % 256 != 0)
        return fail(DRH_ERR_INVALID_ARG, "record must be 256-byte aligned");
    return DRH_OK;
}

drh::RecordHead make_head(int64_t B, int64_t T, int64_t H, int64_t W, float sigma, uint32_t flags) {
    drh::RecordHead h{};
    h.magic = drh::RECORD_MAGIC;
    h.exact = (flags & DRH_EXACT_MATH) ? 1u : 0u;
    h.sigma = sigma;
    h.B = (int32_t)B;
    h.T = (int32_t)T;
    h.H = (int32_t)H;
    h.W = (int32_t)W;
    return h;
}

// Records remembered per context; past this many the registry starts over
// (a record it no longer knows has its head read from the device).
constexpr size_t RECORD_REGISTRY_MAX = 4096;

void remember_record(drh_ctx* ctx, const void* record, const drh::RecordHead& h) {
    std::lock_guard<std::mutex> g(ctx->mu);
    if (ctx->records.size() >= RECORD_REGISTRY_MAX && !ctx->records.count(record)) ctx->records.clear();
    ctx->records[record] = h;
}

// The backward of a record must run with the forward's sizes, sigma and math
// mode: the record's masks and transmittance totals were made with them.
int check_record_head(drh_ctx* ctx, const void* record, const drh::RecordHead& want, hipStream_t s) {
    drh::RecordHead have{};
    bool known = false;
    {
        std::lock_guard<std::mutex> g(ctx->mu);
        auto it = ctx->records.find(record);
        if (it != ctx->records.end()) {
            have = it->second;
            known = true;
        }
    }
    if (!known) {
        HIP_TRY(hipMemcpyAsync(&have, record, sizeof have, hipMemcpyDeviceToHost, s), "read record head");
        int rc = wait_stream(s);
        if (rc) return rc;
        if (have.magic != drh::RECORD_MAGIC)
            return fail(DRH_ERR_INVALID_ARG, "record was not written by drh_render_record");
    }
    if (have.B != want.B || have.T != want.T || have.H != want.H || have.W != want.W)
        return fail(DRH_ERR_INVALID_ARG, "record was made for other sizes (B, T, H, W)");
    if (have.sigma != want.sigma)
        return fail(DRH_ERR_INVALID_ARG, "sigma differs from the sigma of the record's forward pass");
    if (have.exact != want.exact)
        return fail(DRH_ERR_INVALID_ARG, "DRH_EXACT_MATH differs from the record's forward pass");
    return DRH_OK;
}

// ---------------------------------------------------------------- sRGB bytes


// canvas.rs:100-105, with the reference's f32 operations in its order (no
// contraction: the library is built with -ffp-contract=off) and the host
// libm's powf, which is what Rust's f32::powf calls on Linux.
uint8_t encode_srgb_host(float v) {
    if (v < 0.0f) v = 0.0f;  // f32::clamp: NaN passes through
    if (v > 1.0f) v = 1.0f;
    const float s = v <= 0.0031308f ? 12.92f * v : 1.055f * std::pow(v, 1.0f / 2.4f) - 0.055f;
    const float b = s * 255.0f + 0.5f;
    if (!(b >= 0.0f)) return 0;  // `as u8` saturates, NaN -> 0
    if (b >= 255.0f) return 255;
    return (uint8_t)b;
}

// canvas.rs:108-115
float decode_srgb_host(uint8_t byte) {
    const float v = (float)byte / 255.0f;
    if (v <= 0.04045f) return v / 12.92f;
    return std::pow((v + 0.055f) / 1.055f, 2.4f);
}

float float_of_bits(uint32_t b) {
    float f;
    std::memcpy(&f, &b, sizeof f);
    return f;
}

struct SrgbTables {
    drh::SrgbTable thresholds, values;
};

// Entry k of the thresholds: the smallest float in [0, 1] that encodes to k or
// more, by bisection over the bit patterns (ordered like the values there);
// the encoding is monotonic on [0, 1].
const SrgbTables& srgb_tables() {
    static SrgbTables t;
    static std::once_flag once;
    std::call_once(once, [] {
        t.thresholds.v[0] = 0.0f;
        for (int k = 1; k < 256; k++) {
            uint32_t lo = 0, hi = 0x3F800000u;  // encode(0) = 0 < k <= encode(1) = 255
            while (lo + 1 < hi) {
                const uint32_t mid = lo + (hi - lo) / 2;
                if (encode_srgb_host(float_of_bits(mid)) >= k)
                    hi = mid;
                else
                    lo = mid;
            }
            t.thresholds.v[k] = float_of_bits(hi);
        }
        for (int b = 0; b < 256; b++) t.values.v[b] = decode_srgb_host((uint8_t)b);
    });
    return t;
}

}  // namespace

extern "C" {

const char* drh_last_error(void) { return last_error_text(); }

int drh_params_per_triangle(void) { return NP; }

int drh_create(drh_ctx** out) {
    if (!out) return fail(DRH_ERR_INVALID_ARG, "out is NULL");
    *out = nullptr;
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n == 0)
        return fail(DRH_ERR_NO_DEVICE, "no HIP device found; there is no CPU path");
    int dev = 0;
    HIP_TRY(hipGetDevice(&dev), "hipGetDevice");
    hipDeviceProp_t prop;
    HIP_TRY(hipGetDeviceProperties(&prop, dev), "hipGetDeviceProperties");
    auto* c = new drh_ctx();
    c->device = dev;
    c->discrete = prop.integrated == 0;
    c->cus = prop.multiProcessorCount;
    c->pool_limit = std::max<uint64_t>(POOL_BYTE_LIMIT, (uint64_t)prop.totalGlobalMem / POOL_MEMORY_SHARE);
    char buf[512];
    std::snprintf(buf, sizeof buf, "%s (%s, %d CUs, HIP)", prop.name, prop.gcnArchName, prop.multiProcessorCount);
    c->info = buf;
    int rc = scratch_init(dev);
    if (rc) {
        delete c;
        return rc;
    }
    *out = c;
    return DRH_OK;
}

int drh_destroy(drh_ctx* ctx) {
    if (!ctx) return DRH_OK;
    drh_clear_pool(ctx);
    delete ctx;
    return DRH_OK;
}

int drh_device_info(const drh_ctx* ctx, char* buf, size_t len) {
    if (!ctx || !buf || len == 0) return fail(DRH_ERR_INVALID_ARG, "bad arguments");
    std::snprintf(buf, len, "%s", ctx->info.c_str());
    return DRH_OK;
}

int drh_is_discrete(const drh_ctx* ctx) { return ctx && ctx->discrete ? 1 : 0; }

int drh_pool_stats(drh_ctx* ctx, uint64_t* hits, uint64_t* misses, uint64_t* bytes) {
    if (!ctx) return fail(DRH_ERR_INVALID_ARG, "context is NULL");
    std::lock_guard<std::mutex> g(ctx->mu);
    if (hits) *hits = ctx->hits;
    if (misses) *misses = ctx->misses;
    if (bytes) *bytes = ctx->bytes;
    return DRH_OK;
}

int drh_clear_pool(drh_ctx* ctx) {
    if (!ctx) return fail(DRH_ERR_INVALID_ARG, "context is NULL");
    DeviceGuard dg(ctx->device);
    std::lock_guard<std::mutex> g(ctx->mu);
    for (auto& kv : ctx->free_bufs) {
        for (auto& b : kv.second) {
            (void)hipEventSynchronize(b.ev);
            (void)hipEventDestroy(b.ev);
            (void)hipFree(b.ptr);
        }
    }
    ctx->free_bufs.clear();
    ctx->bytes = 0;
    return DRH_OK;
}

int drh_timing_enable(drh_ctx* ctx, int enable) {
    if (!ctx) return fail(DRH_ERR_INVALID_ARG, "context is NULL");
    std::lock_guard<std::mutex> g(ctx->mu);
    ctx->timing = enable != 0;
    return DRH_OK;
}

int drh_phases_read(drh_phase_timings* out) {
    if (!out) return fail(DRH_ERR_INVALID_ARG, "out is NULL");
    *out = g_phases;
    return DRH_OK;
}

int drh_timing_read(drh_ctx* ctx, drh_timings* out) {
    if (!ctx || !out) return fail(DRH_ERR_INVALID_ARG, "bad arguments");
    std::vector<TimedLaunch> launches;
    {
        std::lock_guard<std::mutex> g(ctx->mu);
        launches.swap(ctx->pending);
    }
    double ms[TK_COUNT] = {};
    int64_t n[TK_COUNT] = {};
    int rc = DRH_OK;
    for (auto& l : launches) {
        float t = 0.0f;
        if (rc == DRH_OK) {
            hipError_t e = hipEventSynchronize(l.stop);
            if (e == hipSuccess) e = hipEventElapsedTime(&t, l.start, l.stop);
            if (e != hipSuccess) rc = hip_fail(e, "kernel timing");
        }
        ms[l.kernel] += t;
        n[l.kernel] += 1;
        (void)hipEventDestroy(l.start);
        (void)hipEventDestroy(l.stop);
    }
    out->setup_ms = ms[TK_SETUP];
    out->raster_ms = ms[TK_RASTER];
    out->reduce_ms = ms[TK_REDUCE];
    out->adam_ms = ms[TK_ADAM];
    out->setup_n = n[TK_SETUP];
    out->raster_n = n[TK_RASTER];
    out->reduce_n = n[TK_REDUCE];
    out->adam_n = n[TK_ADAM];
    out->backward_ms = ms[TK_BACKWARD];
    out->backward_n = n[TK_BACKWARD];
    return rc;
}

int drh_render(drh_ctx* ctx, const float* params, const float* backgrounds, int64_t B, int64_t T, int64_t H,
               int64_t W, float sigma, float* out_images, void* stream, uint32_t flags) {
    int rc = check_shape(ctx, B, T, H, W, sigma);
    if (rc) return rc;
    if (B == 0) return DRH_OK;
    if (!out_images || !backgrounds) return fail(DRH_ERR_INVALID_ARG, "output or background pointer is NULL");
    DeviceGuard dg(ctx->device);
    hipStream_t s = (hipStream_t)stream;
    bool host = flags & DRH_HOST_PTRS;
    PhaseClock pc(flags, s);
    Staged p, bg;
    Out img;
    if ((rc = stage_in(ctx, p, K_IN_PARAMS, params, (size_t)B * T * NP, host, s))) return rc;
    if ((rc = stage_in(ctx, bg, K_IN_BG, backgrounds, (size_t)B * 3, host, s))) return rc;
    if ((rc = pc.lap(PH_PACK))) return rc;
    if ((rc = stage_out(ctx, img, K_OUT_IMAGES, out_images, (size_t)B * H * W * 3, host, s))) return rc;
    if ((rc = pc.lap(PH_ALLOC))) return rc;
    if ((rc = run_raster(ctx, drh::MODE_RENDER, p.dev, bg.dev, nullptr, (int)B, (int)T, (int)H, (int)W, sigma,
                         img.dev, nullptr, nullptr, flags, s)))
        return rc;
    if ((rc = pc.lap(PH_DISPATCH))) return rc;
    if ((rc = copy_back(img, s))) return rc;
    if ((rc = finish(flags, s)) || (rc = pc.lap(PH_READBACK))) return rc;
    pc.publish();
    return DRH_OK;
}

int drh_fused_loss_backward(drh_ctx* ctx, const float* params, const float* backgrounds, const float* targets,
                            int64_t B, int64_t T, int64_t H, int64_t W, float sigma, float* out_losses,
                            float* out_grads, float* out_images, void* stream, uint32_t flags) {
    int rc = check_shape(ctx, B, T, H, W, sigma);
    if (rc) return rc;
    if (B == 0) return DRH_OK;
    if (!out_losses || !backgrounds || (T > 0 && !out_grads))
        return fail(DRH_ERR_INVALID_ARG, "output or background pointer is NULL");
    DeviceGuard dg(ctx->device);
    hipStream_t s = (hipStream_t)stream;
    bool host = flags & DRH_HOST_PTRS;
    PhaseClock pc(flags, s);
    Staged p, bg, tg;
    Out losses, grads, img;
    if ((rc = stage_in(ctx, p, K_IN_PARAMS, params, (size_t)B * T * NP, host, s))) return rc;
    if ((rc = stage_in(ctx, bg, K_IN_BG, backgrounds, (size_t)B * 3, host, s))) return rc;
    if ((rc = pc.lap(PH_PACK))) return rc;
    if ((rc = stage_in(ctx, tg, K_IN_IMAGES, targets, (size_t)B * H * W * 3, host, s))) return rc;
    if ((rc = stage_out(ctx, losses, K_OUT_LOSSES, out_losses, (size_t)B, host, s))) return rc;
    if ((rc = stage_out(ctx, grads, K_OUT_GRADS, out_grads, (size_t)B * T * NP, host, s))) return rc;
    if ((rc = stage_out(ctx, img, K_OUT_IMAGES, out_images, (size_t)B * H * W * 3, host, s))) return rc;
    if ((rc = pc.lap(PH_ALLOC))) return rc;
    if ((rc = run_raster(ctx, drh::MODE_LOSS, p.dev, bg.dev, tg.dev, (int)B, (int)T, (int)H, (int)W, sigma, img.dev,
                         grads.dev, losses.dev, flags, s)))
        return rc;
    if ((rc = pc.lap(PH_DISPATCH))) return rc;
    if ((rc = copy_back(losses, s)) || (rc = copy_back(grads, s)) || (rc = copy_back(img, s))) return rc;
    if ((rc = finish(flags, s)) || (rc = pc.lap(PH_READBACK))) return rc;
    pc.publish();
    return DRH_OK;
}

int drh_backward_from_grad(drh_ctx* ctx, const float* params, const float* backgrounds, const float* grad_images,
                           int64_t B, int64_t T, int64_t H, int64_t W, float sigma, float* out_grads, void* stream,
                           uint32_t flags) {
    int rc = check_shape(ctx, B, T, H, W, sigma);
    if (rc) return rc;
    if (B == 0 || T == 0) return DRH_OK;
    if (!out_grads || !backgrounds) return fail(DRH_ERR_INVALID_ARG, "output or background pointer is NULL");
    DeviceGuard dg(ctx->device);
    hipStream_t s = (hipStream_t)stream;
    bool host = flags & DRH_HOST_PTRS;
    PhaseClock pc(flags, s);
    Staged p, bg, gi;
    Out grads;
    if ((rc = stage_in(ctx, p, K_IN_PARAMS, params, (size_t)B * T * NP, host, s))) return rc;
    if ((rc = stage_in(ctx, bg, K_IN_BG, backgrounds, (size_t)B * 3, host, s))) return rc;
    if ((rc = pc.lap(PH_PACK))) return rc;
    if ((rc = stage_in(ctx, gi, K_IN_IMAGES, grad_images, (size_t)B * H * W * 3, host, s))) return rc;
    if ((rc = stage_out(ctx, grads, K_OUT_GRADS, out_grads, (size_t)B * T * NP, host, s))) return rc;
    if ((rc = pc.lap(PH_ALLOC))) return rc;
    if ((rc = run_raster(ctx, drh::MODE_GRAD_IN, p.dev, bg.dev, gi.dev, (int)B, (int)T, (int)H, (int)W, sigma,
                         nullptr, grads.dev, nullptr, flags, s)))
        return rc;
    if ((rc = pc.lap(PH_DISPATCH))) return rc;
    if ((rc = copy_back(grads, s))) return rc;
    if ((rc = finish(flags, s)) || (rc = pc.lap(PH_READBACK))) return rc;
    pc.publish();
    return DRH_OK;
}

int drh_record_bytes(int64_t B, int64_t T, int64_t H, int64_t W, uint64_t* out_bytes) {
    if (!out_bytes) return fail(DRH_ERR_INVALID_ARG, "out_bytes is NULL");
    int rc = check_sizes(B, T, H, W);
    if (rc) return rc;
    *out_bytes = record_layout(B, T, H, W).total;
    return DRH_OK;
}

int drh_render_record(drh_ctx* ctx, const float* params, const float* backgrounds, int64_t B, int64_t T,
                      int64_t H, int64_t W, float sigma, float* out_images, void* record, uint64_t record_bytes,
                      void* stream, uint32_t flags) {
    int rc = check_shape(ctx, B, T, H, W, sigma);
    if (rc) return rc;
    if (B == 0) return DRH_OK;
    if (!out_images || !backgrounds) return fail(DRH_ERR_INVALID_ARG, "output or background pointer is NULL");
    const RecordLayout L = record_layout(B, T, H, W);
    if ((rc = check_record(record, record_bytes, L))) return rc;
    DeviceGuard dg(ctx->device);
    hipStream_t s = (hipStream_t)stream;
    const bool host = flags & DRH_HOST_PTRS;
    Staged p, bg;
    Out img;
    if ((rc = stage_in(ctx, p, K_IN_PARAMS, params, (size_t)B * T * NP, host, s))) return rc;
    if ((rc = stage_in(ctx, bg, K_IN_BG, backgrounds, (size_t)B * 3, host, s))) return rc;
    if ((rc = stage_out(ctx, img, K_OUT_IMAGES, out_images, (size_t)B * H * W * 3, host, s))) return rc;
    char* base = static_cast<char*>(record);
    drh::RasterArgs a{};
    drh::set_sizes(a, (int)B, (int)T, (int)H, (int)W, sigma);
    a.rec = reinterpret_cast<float*>(base + L.rec);
    a.bg = reinterpret_cast<float*>(base + L.bg);
    a.out_img = img.dev;
    a.pq = reinterpret_cast<float*>(base + L.pq);
    a.pze = reinterpret_cast<int2*>(base + L.pze);
    a.tl_ent = reinterpret_cast<drh::TileEnt*>(base + L.tl_ent);
    a.cap2 = L.cap2;
    a.tl_n = reinterpret_cast<int*>(base + L.tl_n);
    a.chw = (flags & DRH_CHANNELS_FIRST) ? 1 : 0;
    const dim3 grid = drh::raster_grid(a.B, a.W, a.H);
    drh::OrderArgs ord{};
    if (use_order(ctx, a.B, (int)grid.x, (int)grid.y)) ord = {reinterpret_cast<int*>(base + L.ord), (int)grid.x, (int)grid.y};
    a.perm_fwd = a.T <= FWD_ORDER_MAX_T ? ord.perm : nullptr;
    a.gx = (int)grid.x;
    a.gy = (int)grid.y;
    a.nseg = 1;
    {
        KernelTimer kt(ctx, TK_SETUP);
        const drh::RecordHead head = make_head(B, T, H, W, sigma, flags);
        HIP_TRY(drh::launch_setup(p.dev, a.B, a.T, a.W, a.H, sigma, drh::SETUP_RECORD, const_cast<float*>(a.rec),
                                  nullptr, s, bg.dev, const_cast<float*>(a.bg), ord, nullptr,
                                  reinterpret_cast<drh::RecordHead*>(base + L.head), head),
                "setup_records launch");
        remember_record(ctx, record, head);
    }
    {
        KernelTimer kt(ctx, TK_RASTER);
        HIP_TRY(drh::launch_forward(drh::MODE_RECORD, !(flags & DRH_EXACT_MATH), a, s), "forward_kernel launch");
    }
    if ((rc = copy_back(img, s))) return rc;
    return finish(flags, s);
}

int drh_backward_recorded(drh_ctx* ctx, const void* record, uint64_t record_bytes, const float* grad_images,
                          int64_t B, int64_t T, int64_t H, int64_t W, float sigma, float* out_grads, void* stream,
                          uint32_t flags) {
    int rc = check_shape(ctx, B, T, H, W, sigma);
    if (rc) return rc;
    if (B == 0 || T == 0) return DRH_OK;
    if (!out_grads) return fail(DRH_ERR_INVALID_ARG, "output pointer is NULL");
    const RecordLayout L = record_layout(B, T, H, W);
    if ((rc = check_record(record, record_bytes, L))) return rc;
    DeviceGuard dg(ctx->device);
    hipStream_t s = (hipStream_t)stream;
    if ((rc = check_record_head(ctx, record, make_head(B, T, H, W, sigma, flags), s))) return rc;
    const bool host = flags & DRH_HOST_PTRS;
    const bool det = (flags & DRH_DETERMINISTIC) != 0;
    Staged gi;
    Out grads;
    Lease partials;
    if ((rc = stage_in(ctx, gi, K_IN_IMAGES, grad_images, (size_t)B * H * W * 3, host, s))) return rc;
    if ((rc = stage_out(ctx, grads, K_OUT_GRADS, out_grads, (size_t)B * T * NP, host, s))) return rc;
    const dim3 grid = drh::raster_grid((int)B, (int)W, (int)H);
    const int nblk = (int)(grid.x * grid.y);
    if (det && (rc = partials.acquire(ctx, K_PARTIALS, (size_t)B * nblk * T * NP * sizeof(float), s))) return rc;
    const char* base = static_cast<const char*>(record);
    drh::RasterArgs a{};
    drh::set_sizes(a, (int)B, (int)T, (int)H, (int)W, sigma);
    a.rec = reinterpret_cast<const float*>(base + L.rec);
    a.bg = reinterpret_cast<const float*>(base + L.bg);
    a.grad_in = gi.dev;
    a.partials = partials.get<float>();
    // read only by the backward kernel; the casts follow RasterArgs' field types
    a.pq = reinterpret_cast<float*>(const_cast<char*>(base + L.pq));
    a.pze = reinterpret_cast<int2*>(const_cast<char*>(base + L.pze));
    a.tl_ent = reinterpret_cast<drh::TileEnt*>(const_cast<char*>(base + L.tl_ent));
    a.cap2 = L.cap2;
    a.tl_n = reinterpret_cast<int*>(const_cast<char*>(base + L.tl_n));
    // the block order the record's setup made (use_order decides alike)
    if (use_order(ctx, a.B, (int)grid.x, (int)grid.y)) a.perm_bwd = reinterpret_cast<const int*>(base + L.ord);
    a.gx = (int)grid.x;
    a.gy = (int)grid.y;
    a.nseg = 1;
    a.grads = grads.dev;
    a.deterministic = det ? 1 : 0;
    a.chw = (flags & DRH_CHANNELS_FIRST) ? 1 : 0;
    if (!det) {
        KernelTimer kt(ctx, TK_SETUP);
        HIP_TRY(drh::launch_zero(grads.dev, (size_t)B * T * NP, s), "zero_floats launch");
    }
    {
        KernelTimer kt(ctx, TK_BACKWARD);
        HIP_TRY(drh::launch_backward(drh::MODE_GRAD_IN, !(flags & DRH_EXACT_MATH), L.cap2 < T, a, s),
                "backward_kernel launch");
    }
    if (det) {
        KernelTimer kt(ctx, TK_REDUCE);
        HIP_TRY(drh::launch_reduce(a.partials, nullptr, a.B, nblk, 1, a.T, 3.0 * a.H * (double)a.W, grads.dev, nullptr, s),
                "reduce_partials launch");
    }
    if ((rc = copy_back(grads, s))) return rc;
    return finish(flags, s);
}

int drh_adam_project_step(drh_ctx* ctx, float* params, const float* grads, float* m, float* v, const float* lr,
                          int64_t n, uint32_t step, float beta1, float beta2, float eps, int project, void* stream,
                          uint32_t flags) {
    if (!ctx) return fail(DRH_ERR_INVALID_ARG, "context is NULL");
    if (n < 0 || n > INT32_MAX) return fail(DRH_ERR_INVALID_ARG, "bad parameter count");
    if (project && n % NP != 0) return fail(DRH_ERR_INVALID_ARG, "projection needs whole triangles (n % 10 == 0)");
    if (step == 0) return fail(DRH_ERR_INVALID_ARG, "step counts from 1");
    if (n == 0) return DRH_OK;
    if (!params || !grads || !m || !v || !lr) return fail(DRH_ERR_INVALID_ARG, "NULL array");
    DeviceGuard dg(ctx->device);
    hipStream_t s = (hipStream_t)stream;
    bool host = flags & DRH_HOST_PTRS;
    // optim.rs:309-310 bias corrections
    float bc1 = 1.0f - powi_f32(beta1, (int32_t)step);
    float bc2 = 1.0f - powi_f32(beta2, (int32_t)step);
    int rc;
    Staged g, l, pin, min_, vin;
    if ((rc = stage_in(ctx, g, K_IN_IMAGES, grads, (size_t)n, host, s))) return rc;
    if ((rc = stage_in(ctx, l, K_IN_BG, lr, (size_t)n, host, s))) return rc;
    if ((rc = stage_in(ctx, pin, K_IN_PARAMS, params, (size_t)n, host, s))) return rc;
    if ((rc = stage_in(ctx, min_, K_FIT_F32, m, (size_t)n, host, s))) return rc;
    if ((rc = stage_in(ctx, vin, K_OUT_GRADS, v, (size_t)n, host, s))) return rc;
    float* dp = const_cast<float*>(pin.dev);
    float* dm = const_cast<float*>(min_.dev);
    float* dv = const_cast<float*>(vin.dev);
    {
        KernelTimer kt(ctx, TK_ADAM);
        HIP_TRY(drh::launch_adam(dp, g.dev, dm, dv, l.dev, (int)n, beta1, beta2, eps, bc1, bc2, project, s),
                "adam_project launch");
    }
    if (host) {
        HIP_TRY(hipMemcpyAsync(params, dp, n * sizeof(float), hipMemcpyDeviceToHost, s), "hipMemcpyAsync D2H");
        HIP_TRY(hipMemcpyAsync(m, dm, n * sizeof(float), hipMemcpyDeviceToHost, s), "hipMemcpyAsync D2H");
        HIP_TRY(hipMemcpyAsync(v, dv, n * sizeof(float), hipMemcpyDeviceToHost, s), "hipMemcpyAsync D2H");
    }
    return finish(flags, s);
}

int drh_encode_srgb(drh_ctx* ctx, const float* values, int64_t n, uint8_t* out, void* stream, uint32_t flags) {
    if (!ctx) return fail(DRH_ERR_INVALID_ARG, "context is NULL");
    if (n < 0) return fail(DRH_ERR_INVALID_ARG, "negative count");
    if (n == 0) return DRH_OK;
    if (!values || !out) return fail(DRH_ERR_INVALID_ARG, "NULL array");
    DeviceGuard dg(ctx->device);
    hipStream_t s = (hipStream_t)stream;
    const bool host = flags & DRH_HOST_PTRS;
    Staged in;
    int rc;
    if ((rc = stage_in(ctx, in, K_SRGB_F32, values, (size_t)n, host, s))) return rc;
    Lease ob;
    uint8_t* dout = out;
    if (host) {
        if ((rc = ob.acquire(ctx, K_SRGB_U8, (size_t)n, s))) return rc;
        dout = ob.get<uint8_t>();
    }
    HIP_TRY(drh::launch_encode_srgb(in.dev, n, dout, srgb_tables().thresholds, s), "encode_srgb launch");
    if (host) {
        hipError_t e = hipMemcpyAsync(out, dout, (size_t)n, hipMemcpyDeviceToHost, s);
        if (e != hipSuccess) return fail(DRH_ERR_READBACK, std::string("hipMemcpyAsync D2H: ") + hipGetErrorString(e));
    }
    return finish(flags, s);
}

int drh_decode_srgb(drh_ctx* ctx, const uint8_t* bytes, int64_t n, float* out, void* stream, uint32_t flags) {
    if (!ctx) return fail(DRH_ERR_INVALID_ARG, "context is NULL");
    if (n < 0) return fail(DRH_ERR_INVALID_ARG, "negative count");
    if (n == 0) return DRH_OK;
    if (!bytes || !out) return fail(DRH_ERR_INVALID_ARG, "NULL array");
    DeviceGuard dg(ctx->device);
    hipStream_t s = (hipStream_t)stream;
    const bool host = flags & DRH_HOST_PTRS;
    Lease ib;
    const uint8_t* din = bytes;
    int rc;
    if (host) {
        if ((rc = ib.acquire(ctx, K_SRGB_U8, (size_t)n, s))) return rc;
        HIP_TRY(hipMemcpyAsync(ib.get<uint8_t>(), bytes, (size_t)n, hipMemcpyHostToDevice, s), "hipMemcpyAsync H2D");
        din = ib.get<uint8_t>();
    }
    Out o;
    if ((rc = stage_out(ctx, o, K_SRGB_F32, out, (size_t)n, host, s))) return rc;
    HIP_TRY(drh::launch_decode_srgb(din, n, o.dev, srgb_tables().values, s), "decode_srgb launch");
    if ((rc = copy_back(o, s))) return rc;
    return finish(flags, s);
}

}  // extern "C"
