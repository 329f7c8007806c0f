// Internal declarations shared by the host sources behind the C ABI
// (runtime.hip: context, pool, raster entry points; fit.hip: the fit loop and
// the step-wise fitter; scratch.hip: the entry point that allocates nothing;
// resize.hip: the Lanczos3 image resize).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

#include "diffrast_hip.h"
#include "kernels.h"

namespace drh_rt {

// Sets the calling thread's drh_last_error() message and returns `code`.
int fail(int code, const std::string& msg);
const char* last_error_text();
int hip_fail(hipError_t e, const char* what);

#define HIP_TRY(expr, what)                                       \
    do {                                                          \
        hipError_t _e = (expr);                                   \
        if (_e != hipSuccess) return ::drh_rt::hip_fail(_e, what); \
    } while (0)

// What a pooled buffer holds; part of the pool key so that, as in the
// reference pool (crates/diffrast-gpu/src/lib.rs:132-143), a buffer is only
// reused for the same purpose at exactly the same size.
enum Kind : uint64_t {
    K_REC = 1,
    K_PARTIALS,
    K_PLOSS,
    K_IN_PARAMS,
    K_IN_BG,
    K_IN_IMAGES,
    K_OUT_IMAGES,
    K_OUT_GRADS,
    K_OUT_LOSSES,
    K_FIT_F32,
    K_FIT_STATE,
    K_PIXSTATE,
    K_PIX_G0,
    K_PIX_ZE,
    K_TILE_ENT,
    K_TILE_N,
    K_SRGB_F32,
    K_SRGB_U8,
    K_ORDER,
    K_FIT_TARGET,
    K_RESIZE_U8,
    K_RESIZE_TAB,
    K_RESIZE_TMP,
    K_CKPT,
    K_ROWS,
};

// Bytes the pool keeps at least (crates/diffrast-gpu/src/lib.rs:123-130);
// buffers released beyond a context's limit are freed. The reference's 512 MiB
// suits a 24 GB card; a context keeps max(512 MiB, 1/32 of the device's memory)
// (9 GB on a 288 GB MI355X), so that batches of 64 scenes at 256x256 reuse
// their buffers instead of freeing them (a stream wait) on every call.
constexpr uint64_t POOL_BYTE_LIMIT = 512ull << 20;
constexpr uint64_t POOL_MEMORY_SHARE = 32;

struct PoolBuf {
    void* ptr = nullptr;
    size_t bytes = 0;
    hipEvent_t ev = nullptr;       // recorded when the last user released it (multi-stream)
    hipStream_t stream = nullptr;  // stream of that last use
    bool used = false;
    bool ev_recorded = false;      // `ev` marks the end of the last use
};

enum TimedKernel : int { TK_SETUP = 0, TK_RASTER, TK_REDUCE, TK_ADAM, TK_BACKWARD, TK_COUNT };
struct TimedLaunch {
    int kernel;
    hipEvent_t start, stop;
};

}  // namespace drh_rt

struct drh_ctx {
    int device = 0;
    int cus = 0;  // compute units of the device
    bool discrete = true;
    std::string info;
    std::mutex mu;
    std::unordered_map<uint64_t, std::vector<drh_rt::PoolBuf>> free_bufs;
    uint64_t hits = 0, misses = 0, bytes = 0;
    uint64_t pool_limit = drh_rt::POOL_BYTE_LIMIT;  // bytes the pool keeps (set by drh_create)
    // Set once buffers have been used on more than one stream. Until then
    // every use of a buffer is ordered by the one stream and releases record
    // no event (an event record costs a GPU-side marker per buffer per call).
    bool multi_stream = false;
    // kernel timing (drh_timing_enable / drh_timing_read)
    bool timing = false;
    std::vector<drh_rt::TimedLaunch> pending;
    // Heads of the forward records this context made (record address -> head),
    // so that drh_backward_recorded checks its arguments without reading the
    // device; a record made elsewhere has its head read from the device.
    std::unordered_map<const void*, drh::RecordHead> records;
};

namespace drh_rt {

inline uint64_t pool_key(uint64_t kind, size_t bytes) { return (kind << 56) | (uint64_t)bytes; }

// A buffer borrowed from the pool for the duration of one call (or of a
// fitter's life). Reuse on the stream of the last use is ordered by that
// stream. Once a context sees a second stream, releases record an event that a
// user on another stream waits for; at that first switch the device is
// synchronized once, since the earlier uses recorded none. Either way reuse
// never races queued work.
class Lease {
  public:
    Lease() = default;
    Lease(const Lease&) = delete;
    Lease& operator=(const Lease&) = delete;
    ~Lease() { release(); }

    int acquire(drh_ctx* ctx, uint64_t kind, size_t bytes, hipStream_t s);
    template <class T>
    T* get() const {
        return static_cast<T*>(buf_.ptr);
    }
    void release();

  private:
    drh_ctx* ctx_ = nullptr;
    uint64_t kind_ = 0;
    hipStream_t stream_ = nullptr;
    PoolBuf buf_;
};

// Restores the caller's current device on scope exit.
struct DeviceGuard {
    int prev = -1;
    bool ok = true;
    explicit DeviceGuard(int dev) {
        if (hipGetDevice(&prev) != hipSuccess) prev = -1;
        if (prev != dev) ok = hipSetDevice(dev) == hipSuccess;
    }
    ~DeviceGuard() {
        int cur = -1;
        if (prev >= 0 && hipGetDevice(&cur) == hipSuccess && cur != prev) (void)hipSetDevice(prev);
    }
};

// Host wait bounded like GpuRasterizer::POLL_TIMEOUT (crates/diffrast-gpu/src/lib.rs:229).
int wait_stream(hipStream_t s);

// Argument checks shared by the raster entry points, with the reference
// binding's messages (crates/diffrast-py/src/lib.rs:162-195).
int check_sizes(int64_t B, int64_t T, int64_t H, int64_t W);
int check_shape(drh_ctx* ctx, int64_t B, int64_t T, int64_t H, int64_t W, float sigma);

// Device view of an input array: the pointer itself, or a pooled copy.
struct Staged {
    Lease lease;
    const float* dev = nullptr;
};
int stage_in(drh_ctx* ctx, Staged& st, uint64_t kind, const float* src, size_t n, bool host, hipStream_t s);

// Device output: the caller's pointer, or a pooled buffer copied back by copy_back.
struct Out {
    Lease lease;
    float* dev = nullptr;
    float* host_dst = nullptr;
    size_t n = 0;
};
int stage_out(drh_ctx* ctx, Out& o, uint64_t kind, float* dst, size_t n, bool host, hipStream_t s);
int copy_back(Out& o, hipStream_t s);

// With host pointers, DRH_SYNC or DRH_PHASES: waits for the stream.
int finish(uint32_t flags, hipStream_t s);

// Host phases of one call under DRH_PHASES (drh_phases_read). lap() waits for
// the stream and charges the time since the previous lap to `phase`; publish()
// makes the laps the calling thread's last phases. Without the flag both do
// nothing.
enum Phase : int { PH_PACK = 0, PH_ALLOC, PH_DISPATCH, PH_READBACK, PH_COUNT };
class PhaseClock {
  public:
    PhaseClock(uint32_t flags, hipStream_t s);
    int lap(int phase);
    void publish() const;

  private:
    bool on_;
    hipStream_t s_;
    double t_ = 0.0;
    double ms_[PH_COUNT] = {};
};

// f32::powi with a runtime exponent (square-and-multiply, as the
// compiler-builtins __powisf2 that the reference's Adam calls).
float powi_f32(float a, int32_t b);

// Brackets one kernel launch with events when the context is timing.
class KernelTimer {
  public:
    KernelTimer(drh_ctx* ctx, int kernel, bool enabled = true);
    ~KernelTimer();

  private:
    drh_ctx* ctx_;
    TimedLaunch l_{};
    bool on_ = false;
};

// Entries the forward kernel records per tile: all T while that fits `budget`
// bytes, else as many as fit (at least `min_cap`); DRH_MAX_TILE_ENTRIES in the
// environment lowers the cap, so tests can force the rebuild path.
constexpr size_t TILE_ENT_BUDGET = 1ull << 30;
int tile_entries(size_t ntiles, int T, size_t budget = TILE_ENT_BUDGET, size_t min_cap = drh::CAP2_MIN);

// The forward kernel follows the block order when its lists are short.
constexpr int FWD_ORDER_MAX_T = 256;
bool use_order(const drh_ctx* ctx, int B, int gx, int gy);

// Device buffers of one raster call besides its inputs and outputs.
struct RasterBufs {
    float* rec = nullptr;           // B*T*REC
    float* partials = nullptr;      // B*nblk*T*NP (deterministic gradient modes)
    double* ploss = nullptr;        // B*nblk (gradient modes)
    float* pq = nullptr;            // B*H*W (gradient modes)
    float* pg0 = nullptr;           // B*H*W*3 (MODE_LOSS)
    int2* pze = nullptr;            // ntiles*64 (gradient modes)
    drh::TileEnt* tent = nullptr;   // ntiles*cap2 (gradient modes)
    int* tn = nullptr;              // ntiles*2 (gradient modes)
    int* order = nullptr;           // B*nblk, or null: launch order
    int cap2 = 0;
    float* ckpt = nullptr;          // split backward's checkpoints, or null: no split
    int nseg = 1, seg_m = 0, nsplit = 0;  // its segments, entries per segment, split blocks per scene
    bool fused = false;             // one fused kernel (fused_gradients); pq, pg0, pze, tn unused
    bool order_tiles = false;       // `order` ranks 8x8 tiles (one-wave fused kernel only), not blocks
    int* rows = nullptr;            // with order_tiles: B*2gy*T triangle indices per 8x8-tile row, or null
    int* row_n = nullptr;           // B*2gy counts
    int segw = 0;                   // fused_seg_kernel's waves per tile (RasterArgs::segw), or 0
};

// fused_seg_kernel takes the gradient calls (fused, outside the split backward)
// whose grids hold at most SEG_MAX_TILES 8x8 tiles, two per SIMD of the
// device: there the one-wave kernel runs about one wave per SIMD, bound by
// each tile's chain of dependent waits, and splitting a tile's triangles over
// SEG_WAVES waves shortens that chain. From SEG_MIN_T triangles (a couple per
// wave) up to drh::SEG_MAX_T. DRH_NO_SEGMENTS=1 in the environment keeps the
// other fused kernels (for comparing the paths).
constexpr size_t SEG_MAX_TILES = 2048;
constexpr int SEG_MIN_T = 2 * drh::SEG_WAVES;
bool use_segments(int mode, size_t ntiles, int T);

// The one-wave fused kernel's lists scan the triangles of their tile row
// (OrderArgs::rows) from this many triangles on. Below it a tile's box tests
// are at most a few passes of 64 and making the row lists costs setup_records
// more than it saves (measured at T = 128: +3.3 us of setup, the fused kernel
// unchanged; at T = 512 with small triangles the fused kernel 35.7 -> 31.7 us).
constexpr int ROW_LISTS_MIN_T = 256;

// Split of the backward's sweep over a tile's recorded entries. A tile's sweep
// is sequential, and the tiles with the longest lists sit together (a block's
// four tiles are alike). A grid that does not fill the device (fewer blocks
// than SPLIT_MAX_BLOCKS_PER_CU per compute unit) runs about one round of
// blocks, so its heaviest blocks bound the backward kernel's time: there the
// heaviest quarter of each scene's blocks by setup_records' estimate get
// SPLIT_SEGMENTS waves per tile, each over ceil(T / SPLIT_DIVISOR) entries (the
// last to the end), from checkpoints the forward kernel leaves. A grid of
// several rounds is bound by throughput instead, and the split's extra blocks
// and checkpoints only cost time there (measured: B=16 256x256 T=128). Used
// with a block order, when gradients are summed with atomics and every entry
// is recorded (the backward's variant with neither fixed-order sums nor the
// rebuild path) and T is large enough for long lists; 1 (no split) otherwise.
constexpr int SPLIT_SEGMENTS = 3, SPLIT_DIVISOR = 6, SPLIT_MIN_T = 48, SPLIT_BLOCK_SHARE = 4,
              SPLIT_MAX_BLOCKS_PER_CU = 6;
int backward_segments(int T, int cap2, bool det, size_t blocks, int cus);

// The shared raster sequence over given buffers: records, the forward pass,
// and (gradient modes) the backward pass and the partial-row reduction. With
// `halt`, every kernel does nothing once *halt >= 0.
// `timed`: the launches take part in drh_timing_* (events are created for them).
// Whether a gradient-mode call runs as one fused kernel (forward and backward
// sweeps of each block together, both in the backward's block order): when
// every list is recorded whole in line-aligned regions (cap2 >= T, cap2 % 8 ==
// 0) and without the split backward (which a grid too small to fill the
// device takes instead). DRH_UNFUSED=1 in the environment keeps the two
// kernels (for comparing the two paths).
bool fused_gradients(int mode, int nseg, int cap2, int T);

// `tail` (the fit loop, deterministic MODE_LOSS, B = 1): fit_step in place of
// reduce_partials, the iteration's bookkeeping and Adam in the same kernel.
int run_raster_bufs(drh_ctx* ctx, int mode, const float* params, const float* bgs, const float* img_in, int B,
                    int T, int H, int W, float sigma, float* out_img, float* out_grads, float* out_losses,
                    uint32_t flags, const RasterBufs& bufs, hipStream_t s, const int* halt = nullptr,
                    bool timed = true, const drh::FitTail* tail = nullptr);

// run_raster_bufs over pooled buffers.
int run_raster(drh_ctx* ctx, int mode, const float* params, const float* bgs, const float* img_in, int B, int T,
               int H, int W, float sigma, float* out_img, float* out_grads, float* out_losses, uint32_t flags,
               hipStream_t s, const int* halt = nullptr, const drh::FitTail* tail = nullptr);

// Called by drh_create with the context's device current: takes the device
// address of the scratch array of drh_fused_loss_backward_noalloc on that
// device (once per device).
int scratch_init(int device);

}  // namespace drh_rt
