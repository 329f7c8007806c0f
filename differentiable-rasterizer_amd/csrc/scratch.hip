// drh_fused_loss_backward_noalloc: drh_fused_loss_backward for callers that
// cannot allocate device memory (code under HIP graph capture, tight serving
// loops, harnesses that forbid hipMalloc). Its buffers besides the caller's
// inputs and outputs (triangle records, per-pixel hand-over, per-tile entry
// lists, loss partials, block order, and with DRH_DETERMINISTIC the partial
// gradient rows) live in one file-scope device array of SCRATCH_BYTES, which
// every GPU the library runs on holds until the process ends. The entry point
// calls no hipMalloc, hipFree or other allocating routine.
//
// In host code `scratch` is a host-side stand-in for the array, not a device
// address: scratch_init takes the device address once per device (with that
// device current) and only that address is used afterwards. Every call on a
// GPU shares that GPU's array, so the calls on one GPU are serialized: a call
// enqueues its launches under that GPU's mutex and then records the GPU's
// event on its stream, and a call on another stream first makes its stream
// wait for that event. Calls from several threads and streams therefore run
// one after another on the device. Under graph capture no event is recorded or
// waited for (an event of an eager call cannot order a graph's replays): the
// caller orders the replays of a captured call against other calls.

#include <hip/hip_runtime.h>

#include <memory>
#include <mutex>
#include <string>
#include <vector>

#include "runtime.h"

using drh::NP;
using namespace drh_rt;

constexpr size_t SCRATCH_BYTES = 128ull << 20;  // 128 MiB per GPU
static __device__ __align__(256) unsigned char scratch[SCRATCH_BYTES];

namespace {

// One per device: the device address of `scratch` and what orders the calls
// that share it.
struct DeviceSlot {
    void* addr = nullptr;
    std::mutex call;             // held while a call enqueues its launches
    hipEvent_t done = nullptr;   // recorded after the last call's last launch
    hipStream_t last = nullptr;  // the stream it was recorded on
    bool recorded = false;
};

std::mutex g_mu;
std::vector<std::unique_ptr<DeviceSlot>> g_dev;

DeviceSlot* device_slot(int device) {
    std::lock_guard<std::mutex> g(g_mu);
    return device >= 0 && (size_t)device < g_dev.size() ? g_dev[device].get() : nullptr;
}

// Offsets of the buffers of one call in the scratch array, each at a 256-byte
// boundary; the tile-entry lists take what the rest leaves (all T entries per
// tile when they fit, else fewer, and tiles past them rebuild their lists in
// the backward kernel).
struct ScratchLayout {
    size_t rec = 0, ploss = 0, pq = 0, pg0 = 0, pze = 0, tn = 0, order = 0, partials = 0, tent = 0, total = 0;
    int cap2 = 0;
    int segw = 0;  // fused_seg_kernel, as drh_fused_loss_backward takes it
    bool ordered = false;
};

ScratchLayout scratch_layout(const drh_ctx* ctx, int B, int T, int H, int W, bool det) {
    ScratchLayout L;
    const dim3 grid = drh::raster_grid(B, W, H);
    const size_t nblk = (size_t)grid.x * grid.y, ntiles = (size_t)B * nblk * drh::WAVES;
    auto up = [](size_t x) { return (x + 255) & ~(size_t)255; };
    size_t off = 0;
    L.rec = off;
    off = up(off + (size_t)B * T * drh::REC * sizeof(float));
    L.ploss = off;
    off = up(off + (size_t)B * nblk * drh::WAVES * sizeof(double));  // per tile
    L.pq = off;
    off = up(off + (size_t)B * H * W * sizeof(float));
    L.pg0 = off;
    off = up(off + (size_t)B * H * W * 3 * sizeof(float));
    L.pze = off;
    off = up(off + ntiles * 64 * sizeof(int2));
    L.tn = off;
    off = up(off + ntiles * 2 * sizeof(int));
    L.ordered = use_order(ctx, B, (int)grid.x, (int)grid.y);
    L.order = off;
    if (L.ordered) off = up(off + (size_t)B * nblk * sizeof(int));
    // the call takes fused_seg_kernel where drh_fused_loss_backward would
    const int seg_cap2 = drh::seg_cap2((int)T);
    L.segw = use_segments(drh::MODE_LOSS, ntiles, T) && fused_gradients(drh::MODE_LOSS, 1, seg_cap2, T)
                 ? drh::SEG_WAVES
                 : 0;
    L.partials = off;
    if (det) off = up(off + (size_t)B * nblk * (L.segw ? drh::WAVES : 1) * T * NP * sizeof(float));
    L.tent = off;
    const size_t left = SCRATCH_BYTES > off ? SCRATCH_BYTES - off : 0;
    // whole 64-byte lines per tile and one slot past T entries, as the fused kernel needs
    L.cap2 = tile_entries(ntiles, (T + 8) & ~7, left, 1);
    if (L.segw && (size_t)seg_cap2 * ntiles * sizeof(drh::TileEnt) <= left)
        L.cap2 = seg_cap2;
    else
        L.segw = 0;
    L.total = up(off + ntiles * (size_t)L.cap2 * sizeof(drh::TileEnt));
    return L;
}

}  // namespace

namespace drh_rt {

int scratch_init(int device) {
    std::lock_guard<std::mutex> g(g_mu);
    if (device < 0) return fail(DRH_ERR_DEVICE, "no device");
    if ((size_t)device >= g_dev.size()) g_dev.resize((size_t)device + 1);
    if (g_dev[device]) return DRH_OK;
    auto d = std::make_unique<DeviceSlot>();
    hipError_t e = hipGetSymbolAddress(&d->addr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !d->addr)
        return hip_fail(e != hipSuccess ? e : hipErrorInvalidSymbol, "hipGetSymbolAddress(scratch)");
    e = hipEventCreateWithFlags(&d->done, hipEventDisableTiming);
    if (e != hipSuccess) return hip_fail(e, "hipEventCreate (scratch)");
    g_dev[device] = std::move(d);
    return DRH_OK;
}

}  // namespace drh_rt

extern "C" {

int drh_fused_loss_backward_noalloc(drh_ctx* ctx, const float* params, const float* backgrounds,
                                    const float* targets, int64_t B, int64_t T, int64_t H, int64_t W, float sigma,
                                    float* out_losses, float* out_grads, float* out_images, void* stream,
                                    uint32_t flags) {
    int rc = check_shape(ctx, B, T, H, W, sigma);
    if (rc) return rc;
    if (flags & DRH_HOST_PTRS)
        return fail(DRH_ERR_INVALID_ARG, "drh_fused_loss_backward_noalloc takes device pointers only "
                                         "(host arrays would need staging buffers)");
    if (B == 0) return DRH_OK;
    if (!params && T > 0) return fail(DRH_ERR_INVALID_ARG, "input pointer is NULL");
    if (!targets || !out_losses || !backgrounds || (T > 0 && !out_grads))
        return fail(DRH_ERR_INVALID_ARG, "output, target or background pointer is NULL");
    const bool det = (flags & DRH_DETERMINISTIC) != 0;
    const ScratchLayout L = scratch_layout(ctx, (int)B, (int)T, (int)H, (int)W, det);
    if (L.total > SCRATCH_BYTES)
        return fail(DRH_ERR_TOO_LARGE, "these sizes need " + std::to_string(L.total) + " bytes of scratch; the " +
                                           "entry point that allocates nothing has " +
                                           std::to_string(SCRATCH_BYTES) + " (use drh_fused_loss_backward)");
    DeviceGuard dg(ctx->device);
    DeviceSlot* d = device_slot(ctx->device);
    if (!d) return fail(DRH_ERR_DEVICE, "scratch array not initialised on this device");
    char* base = static_cast<char*>(d->addr);
    hipStream_t s = (hipStream_t)stream;
    // one call at a time per device: see the head of this file
    std::lock_guard<std::mutex> one(d->call);
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    HIP_TRY(hipStreamIsCapturing(s, &cap), "hipStreamIsCapturing");
    const bool eager = cap == hipStreamCaptureStatusNone;
    if (eager && d->recorded && d->last != s) HIP_TRY(hipStreamWaitEvent(s, d->done, 0), "hipStreamWaitEvent (scratch)");
    RasterBufs bufs;
    bufs.rec = reinterpret_cast<float*>(base + L.rec);
    bufs.ploss = reinterpret_cast<double*>(base + L.ploss);
    bufs.pq = reinterpret_cast<float*>(base + L.pq);
    bufs.pg0 = reinterpret_cast<float*>(base + L.pg0);
    bufs.pze = reinterpret_cast<int2*>(base + L.pze);
    bufs.tn = reinterpret_cast<int*>(base + L.tn);
    bufs.order = L.ordered ? reinterpret_cast<int*>(base + L.order) : nullptr;
    bufs.partials = det ? reinterpret_cast<float*>(base + L.partials) : nullptr;
    bufs.tent = reinterpret_cast<drh::TileEnt*>(base + L.tent);
    bufs.cap2 = L.cap2;
    bufs.fused = fused_gradients(drh::MODE_LOSS, bufs.nseg, bufs.cap2, (int)T);
    bufs.segw = bufs.fused ? L.segw : 0;
    // Nothing in the scratch array needs to start at zero: every buffer is
    // written by this call's kernels before it is read (the gradients are the
    // caller's output and setup_records clears them).
    rc = run_raster_bufs(ctx, drh::MODE_LOSS, params, backgrounds, targets, (int)B, (int)T, (int)H, (int)W, sigma,
                         out_images, out_grads, out_losses, flags, bufs, s, nullptr, false);
    if (eager) {
        // also after a failed launch: whatever was enqueued is ordered before the next call
        hipError_t e = hipEventRecord(d->done, s);
        if (e != hipSuccess) return rc ? rc : hip_fail(e, "hipEventRecord (scratch)");
        d->recorded = true;
        d->last = s;
    }
    if (rc) return rc;
    if (flags & DRH_SYNC) HIP_TRY(hipStreamSynchronize(s), "hipStreamSynchronize");
    return DRH_OK;
}

}  // extern "C"
