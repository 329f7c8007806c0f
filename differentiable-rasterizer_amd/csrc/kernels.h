// Shared definitions between the HIP kernels and the host runtime.
#pragma once

#include <cmath>

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace drh {

constexpr int NP = 10;    // parameters per triangle (scene.rs:21)
constexpr int TILE = 8;   // a wave covers an 8x8 pixel tile, one pixel per lane
constexpr int WAVES = 4;  // waves per block: 2x2 tiles, a 16x16 pixel region
constexpr int CH = 128;   // triangles per chunk (LDS accumulators are per chunk)
static_assert((CH * NP) % 4 == 0, "accumulator rows are cleared and summed four floats at a time");

// Per-triangle record, REC floats, written by setup_records. The hot loops
// load fields [0, REC_HOT) of one record per list entry; the rest is read
// only while building a tile's list.
constexpr int REC = 76;
constexpr int REC_HOT = 40;
enum RecField : int {
    R_V = 0,       // 6: vertices x0 y0 x1 y1 x2 y2
    R_C = 6,       // 3: colour
    R_A = 9,       // clamped alpha (NaN preserved)
    R_BOX = 10,    // 4 ints: x0 y0 x1 y1, half-open; all 0 when not live
    R_FLAGS = 14,  // int: F_*
    R_SPARE = 15,
    R_E = 16,      // 6: edge vectors b - a for (v0,v1) (v1,v2) (v2,v0)
    R_LEN2 = 22,   // 3: |e|^2
    R_RLEN2 = 25,  // 3: 1/|e|^2, 0 when |e|^2 <= 1e-20
    R_N = 28,      // 6: outward unit normals (0 when the fast path is off)
    R_OFF = 34,    // 3: a . n per edge
    R_FAR = 37,    // max outward distance above which w < MIN_WEIGHT
    R_DEEP = 38,   // max outward distance below which coverage == 1.0f
    R_SLACK = 39,  // rounding slack of the edge-line distances
    R_D = 40,      // 6: unit edge directions (fast path only)
    R_SOFF = 46,   // 3: a . d per edge
    R_LEN = 49,    // 3: |e|
    R_EB = 52,     // 3 x 8: per edge a.x a.y e.x e.y |e|^2 1/|e|^2 (+-1: F_CCW) 0 (scalar-loaded by edge index)
};
// F_CCW: the cross products of inside points are >= 0 (else <= 0).
// F_LIVE: drawn by this call's forward pass. F_TAPE: live for the taped forward
// of the gradient paths, which culls a NaN alpha that a render composites; it
// differs from F_LIVE only in records made by a render kept for a backward.
enum : int { F_LIVE = 1, F_ACTIVE = 2, F_FAST = 4, F_CCW = 8, F_TAPE = 16 };

// MODE_RECORD is a forward pass only: MODE_RENDER's image plus MODE_GRAD_IN's
// hand-over to the backward kernel, for a render whose backward comes later.
enum : int { MODE_RENDER = 0, MODE_LOSS = 1, MODE_GRAD_IN = 2, MODE_RECORD = 3 };
// setup_records liveness: a render's, the taped forward's, or a render's with
// F_TAPE marking the taped forward's (MODE_RECORD).
enum : int { SETUP_RENDER = 0, SETUP_TAPE = 1, SETUP_RECORD = 2 };

// Contributing entries the forward kernel records per tile for the backward
// kernel (over all chunks) are RasterArgs::cap2, at least CAP2_MIN. When cap2
// covers T every tile's list is recorded whole and the backward kernel is the
// variant without the rebuild path; otherwise a tile past cap2 rebuilds and
// reclassifies its remaining chunks there.
constexpr int CAP2_MIN = 128;

// fused_seg_kernel: waves per tile, and the most triangles per scene (its LDS
// holds a 288-byte record per triangle of the scene, 45 KB at 160). Eight
// waves measured faster than four (B=1 64x64 T=32: 18.0 -> 15.3 us; the
// 176x176 T=150 fit: 26.4 -> 23.4 us per iteration).
constexpr int SEG_WAVES = 8;
constexpr int SEG_MAX_T = 160;
// Its entry region per tile: SEG_WAVES segments of whole 64-byte lines (8
// entries) of more than T / SEG_WAVES entries each, so that cap2 > T, as the
// fused paths require.
__host__ __device__ constexpr int seg_cap2(int T) { return SEG_WAVES * (((T + SEG_WAVES - 1) / SEG_WAVES + 8) & ~7); }
// A loss slot not yet written (RasterArgs::loss_tail): a signalling NaN with
// the lowest mantissa bit set. Arithmetic only returns quiet NaNs, and NaNs
// that reach the loss from float inputs have their low 29 mantissa bits clear,
// so no partial loss has these bits.
constexpr uint64_t LOSS_PENDING = 0xFFF4C0DE5EED0001ull;

// One recorded entry of a tile's list, written by the forward kernel and read
// (with scalar loads) by the backward kernel.
struct TileEnt {
    uint32_t k;     // (k << 8) | the list entry's low byte (kind bits, plan, edge-block offset, in-box bit)
    uint32_t row;   // byte offset of the triangle's row in a chunk's per-wave accumulator
    uint64_t on;    // lanes with w > MIN_WEIGHT
    uint64_t band;  // of those, lanes on the exact path
};
static_assert(sizeof(TileEnt) == 24, "TileEnt is read as 2 + 4 dwords");

// Per-pixel state the forward kernel hands to the backward kernel, field-major:
//   q   B*H*W floats: the pixel's total transmittance, the product of its
//       nonzero (1 - w) factors, kept in [2^-64, 1];
//   g0  B*H*W*3 floats: dL/dpixel (MODE_LOSS; MODE_GRAD_IN reads the caller's);
//   ze  per tile and lane: the count of zero factors and of 2^64 rescalings of
//       q, written only for a tile where some lane has either (TN_IRREGULAR set
//       in its tl_n[2 tile + 1]); zero for every other tile.
// 16 bytes per pixel in MODE_LOSS and 4 otherwise, against 24 with all five
// words per pixel: the counts are zero for nearly every pixel.
constexpr int TN_IRREGULAR = 1 << 30;

// The raster kernels' block order, made by setup_records (perm null: none):
// perm[b * gx*gy + r] is the scene-local index of scene b's r-th heaviest cell;
// gx, gy: cells per scene row and column, (gx + 1) * (gy + 1) <= ORD_MAX_CELLS.
// A cell is a 16x16 block (shift 4) or, for the one-wave fused kernel, an 8x8
// tile (shift 3; gx, gy then twice the blocks', so dead tiles of a partial
// block are cells too).
struct OrderArgs {
    int* perm;
    int gx, gy;
    int shift = 4;
    // Optional (the tile order, gy ceil(T / 32) <= ORD_ROW_WORDS): the live
    // triangles whose cull box meets each cell row, in index order:
    // rows[(b gy + y) T + i] for i < row_n[b gy + y].
    int* rows = nullptr;
    int* row_n = nullptr;
    // Scalings of the reach estimate, set by launch_setup from W, H and shift:
    // 1/H, a cell's height 2^shift / H, W / 2^shift, and the offsets of the
    // cell-index bounds (0.5 - 2^shift) / 2^shift and -0.5 / 2^shift.
    float r_h = 0, cell_h = 0, w_cells = 0, c0_off = 0, c1_off = 0;
};
constexpr int ORD_MAX_CELLS = 8192;
constexpr int ORD_ROW_WORDS = 2048;  // LDS bit-mask words of the row lists (one bit per triangle and row)

struct RasterArgs {
    int B, T, H, W;
    float sigma;
    // Wave-uniform quotients, divided once on the host (IEEE, as the kernels
    // would): rsig = 1 / max(sigma, 1e-8), lscale = 2 / (3 H W) (dL/dpixel).
    // Set with set_sizes, which also fills B, T, H, W and sigma.
    float rsig, lscale;
    const float* rec;      // B*T*REC
    const float* bg;       // B*3
    const float* target;   // B*H*W*3 (MODE_LOSS)
    const float* grad_in;  // B*H*W*3 (MODE_GRAD_IN)
    float* out_img;        // B*H*W*3 (MODE_RENDER, MODE_RECORD; optional in MODE_LOSS)
    float* partials;       // B*nblk*T*NP
    double* partial_loss;  // B*nblk
    float* pq;             // B*H*W total transmittance
    float* pg0;            // B*H*W*3 dL/dpixel (MODE_LOSS)
    int2* pze;             // ntiles*64 zero and rescaling counts (irregular tiles)
    TileEnt* tl_ent;       // ntiles*cap2 recorded entries
    int cap2;              // entries recorded per tile
    // fused_seg_kernel's waves per tile (SEG_WAVES), or 0: the fused path
    // takes the other kernels. cap2 is then SEG_WAVES x a multiple of 8, and
    // with DRH_DETERMINISTIC the partial rows and loss partials are per tile.
    int segw;
    int* tl_n;             // ntiles*2: entries recorded, chunks fully recorded | TN_IRREGULAR
    float* grads;          // B*T*NP, accumulated with atomics unless deterministic
    float* losses;         // B (MODE_LOSS)
    // MODE_LOSS, the fused kernels outside the fixed-order mode (one-wave and
    // segmented): the grid's last B workgroups sum each
    // scene's per-tile loss partials into `losses` (no sum_losses launch). The
    // tiles store their partials with device-scope atomic stores into slots
    // that setup_records filled with LOSS_PENDING, and each summing workgroup
    // polls its scene's slots (device-scope atomic loads) until none is pending.
    int loss_tail;
    int deterministic;     // per-block partial rows + reduce_partials instead of atomics
    int chw;               // images, targets and grad_in are B x 3 x H x W (else B x H x W x 3)
    const int* perm_fwd;   // block order of the forward kernel (OrderArgs::perm) or null
    const int* perm_bwd;   // block order of the backward kernel or null
    int perm_tiles;        // perm_bwd orders 8x8 tiles (one-wave fused kernel), not blocks
    // ceil(2^32 / (2 gx)), set by the one-wave fused kernel's launch: an ordered
    // tile's row in its scene's tile grid by one multiply-high instead of a division
    uint32_t tdiv_m;
    // OrderArgs::rows / row_n of 8x8-tile rows (row_gy per scene), or null:
    // the one-wave fused kernel's lists then scan every triangle
    const int* rows;
    const int* row_n;
    int row_gy;
    const int* halt;       // null, or a flag: every block returns at entry once it is >= 0
    // Split backward (nseg > 1, with a block order): in the nsplit heaviest
    // blocks of each scene, segment s of a tile's recorded entries,
    // [s seg_m, (s + 1) seg_m) (the last one to the end), is swept by its own
    // wave, starting from the pixel state the forward kernel checkpointed
    // before entry s seg_m: ckpt holds CKPT_WORDS x 64 words per (tile, s >= 1).
    int nseg;              // segments per split tile, 0 or 1: no split
    int seg_m;             // entries per segment
    int nsplit;            // split blocks per scene
    int gx, gy;            // blocks per scene row and column
    float* ckpt;           // ntiles * (nseg - 1) * CKPT_WORDS * 64
};

inline void set_sizes(RasterArgs& a, int B, int T, int H, int W, float sigma) {
    a.B = B;
    a.T = T;
    a.H = H;
    a.W = W;
    a.sigma = sigma;
    a.rsig = 1.0f / std::fmax(sigma, 1e-8f);
    a.lscale = 2.0f / (float)(3 * (size_t)W * H);
}

// A checkpoint word per lane: colour (3), transmittance q, zero count z and
// rescaling count e (as int bits).
constexpr int CKPT_WORDS = 6;

// Head of a forward record (drh_render_record), written by setup_records:
// what a later backward of the record must agree with.
constexpr uint32_t RECORD_MAGIC = 0x44524831u;  // "DRH1"
struct RecordHead {
    uint32_t magic;
    uint32_t exact;  // the forward ran with IEEE geometry (DRH_EXACT_MATH)
    float sigma;
    int32_t B, T, H, W;
    uint32_t pad;
};

// Device-side state of a running fit (fit.rs:197-211).
enum : int { STOP_COMPLETED = 0, STOP_CONVERGED = 1, STOP_DIVERGED = 2 };
struct FitState {
    float best_loss;
    int best_iter;
    int since;
    int n_losses;
    int stop;  // -1 while running, else STOP_*
};

// The fit loop's step after the deterministic raster kernels (fit_step): the
// partial rows' reduction, the fit bookkeeping and Adam with the projection.
// The state is double-buffered by iteration parity: iteration i reads st[i & 1]
// and its first block writes st[(i + 1) & 1], so every block decides from the
// same state; `halt` mirrors the stop code for the next iterations' kernels.
struct FitTail {
    int iter;
    float* loss;  // the iteration's loss (1 float)
    float *params, *grads, *m, *v;
    const float* lr;
    float beta1, beta2, eps, bc1, bc2, min_delta;
    long long patience;
    FitState* st;  // 2 states
    int* halt;
    float *losses_out, *best;
    // The fit's triangle records, or null (pooled per call). rec_ready: they
    // already hold this iteration's (the previous fit_step made them), so
    // setup_records is not launched. fit_step makes the next iteration's, at
    // sigma_next on the W x H canvas, from its updated parameters: a fit
    // iteration is then two kernels.
    float* rec;
    int rec_ready;
    float sigma_next;
    int W, H;
};
// fit_step's parameter columns per block: whole triangles, so that a block
// can make its triangles' records once it has updated them.
constexpr int FIT_TRIS = 6;

// Events that the calling thread's next kernel launch in this library takes
// as its start and stop (hipExtLaunchKernel: the kernel's own start and end,
// with no event packets of their own around it), or null; `used` is set by the
// launch. The runtime's per-kernel timing (drh_timing_enable) sets them.
struct LaunchEvents {
    hipEvent_t start = nullptr, stop = nullptr;
    bool used = false;
};
LaunchEvents& launch_events();

dim3 raster_grid(int B, int W, int H);
// nblk partial rows (and loss partials) per scene, loss_per of which form a
// block's loss (1, or WAVES for fused_seg_kernel's per-tile rows).
hipError_t launch_fit_step(const float* partials, const double* partial_loss, int nblk, int loss_per, int T,
                           double npix3, const FitTail& ft, hipStream_t s);
// bg_dst (optional) receives a copy of the B x 3 backgrounds at bg_src; with
// o.cnt, the block order is made (OrderArgs).
// halt (optional): the kernel does nothing once *halt >= 0 (a stopped fit).
// head (optional): receives head_val (a forward record's head).
hipError_t launch_setup(const float* params, int B, int T, int W, int H, float sigma, int setup_mode,
                        float* rec, float* zero_grads, hipStream_t s, const float* bg_src = nullptr,
                        float* bg_dst = nullptr, const OrderArgs& o = OrderArgs{}, const int* halt = nullptr,
                        RecordHead* head = nullptr, const RecordHead& head_val = RecordHead{},
                        double* pending = nullptr, int npending = 0);
// n floats set to zero by a kernel (no memset node, so callers may capture it).
hipError_t launch_zero(float* p, size_t n, hipStream_t s);
hipError_t launch_forward(int mode, bool fast, const RasterArgs& a, hipStream_t s);
hipError_t launch_backward(int mode, bool fast, bool rebuild, const RasterArgs& a, hipStream_t s);
// Forward and backward of a gradient mode in one kernel (hipErrorInvalidValue
// unless cap2 >= T, cap2 % 8 == 0 and no split); then launch_reduce
// (deterministic) or, in MODE_LOSS, launch_sum_losses forms the results from
// its per-block sums.
hipError_t launch_fused(int mode, bool fast, const RasterArgs& a, hipStream_t s);
// per: loss partials per block (1, or WAVES for the fused kernel's per-tile partials outside the
// deterministic mode; hipErrorInvalidValue otherwise, or for nblk < 1).
hipError_t launch_sum_losses(const double* partial_loss, int B, int nblk, int per, double npix3, float* losses,
                             hipStream_t s, const int* halt = nullptr);
// Loss partials per block that a gradient call's raster kernels write.
constexpr int loss_partials_per_block(bool fused, bool deterministic) { return fused && !deterministic ? WAVES : 1; }
// npix3: 3 H W, the divisor of the per-item loss (canvas.rs:45-58)
hipError_t launch_reduce(const float* partials, const double* partial_loss, int B, int nblk, int loss_per, int T,
                         double npix3, float* grads, float* losses, hipStream_t s, const int* halt = nullptr);
// 256 floats passed by value to the sRGB kernels: the byte thresholds of the
// encoding (entry k the smallest linear value whose byte is k; entry 0 unused)
// or the decoded value of each byte.
struct SrgbTable {
    float v[256];
};
hipError_t launch_encode_srgb(const float* in, int64_t n, uint8_t* out, const SrgbTable& thresholds, hipStream_t s);
hipError_t launch_decode_srgb(const uint8_t* in, int64_t n, float* out, const SrgbTable& values, hipStream_t s);

hipError_t launch_adam(float* params, const float* grads, float* m, float* v, const float* lr, int n,
                       float beta1, float beta2, float eps, float bc1, float bc2, int project,
                       hipStream_t s);

}  // namespace drh
