// Issue cost of wave64 instruction classes on one gfx950 SIMD, from streams of
// independent operations: 4096 workgroups of 256 threads (8 waves per SIMD on
// 256 CUs), each wave running `iters` x (16 x 8) instructions of a stream on
// eight independent registers. Prints SIMD cycles per instruction, taking the
// shader clock from s_memtime against the 100 MHz s_memrealtime over each run.
//
// Build: hipcc --offload-arch=gfx950 -O3 -Xclang -target-feature -Xclang -packed-fp32-ops
//        issue_cost.hip -o issue_cost
//
// The raster kernels' cost model follows from what this prints: plain VGPR
// arithmetic issues about every 2 cycles, while an operand read from an SGPR,
// compares, selects, min/max/med3, shifts, conversions and transcendentals
// occupy about 4 (8 for transcendentals) unless mixed with plain arithmetic.
#include <hip/hip_runtime.h>
#include <cstdio>

#define R8(S) S S S S S S S S
#define OUTS "+v"(v0), "+v"(v1), "+v"(v2), "+v"(v3), "+v"(v4), "+v"(v5), "+v"(v6), "+v"(v7)
#define ALL8(I) I("%0") I("%1") I("%2") I("%3") I("%4") I("%5") I("%6") I("%7")

// One stream step over the eight registers, per instruction form.
#define ADD(d) "v_add_f32 " d ", " d ", %8\n"
#define FMA(d) "v_fma_f32 " d ", " d ", %8, %9\n"
#define FMA_S(d) "v_fma_f32 " d ", " d ", %8, %10\n"
#define MUL_S(d) "v_mul_f32_e64 " d ", " d ", %10\n"
#define MAXV(d) "v_max_f32 " d ", " d ", %8\n"
#define CMP(d) "v_cmp_lt_f32_e64 s[60:61], " d ", %8\n"
#define CND(d) "v_cndmask_b32_e64 " d ", " d ", %8, %11\n"
#define LSHL(d) "v_lshlrev_b32 " d ", 1, " d "\n"
#define CVT(d) "v_cvt_f32_i32 " d ", " d "\n"
#define EXP(d) "v_exp_f32 " d ", " d "\n"
#define ADD_MAX(d) "v_add_f32 " d ", " d ", %8\nv_max_f32 " d ", " d ", %8\n"
#define ADD_FMAS(d) "v_add_f32 " d ", " d ", %8\nv_fma_f32 " d ", " d ", %8, %10\n"
#define ADD7_EXP(d) "v_add_f32 " d ", " d ", %8\n"
#define SADD(d) "s_add_u32 " d ", " d ", %8\n"
#define SOUTS "+s"(u0), "+s"(u1), "+s"(u2), "+s"(u3), "+s"(u4), "+s"(u5), "+s"(u6), "+s"(u7)
#define VS(d) "v_add_f32 " d ", " d ", %16\n"
#define SV(d) "s_add_u32 " d ", " d ", %17\n"
#define ALL8S(I) I("%8") I("%9") I("%10") I("%11") I("%12") I("%13") I("%14") I("%15")

template <int KIND>
__global__ void __launch_bounds__(256) stream(float* out, int iters, float s, unsigned long long* clk) {
    float v0 = threadIdx.x, v1 = v0 + 1, v2 = v0 + 2, v3 = v0 + 3, v4 = v0 + 4, v5 = v0 + 5, v6 = v0 + 6,
          v7 = v0 + 7;
    const float w = threadIdx.x * 0.5f, w2 = w + 0.25f;
    const unsigned long long m = __ballot(threadIdx.x & 1);
    uint32_t u0 = __builtin_amdgcn_readfirstlane(iters), u1 = u0 + 1, u2 = u0 + 2, u3 = u0 + 3, u4 = u0 + 4,
             u5 = u0 + 5, u6 = u0 + 6, u7 = u0 + 7;
    const uint32_t su = __builtin_amdgcn_readfirstlane(blockIdx.x);
    const unsigned long long c0 = clock64(), r0 = wall_clock64();
    for (int i = 0; i < iters; ++i) {
        // 128 instructions per iteration (512 for the add/exp mix)
        if (KIND == 0) asm volatile(R8(ALL8(ADD) ALL8(ADD)) : OUTS : "v"(w), "v"(w2), "s"(s), "s"(m) : "s60", "s61");
        if (KIND == 1) asm volatile(R8(ALL8(FMA) ALL8(FMA)) : OUTS : "v"(w), "v"(w2), "s"(s), "s"(m) : "s60", "s61");
        if (KIND == 2) asm volatile(R8(ALL8(FMA_S) ALL8(FMA_S)) : OUTS : "v"(w), "v"(w2), "s"(s), "s"(m) : "s60", "s61");
        if (KIND == 3) asm volatile(R8(ALL8(MUL_S) ALL8(MUL_S)) : OUTS : "v"(w), "v"(w2), "s"(s), "s"(m) : "s60", "s61");
        if (KIND == 4) asm volatile(R8(ALL8(MAXV) ALL8(MAXV)) : OUTS : "v"(w), "v"(w2), "s"(s), "s"(m) : "s60", "s61");
        if (KIND == 5) asm volatile(R8(ALL8(CMP) ALL8(CMP)) : OUTS : "v"(w), "v"(w2), "s"(s), "s"(m) : "s60", "s61");
        if (KIND == 6) asm volatile(R8(ALL8(CND) ALL8(CND)) : OUTS : "v"(w), "v"(w2), "s"(s), "s"(m) : "s60", "s61");
        if (KIND == 7) asm volatile(R8(ALL8(LSHL) ALL8(LSHL)) : OUTS : "v"(w), "v"(w2), "s"(s), "s"(m) : "s60", "s61");
        if (KIND == 8) asm volatile(R8(ALL8(CVT) ALL8(CVT)) : OUTS : "v"(w), "v"(w2), "s"(s), "s"(m) : "s60", "s61");
        if (KIND == 9) asm volatile(R8(ALL8(EXP) ALL8(EXP)) : OUTS : "v"(w), "v"(w2), "s"(s), "s"(m) : "s60", "s61");
        if (KIND == 10) asm volatile(R8(ALL8(ADD_MAX)) : OUTS : "v"(w), "v"(w2), "s"(s), "s"(m) : "s60", "s61");
        if (KIND == 11) asm volatile(R8(ALL8(ADD_FMAS)) : OUTS : "v"(w), "v"(w2), "s"(s), "s"(m) : "s60", "s61");
        if (KIND == 12)  // 7 adds and one exp per register: 8 x 64 instructions
            asm volatile(R8(ALL8(ADD7_EXP) ALL8(ADD7_EXP) ALL8(ADD7_EXP) ALL8(ADD7_EXP) ALL8(ADD7_EXP) ALL8(ADD7_EXP)
                                ALL8(ADD7_EXP) ALL8(EXP)) : OUTS : "v"(w), "v"(w2), "s"(s), "s"(m) : "s60", "s61");
        // s_add_u32 writes SCC, which the loop's own compare and branch use
        if (KIND == 13) asm volatile(R8(ALL8(SADD) ALL8(SADD)) : SOUTS : "s"(su) : "scc");
        if (KIND == 14)  // a scalar add beside every vector add: 128 of each
            asm volatile(R8(ALL8(VS) ALL8S(SV) ALL8(VS) ALL8S(SV)) : OUTS, SOUTS : "v"(w), "s"(su) : "scc");
    }
    const unsigned long long c1 = clock64(), r1 = wall_clock64();
    v0 += (float)(u0 + u1 + u2 + u3 + u4 + u5 + u6 + u7);
    out[(size_t)blockIdx.x * blockDim.x + threadIdx.x] = v0 + v1 + v2 + v3 + v4 + v5 + v6 + v7;
    if (threadIdx.x == 0) {
        clk[2 * blockIdx.x] = c1 - c0;
        clk[2 * blockIdx.x + 1] = r1 - r0;
    }
}

#define CHECK(x)                                                                           \
    do {                                                                                   \
        hipError_t e_ = (x);                                                               \
        if (e_ != hipSuccess) {                                                            \
            printf("HIP error %s at line %d\n", hipGetErrorString(e_), __LINE__);          \
            return 1;                                                                      \
        }                                                                                  \
    } while (0)

constexpr int BLOCKS = 4096, ITERS = 100, SIMDS = 1024;

template <int KIND>
int run(const char* name, int per_iter, float* out, unsigned long long* clk, unsigned long long* host) {
    hipEvent_t e0, e1;
    CHECK(hipEventCreate(&e0));
    CHECK(hipEventCreate(&e1));
    float best = 1e30f;
    for (int rep = 0; rep < 3; ++rep) {
        CHECK(hipEventRecord(e0));
        stream<KIND><<<BLOCKS, 256>>>(out, ITERS, 0.5f, clk);
        CHECK(hipGetLastError());
        CHECK(hipEventRecord(e1));
        CHECK(hipEventSynchronize(e1));
        float ms;
        CHECK(hipEventElapsedTime(&ms, e0, e1));
        best = ms < best ? ms : best;
    }
    CHECK(hipMemcpy(host, clk, sizeof(unsigned long long) * 2 * BLOCKS, hipMemcpyDeviceToHost));
    double cyc = 0, rt = 0;
    for (int i = 0; i < BLOCKS; ++i) {
        cyc += (double)host[2 * i];
        rt += (double)host[2 * i + 1];
    }
    const double ghz = cyc / rt * 0.1;
    const double per_simd = (double)BLOCKS * 4 * ITERS * per_iter / SIMDS;
    printf("%-34s %8.4f ms  %5.3f GHz  %5.2f cycles/instr\n", name, best, ghz, best * 1e-3 * ghz * 1e9 / per_simd);
    return 0;
}

int main() {
    setvbuf(stdout, nullptr, _IOLBF, 0);
    float* out;
    unsigned long long* clk;
    CHECK(hipMalloc(&out, sizeof(float) * BLOCKS * 256));
    CHECK(hipMalloc(&clk, sizeof(unsigned long long) * 2 * BLOCKS));
    unsigned long long* host = new unsigned long long[2 * BLOCKS];
    for (int i = 0; i < 20; ++i) stream<0><<<BLOCKS, 256>>>(out, ITERS, 0.5f, clk);
    CHECK(hipDeviceSynchronize());
    int rc = 0;
    rc |= run<0>("v_add_f32 v, v", 128, out, clk, host);
    rc |= run<1>("v_fma_f32 v, v, v", 128, out, clk, host);
    rc |= run<2>("v_fma_f32 v, v, s", 128, out, clk, host);
    rc |= run<3>("v_mul_f32 v, s", 128, out, clk, host);
    rc |= run<4>("v_max_f32 v, v", 128, out, clk, host);
    rc |= run<5>("v_cmp_lt_f32 -> s[2]", 128, out, clk, host);
    rc |= run<6>("v_cndmask_b32 v, v, s[2]", 128, out, clk, host);
    rc |= run<7>("v_lshlrev_b32", 128, out, clk, host);
    rc |= run<8>("v_cvt_f32_i32", 128, out, clk, host);
    rc |= run<9>("v_exp_f32", 128, out, clk, host);
    rc |= run<10>("mix: v_add + v_max", 128, out, clk, host);
    rc |= run<11>("mix: v_add + v_fma v, v, s", 128, out, clk, host);
    rc |= run<12>("mix: 7 v_add + 1 v_exp", 512, out, clk, host);
    rc |= run<13>("s_add_u32 (per SIMD: 8 waves)", 128, out, clk, host);
    rc |= run<14>("mix: v_add + s_add (per pair)", 128, out, clk, host);
    delete[] host;
    return rc;
}
