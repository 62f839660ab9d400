// Dequant GEMM for large batches (q4t_matmat / q4tp_matmat with b > 16,
// qtensor.rs:5830-5960 / 5422-5680, and the prefill's dense contractions):
// Y[b][n] = sum_k X[b][k] W[n][k] for b < M (any M), W in the q4t / q4tp
// device layout of the GEMV kernels.
//
// Tiling (MFMA f32 16x16x32 f16): a workgroup of 4 waves owns 64 batch rows
// x 64 GRB weight rows (wave w holds GRB row blocks in registers), and walks
// K in steps of 128 columns (4 tiles):
//   - the operand step (hi / lo f16 planes of 64 rows x 4 tiles and their
//     two tables of tile biases, 34 KiB) is loaded into registers one step ahead and
//     written to the other half of a double-buffered LDS tile after the
//     current step's MFMAs (one barrier per step);
//   - the weights of the next step (4 row blocks x 1 KiB + scales per wave)
//     are requested before the current step is computed;
//   - per tile and row block: the nibbles become f16 denormals n * 2^-24
//     (one mask per pair); the hi and lo planes (fixed point, prep16_row)
//     take one MFMA each, each started at its plane's tile bias
//     -8 * 2^-24 * sum (so D = 2^-24 * sum((n - 8) x) / xs exactly), and the
//     tile scale multiplies D in f32 as q4t_row_exact does
//     (qtensor.rs:4418-4432).
#include <mutex>
#include <set>

#include "gemv_kern.h"
#include "runtime.h"

namespace cmf {

struct GemmArgs {
    const void* w;        // [rb][group of 4 tiles][lane][16 B]   (q8: [rb][64-column chunk][lane][16 B])
    const void* scale;    // q4t f16 [rb][group][16][4]; q4tp u32 codes; q8 f32 row scales
    const float2* rowp;   // q4tp (2^lo, 2^step) per row
    const uint8_t* planes;  // hi [item][Mp], lo [item][Mp] (16 B), biases hi / lo [tile][Mp] f32 (q8: q0 q1 q2 [item][Mp])
    const float* xs;      // [Mp] 2^-e per batch row (q8: amax / 127)
    float* y;
    int ldy, M, Mp, N, ntg, nrb, resid;
    // split K: workgroup z takes K steps [z gsteps, (z + 1) gsteps) and
    // writes its partial sums to part [z][M][N] (part == nullptr: one part,
    // y written directly)
    int gsteps;
    float* part;
};

constexpr int GB = 64;             // batch rows per workgroup
constexpr int GCH = 34;            // 1 KiB operand chunks per K step (16 hi + 16 lo items, hi and lo biases)
constexpr int GJ = (GCH + 3) / 4;  // chunks per wave (clamped)
// k_gemm_q4's dynamic LDS: the operand tile [2][GCH][64] x 16 B, then the
// weight rows' tile scales [2][4 waves] x 1 KiB
constexpr size_t GEMM_AT_BYTES = (size_t)2 * GCH * 64 * 16 + (size_t)2 * 4 * 1024;

// s_waitcnt lgkmcnt(0) + s_barrier: an LDS-only workgroup barrier (the
// weight loads in flight are not waited for, as __syncthreads would)
__device__ __forceinline__ void lds_sync() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// GRB: row blocks per wave (4 for large batches; 1 gives small batches 4x
// the workgroups).
template <int FMT, int GRB>
__global__ __launch_bounds__(256, 2) void k_gemm_q4(GemmArgs a) {
    constexpr bool TP = FMT == DT_Q4TP;
    // the double-buffered operand tile [2][GCH chunks][64 lanes] x 16 B,
    // filled by direct global -> LDS loads (dynamic LDS: with a static array
    // as the load target the compiler waits for every load in flight before
    // each LDS read)
    extern __shared__ __align__(16) uint4 gemm_at[];
    __shared__ float lad[TP ? 4 : 1][TP ? GRB * 16 * 33 : 1];
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int r = lane & 15, s = lane >> 4;
    const int by = blockIdx.y, rbw = (blockIdx.x * 4 + wave) * GRB;  // first row block of this wave
    const int ntg = a.ntg, Mp = a.Mp;
    const size_t items = (size_t)ntg * 16;  // operand items (4 per tile)
    const uint4* PH = (const uint4*)a.planes;
    const uint4* PL = PH + items * Mp;
    const float* PB = (const float*)(PL + items * Mp);
    const float* PB2 = PB + (size_t)ntg * 4 * Mp;  // the lo plane's biases

    // operand chunk c of step g for this lane: 16 hi items, 16 lo items, the
    // hi biases, the lo biases.  One unconditional load per chunk, the source
    // picked by selects (a load under a branch makes the compiler wait for it
    // at once); chunk j of this wave is held in its own register quad (RA).
    auto src_a = [&](int j, int g) __attribute__((always_inline)) -> const uint4* {
        const int c = min(wave + 4 * j, GCH - 1);
        const uint4* ph = PH + (size_t)(16 * g + c) * Mp + GB * by + lane;
        const uint4* pl = PL + (size_t)(16 * g + c - 16) * Mp + GB * by + lane;
        const size_t bo = (size_t)(4 * g + (lane >> 4)) * Mp + GB * by + 4 * (lane & 15);
        const uint4* pb = (const uint4*)((c == 32 ? PB : PB2) + bo);
        return c < 16 ? ph : c < 32 ? pl : pb;
    };
    // chunk j of this wave in buffer buf: the wave-uniform 1 KiB it fills
    // (lane l's 16 bytes land at + 16 l); the clamped chunk (the lo biases)
    // is written by every wave with the same data
    auto dma_a = [&](int j, int g, int buf) __attribute__((always_inline)) {
        uint4* dst = gemm_at + ((size_t)buf * GCH + min(wave + 4 * j, GCH - 1)) * 64;
        __builtin_amdgcn_global_load_lds((const void*)src_a(j, g), (__attribute__((address_space(3))) void*)dst, 16,
                                         0, 0);
    };
    // weights of step g for the wave's row blocks (clamped to the last block)
    auto load_w = [&](uint4* wv, int g) __attribute__((always_inline)) {
#pragma unroll
        for (int q = 0; q < GRB; q++) {
            const size_t t = (size_t)min(rbw + q, a.nrb - 1) * ntg + g;
            wv[q] = ((const uint4*)a.w)[t * 64 + lane];
        }
    };
    // the tile scales of step g for the wave's rows into its 1 KiB of the
    // scale area (buffer buf) by one direct load: q4t 16 B per lane = two
    // rows' four f16 scales, lane l -> row block l / 8, rows 2 (l % 8) ..;
    // q4tp 4 B per lane = one row's four rung codes, lane l -> row block
    // l / 16, row l % 16 (lanes past the wave's rows repeat the last block)
    uint8_t* sarea = (uint8_t*)(gemm_at + (size_t)2 * GCH * 64);
    auto dma_s = [&](int g, int buf) __attribute__((always_inline)) {
        uint8_t* dst = sarea + (size_t)(buf * 4 + wave) * 1024;
        if constexpr (TP) {
            const int q = min(lane >> 4, GRB - 1);
            const size_t t = (size_t)min(rbw + q, a.nrb - 1) * ntg + g;
            __builtin_amdgcn_global_load_lds((const void*)((const uint32_t*)a.scale + t * 16 + (lane & 15)),
                                             (__attribute__((address_space(3))) void*)dst, 4, 0, 0);
        } else {
            const int q = min(lane >> 3, GRB - 1);
            const size_t t = (size_t)min(rbw + q, a.nrb - 1) * ntg + g;
            __builtin_amdgcn_global_load_lds((const void*)((const uint2*)a.scale + t * 16 + 2 * (lane & 7)),
                                             (__attribute__((address_space(3))) void*)dst, 16, 0, 0);
        }
    };
    if constexpr (TP) {  // 32-rung ladders of the wave's rows (quant.rs:399-410)
#pragma unroll
        for (int q = 0; q < GRB; q++) {
            if (s == 0) {
                const float2 p = a.rowp[min(rbw + q, a.nrb - 1) * 16 + r];
                float tv = p.x;
                lad[wave][(q * 16 + r) * 33] = tv;
                for (int c = 1; c < 32; c++) {
                    tv = tv * p.y;
                    lad[wave][(q * 16 + r) * 33 + c] = tv;
                }
            }
        }
    }
    float4v acc[GRB][4];
#pragma unroll
    for (int q = 0; q < GRB; q++)
#pragma unroll
        for (int mb = 0; mb < 4; mb++) acc[q][mb] = float4v{0.f, 0.f, 0.f, 0.f};

    const int gs0 = blockIdx.z * a.gsteps, gs1 = min(ntg, gs0 + a.gsteps);  // this part's K steps
    uint4 wA[GRB], wB[GRB];
#pragma unroll
    for (int j = 0; j < GJ; j++) dma_a(j, gs0, 0);
    dma_s(gs0, 0);
    load_w(wA, gs0);
    wait_vmcnt<0>();
    __syncthreads();

    auto compute = [&](int buf, const uint4* wv) __attribute__((always_inline)) {
        const uint4* A = gemm_at + (size_t)buf * GCH * 64;
        // this step's scale words of the lane's rows in LDS (q4t: [q][r] four
        // f16; q4tp: [q][r] u32 of four 5-bit codes), read per tile
        const uint8_t* sb = sarea + (size_t)(buf * 4 + wave) * 1024;
        const float4v* Bias = (const float4v*)(A + 32 * 64);   // hi plane's [tile][64 rows] f32
        const float4v* BiasL = (const float4v*)(A + 33 * 64);  // lo plane's
#pragma unroll 1
        for (int t = 0; t < 4; t++) {
            half8 bq[GRB];
            float sc[GRB];
#pragma unroll
            for (int q = 0; q < GRB; q++) {
                const uint32_t wd = t == 0 ? wv[q].x : t == 1 ? wv[q].y : t == 2 ? wv[q].z : wv[q].w;
                bq[q] = dq_nib_word(wd);
                if constexpr (TP) {
                    const uint32_t code = ((const uint32_t*)sb)[q * 16 + r];
                    sc[q] = lad[wave][(q * 16 + r) * 33 + ((code >> (5 * t)) & 31)];
                } else {
                    sc[q] = f16_bits_to_f32(((const uint16_t*)sb)[(q * 16 + r) * 4 + t]);
                }
            }
#pragma unroll
            for (int mb = 0; mb < 4; mb++) {
                const half8 xh = __builtin_bit_cast(half8, A[(4 * t + s) * 64 + 16 * mb + r]);
                const half8 xl = __builtin_bit_cast(half8, A[(16 + 4 * t + s) * 64 + 16 * mb + r]);
                const float4v cb = Bias[t * 16 + 4 * mb + s];  // rows 16 mb + 4 s .. + 3
                const float4v cbl = BiasL[t * 16 + 4 * mb + s];
#pragma unroll
                for (int q = 0; q < GRB; q++) {
                    // hi and lo in accumulators of their own: each tile sum is
                    // exact only within one plane
                    float4v d = __builtin_amdgcn_mfma_f32_16x16x32_f16(xh, bq[q], cb, 0, 0, 0);
                    d += __builtin_amdgcn_mfma_f32_16x16x32_f16(xl, bq[q], cbl, 0, 0, 0);
                    acc[q][mb] += d * sc[q];
                }
            }
        }
    };

    // The next step's operand and tile scales (into the other buffer,
    // directly) and weights go out before this step's MFMAs; the wait covers
    // the direct loads only (the GRB weight loads after them stay in flight), and the barrier
    // lets every wave's chunks land before they are read and keeps the
    // buffer being read from being refilled.  Past the last step the loads
    // repeat it into the buffer no one reads.
    for (int g = gs0; g < gs1; g += 2) {
        {
            const int g_ = min(g + 1, gs1 - 1);
#pragma unroll
            for (int j = 0; j < GJ; j++) dma_a(j, g_, 1);
            dma_s(g_, 1);
            load_w(wB, g_);
            compute(0, wA);
            wait_vmcnt<GRB>();
        }
        lds_sync();
        if (g + 1 >= gs1) break;
        {
            const int g_ = min(g + 2, gs1 - 1);
#pragma unroll
            for (int j = 0; j < GJ; j++) dma_a(j, g_, 0);
            dma_s(g_, 0);
            load_w(wA, g_);
            compute(1, wB);
            wait_vmcnt<GRB>();
        }
        lds_sync();
    }
#pragma unroll
    for (int q = 0; q < GRB; q++) {
        const int n = (rbw + q) * 16 + r;
        if (rbw + q >= a.nrb || n >= a.N) continue;
#pragma unroll
        for (int mb = 0; mb < 4; mb++)
#pragma unroll
            for (int v = 0; v < 4; v++) {
                const int b = GB * by + 16 * mb + 4 * s + v;
                if (b < a.M) {
                    const float val = acc[q][mb][v] * a.xs[b] * 16777216.0f;
                    if (a.part) {
                        a.part[((size_t)blockIdx.z * a.M + b) * a.N + n] = val;
                    } else {
                        float* yp = a.y + (size_t)b * a.ldy + n;
                        *yp = a.resid ? *yp + val : val;
                    }
                }
            }
    }
}

// ---------------------------------------------------------------------------
// q8 (qmatvec's exact arm in batches, qtensor.rs:9980-10047): int8 weights
// times the operand carried as three int8 planes x ~= sx (q0 + q1/128 +
// q2/16384) (prep8_row), on v_mfma_i32_16x16x64_i8.  A workgroup of 4 waves
// owns 64 batch rows x 64 Q8RB weight rows and walks K in steps of two
// 64-column chunks: the step's operand (3 planes x 2 chunks x 64 rows x
// 64 B = 24 KiB) is staged one step ahead through registers into a
// double-buffered LDS tile, the next step's weights are requested before the
// current MFMAs.  Each plane keeps its own int32 accumulators over the whole
// K (exact: |sum| <= 127 * 127 * K < 2^31 for K <= 16384), combined in f32
// at the end as the GEMV does: ((s0 + s1/128 + s2/16384) * sx) * rs.
// ---------------------------------------------------------------------------
constexpr int Q8CH = 24;              // 1 KiB operand chunks per step
constexpr int Q8J = Q8CH / 4;         // per wave
constexpr size_t GEMM_Q8_AT_BYTES = (size_t)2 * Q8CH * 64 * 16;  // k_gemm_q8's dynamic LDS
template <int Q8RB>
__global__ __launch_bounds__(256) void k_gemm_q8(GemmArgs a) {
    // double-buffered operand tile [2][Q8CH chunks][64 lanes] x 16 B, filled
    // by direct global -> LDS loads (as k_gemm_q4)
    extern __shared__ __align__(16) int4v gemm_at8[];
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int r = lane & 15, s = lane >> 4;
    const int by = blockIdx.y, rbw = (blockIdx.x * 4 + wave) * Q8RB;
    const int nk = a.ntg, Mp = a.Mp;
    const int4v* P = (const int4v*)a.planes;  // plane p, item (kc * 4 + s): P[(p * nk * 4 + item) * Mp + row]
    // operand chunk c of step g: plane c / 8, chunk 2g + (c / 4) % 2, quarter c % 4
    auto src_a = [&](int j, int g) __attribute__((always_inline)) -> const int4v* {
        const int c = wave + 4 * j;
        const int p = c >> 3, kc = min(2 * g + ((c >> 2) & 1), nk - 1), q = c & 3;
        return P + ((size_t)p * nk * 4 + kc * 4 + q) * Mp + GB * by + lane;
    };
    auto load_w = [&](int4v (*wv)[2], int g) __attribute__((always_inline)) {
#pragma unroll
        for (int q = 0; q < Q8RB; q++)
#pragma unroll
            for (int h = 0; h < 2; h++) {
                const size_t t = (size_t)min(rbw + q, a.nrb - 1) * nk + min(2 * g + h, nk - 1);
                wv[q][h] = ld_stream((const int4v*)a.w + t * 64 + lane);
            }
    };
    int4v acc[Q8RB][4][3];
#pragma unroll
    for (int q = 0; q < Q8RB; q++)
#pragma unroll
        for (int mb = 0; mb < 4; mb++)
#pragma unroll
            for (int p = 0; p < 3; p++) acc[q][mb][p] = int4v{0, 0, 0, 0};
    int4v wA[Q8RB][2], wB[Q8RB][2];
    const int nst = (nk + 1) / 2;
    const int gs0 = blockIdx.z * a.gsteps, gs1 = min(nst, gs0 + a.gsteps);  // this part's K steps
    auto dma_a = [&](int g, int buf) __attribute__((always_inline)) {
#pragma unroll
        for (int j = 0; j < Q8J; j++) {
            int4v* dst = gemm_at8 + ((size_t)buf * Q8CH + wave + 4 * j) * 64;
            __builtin_amdgcn_global_load_lds((const void*)src_a(j, g), (__attribute__((address_space(3))) void*)dst,
                                             16, 0, 0);
        }
    };
    dma_a(gs0, 0);
    load_w(wA, gs0);
    wait_vmcnt<0>();
    __syncthreads();

    auto compute = [&](int buf, int4v (*wv)[2], int g) __attribute__((always_inline)) {
        const int4v* A = gemm_at8 + (size_t)buf * Q8CH * 64;
#pragma unroll
        for (int h = 0; h < 2; h++) {
            if (2 * g + h >= nk) break;  // uniform: an odd chunk count's last step
#pragma unroll
            for (int mb = 0; mb < 4; mb++) {
                const int4v x0 = A[(0 * 8 + h * 4 + s) * 64 + 16 * mb + r];
                const int4v x1 = A[(1 * 8 + h * 4 + s) * 64 + 16 * mb + r];
                const int4v x2 = A[(2 * 8 + h * 4 + s) * 64 + 16 * mb + r];
#pragma unroll
                for (int q = 0; q < Q8RB; q++) {
                    acc[q][mb][0] = __builtin_amdgcn_mfma_i32_16x16x64_i8(x0, wv[q][h], acc[q][mb][0], 0, 0, 0);
                    acc[q][mb][1] = __builtin_amdgcn_mfma_i32_16x16x64_i8(x1, wv[q][h], acc[q][mb][1], 0, 0, 0);
                    acc[q][mb][2] = __builtin_amdgcn_mfma_i32_16x16x64_i8(x2, wv[q][h], acc[q][mb][2], 0, 0, 0);
                }
            }
        }
    };
    // as k_gemm_q4: the next step's operand straight into the other buffer,
    // a wait for those loads only, an LDS-only barrier
    for (int g = gs0; g < gs1; g += 2) {
        {
            const int gn = min(g + 1, gs1 - 1);
            dma_a(gn, 1);
            load_w(wB, gn);
            compute(0, wA, g);
            wait_vmcnt<2 * Q8RB>();
        }
        lds_sync();
        if (g + 1 >= gs1) break;
        {
            const int gn = min(g + 2, gs1 - 1);
            dma_a(gn, 0);
            load_w(wA, gn);
            compute(1, wB, g + 1);
            wait_vmcnt<2 * Q8RB>();
        }
        lds_sync();
    }
#pragma unroll
    for (int q = 0; q < Q8RB; q++) {
        const int n = (rbw + q) * 16 + r;
        if (rbw + q >= a.nrb || n >= a.N) continue;
        const float rs = ((const float*)a.scale)[n];
#pragma unroll
        for (int mb = 0; mb < 4; mb++)
#pragma unroll
            for (int v = 0; v < 4; v++) {
                const int b = GB * by + 16 * mb + 4 * s + v;
                if (b < a.M) {
                    const float tt = (float)acc[q][mb][0][v] + (float)acc[q][mb][1][v] * 0.0078125f +
                                     (float)acc[q][mb][2][v] * 6.103515625e-05f;
                    const float val = (tt * a.xs[b]) * rs;
                    if (a.part) {
                        a.part[((size_t)blockIdx.z * a.M + b) * a.N + n] = val;
                    } else {
                        float* yp = a.y + (size_t)b * a.ldy + n;
                        *yp = a.resid ? *yp + val : val;
                    }
                }
            }
    }
}

// y = (resid ? y : 0) + sum over the parts in part order (split K).
__global__ __launch_bounds__(256) void k_gemm_reduce(const float* __restrict__ part, int nz, int M, int N,
                                                     float* __restrict__ y, int ldy, int resid) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= M * N) return;
    const int b = i / N, n = i - b * N;
    float acc = part[i];
    for (int z = 1; z < nz; z++) acc += part[(size_t)z * M * N + i];
    float* yp = y + (size_t)b * ldy + n;
    *yp = resid ? *yp + acc : acc;
}

// Operand planes of the GEMM (grown on demand).
// operand planes, row scales and split-K partial sums, grown on demand, per
// host thread (each thread runs on its own stream); a GEMM is never part of
// a captured graph (the decode rounds' batches are <= 16 rows)
static thread_local uint8_t* g_gemm_planes = nullptr;
static thread_local size_t g_gemm_cap = 0;
static thread_local float* g_gemm_xs = nullptr;
static thread_local size_t g_gemm_xs_cap = 0;
static thread_local float* g_gemm_part = nullptr;  // split-K partial sums
static thread_local size_t g_gemm_part_cap = 0;

// K parts for a grid of base workgroups over nsteps K steps: doubled while
// the grid is below one workgroup per CU (256), at least 4 steps a part.
// Measured on MI355X: at m = 256 (prefill chunks) the down projection
// 1024x3072 (64 workgroups unsplit) and wo 1024x2048 take 4 parts; q4t
// 12288x4096 at m = 64 (192 workgroups) 2 parts, 71 -> 56 us; qkv at
// m = 256 (256 workgroups) split in 2 made the prefill slower (32.9 ->
// 33.6 ms).
static int gemm_kparts(long base, int nsteps) {
    static const int env = [] {
        const char* e = getenv("CMF_GEMM_SPLITK");
        return e ? atoi(e) : -1;
    }();
    if (env == 0) return 1;
    int z = 1;
    while (base * z < 256 && nsteps / (z * 2) >= 4) z *= 2;
    return z;
}

size_t gemm_planes_bytes(const DevWeight& w, int mp) {
    // q8: three planes of nk * 64 * Mp B; q4: hi + lo 2 * items * Mp * 16 B
    // and the two tables of tile biases 2 * tiles * Mp * 4 B
    if (w.dtype == DT_Q8ROW) return (size_t)w.kchunks * 64 * mp * 3;
    return (size_t)w.kchunks * 16 * mp * 32 + (size_t)w.kchunks * 4 * mp * 8;
}

int gemm(const DevWeight& w, const XSrc& src, int m, float* y, int ldy, bool resid, hipStream_t st) {
    if (w.dtype != DT_Q4T && w.dtype != DT_Q4TP && w.dtype != DT_Q8ROW) return fail("gemm: q8 / q4t / q4tp weights");
    if (m < 1 || m > 65535) return fail("gemm: batch must be 1..65535");
    const int mp = (m + GB - 1) / GB * GB;
    const size_t pb = gemm_planes_bytes(w, mp);
    if (g_gemm_cap < pb) {
        (void)hipStreamSynchronize(st);
        if (g_gemm_planes) (void)hipFree(g_gemm_planes);
        g_gemm_planes = nullptr;
        g_gemm_cap = 0;
        CMF_HIP(hipMalloc(&g_gemm_planes, pb));
        g_gemm_cap = pb;
    }
    if (g_gemm_xs_cap < (size_t)mp) {
        (void)hipStreamSynchronize(st);
        if (g_gemm_xs) (void)hipFree(g_gemm_xs);
        g_gemm_xs = nullptr;
        g_gemm_xs_cap = 0;
        CMF_HIP(hipMalloc(&g_gemm_xs, (size_t)mp * sizeof(float)));
        g_gemm_xs_cap = mp;
    }
    int rc = launch_prep_src_gemm(w, src, m, mp, g_gemm_planes, g_gemm_xs, st);
    if (rc != CMF_OK) return rc;
    GemmArgs a;
    a.w = w.w;
    a.scale = w.scale;
    a.rowp = w.rowp;
    a.planes = g_gemm_planes;
    a.xs = g_gemm_xs;
    a.y = y;
    a.ldy = ldy;
    a.M = m;
    a.Mp = mp;
    a.N = w.rows;
    a.ntg = w.kchunks;
    a.nrb = w.rows_pad / 16;
    a.resid = resid ? 1 : 0;
    a.part = nullptr;
    // split K (nz parts into the partial buffer, then k_gemm_reduce)
    auto split = [&](long base, int nsteps) -> int {
        const int nz = gemm_kparts(base, nsteps);
        a.gsteps = (nsteps + nz - 1) / nz;
        if (nz == 1) return 1;
        const size_t need = (size_t)nz * m * w.rows;
        if (g_gemm_part_cap < need) {
            (void)hipStreamSynchronize(st);
            if (g_gemm_part) (void)hipFree(g_gemm_part);
            g_gemm_part = nullptr;
            g_gemm_part_cap = 0;
            if (hipMalloc(&g_gemm_part, need * sizeof(float)) != hipSuccess) return -1;
            g_gemm_part_cap = need;
        }
        a.part = g_gemm_part;
        return (nsteps + a.gsteps - 1) / a.gsteps;
    };
    auto reduce = [&](int nz) -> int {
        if (nz > 1)
            hipLaunchKernelGGL(k_gemm_reduce, dim3((m * w.rows + 255) / 256), dim3(256), 0, st, g_gemm_part, nz, m,
                               w.rows, y, ldy, a.resid);
        CMF_HIP(hipGetLastError());
        return CMF_OK;
    };
    if (w.dtype == DT_Q8ROW) {
        // two row blocks per wave once that still leaves ~4 workgroups per CU
        const bool big = (long)((a.nrb + 7) / 8) * (mp / GB) >= 1024;
        const int rbwg = big ? 8 : 4;
        const int gx = (a.nrb + rbwg - 1) / rbwg, nz = split((long)gx * (mp / GB), (a.ntg + 1) / 2);
        if (nz < 0) return fail("gemm: split-K buffer");
        const dim3 grid(gx, mp / GB, nz);
        if (big) hipLaunchKernelGGL((k_gemm_q8<2>), grid, dim3(256), GEMM_Q8_AT_BYTES, st, a);
        else hipLaunchKernelGGL((k_gemm_q8<1>), grid, dim3(256), GEMM_Q8_AT_BYTES, st, a);
        return reduce(nz);
    }
    // four row blocks per wave once that still leaves ~4 workgroups per CU
    const bool big = (long)((a.nrb + 15) / 16) * (mp / GB) >= 1024;
    // two row blocks per wave (half the operand re-reads) while that still
    // gives >= 384 workgroups: measured 12288x4096 m=256 160 -> 126 us, but
    // 6144x1024 m=256 (192 workgroups) 30.7 -> 38.8 us
    const int grb_small = !big && (long)((a.nrb + 7) / 8) * (mp / GB) >= 384 ? 2 : 1;
    const int rbwg = big ? 16 : 4 * grb_small;
    const int gx = (a.nrb + rbwg - 1) / rbwg, nz = split((long)gx * (mp / GB), a.ntg);
    if (nz < 0) return fail("gemm: split-K buffer");
    const dim3 grid(gx, mp / GB, nz);
    const void* kf = w.dtype == DT_Q4T
                         ? (big ? (const void*)k_gemm_q4<DT_Q4T, 4>
                                : (grb_small == 2 ? (const void*)k_gemm_q4<DT_Q4T, 2> : (const void*)k_gemm_q4<DT_Q4T, 1>))
                         : (big ? (const void*)k_gemm_q4<DT_Q4TP, 4>
                                : (grb_small == 2 ? (const void*)k_gemm_q4<DT_Q4TP, 2> : (const void*)k_gemm_q4<DT_Q4TP, 1>));
    {
        // the operand tile's dynamic LDS is above the default 64 KiB limit
        static std::mutex mu;
        static std::set<const void*> done;
        std::lock_guard<std::mutex> g(mu);
        if (done.insert(kf).second)
            CMF_HIP(hipFuncSetAttribute(kf, hipFuncAttributeMaxDynamicSharedMemorySize, (int)GEMM_AT_BYTES));
    }
    void* args[] = {&a};
    CMF_HIP(hipLaunchKernel(kf, grid, dim3(256), args, GEMM_AT_BYTES, st));
    return reduce(nz);
}

int gemm_q4(const DevWeight& w, const float* x, int ldx, int m, float* y, int ldy, hipStream_t st) {
    XSrc r{};
    r.mode = XS_ROWS;
    r.x = x;
    r.ldx = ldx;
    return gemm(w, r, m, y, ldy, false, st);
}

}  // namespace cmf
