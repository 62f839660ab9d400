// Dequant GEMV / skinny GEMM kernels for gfx950 (MI355X).
//
// y[b][r] = sum_k W[r][k] * x[b][k] for b < M <= 16 and the three weight
// codecs of the engine (q8 per-row, q4_tiled, q4tp).  Work split:
//   - a workgroup of KS waves owns one block of 16 weight rows at a time
//     (the grid is sized to what the CUs hold at once, so one block per
//     workgroup unless the matrix is taller); its waves split K and reduce
//     in LDS in a fixed order (deterministic);
//   - every wave streams 1 KiB of packed weights per step with one 128-bit
//     load per lane, its whole K share (SP steps) requested at once;
//   - the activations are the MFMA A operand (16 batch rows, zero-padded),
//     the weights the B operand (16 weight rows):
//       q8  : v_mfma_i32_16x16x64_i8 on the raw int8 weights; x is carried
//             as three int8 planes, x ~= sx*(q0 + q1/128 + q2/16384)
//             (|error| <= 2^-22 max|x|), each summed exactly in int32;
//       q4* : v_mfma_f32_16x16x32_f16, one tile (32 columns, one scale) per
//             MFMA; nibbles become the exact f16 denormals n * 2^-24 in
//             registers (one mask per pair), the format's -8 offset enters
//             as the accumulator input -8 * 2^-24 * sum(x) of the tile, and
//             x is carried as f16 hi + lo of x*2^e (22-bit significand).
//             Each tile's product is scaled by its tile scale and
//             accumulated in f32, as q4t_row_exact does
//             (qtensor.rs:4418-4432).
//   - the activation operand is built once per workgroup into LDS from its
//     producer (RMSNorm of the residual rows, SwiGLU of the gate/up rows,
//     plain rows, the MTP [enorm(embed); hnorm(h)] concat, or a prepared
//     buffer), so the producer needs no kernel of its own; when it does not
//     fit in LDS the prepared planes are read from global memory (L2).
//   - optional residual epilogue: y is added into the output (h += W x).
#pragma once

#include "common.h"
#include "gemv.h"

namespace cmf {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float float4v __attribute__((ext_vector_type(4)));
typedef int int4v __attribute__((ext_vector_type(4)));

constexpr int LDSX_MAX = 128 * 1024;  // largest LDS-staged activation operand (+ scratch)

// Four nibble bytes (8 weights: elements 8s..8s+7 of a tile) to the f16
// denormals n * 2^-24 (exact, the raw nibble under a zero exponent) in the
// in-slot order {0,4,2,6,1,5,3,7}: one mask (and shift) per pair.  The -8
// offset of the format enters through the MFMA accumulator (q4_tile_bias).
__device__ __forceinline__ half8 dq_nib_word(uint32_t w) {
    constexpr uint32_t K = 0x000F000Fu;
    const uint32_t p0 = w & K;          // elements 0, 4
    const uint32_t p1 = (w >> 8) & K;   // 2, 6
    const uint32_t p2 = (w >> 4) & K;   // 1, 5
    const uint32_t p3 = (w >> 12) & K;  // 3, 7
    return __builtin_bit_cast(half8, make_uint4(p0, p1, p2, p3));
}

__device__ __forceinline__ float f16_bits_to_f32(uint32_t h) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
}

// ---------------------------------------------------------------------------
// Activation staging (once per workgroup)
// ---------------------------------------------------------------------------
constexpr int SEGJ = 8;            // float4 per lane per staging unit
constexpr int SEG4 = 64 * SEGJ;    // float4 per staging unit (2048 elements)
constexpr int SEGMAX = 8;          // staging units per row (operands up to 16384 elements)

__device__ __forceinline__ float silu_mul(float g, float u) { return (g / (1.0f + expf(-g))) * u; }

__device__ __forceinline__ float amax4(float m, float4v v) {
    return fmaxf(fmaxf(m, fmaxf(fabsf(v.x), fabsf(v.y))), fmaxf(fabsf(v.z), fabsf(v.w)));
}
__device__ __forceinline__ double sq4(float4v v) {
    return (double)v.x * (double)v.x + (double)v.y * (double)v.y + (double)v.z * (double)v.z +
           (double)v.w * (double)v.w;
}

// Phase 1 of one staging unit u (row b = u / S): lane element groups
// k4 = base + 64*j + lane (4 elements each) are all requested at once (row 0
// also requests the norm weights), the raw values stored to the scratch rows,
// and the unit's sums of squares (norm producers) or max|x| reduced to LDS.
template <int MODE>
__device__ __forceinline__ void unit_phase1(const XSrc& s, int u, int S, int K4, int kp4, int H4, float4v* xf4,
                                            float4v* wl4, double* red1, double* red2, float* mred) {
    const int lane = threadIdx.x & 63;
    const int b = u / S, base = (u % S) * SEG4;
    constexpr bool nrm = MODE == XS_NORM || MODE == XS_CAT;
    const bool ldw = nrm && b == 0;
    float4v v[SEGJ], wv[SEGJ];
    const float4v z4 = float4v{0.f, 0.f, 0.f, 0.f};
    const float* row = s.x + (size_t)b * s.ldx;
    if constexpr (MODE == XS_SILU) {
        float4v g[SEGJ], u[SEGJ];
#pragma unroll
        for (int j = 0; j < SEGJ; j++) {
            const int k4 = base + 64 * j + lane;
            g[j] = k4 < K4 ? ((const float4v*)row)[k4] : z4;
            u[j] = k4 < K4 ? ((const float4v*)(row + s.K))[k4] : z4;
        }
#pragma unroll
        for (int j = 0; j < SEGJ; j++)
            v[j] = float4v{silu_mul(g[j].x, u[j].x), silu_mul(g[j].y, u[j].y), silu_mul(g[j].z, u[j].z),
                               silu_mul(g[j].w, u[j].w)};
    } else if constexpr (MODE == XS_CAT) {
        const int tok = s.toks[b];
        const EmbedSrc& e = s.emb;
        const bool tv = tok >= 0 && tok < e.rows;
        const int rb = tok >> 4, r = tok & 15;
        const float rs = tv ? e.rs[tok] : 0.f;
#pragma unroll
        for (int j = 0; j < SEGJ; j++) {
            const int k4 = base + 64 * j + lane;
            // four consecutive int8 of the token's row in the q8 device layout
            const int k = 4 * k4, kc = k >> 6, sl = (k >> 4) & 3, jj = k & 15;
            uint32_t q = 0u;
            float4v xr = z4;
            if (k4 < K4 && k4 < H4 && tv)
                q = *(const uint32_t*)(e.w + (((size_t)rb * e.nkc + kc) * 64 + 16 * sl + r) * 16 + jj);
            if (k4 < K4 && k4 >= H4) xr = ((const float4v*)row)[k4 - H4];
            v[j] = k4 < H4 ? float4v{(float)(int8_t)(q & 0xFF), (float)(int8_t)((q >> 8) & 0xFF),
                                         (float)(int8_t)((q >> 16) & 0xFF), (float)(int8_t)(q >> 24)}
                           : xr;
            wv[j] = ldw && k4 < K4 ? (k4 < H4 ? ((const float4v*)s.w)[k4] : ((const float4v*)s.w2)[k4 - H4]) : z4;
        }
#pragma unroll
        for (int j = 0; j < SEGJ; j++) {
            const int k4 = base + 64 * j + lane;
            if (k4 < H4) v[j] = float4v{v[j].x * rs, v[j].y * rs, v[j].z * rs, v[j].w * rs};
        }
    } else {
#pragma unroll
        for (int j = 0; j < SEGJ; j++) {
            const int k4 = base + 64 * j + lane;
            v[j] = k4 < K4 ? ((const float4v*)row)[k4] : z4;
            if constexpr (MODE == XS_NORM) wv[j] = ldw && k4 < K4 ? ((const float4v*)s.w)[k4] : z4;
        }
    }
    double s1 = 0.0, s2 = 0.0;
    float am = 0.f;
#pragma unroll
    for (int j = 0; j < SEGJ; j++) {
        const int k4 = base + 64 * j + lane;
        if (k4 < kp4) {
            xf4[(size_t)b * kp4 + k4] = v[j];
            if (ldw) wl4[k4] = wv[j];
        }
        if constexpr (nrm) {
            if (k4 < H4) s1 += sq4(v[j]);
            else s2 += sq4(v[j]);
        } else {
            am = amax4(am, v[j]);
        }
    }
    if constexpr (nrm) {
        for (int o = 32; o > 0; o >>= 1) {
            s1 += __shfl_xor(s1, o);
            s2 += __shfl_xor(s2, o);
        }
        if (lane == 0) {
            red1[u] = s1;
            red2[u] = s2;
        }
    } else {
        for (int o = 32; o > 0; o >>= 1) am = fmaxf(am, __shfl_xor(am, o));
        if (lane == 0) mred[u] = am;
    }
}

// Builds the operand of all M batch rows in LDS with the whole workgroup.
// Rows are cut into units of 2048 elements; the waves take units round-robin.
//   phase 1: every input element (and the norm weights) is requested at
//            once, raw values go to the f32 scratch xf [M][kpad], per-unit
//            sums of squares (f64) or max|x| to LDS;
//   phase 2 (RMSNorm producers): inv = 1/sqrt(mean + eps) from the unit sums
//            in a fixed order, x = (raw * inv) * w in place, per-unit max|x|;
//   phase 3: operand planes, one 16-byte item per thread step:
//     q4: hi plane then lo plane, [tile*4 + s][b] x 16 B; lxs[b] = 2^-e;
//         then the tile biases [tile][16] f32 (q4_tile_bias)
//     q8: planes q0,q1,q2, [chunk*4 + s][b] x 16 B;      lxs[b] = sx
__device__ __forceinline__ void stage_fused(const XSrc& s, int M, int fmt, int nk, uint8_t* lx, float* lxs,
                                            float* xf) {
    __shared__ double red1[MAXB * SEGMAX], red2[MAXB * SEGMAX];
    __shared__ float mred[MAXB * SEGMAX];
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), nw = blockDim.x >> 6;
    const int kpad = fmt == DT_Q8ROW ? nk * 64 : nk * 32;  // nk: q8 chunks / q4 tiles
    const int K4 = s.K >> 2, kp4 = kpad >> 2;
    const int S = (kp4 + SEG4 - 1) / SEG4, units = M * S;
    const bool nrm = s.mode == XS_NORM || s.mode == XS_CAT;
    const int H4 = s.mode == XS_CAT ? s.H >> 2 : 0x7fffffff;
    float4v* xf4 = (float4v*)xf;
    float4v* wl4 = xf4 + (size_t)M * kp4;  // norm weight of every element
    const float4v z4 = float4v{0.f, 0.f, 0.f, 0.f};
    for (int u = wave; u < units; u += nw) {
        switch (s.mode) {
            case XS_SILU: unit_phase1<XS_SILU>(s, u, S, K4, kp4, H4, xf4, wl4, red1, red2, mred); break;
            case XS_CAT: unit_phase1<XS_CAT>(s, u, S, K4, kp4, H4, xf4, wl4, red1, red2, mred); break;
            case XS_NORM: unit_phase1<XS_NORM>(s, u, S, K4, kp4, H4, xf4, wl4, red1, red2, mred); break;
            default: unit_phase1<XS_ROWS>(s, u, S, K4, kp4, H4, xf4, wl4, red1, red2, mred); break;
        }
    }
    __syncthreads();
    if (nrm) {
        const int n1 = s.mode == XS_CAT ? s.H : s.K;
        for (int u = wave; u < units; u += nw) {
            const int b = u / S, sg = u % S;
            double t1 = 0.0, t2 = 0.0;
            for (int q = 0; q < S; q++) {
                t1 += red1[b * S + q];
                t2 += red2[b * S + q];
            }
            const float inv1 = 1.0f / (float)sqrt(t1 / (double)n1 + s.eps);
            const float inv2 = s.mode == XS_CAT ? 1.0f / (float)sqrt(t2 / (double)s.H + s.eps) : 1.f;
            float am = 0.f;
#pragma unroll
            for (int j = 0; j < SEGJ; j++) {
                const int k4 = sg * SEG4 + 64 * j + lane;
                if (k4 < K4) {
                    const float iv = k4 < H4 ? inv1 : inv2;
                    const float4v x = xf4[(size_t)b * kp4 + k4], w = wl4[k4];
                    const float4v y = float4v{x.x * iv * w.x, x.y * iv * w.y, x.z * iv * w.z, x.w * iv * w.w};
                    xf4[(size_t)b * kp4 + k4] = y;
                    am = amax4(am, y);
                }
            }
            for (int o = 32; o > 0; o >>= 1) am = fmaxf(am, __shfl_xor(am, o));
            if (lane == 0) mred[u] = am;
        }
        __syncthreads();
    }
    const int nitems = nk * 4;
    const size_t pl = (size_t)nitems * M * 16;
    for (int i = threadIdx.x; i < M * nitems; i += blockDim.x) {
        const int b = i / nitems, item = i - b * nitems;
        float am = 0.f;
        for (int q = 0; q < S; q++) am = fmaxf(am, mred[b * S + q]);
        const float* xr = xf + (size_t)b * kpad;
        const size_t off = ((size_t)item * M + b) * 16;
        if (fmt == DT_Q8ROW) {
            const float sx = am > 0.f ? am / 127.0f : 1.0f, inv = 1.0f / sx;
            if (item == 0) lxs[b] = sx;
            uint32_t w0[4], w1[4], w2[4];
#pragma unroll
            for (int c = 0; c < 4; c++) {
                const float4v xv = *(const float4v*)(xr + item * 16 + 4 * c);
                const float xs4[4] = {xv.x, xv.y, xv.z, xv.w};
                uint32_t a = 0, bb = 0, cc = 0;
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const float x = xs4[j] * inv;
                    const float q0 = fminf(127.f, fmaxf(-127.f, rintf(x)));
                    const float r1 = (x - q0) * 128.0f;
                    const float q1 = fminf(127.f, fmaxf(-127.f, rintf(r1)));
                    const float q2 = fminf(127.f, fmaxf(-127.f, rintf((r1 - q1) * 128.0f)));
                    a |= (uint32_t)(uint8_t)(int8_t)q0 << (8 * j);
                    bb |= (uint32_t)(uint8_t)(int8_t)q1 << (8 * j);
                    cc |= (uint32_t)(uint8_t)(int8_t)q2 << (8 * j);
                }
                w0[c] = a;
                w1[c] = bb;
                w2[c] = cc;
            }
            *(uint4*)(lx + off) = make_uint4(w0[0], w0[1], w0[2], w0[3]);
            *(uint4*)(lx + pl + off) = make_uint4(w1[0], w1[1], w1[2], w1[3]);
            *(uint4*)(lx + 2 * pl + off) = make_uint4(w2[0], w2[1], w2[2], w2[3]);
        } else {
            int ex = 0;
            if (am > 0.f) frexpf(am, &ex);
            const float sc = am > 0.f ? ldexpf(1.0f, 15 - ex) : 1.0f;
            if (item == 0) lxs[b] = am > 0.f ? ldexpf(1.0f, ex - 15) : 1.0f;
            const float4v xa = *(const float4v*)(xr + item * 8), xb = *(const float4v*)(xr + item * 8 + 4);
            // in-slot order {0,4,2,6,1,5,3,7}
            const float xo[8] = {xa.x, xb.x, xa.z, xb.z, xa.y, xb.y, xa.w, xb.w};
            uint32_t hv[4], lv[4];
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const float x0 = xo[2 * j] * sc, x1 = xo[2 * j + 1] * sc;
                const _Float16 h0 = (_Float16)x0, h1 = (_Float16)x1;
                const _Float16 l0 = (_Float16)(x0 - (float)h0), l1 = (_Float16)(x1 - (float)h1);
                hv[j] = __builtin_bit_cast(uint16_t, h0) | ((uint32_t)__builtin_bit_cast(uint16_t, h1) << 16);
                lv[j] = __builtin_bit_cast(uint16_t, l0) | ((uint32_t)__builtin_bit_cast(uint16_t, l1) << 16);
            }
            *(uint4*)(lx + off) = make_uint4(hv[0], hv[1], hv[2], hv[3]);
            *(uint4*)(lx + pl + off) = make_uint4(lv[0], lv[1], lv[2], lv[3]);
        }
    }
    if (fmt != DT_Q8ROW) {
        // tile biases [tile][16] after the planes (q4_tile_bias; zero rows >= M)
        float* bias = (float*)(lx + 2 * pl);
        for (int i = threadIdx.x; i < nk * 16; i += blockDim.x) {
            const int t = i >> 4, b = i & 15;
            float v = 0.f;
            if (b < M) {
                float am = 0.f;
                for (int q = 0; q < S; q++) am = fmaxf(am, mred[b * S + q]);
                int ex = 0;
                if (am > 0.f) frexpf(am, &ex);
                const float sc = am > 0.f ? ldexpf(1.0f, 15 - ex) : 1.0f;
                v = q4_tile_bias(xf + (size_t)b * kpad, kpad, t * 32, sc);
            }
            bias[i] = v;
        }
    }
}

// Operand staging of a whole workgroup; XS_GLOBAL planes have the LDS
// layout already and are copied as they are.
template <bool FU>
__device__ __forceinline__ void stage_x(const XSrc& s, int M, int fmt, int nk, uint8_t* lx, float* lxs) {
    if constexpr (!FU) {
        const int n = nk * 4 * M * (fmt == DT_Q8ROW ? 3 : 2);  // 16-byte items
        const uint4* g = (const uint4*)s.planes;
        uint4* l = (uint4*)lx;
        for (int i = threadIdx.x; i < n; i += blockDim.x) l[i] = g[i];
        if (threadIdx.x < 16) lxs[threadIdx.x] = s.xs[threadIdx.x];
    } else {
        // planes (+ q4 tile biases), then the f32 scratch
        const size_t pbytes = fmt == DT_Q8ROW ? (size_t)nk * 4 * M * 16 * 3 : (size_t)nk * (128 * M + 64);
        stage_fused(s, M, fmt, nk, lx, lxs, (float*)(lx + pbytes));
    }
    __syncthreads();
}

// Prepared planes go to LDS by direct global->LDS loads (no registers),
// issued before the weight stream: the loads of a wave complete in order, so
// the operand is in LDS once at most the weight loads issued after it are
// outstanding (vmcnt).  Wave w copies 1 KiB chunks w, w + nw, ... (indices
// clamped to the last item, so the copy never reads past the planes).
__device__ __forceinline__ void x_dma(const XSrc& s, int n, uint8_t* lx) {
    const uint4* g = (const uint4*)s.planes;
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int nw = blockDim.x >> 6;
    for (int c = wave; c * 64 < n; c += nw)
        __builtin_amdgcn_global_load_lds((const void*)(g + min(c * 64 + lane, n - 1)),
                                         (__attribute__((address_space(3))) void*)(lx + c * 1024), 16, 0, 0);
}
// s_waitcnt vmcnt(N) lgkmcnt(0) (gfx9 encoding: vmcnt bits 3:0 and 15:14,
// expcnt 6:4 left at 7, lgkmcnt 11:8)
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4));
}

// ---------------------------------------------------------------------------
// q4t / q4tp
// ---------------------------------------------------------------------------
// Workgroup g walks the work units (row block rb, K part kp) of row blocks
// g, g + grid, ...; a K part is KS*SP steps of 1 KiB (one step = 16 rows x
// 128 columns), SP consecutive steps per wave, all requested at once.  After
// the last K part the KS partial sums are reduced in LDS in wave order
// (deterministic).  (A variant that requested the next unit's weights before
// computing the current one held twice the registers, lost occupancy and was
// no faster on MI355X.)
// HL (m <= 8): A rows 0..7 carry the f16 hi plane of batch row r and rows
// 8..15 the lo plane of batch row r - 8, one MFMA per tile; the two halves
// are added at the end.  XM: where the activation operand comes from
// (XM_PREP prepared planes copied to LDS, XM_FUSED a fused producer staged
// into LDS by stage_fused, XM_GLOBAL prepared planes read in place).
constexpr int SP = 4;  // weight steps per wave and work unit
enum { XM_PREP = 0, XM_FUSED = 1, XM_GLOBAL = 2 };

template <int FMT, int NV, int KS, bool HL, int XM>
__global__ __launch_bounds__(64 * KS) void k_gemv_q4(GemvArgs a) {
    extern __shared__ __align__(16) uint8_t smem[];
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int r = lane & 15, s = lane >> 4;
    const int M = a.m, ntg = a.nk;  // nk = groups of 4 tiles
    constexpr bool TP = FMT == DT_Q4TP;
    __shared__ float lad[TP ? 2 : 1][TP ? 16 * 33 : 1];  // ladders of the current / next row block
    __shared__ float4v part[KS][64];
    __shared__ float lxs[16];
    const int P = (ntg + KS * SP - 1) / (KS * SP);  // K parts per row block
    int rb = blockIdx.x, kp = 0;
    if (rb >= a.nrb) return;  // uniform over the workgroup
    // weights + tile scales of a unit (q4tp: and the row ladder parameters
    // of its row block), all unconditional (steps past the row clamped to
    // its last one): a load under a branch makes the compiler wait for it
    // at once.  NL = loads per call.
    constexpr int NL = 2 * SP + (TP ? 1 : 0);
    auto load = [&](uint4* wv, uint2* sv, float2& pv, int rbl, int kpl) {
        const size_t wbase = (size_t)(a.rb0 + rbl) * ntg;
        const int t0 = kpl * KS * SP + wave * SP;
#pragma unroll
        for (int u = 0; u < SP; u++) {
            const size_t t = wbase + min(t0 + u, ntg - 1);
            wv[u] = ((const uint4*)a.w)[t * 64 + lane];
            if constexpr (TP) sv[u] = make_uint2(((const uint32_t*)a.scale)[t * 16 + r], 0u);
            else sv[u] = ((const uint2*)a.scale)[t * 16 + r];
        }
        if constexpr (TP) pv = a.rowp[(a.rb0 + rbl) * 16 + r];
    };
    // the 32-rung ladder of each row of a row block: t[c] = t[c-1] * ratio
    // (quant.rs:399-410), by 16 threads of the second wave (the first one
    // reduces meanwhile)
    auto ladder = [&](int buf, float2 p) {
        if constexpr (TP) {
            const int lt = (int)threadIdx.x - (KS > 1 ? 64 : 0);
            if (lt >= 0 && lt < 16) {
                float tv = p.x;
                lad[buf][lt * 33] = tv;
                for (int c = 1; c < 32; c++) {
                    tv = tv * p.y;
                    lad[buf][lt * 33 + c] = tv;
                }
            }
        }
    };
    uint4 wA[SP];
    uint2 sA[SP];
    float2 pA{};
    float xsv = 0.f;
    if constexpr (XM == XM_PREP) {
        x_dma(a.src, ntg * (32 * M + 16), smem);  // hi + lo planes + tile biases
        xsv = a.src.xs[threadIdx.x & 15];
    }
    __builtin_amdgcn_sched_barrier(0);
    load(wA, sA, pA, rb, 0);
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (XM == XM_PREP) {
        wait_vmcnt<NL>();  // operand planes and xs are in
        if (threadIdx.x < 16) lxs[threadIdx.x] = xsv;
    } else if constexpr (XM == XM_FUSED) {
        stage_x<true>(a.src, M, FMT, ntg * 4, smem, lxs);
    } else if (threadIdx.x < 16) {
        lxs[threadIdx.x] = a.src.xs[threadIdx.x];
    }
    ladder(0, pA);
    __syncthreads();
    // operand planes [item][b] x 16 B, hi then lo: in LDS, or read in place
    const uint4* LH = XM != XM_GLOBAL ? (const uint4*)smem : (const uint4*)a.src.planes;
    const uint4* LL = LH + ntg * 4 * 4 * M;
    const float4v* LB = (const float4v*)(LL + ntg * 4 * 4 * M);  // tile biases [tile][16]
    // lanes whose A row is past the batch read batch row 0: their D rows are
    // never stored, and every lane loads unconditionally
    const uint4* LX = HL ? (r < 8 ? LH : LL) : LH;
    const int xb = HL ? ((r & 7) < M ? (r & 7) : 0) : (r < M ? r : 0);
    const int xoff = s * M + xb, M4 = 4 * M;
    const float4v zero = {0.f, 0.f, 0.f, 0.f};
    float4v acc = zero;
    int buf = 0;

    // one work unit: rb/kp current, rn/kn the next one (rn >= nrb: none)
    auto process = [&](const uint4* wv, const uint2* sv, const float2& pn, int rn) {
        const int t0 = kp * KS * SP + wave * SP;
#pragma unroll
        for (int u = 0; u < SP; u++) {
            if (t0 + u < ntg) {
                const int tg = t0 + u;
                float sc[4];
                if constexpr (!TP) {
                    sc[0] = f16_bits_to_f32(sv[u].x & 0xFFFFu);
                    sc[1] = f16_bits_to_f32(sv[u].x >> 16);
                    sc[2] = f16_bits_to_f32(sv[u].y & 0xFFFFu);
                    sc[3] = f16_bits_to_f32(sv[u].y >> 16);
                } else {
                    const uint32_t cw = sv[u].x;
                    sc[0] = lad[buf][r * 33 + (cw & 31)];
                    sc[1] = lad[buf][r * 33 + ((cw >> 5) & 31)];
                    sc[2] = lad[buf][r * 33 + ((cw >> 10) & 31)];
                    sc[3] = lad[buf][r * 33 + ((cw >> 15) & 31)];
                }
                const uint32_t ww[4] = {wv[u].x, wv[u].y, wv[u].z, wv[u].w};
#pragma unroll
                for (int t = 0; t < 4; t++) {
                    const int item = (tg * 4 + t) * M4 + xoff;
                    const half8 bq = dq_nib_word(ww[t]);
                    const float4v cb = LB[(tg * 4 + t) * 4 + s];  // rows 4s..4s+3
                    float4v d;
                    if constexpr (HL) {
                        const half8 xa = __builtin_bit_cast(half8, LX[item]);
                        d = __builtin_amdgcn_mfma_f32_16x16x32_f16(xa, bq, cb, 0, 0, 0);
                    } else {
                        const half8 xh = __builtin_bit_cast(half8, LH[item]);
                        const half8 xl = __builtin_bit_cast(half8, LL[item]);
                        d = __builtin_amdgcn_mfma_f32_16x16x32_f16(xh, bq, cb, 0, 0, 0);
                        d = __builtin_amdgcn_mfma_f32_16x16x32_f16(xl, bq, d, 0, 0, 0);
                    }
#pragma unroll
                    for (int v = 0; v < NV; v++) acc[v] += d[v] * sc[t];
                }
            }
        }
        if (kp < P - 1) return;  // the row block continues in the next unit
        if constexpr (KS > 1) {
            part[wave][lane] = acc;
            __syncthreads();
        }
        if (wave == 0) {
#pragma unroll
            for (int q = 1; q < KS; q++) {
                const float4v o = part[q][lane];
#pragma unroll
                for (int v = 0; v < NV; v++) acc[v] += o[v];
            }
            if constexpr (HL) {
                // hi rows (lanes s = 0, 1) + lo rows (lanes s = 2, 3)
#pragma unroll
                for (int v = 0; v < NV; v++) acc[v] += __shfl_xor(acc[v], 32);
            }
            const int row = (a.rb0 + rb) * 16 + r;
            if (row >= a.row_lo && row < a.row_hi && (!HL || s < 2)) {
#pragma unroll
                for (int v = 0; v < NV; v++) {
                    const int b = 4 * s + v;
                    if (b < M) {
                        float* yp = a.y + (size_t)b * a.ldy + (row - a.row_lo);
                        const float val = acc[v] * lxs[b] * 16777216.0f;  // 2^24: denormal nibbles
                        *yp = a.resid ? *yp + val : val;
                    }
                }
            }
        }
        acc = zero;
        if (rn < a.nrb) ladder(buf ^ 1, pn);
        buf ^= 1;
        if constexpr (KS > 1 || TP) __syncthreads();
    };

    for (;;) {
        int rn = rb, kn = kp + 1;
        if (kn == P) {
            kn = 0;
            rn += gridDim.x;
        }
        float2 pn{};
        if constexpr (TP)
            if (rn < a.nrb) pn = a.rowp[(a.rb0 + rn) * 16 + r];
        process(wA, sA, pn, rn);
        if (rn >= a.nrb) break;
        rb = rn;
        kp = kn;
        load(wA, sA, pA, rb, kp);
    }
}

// ---------------------------------------------------------------------------
// q8
// ---------------------------------------------------------------------------
// Same schedule as k_gemv_q4 with 64-column int8 chunks as the 1 KiB steps
// (v_mfma_i32_16x16x64_i8).  PK (m <= 5): the three activation planes share
// one MFMA, A row p*m + b holding plane p of batch row b; otherwise one MFMA
// per plane.
template <int KS, bool PK, int XM>
__global__ __launch_bounds__(64 * KS) void k_gemv_q8(GemvArgs a) {
    extern __shared__ __align__(16) uint8_t smem[];
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int r = lane & 15, s = lane >> 4;
    const int M = a.m, nkc = a.nk;
    __shared__ float4v part[KS > 1 ? KS : 1][PK ? 1 : 3][64];
    __shared__ float lxs[16];
    __shared__ float dm[PK ? 16 * 17 : 1];
    const int P = (nkc + KS * SP - 1) / (KS * SP);
    int rb = blockIdx.x, kp = 0;
    if (rb >= a.nrb) return;  // uniform over the workgroup
    auto load = [&](int4v* wv, int rbl, int kpl) {
        const size_t wbase = (size_t)(a.rb0 + rbl) * nkc;
        const int c0 = kpl * KS * SP + wave * SP;
        // unconditional loads (steps past the row clamped to its last one)
#pragma unroll
        for (int u = 0; u < SP; u++) wv[u] = ((const int4v*)a.w)[(wbase + min(c0 + u, nkc - 1)) * 64 + lane];
    };
    int4v wA[SP];
    float xsv = 0.f;
    if constexpr (XM == XM_PREP) {
        x_dma(a.src, nkc * 4 * M * 3, smem);  // three planes
        xsv = a.src.xs[threadIdx.x & 15];
    }
    __builtin_amdgcn_sched_barrier(0);
    load(wA, rb, 0);
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (XM == XM_PREP) {
        wait_vmcnt<SP>();  // operand planes and xs are in
        if (threadIdx.x < 16) lxs[threadIdx.x] = xsv;
    } else if constexpr (XM == XM_FUSED) {
        stage_x<true>(a.src, M, DT_Q8ROW, nkc, smem, lxs);
    } else if (threadIdx.x < 16) {
        lxs[threadIdx.x] = a.src.xs[threadIdx.x];
    }
    __syncthreads();
    // operand planes [item][b] x 16 B, q0 q1 q2: in LDS, or read in place
    const int lpl = nkc * 4 * M;
    const int4v* L0 = XM != XM_GLOBAL ? (const int4v*)smem : (const int4v*)a.src.planes;
    // PK: lane r reads plane pr of batch row br
    // lanes whose A row is past the batch read batch row 0 of plane 0: their
    // D rows are never used, and every lane loads unconditionally
    const bool xin = PK ? r < 3 * M : r < M;
    const int pr = PK && xin ? r / M : 0, br = xin ? (PK ? r - pr * M : r) : 0;
    const int4v* LP = L0 + pr * lpl;
    const int xoff = s * M + br, M4 = 4 * M;
    int4v a0 = {0, 0, 0, 0}, a1 = {0, 0, 0, 0}, a2 = {0, 0, 0, 0};

    auto process = [&](const int4v* wv) {
        const int c0 = kp * KS * SP + wave * SP;
#pragma unroll
        for (int u = 0; u < SP; u++) {
            if (c0 + u < nkc) {
                const int o = (c0 + u) * M4 + xoff;
                if constexpr (PK) {
                    const int4v x0 = LP[o];
                    a0 = __builtin_amdgcn_mfma_i32_16x16x64_i8(x0, wv[u], a0, 0, 0, 0);
                } else {
                    const int4v x0 = L0[o], x1 = L0[lpl + o], x2 = L0[2 * lpl + o];
                    a0 = __builtin_amdgcn_mfma_i32_16x16x64_i8(x0, wv[u], a0, 0, 0, 0);
                    a1 = __builtin_amdgcn_mfma_i32_16x16x64_i8(x1, wv[u], a1, 0, 0, 0);
                    a2 = __builtin_amdgcn_mfma_i32_16x16x64_i8(x2, wv[u], a2, 0, 0, 0);
                }
            }
        }
        if (kp < P - 1) return;  // the row block continues in the next unit
        // per-wave partials in f32 (exact while |partial| < 2^24, i.e. for K
        // shares up to 1024 columns), summed over waves in wave order
        float4v f0 = {(float)a0[0], (float)a0[1], (float)a0[2], (float)a0[3]};
        float4v f1 = {(float)a1[0], (float)a1[1], (float)a1[2], (float)a1[3]};
        float4v f2 = {(float)a2[0], (float)a2[1], (float)a2[2], (float)a2[3]};
        a0 = int4v{0, 0, 0, 0};
        a1 = a0;
        a2 = a0;
        if constexpr (KS > 1) {
            part[wave][0][lane] = f0;
            if constexpr (!PK) {
                part[wave][1][lane] = f1;
                part[wave][2][lane] = f2;
            }
            __syncthreads();
        }
        if (wave == 0) {
#pragma unroll
            for (int q = 1; q < KS; q++) {
                f0 += part[q][0][lane];
                if constexpr (!PK) {
                    f1 += part[q][1][lane];
                    f2 += part[q][2][lane];
                }
            }
            if constexpr (PK) {
                // D[4s + v][r] through LDS to rows p*M + b of plane p (wave 0 only)
#pragma unroll
                for (int v = 0; v < 4; v++) dm[(4 * s + v) * 17 + r] = f0[v];
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                __builtin_amdgcn_wave_barrier();
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
                for (int v = 0; v < 4; v++) {
                    const int b = 4 * s + v;
                    if (b < M) {
                        f0[v] = dm[b * 17 + r];
                        f1[v] = dm[(M + b) * 17 + r];
                        f2[v] = dm[(2 * M + b) * 17 + r];
                    }
                }
                // dm is rewritten only by this wave's next row block
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                __builtin_amdgcn_wave_barrier();
            }
            const int row = (a.rb0 + rb) * 16 + r;
            if (row >= a.row_lo && row < a.row_hi) {
                const float rs = ((const float*)a.scale)[row];
#pragma unroll
                for (int v = 0; v < 4; v++) {
                    const int b = 4 * s + v;
                    if (b < M) {
                        const float tt = f0[v] + f1[v] * 0.0078125f + f2[v] * 6.103515625e-05f;
                        float* yp = a.y + (size_t)b * a.ldy + (row - a.row_lo);
                        const float val = (tt * lxs[b]) * rs;
                        *yp = a.resid ? *yp + val : val;
                    }
                }
            }
        }
        if constexpr (KS > 1) __syncthreads();
    };

    for (;;) {
        int rn = rb, kn = kp + 1;
        if (kn == P) {
            kn = 0;
            rn += gridDim.x;
        }
        process(wA);
        if (rn >= a.nrb) break;
        rb = rn;
        kp = kn;
        load(wA, rb, kp);
    }
}

// ---------------------------------------------------------------------------
// Kernel instance tables (one translation unit per weight codec).
// ---------------------------------------------------------------------------
template <int FMT, int NV, bool HL, int XM>
GemvKernel q4_by_ks(int ks) {
    switch (ks) {
        case 1: return k_gemv_q4<FMT, NV, 1, HL, XM>;
        case 2: return k_gemv_q4<FMT, NV, 2, HL, XM>;
        case 4: return k_gemv_q4<FMT, NV, 4, HL, XM>;
        case 8: return k_gemv_q4<FMT, NV, 8, HL, XM>;
    }
    // two MFMAs per tile need more than the 128 registers a 16-wave
    // workgroup leaves each wave
    if constexpr (HL)
        if (ks == 16) return k_gemv_q4<FMT, NV, 16, HL, XM>;
    return nullptr;
}
template <int FMT, int NV, bool HL>
GemvKernel q4_by_xm(int xm, int ks) {
    switch (xm) {
        case XM_PREP: return q4_by_ks<FMT, NV, HL, XM_PREP>(ks);
        case XM_FUSED: return q4_by_ks<FMT, NV, HL, XM_FUSED>(ks);
        case XM_GLOBAL: return q4_by_ks<FMT, NV, HL, XM_GLOBAL>(ks);
    }
    return nullptr;
}
template <int FMT>
GemvKernel q4_pick(int m, int xm, int ks) {
    if (m == 1) return q4_by_xm<FMT, 1, true>(xm, ks);
    if (m <= 8) return q4_by_xm<FMT, 4, true>(xm, ks);
    return q4_by_xm<FMT, 4, false>(xm, ks);
}
template <bool PK, int XM>
GemvKernel q8_by_ks(int ks) {
    switch (ks) {
        case 1: return k_gemv_q8<1, PK, XM>;
        case 2: return k_gemv_q8<2, PK, XM>;
        case 4: return k_gemv_q8<4, PK, XM>;
        case 8: return k_gemv_q8<8, PK, XM>;
        case 16: return k_gemv_q8<16, PK, XM>;
    }
    return nullptr;
}
template <bool PK>
GemvKernel q8_by_xm(int xm, int ks) {
    switch (xm) {
        case XM_PREP: return q8_by_ks<PK, XM_PREP>(ks);
        case XM_FUSED: return q8_by_ks<PK, XM_FUSED>(ks);
        case XM_GLOBAL: return q8_by_ks<PK, XM_GLOBAL>(ks);
    }
    return nullptr;
}

}  // namespace cmf
