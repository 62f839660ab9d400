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
//             as the accumulator input -8 * 2^-24 * sum(x) of the tile (prep16_row), and
//             x is carried as f16 hi + lo of x*2^e (22-bit significand).
//             Each tile's product is scaled by its tile scale and
//             accumulated in f32, as q4t_row_exact does
//             (qtensor.rs:4418-4432).
//   - the activation operand arrives prepared (planes written by a producer
//     kernel: RMSNorm of the residual rows, SwiGLU of the gate/up rows, the
//     MTP [enorm(embed); hnorm(h)] concat or plain rows) and is copied to
//     LDS by direct global->LDS loads; when it does not fit in LDS the
//     planes are read from global memory (L2) in place.
//   - optional residual epilogue: y is added into the output (h += W x).
#pragma once

#include "common.h"
#include "gemv.h"
#include "wave.h"

namespace cmf {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float float4v __attribute__((ext_vector_type(4)));
typedef int int4v __attribute__((ext_vector_type(4)));

// Weight words are read exactly once per launch: nontemporal loads keep the
// stream from displacing the operand planes and partials in L2 (measured on
// a plain 28 MB read: 5.8 -> 5.6 us; 108 MB: 19.0 -> 17.6 us).
// Every load issued while the operand's direct-to-LDS copy is in flight
// goes through a global-address-space pointer: a generic (flat) load may
// alias LDS, so the compiler waits for the whole copy (vmcnt(0)) before
// issuing it, which put a full memory round trip in front of the weight
// stream.
template <class T>
__device__ __forceinline__ const __attribute__((address_space(1))) T* gptr(const T* p) {
    return (const __attribute__((address_space(1))) T*)p;
}
// (scalar and ext_vector types only: the HIP vector classes cannot be copied
// out of another address space)
template <class T>
__device__ __forceinline__ T ldg(const T* p) {
    return *gptr(p);
}
__device__ __forceinline__ float2 ldg_f2(const float2* p) {
    const uint64_t u = ldg((const uint64_t*)p);
    return make_float2(__uint_as_float((uint32_t)u), __uint_as_float((uint32_t)(u >> 32)));
}
__device__ __forceinline__ int4v ld_stream(const int4v* p) { return __builtin_nontemporal_load(gptr(p)); }
__device__ __forceinline__ uint4 ld_stream(const uint4* p) {
    const int4v v = __builtin_nontemporal_load(gptr((const int4v*)p));
    return make_uint4((uint32_t)v.x, (uint32_t)v.y, (uint32_t)v.z, (uint32_t)v.w);
}

constexpr int LDSX_MAX = 128 * 1024;  // largest LDS-staged activation operand (+ scratch)
constexpr int LDSX_MAX_G3 = 144 * 1024;  // ... of a grouped (one per CU) workgroup

// Four nibble bytes (8 weights: elements 8s..8s+7 of a tile) to the f16
// denormals n * 2^-24 (exact, the raw nibble under a zero exponent) in the
// in-slot order {0,4,2,6,1,5,3,7}: one mask (and shift) per pair.  The -8
// offset of the format enters through the MFMA accumulator (the tile biases
// written by prep16_row).
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

// Prepared planes go to LDS by direct global->LDS loads (no registers),
// issued before the weight stream: the loads of a wave complete in order, so
// the operand is in LDS once at most the weight loads issued after it are
// outstanding (vmcnt).  Wave w copies 1 KiB chunks w, w + nw, ... (indices
// clamped to the last item, so the copy never reads past the planes).
__device__ __forceinline__ void x_dma_ptr(const void* src, int n, uint8_t* lx) {
    const uint4* g = (const uint4*)src;
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int nw = blockDim.x >> 6;
    for (int c = wave; c * 64 < n; c += nw)
        __builtin_amdgcn_global_load_lds((const void*)(g + min(c * 64 + lane, n - 1)),
                                         (__attribute__((address_space(3))) void*)(lx + c * 1024), 16, 0, 0);
}
__device__ __forceinline__ void x_dma(const XSrc& s, int n, uint8_t* lx) {
    const uint4* g = (const uint4*)s.planes;
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int nw = blockDim.x >> 6;
    for (int c = wave; c * 64 < n; c += nw)
        __builtin_amdgcn_global_load_lds((const void*)(g + min(c * 64 + lane, n - 1)),
                                         (__attribute__((address_space(3))) void*)(lx + c * 1024), 16, 0, 0);
}
// Fused operand (XM_FUSED): the raw rows b < m of the operand (K floats at
// x + b*ldx) and, for XS_NORM, the norm weight (K floats) go to LDS by
// direct loads, issued before the weight stream like x_dma; stage_fused then
// evaluates the producer in every workgroup while its weights are in flight.
// raw[] sits after the planes at a 1 KiB boundary and its allocation is
// rounded up to 1 KiB, so the clamped tail of the last wave load stays in it.
// XS_CAT (the MTP operand [rms_norm(embed(tok)) * w ; rms_norm(x) * w2], H
// columns each, pipeline.rs:3085-3094): after the m output rows raw[m][K]
// (1 KiB aligned) sit the rows x [m][H], w [H], w2 [H] (f32), the tokens'
// int8 embedding rows [m][cat_row_bytes(H)] and their row scales [m] (0 for
// a token outside the table).  The host admits it for H % 256 == 0, so the
// f32 part is a whole number of wave loads and needs no clamped tail.
__device__ __forceinline__ int cat_row_bytes(int H) { return (H + 1023) & ~1023; }
__device__ __forceinline__ float* cat_area(float* raw, int m, int K) {
    return raw + ((((size_t)m * K * 4) + 1023) & ~(size_t)1023) / 4;
}

__device__ __forceinline__ void x_dma_cat(const XSrc& s, int m, float* raw) {
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int nw = blockDim.x >> 6;
    const int H = s.H, c16 = H >> 2;
    float* area = cat_area(raw, m, 2 * H);
    const int n = (m + 2) * c16;  // a multiple of 64
    for (int c = wave * 64; c < n; c += nw * 64) {
        const int idx = c + lane;
        const int b = idx / c16, j = idx - b * c16;
        const float* g = b < m ? s.x + (size_t)b * s.ldx + 4 * j : (b == m ? s.w : s.w2) + 4 * j;
        __builtin_amdgcn_global_load_lds((const void*)g, (__attribute__((address_space(3))) void*)(area + 4 * c), 16,
                                         0, 0);
    }
    // embedding row of token t: the 16-byte chunk j (columns 16j..16j+15) of
    // the q8 device layout sits at ((t/16 * nkc + j/4) * 64 + 16 (j%4) + t%16) * 16
    uint8_t* eq = (uint8_t*)(area + (size_t)(m + 2) * H);
    const int EH = cat_row_bytes(H), e16 = H >> 4;
    float* crs = (float*)(eq + (size_t)m * EH);
    for (int b = wave; b < m; b += nw) {
        const int tok = s.toks[b];
        const bool tv = tok >= 0 && tok < s.emb.rows;
        const int t = tv ? tok : 0;
        const int8_t* rowbase = s.emb.w + ((size_t)(t >> 4) * s.emb.nkc * 64 + (t & 15)) * 16;
        for (int j0 = 0; j0 < e16; j0 += 64) {
            const int j = min(j0 + lane, e16 - 1);  // the tail stays inside the row's EH bytes
            __builtin_amdgcn_global_load_lds((const void*)(rowbase + ((size_t)(j >> 2) * 64 + 16 * (j & 3)) * 16),
                                             (__attribute__((address_space(3))) void*)(eq + (size_t)b * EH + 16 * j0),
                                             16, 0, 0);
        }
        const float rs = ldg(s.emb.rs + t);
        if (lane == 0) crs[b] = tv ? rs : 0.f;
    }
}

__device__ __forceinline__ void x_dma_rows(const XSrc& s, int m, int K, float* raw) {
    if (s.mode == XS_CAT) {
        x_dma_cat(s, m, raw);
        return;
    }
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int nw = blockDim.x >> 6;
    const int c16 = K >> 2;  // 16-byte chunks per row
    const int n = (m + (s.mode == XS_NORM ? 1 : 0)) * c16;
    for (int c = wave * 64; c < n; c += nw * 64) {
        const int idx = min(c + lane, n - 1);
        const int b = idx / c16, j = idx - b * c16;
        const float* g = b < m ? s.x + (size_t)b * s.ldx + 4 * j : s.w + 4 * j;
        __builtin_amdgcn_global_load_lds((const void*)g, (__attribute__((address_space(3))) void*)(raw + 4 * c), 16,
                                         0, 0);
    }
}

// The producer of k_prep_src (XS_NORM: rms_norm(x) * w, inference.rs:33-50;
// XS_ROWS: the rows) for the m rows in raw[] (in place), then their planes
// (prep8_rows / prep16_rows) into planes and xs, all in LDS.  One wave per
// row (rows wave, wave + nw, ...): sum of squares in f64 and the row's
// max|y| reduce inside the wave, so the rows proceed in parallel with no
// workgroup barrier between them.  Ends with a barrier; the caller has made
// raw[] visible (barrier after the loads).
__device__ __forceinline__ void stage_fused(const XSrc& src, int m, int K, int fmt, int nk, float* raw,
                                            uint8_t* planes, float* xs) {
    const int mode = src.mode;
    const double eps = src.eps;
    __shared__ float amv[MAXB];
    const int tid = threadIdx.x, nt = blockDim.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), nw = nt >> 6;
    const bool nrm = mode == XS_NORM;
    const float* wn = raw + (size_t)m * K;
    // float4 LDS reads, four in flight per lane (K % 4 == 0, rows 16 B
    // aligned): each pass costs about one LDS round trip per 1024 columns
    const int K4 = K >> 2;
    if (mode == XS_CAT) {
        // the two halves: the token's embedding row (int8 * row scale, as
        // k_prep_src) and the hidden row, each rms-normed with its weight
        const int H = K >> 1, H4 = H >> 2;
        const float* area = cat_area(raw, m, K);
        const float4* w1 = (const float4*)(area + (size_t)m * H);
        const float4* w2 = w1 + H4;
        const uint8_t* eq = (const uint8_t*)(area + (size_t)(m + 2) * H);
        const int EH = cat_row_bytes(H);
        const float* crs = (const float*)(eq + (size_t)m * EH);
        for (int b = wave; b < m; b += nw) {
            float4* xr = (float4*)(raw + (size_t)b * K);
            const float4* hr = (const float4*)(area + (size_t)b * H);
            const uint32_t* er = (const uint32_t*)(eq + (size_t)b * EH);
            const float rs = crs[b];
            double a1 = 0.0, a2 = 0.0;
#pragma unroll 4
            for (int i = lane; i < H4; i += 64) {
                const uint32_t q = er[i];
                const float4 e = make_float4((float)(int8_t)(q & 0xFF) * rs, (float)(int8_t)((q >> 8) & 0xFF) * rs,
                                             (float)(int8_t)((q >> 16) & 0xFF) * rs, (float)(int8_t)(q >> 24) * rs);
                xr[i] = e;
                a1 += (double)e.x * (double)e.x + (double)e.y * (double)e.y + (double)e.z * (double)e.z +
                      (double)e.w * (double)e.w;
                const float4 h = hr[i];
                a2 += (double)h.x * (double)h.x + (double)h.y * (double)h.y + (double)h.z * (double)h.z +
                      (double)h.w * (double)h.w;
            }
            const float inv1 = 1.0f / (float)sqrt(wave_sum(a1) / (double)H + eps);
            const float inv2 = 1.0f / (float)sqrt(wave_sum(a2) / (double)H + eps);
            float am = 0.f;
#pragma unroll 4
            for (int i = lane; i < H4; i += 64) {
                const float4 e = xr[i], we = w1[i], h = hr[i], wh = w2[i];
                const float4 y1 = make_float4(e.x * inv1 * we.x, e.y * inv1 * we.y, e.z * inv1 * we.z, e.w * inv1 * we.w);
                const float4 y2 = make_float4(h.x * inv2 * wh.x, h.y * inv2 * wh.y, h.z * inv2 * wh.z, h.w * inv2 * wh.w);
                xr[i] = y1;
                xr[H4 + i] = y2;
                am = fmaxf(am, fmaxf(fmaxf(fabsf(y1.x), fabsf(y1.y)), fmaxf(fabsf(y1.z), fabsf(y1.w))));
                am = fmaxf(am, fmaxf(fmaxf(fabsf(y2.x), fabsf(y2.y)), fmaxf(fabsf(y2.z), fabsf(y2.w))));
            }
            am = wave_max(am);
            if (lane == 0) amv[b] = am;
        }
    }
    for (int b = wave; mode != XS_CAT && b < m; b += nw) {
        float4* xr = (float4*)(raw + (size_t)b * K);
        const float4* w4 = (const float4*)wn;
        float inv = 1.f;
        if (nrm) {
            double acc = 0.0;
#pragma unroll 4
            for (int i = lane; i < K4; i += 64) {
                const float4 v = xr[i];
                acc += (double)v.x * (double)v.x + (double)v.y * (double)v.y + (double)v.z * (double)v.z +
                       (double)v.w * (double)v.w;
            }
            inv = 1.0f / (float)sqrt(wave_sum(acc) / (double)K + eps);
        }
        float am = 0.f;
#pragma unroll 4
        for (int i = lane; i < K4; i += 64) {
            float4 v = xr[i];
            if (nrm) {
                const float4 ww = w4[i];
                v = make_float4(v.x * inv * ww.x, v.y * inv * ww.y, v.z * inv * ww.z, v.w * inv * ww.w);
                xr[i] = v;
            }
            am = fmaxf(am, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
        }
        am = wave_max(am);
        if (lane == 0) amv[b] = am;
    }
    __syncthreads();
    if (fmt == DT_Q8ROW) prep8_rows(raw, K, amv, nk, m, planes, xs, tid, nt);
    else prep16_rows(raw, K, amv, nk, m, planes, xs, tid, nt);
    __syncthreads();
}
// bytes of the prepared planes a GEMV workgroup holds in LDS (1 KiB aligned:
// the raw rows of XM_FUSED follow)
__device__ __forceinline__ int planes_lds_bytes(int fmt, int nk, int m) {
    // (q4, m > 8: the lo-plane bias table T2 too)
    const int b = fmt == DT_Q8ROW ? nk * 192 * m : nk * 16 * (32 * m + (m > 8 ? 32 : 16));
    return (b + 1023) & ~1023;
}

// s_waitcnt vmcnt(N) (gfx9 encoding: vmcnt bits 3:0 and 15:14, expcnt 6:4
// and lgkmcnt 11:8 left at their maxima, i.e. not waited for)
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// The epilogue's global reads for row block rb, issued at the start of the
// kernel: the q8 row scale (rowscale != nullptr) and, for a residual GEMV,
// y[b][row] of the lane's batch rows b = 4s + v (indices clamped, so every
// lane loads; values for rows or batch rows out of range are never used).
__device__ __forceinline__ void prefetch_epilogue(const GemvArgs& a, int rb, int r, int s, int M,
                                                  const float* rowscale, float& rs, float (&yv)[4]) {
    const int row = max(a.row_lo, min((a.rb0 + rb) * 16 + r, a.row_hi - 1));
    rs = rowscale ? ldg(rowscale + row) : 0.f;
    if (a.resid) {
#pragma unroll
        for (int v = 0; v < 4; v++) yv[v] = ldg(a.y + (size_t)min(4 * s + v, M - 1) * a.ldy + (row - a.row_lo));
    }
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
// are added at the end.  XM: where the prepared activation operand is read
// (XM_PREP: copied to LDS first, XM_GLOBAL: in place, for operands larger
// than the LDS budget).  (Producing the operand in every workgroup from the
// raw rows instead of one producer launch per GEMV was measured 1.3-2x
// slower per GEMV on MI355X: the per-workgroup staging sits on the critical
// path of these latency-bound launches.)
constexpr int SP = 4;  // weight steps per wave and work unit
// XM_PREPC (q8): XM_PREP with one scale per (batch row, 64-column chunk)
enum { XM_PREP = 0, XM_FUSED = 1, XM_GLOBAL = 2, XM_PREPC = 3 };

// ONE: every workgroup serves exactly one unit (one K part, its row blocks;
// the host launches it only so): no loop, so the compiler waits for each
// step's weights in turn instead of for all of them before the first MFMA
template <int FMT, int NV, int KS, bool HL, int XM, int RB, int G = 1, int SPW = SP, bool ONE = false>
__global__ __launch_bounds__(64 * KS * G) void k_gemv_q4(GemvArgs args) {
    GemvArgs a = args;
    if (a.jobs) {  // grouped launch: this workgroup serves job blockIdx.y
        const int j = blockIdx.y;
        if (j >= a.jobs[0]) return;  // uniform over the workgroup
        const GemvDesc d = a.desc[a.jobs[1 + j]];
        a.w = d.w;
        a.scale = d.scale;
        a.rowp = d.rowp;
        a.src.planes += j * a.planes_stride;
        if (a.planes_stride) a.src.xs += 16 * j;  // stride 0: one operand for all jobs
        a.y += j * a.y_stride;
    }
    extern __shared__ __align__(16) uint8_t smem[];
    const int lane = threadIdx.x & 63, wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    // G groups of KS waves: group grp owns its own row blocks, wave (K
    // share) within it; the groups share the operand copy
    const int grp = G > 1 ? wv / KS : 0, wave = G > 1 ? wv % KS : wv;
    const int r = lane & 15, s = lane >> 4;
    const int M = a.m, ntg = a.nk;  // nk = groups of 4 tiles
    constexpr bool TP = FMT == DT_Q4TP;
    constexpr int LD = 16 * 33;  // one row block's ladders
    __shared__ float lad[G][TP ? 2 : 1][TP ? RB * LD : 1];  // ladders of the current / next row blocks
    __shared__ float4v part[G][KS][RB][64];
    __shared__ float lxs[16];
    const int P = (ntg + KS * SPW - 1) / (KS * SPW);  // K parts per row block
    const int rstep = gridDim.x * G * RB;
    int rb = (blockIdx.x * G + grp) * RB, kp = 0;  // first of the RB row blocks of the unit
    // groups past the matrix run with clamped loads and store nothing; the
    // workgroup's first group decides (uniform) when the walk ends
    if (blockIdx.x * G * RB >= a.nrb) return;
    // weights + tile scales of a unit (q4tp: and the row ladder parameters
    // of its row blocks), all unconditional (steps past the row clamped to
    // its last one, row blocks past the matrix to its last one): a load
    // under a branch makes the compiler wait for it at once.  NL = loads per
    // call.
    constexpr int NL = RB * (2 * SPW + (TP ? 1 : 0));
    auto load_steps = [&](uint4* wv, uint2* sv, int rbl, int kpl, int u0, int u1) {
        const int t0 = kpl * KS * SPW + wave * SPW;
#pragma unroll
        for (int q = 0; q < RB; q++) {
            const size_t wbase = (size_t)(a.rb0 + min(rbl + q, a.nrb - 1)) * ntg;
#pragma unroll
            for (int u = u0; u < u1; u++) {
                const size_t t = wbase + min(t0 + u, ntg - 1);
                wv[q * SPW + u] = ld_stream((const uint4*)a.w + t * 64 + lane);
                if constexpr (TP) sv[q * SPW + u] = make_uint2(ldg((const uint32_t*)a.scale + t * 16 + r), 0u);
                else {
                    const uint64_t sw = ldg((const uint64_t*)a.scale + t * 16 + r);  // (scalar type: see gptr)
                    sv[q * SPW + u] = make_uint2((uint32_t)sw, (uint32_t)(sw >> 32));
                }
            }
        }
    };
    auto load_rowp = [&](float2* pv, int rbl) {
        if constexpr (TP) {
#pragma unroll
            for (int q = 0; q < RB; q++) pv[q] = ldg_f2(a.rowp + (a.rb0 + min(rbl + q, a.nrb - 1)) * 16 + r);
        }
    };
    auto load = [&](uint4* wv, uint2* sv, float2* pv, int rbl, int kpl) {
        load_steps(wv, sv, rbl, kpl, 0, SPW);
        load_rowp(pv, rbl);
    };
    // the 32-rung ladder of each row of the RB row blocks: t[c] = t[c-1] *
    // ratio (quant.rs:399-410), by 16 threads per row block starting at the
    // second wave (the first one reduces meanwhile)
    auto ladder = [&](int buf, const float2* p) {
        if constexpr (TP) {
            const int lt = (int)threadIdx.x - grp * 64 * KS - (KS > 1 ? 64 : 0);
#pragma unroll
            for (int q = 0; q < RB; q++) {
                if (lt >= 16 * q && lt < 16 * q + 16) {
                    float tv = p[q].x;
                    float* lq = &lad[grp][buf][q * LD + (lt - 16 * q) * 33];
                    lq[0] = tv;
                    for (int c = 1; c < 32; c++) {
                        tv = tv * p[q].y;
                        lq[c] = tv;
                    }
                }
            }
        }
    };
    uint4 wA[RB * SPW];
    uint2 sA[RB * SPW];
    float2 pA[RB] = {};
    float xsv = 0.f;
    float* raw = (float*)(smem + planes_lds_bytes(FMT, ntg, M));
    // the first row blocks' residual rows, requested first (the epilogue
    // then waits for no memory round trip)
    const int rb_first = rb;
    float rs_unused, y_first[RB][4];
#pragma unroll
    for (int q = 0; q < RB; q++) prefetch_epilogue(a, rb + q, r, s, M, nullptr, rs_unused, y_first[q]);
    if constexpr (XM == XM_PREP) {
        x_dma(a.src, ntg * (32 * M + (HL ? 16 : 32)), smem);  // hi + lo planes + tile biases (!HL: both tables)
        xsv = ldg(a.src.xs + (threadIdx.x & 15));
    } else if constexpr (XM == XM_FUSED) {
        x_dma_rows(a.src, M, a.src.K, raw);
        // the raw rows arrive before the weight stream is requested: measured
        // on MI355X, staging overlapped with the stream then starts earlier
        // than with both in flight together (down 1024x3072 m=1: 5.7 vs 6.4 us)
        wait_vmcnt<0>();
    }
    __builtin_amdgcn_sched_barrier(0);
    load(wA, sA, pA, rb, 0);
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (XM == XM_PREP) {
        wait_vmcnt<NL>();  // operand planes and xs are in
        if (threadIdx.x < 16) lxs[threadIdx.x] = xsv;
    } else if constexpr (XM == XM_FUSED) {
        wait_vmcnt<NL>();  // raw rows are in
        __syncthreads();
        stage_fused(a.src, M, a.src.K, FMT, ntg * 4, raw, smem, lxs);
    } else if (threadIdx.x < 16) {
        lxs[threadIdx.x] = a.src.xs[threadIdx.x];
    }
    ladder(0, pA);
    __syncthreads();
    // operand planes [item][b] x 16 B, hi then lo: in LDS, or read in place
    const uint4* LH = XM != XM_GLOBAL ? (const uint4*)smem : (const uint4*)a.src.planes;
    const uint4* LL = LH + ntg * 4 * 4 * M;
    const float4v* LB = (const float4v*)(LL + ntg * 4 * 4 * M);  // tile biases [tile][16] (T1)
    const float4v* LB2 = LB + ntg * 16;                           // the lo plane's (T2), !HL
    // lanes whose A row is past the batch read batch row 0: their D rows are
    // never stored, and every lane loads unconditionally
    const uint4* LX = HL ? (r < 8 ? LH : LL) : LH;
    const int xb = HL ? ((r & 7) < M ? (r & 7) : 0) : (r < M ? r : 0);
    const int xoff = s * M + xb, M4 = 4 * M;
    const float4v zero = {0.f, 0.f, 0.f, 0.f};
    float4v acc[RB];
#pragma unroll
    for (int q = 0; q < RB; q++) acc[q] = zero;
    int buf = 0;

    // one work unit: rb/kp current, rn the next unit's first row block
    // (rn >= nrb: none); one operand read serves the RB row blocks
    auto process = [&](const uint4* wv, const uint2* sv, const float2* pn, int rn) {
        const int t0 = kp * KS * SPW + wave * SPW;
#pragma unroll
        for (int u = 0; u < SPW; u++) {
            if (t0 + u < ntg) {
                const int tg = t0 + u;
                float sc[RB][4];
#pragma unroll
                for (int q = 0; q < RB; q++) {
                    const uint2 sq = sv[q * SPW + u];
                    if constexpr (!TP) {
                        sc[q][0] = f16_bits_to_f32(sq.x & 0xFFFFu);
                        sc[q][1] = f16_bits_to_f32(sq.x >> 16);
                        sc[q][2] = f16_bits_to_f32(sq.y & 0xFFFFu);
                        sc[q][3] = f16_bits_to_f32(sq.y >> 16);
                    } else {
                        const uint32_t cw = sq.x;
                        const float* lq = &lad[grp][buf][q * LD + r * 33];
                        sc[q][0] = lq[cw & 31];
                        sc[q][1] = lq[(cw >> 5) & 31];
                        sc[q][2] = lq[(cw >> 10) & 31];
                        sc[q][3] = lq[(cw >> 15) & 31];
                    }
                }
#pragma unroll
                for (int t = 0; t < 4; t++) {
                    const int item = (tg * 4 + t) * M4 + xoff;
                    const float4v cb = LB[(tg * 4 + t) * 4 + s];  // rows 4s..4s+3
                    float4v cbl = {0.f, 0.f, 0.f, 0.f};
                    if constexpr (!HL) cbl = LB2[(tg * 4 + t) * 4 + s];
                    half8 xa, xh, xl;
                    if constexpr (HL) {
                        xa = __builtin_bit_cast(half8, LX[item]);
                    } else {
                        xh = __builtin_bit_cast(half8, LH[item]);
                        xl = __builtin_bit_cast(half8, LL[item]);
                    }
#pragma unroll
                    for (int q = 0; q < RB; q++) {
                        const uint32_t wq = t == 0 ? wv[q * SPW + u].x
                                            : t == 1 ? wv[q * SPW + u].y
                                            : t == 2 ? wv[q * SPW + u].z
                                                     : wv[q * SPW + u].w;
                        const half8 bq = dq_nib_word(wq);
                        float4v d;
                        if constexpr (HL) {
                            d = __builtin_amdgcn_mfma_f32_16x16x32_f16(xa, bq, cb, 0, 0, 0);
                        } else {
                            // hi and lo in accumulators of their own: each
                            // tile sum is exact only within one plane
                            d = __builtin_amdgcn_mfma_f32_16x16x32_f16(xh, bq, cb, 0, 0, 0);
                            d += __builtin_amdgcn_mfma_f32_16x16x32_f16(xl, bq, cbl, 0, 0, 0);
                        }
#pragma unroll
                        for (int v = 0; v < NV; v++) acc[q][v] += d[v] * sc[q][t];
                    }
                }
            }
        }
        if (kp < P - 1) return;  // the row blocks continue in the next unit
        if constexpr (KS > 1) {
#pragma unroll
            for (int q = 0; q < RB; q++) part[grp][wave][q][lane] = acc[q];
            __syncthreads();
        }
        if (wave == 0) {
#pragma unroll
            for (int q = 0; q < RB; q++) {
                float4v o4 = acc[q];
#pragma unroll
                for (int w = 1; w < KS; w++) {
                    const float4v o = part[grp][w][q][lane];
#pragma unroll
                    for (int v = 0; v < NV; v++) o4[v] += o[v];
                }
                if constexpr (HL) {
                    // hi rows (lanes s = 0, 1) + lo rows (lanes s = 2, 3)
#pragma unroll
                    for (int v = 0; v < NV; v++) o4[v] += __shfl_xor(o4[v], 32);
                }
                const int rbq = rb + q;
                const int row = (a.rb0 + rbq) * 16 + r;
                if (a.epi == EPI_SWIGLU) {
                    // rows r < 8 gate, r + 8 the matching up row (lane ^ 8):
                    // y[b][8 rb + r] = silu(g) * u (inference.rs:14-16)
#pragma unroll
                    for (int v = 0; v < NV; v++) {
                        const int b = 4 * s + v;
                        const float val = o4[v] * lxs[b & 15] * 16777216.0f;
                        const float u = __shfl_xor(val, 8);
                        if (rbq < a.nrb && r < 8 && b < M && (!HL || s < 2))
                            a.y[(size_t)b * a.ldy + (a.rb0 + rbq) * 8 + r] = (val / (1.0f + expf(-val))) * u;
                    }
                } else if (rbq < a.nrb && row >= a.row_lo && row < a.row_hi && (!HL || s < 2)) {
#pragma unroll
                    for (int v = 0; v < NV; v++) {
                        const int b = 4 * s + v;
                        if (b < M) {
                            float* yp = a.y + (size_t)b * a.ldy + (row - a.row_lo);
                            const float val = o4[v] * lxs[b] * 16777216.0f;  // 2^24: denormal nibbles
                            *yp = a.resid ? (rb == rb_first ? y_first[q][v] : *yp) + val : val;
                        }
                    }
                }
            }
        }
#pragma unroll
        for (int q = 0; q < RB; q++) acc[q] = zero;
        if (rn < a.nrb) ladder(buf ^ 1, pn);
        buf ^= 1;
        if constexpr (KS > 1 || TP || G > 1) __syncthreads();
    };

    if constexpr (ONE) {
        const float2 pn[RB] = {};
        process(wA, sA, pn, a.nrb);  // (no next unit)
        return;
    }
    for (;;) {
        int rn = rb, kn = kp + 1;
        if (kn == P) {
            kn = 0;
            rn += rstep;
        }
        float2 pn[RB] = {};
        if constexpr (TP)
            if (rn < a.nrb) {
#pragma unroll
                for (int q = 0; q < RB; q++) pn[q] = ldg_f2(a.rowp + (a.rb0 + min(rn + q, a.nrb - 1)) * 16 + r);
            }
        process(wA, sA, pn, rn);
        if (rn - grp * RB >= a.nrb) break;  // the first group's next unit (uniform)
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
__global__ __launch_bounds__(64 * KS) void k_gemv_q8(GemvArgs args) {
    GemvArgs a = args;
    if (a.jobs) {  // grouped launch: this workgroup serves job blockIdx.y
        const int j = blockIdx.y;
        if (j >= a.jobs[0]) return;  // uniform over the workgroup
        const GemvDesc d = a.desc[a.jobs[1 + j]];
        a.w = d.w;
        a.scale = d.scale;
        a.rowp = d.rowp;
        a.src.planes += j * a.planes_stride;
        if (a.planes_stride) a.src.xs += 16 * j;  // stride 0: one operand for all jobs
        a.y += j * a.y_stride;
    }
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
        for (int u = 0; u < SP; u++) wv[u] = ldg((const int4v*)a.w + (wbase + min(c0 + u, nkc - 1)) * 64 + lane);
    };
    int4v wA[SP];
    float xsv = 0.f;
    float* raw = (float*)(smem + planes_lds_bytes(DT_Q8ROW, nkc, M));
    // the first row block's row scale and residual rows, requested first so
    // that the epilogue does not wait for a memory round trip
    const int rb_first = rb;
    float rs_first, y_first[4];
    prefetch_epilogue(a, rb, r, s, M, (const float*)a.scale, rs_first, y_first);
    // XM_PREPC: the chunk scales [M][nkc] (contiguous, cs_ld == nkc) follow
    // the planes in LDS at a 1 KiB boundary, copied by direct loads like them
    float* lcs = (float*)(smem + planes_lds_bytes(DT_Q8ROW, nkc, M));
    if constexpr (XM == XM_PREP) {
        x_dma(a.src, nkc * 4 * M * 3, smem);  // three planes
        xsv = ldg(a.src.xs + (threadIdx.x & 15));
    } else if constexpr (XM == XM_PREPC) {
        x_dma(a.src, nkc * 4 * M * 3, smem);
        x_dma_ptr(a.src.cs, (M * nkc + 3) / 4, (uint8_t*)lcs);
    } else if constexpr (XM == XM_FUSED) {
        x_dma_rows(a.src, M, a.src.K, raw);
        // the raw rows arrive before the weight stream is requested: measured
        // on MI355X, staging overlapped with the stream then starts earlier
        // than with both in flight together (down 1024x3072 m=1: 5.7 vs 6.4 us)
        wait_vmcnt<0>();
    }
    __builtin_amdgcn_sched_barrier(0);
    load(wA, rb, 0);
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (XM == XM_PREP) {
        wait_vmcnt<SP>();  // operand planes and xs are in
        if (threadIdx.x < 16) lxs[threadIdx.x] = xsv;
    } else if constexpr (XM == XM_PREPC) {
        wait_vmcnt<SP>();  // operand planes are in
        if (threadIdx.x < 16) lxs[threadIdx.x] = 1.f;  // the chunk scales carry the operand's scale
    } else if constexpr (XM == XM_FUSED) {
        wait_vmcnt<SP>();  // raw rows are in
        __syncthreads();
        stage_fused(a.src, M, a.src.K, DT_Q8ROW, nkc, raw, smem, lxs);
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
    // XM_PREPC: per-chunk partials in f32, each chunk's int32 sums scaled
    // by its chunk scale (and, PK, the plane weight of the lane's D rows
    // 4s + v = p M + b)
    float4v c0f = {0.f, 0.f, 0.f, 0.f}, c1f = c0f, c2f = c0f;
    int cb_[4];
    float cpw_[4];
#pragma unroll
    for (int v = 0; v < 4; v++) {
        const int rr = 4 * s + v;
        const int p = PK ? min(rr / M, 2) : 0, b = PK ? rr - p * M : rr;
        cb_[v] = min(b, M - 1);
        cpw_[v] = p == 0 ? 1.f : (p == 1 ? 0.0078125f : 6.103515625e-05f);
    }

    auto process = [&](const int4v* wv) {
        const int c0 = kp * KS * SP + wave * SP;
#pragma unroll
        for (int u = 0; u < SP; u++) {
            if (c0 + u < nkc) {
                const int o = (c0 + u) * M4 + xoff;
                if constexpr (XM == XM_PREPC) {
                    const int cc = c0 + u;
                    const int4v zi = {0, 0, 0, 0};
                    if constexpr (PK) {
                        const int4v d = __builtin_amdgcn_mfma_i32_16x16x64_i8(LP[o], wv[u], zi, 0, 0, 0);
#pragma unroll
                        for (int v = 0; v < 4; v++) c0f[v] += (float)d[v] * (lcs[cb_[v] * nkc + cc] * cpw_[v]);
                    } else {
                        const int4v d0 = __builtin_amdgcn_mfma_i32_16x16x64_i8(L0[o], wv[u], zi, 0, 0, 0);
                        const int4v d1 = __builtin_amdgcn_mfma_i32_16x16x64_i8(L0[lpl + o], wv[u], zi, 0, 0, 0);
                        const int4v d2 = __builtin_amdgcn_mfma_i32_16x16x64_i8(L0[2 * lpl + o], wv[u], zi, 0, 0, 0);
#pragma unroll
                        for (int v = 0; v < 4; v++) {
                            const float sc = lcs[cb_[v] * nkc + cc];
                            c0f[v] += (float)d0[v] * sc;
                            c1f[v] += (float)d1[v] * sc;
                            c2f[v] += (float)d2[v] * sc;
                        }
                    }
                } else if constexpr (PK) {
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
        if constexpr (XM == XM_PREPC) {  // already scaled (plane weights included for PK)
            f0 = c0f;
            f1 = PK ? c0f * 0.f : c1f * 0.0078125f;
            f2 = PK ? c0f * 0.f : c2f * 6.103515625e-05f;
            c0f = float4v{0.f, 0.f, 0.f, 0.f};
            c1f = c0f;
            c2f = c0f;
        }
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
            const bool first = rb == rb_first;
            if (a.epi == EPI_SWIGLU) {
                // rows r < 8 gate, r + 8 the matching up row (lane ^ 8)
                const float rs = first ? rs_first : ((const float*)a.scale)[row];
#pragma unroll
                for (int v = 0; v < 4; v++) {
                    const int b = 4 * s + v;
                    const float tt = XM == XM_PREPC ? f0[v] + f1[v] + f2[v]
                                                    : f0[v] + f1[v] * 0.0078125f + f2[v] * 6.103515625e-05f;
                    const float val = (tt * lxs[b & 15]) * rs;
                    const float u = __shfl_xor(val, 8);
                    if (r < 8 && b < M)
                        a.y[(size_t)b * a.ldy + (a.rb0 + rb) * 8 + r] = (val / (1.0f + expf(-val))) * u;
                }
            } else if (row >= a.row_lo && row < a.row_hi) {
                const float rs = first ? rs_first : ((const float*)a.scale)[row];
#pragma unroll
                for (int v = 0; v < 4; v++) {
                    const int b = 4 * s + v;
                    if (b < M) {
                        const float tt = XM == XM_PREPC ? f0[v] + f1[v] + f2[v]
                                                        : f0[v] + f1[v] * 0.0078125f + f2[v] * 6.103515625e-05f;
                        float* yp = a.y + (size_t)b * a.ldy + (row - a.row_lo);
                        const float val = (tt * lxs[b]) * rs;
                        *yp = a.resid ? (first ? y_first[v] : *yp) + val : val;
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
// M = 1 with a prepared operand (XS_GLOBAL): one workgroup per row block, KS
// waves each owning SPW consecutive 1 KiB steps of its row.  Every wave
// copies only its own slice of the operand planes to LDS by direct loads and
// waits for its own loads alone: no workgroup-wide operand copy and no
// barrier before the MFMAs (measured on MI355X against the general kernel:
// q8 4096x4096 5.78 -> 4.65 us, q4t 12288x4096 7.1 -> 6.85 us; the copy of
// the whole operand by every workgroup, 768 x 24 KiB from L2 for the q4t
// shape, was the largest cost above a plain read of the weights).  The KS
// partial sums are reduced in LDS in wave order (deterministic).  The slices
// live in the dynamic LDS allocation: with a static __shared__ array as the
// direct-load target the compiler waited for every load of the wave
// (vmcnt(0)) before the first LDS read instead of for the slice alone.
// ---------------------------------------------------------------------------

// Row-block epilogue of the M = 1 kernels: wave 0 adds the KS partials in
// wave order and lanes with s == 0 write row r.
template <int KS>
__device__ __forceinline__ float m1_reduce(float (*part)[64], float v, int wave, int lane) {
    part[wave][lane] = v;
    __syncthreads();
    if (wave != 0) return 0.f;  // (only wave 0 writes the outputs)
    float o = part[0][lane];
#pragma unroll
    for (int w = 1; w < KS; w++) o += part[w][lane];
    return o;
}

// q8: v_mfma_i32_16x16x64_i8 with A rows 0..2 the three int8 planes of x
// (the PK layout of k_gemv_q8 at m = 1); exact int32 sums per wave (SPW * 64
// columns * 127 * 127 < 2^24, so the f32 partial is exact), the planes
// combined once at the end.
template <int KS, int SPW, bool RESID>
__global__ __launch_bounds__(64 * KS) void k_gemv_q8_m1(GemvArgs a) {
    static_assert(SPW * 64 * 127 * 127 < (1 << 24), "per-wave int32 partial must stay exact in f32");
    constexpr int NI = SPW * 4 * 3;           // 16-byte operand items of a wave's slice
    constexpr int NCH = (NI + 63) / 64;       // ... in 1 KiB direct loads
    __shared__ float part[KS][64];
    extern __shared__ __align__(16) uint8_t smem[];  // [KS][NCH * 1024]: the waves' operand slices
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int r = lane & 15, s = lane >> 4;
    const int nkc = a.nk, rb = blockIdx.x;
    const int c0 = wave * SPW;
    const int row = (a.rb0 + rb) * 16 + r;
    const int rowc = max(a.row_lo, min(row, a.row_hi - 1));
    // epilogue reads first (row scale, residual), then the slice, then the weights
    const float rs = ldg((const float*)a.scale + row);
    // (every load unconditional: a load under a branch makes the compiler
    // wait for all loads in flight at the branch; RESID is a template
    // argument so that a plain GEMV issues no residual read, 0.2 us)
    const float yold = RESID ? ldg(a.y + (rowc - a.row_lo)) : 0.f;
    const float xs = ldg(a.src.xs);
    uint8_t* lx = smem + wave * (NCH * 1024);
#pragma unroll
    for (int c = 0; c < NCH; c++) {
        // item i = (u * 4 + s') * 3 + p: plane p of step c0 + u, k-slot s' (clamped to the matrix)
        const int i = min(c * 64 + lane, NI - 1);
        const int p = i % 3, us = i / 3, u = us >> 2, sp = us & 3;
        const int step = min(c0 + u, nkc - 1);
        __builtin_amdgcn_global_load_lds((const void*)(a.src.planes + ((size_t)p * nkc * 4 + step * 4 + sp) * 16),
                                         (__attribute__((address_space(3))) void*)(lx + c * 1024), 16, 0, 0);
    }
    __builtin_amdgcn_sched_barrier(0);
    int4v wv[SPW];
    const size_t wbase = (size_t)(a.rb0 + rb) * nkc;
#pragma unroll
    for (int u = 0; u < SPW; u++) wv[u] = ldg((const int4v*)a.w + (wbase + min(c0 + u, nkc - 1)) * 64 + lane);
    __builtin_amdgcn_sched_barrier(0);
    wait_vmcnt<SPW>();  // this wave's slice is in
    const int4v* X = (const int4v*)lx;
    int4v acc = {0, 0, 0, 0};
#pragma unroll
    for (int u = 0; u < SPW; u++) {
        // steps past the row (clamped loads) multiply a zero operand: a
        // select, not a branch, so that each MFMA waits for its own step only
        const int4v z = {0, 0, 0, 0};
        const int4v xv = X[(u * 4 + s) * 3 + min(r, 2)];
        const int4v xa = (r < 3 && c0 + u < nkc) ? xv : z;
        acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(xa, wv[u], acc, 0, 0, 0);
    }
    // lanes s == 0 hold rows 0..2 (the planes) of weight row r
    const float v = (float)acc[0] + (float)acc[1] * 0.0078125f + (float)acc[2] * 6.103515625e-05f;
    const float o = m1_reduce<KS>(part, v, wave, lane);
    if (wave == 0 && s == 0 && row >= a.row_lo && row < a.row_hi && rb < a.nrb) {
        const float val = (o * xs) * rs;
        a.y[row - a.row_lo] = RESID ? yold + val : val;
    }
}

// q4t: the f16 hi / lo planes of the wave's tiles in LDS, A rows 0..7 the
// hi plane and 8..15 the lo plane of batch row 0 (HL); each tile's biases
// -8 * 2^-24 * sum(hi) and -8 * 2^-24 * sum(lo) (the format's -8 offset per
// plane) come from the prepared table into the slice too (SPW * 8 <= 64
// floats after the planes) and are added to the hi and lo rows after the
// MFMA.  (Scalar loads of the biases made the compiler wait for every load
// of the wave before the first MFMA.)
// (RB row blocks per workgroup share its operand slices; measured on
// MI355X, 12288x4096: RB = 2 8.2 us against 7.1 us at RB = 1, which is what
// the dispatch instantiates)
template <int KS, int SPW, bool RESID, int RB = 1>
__global__ __launch_bounds__(64 * KS) void k_gemv_q4t_m1(GemvArgs a) {
    constexpr int NI = SPW * 4 * 4 * 2;  // 16-byte items: step x tile x k-slot x plane
    constexpr int NCH = (NI + 63) / 64;
    __shared__ float part[KS][RB * 64];
    static_assert(SPW * 8 <= 64, "one bias per lane");
    extern __shared__ __align__(16) uint8_t smem[];  // [KS][NCH * 1024 + 256]: the waves' operand slices
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int r = lane & 15, s = lane >> 4, p = r < 8 ? 0 : 1;
    const int ntg = a.nk, rb = blockIdx.x * RB;  // RB row blocks share the operand slices
    const int t0 = wave * SPW;
    float yold[RB];
#pragma unroll
    for (int q = 0; q < RB; q++) {
        const int row = (a.rb0 + rb + q) * 16 + r;
        const int rowc = max(a.row_lo, min(row, a.row_hi - 1));
        yold[q] = RESID ? ldg(a.y + (rowc - a.row_lo)) : 0.f;  // (as in k_gemv_q8_m1)
    }
    const float xs = ldg(a.src.xs);
    const uint8_t* hi = a.src.planes;
    const uint8_t* lo = hi + (size_t)ntg * 4 * 4 * 16;
    const float* btab = (const float*)(lo + (size_t)ntg * 4 * 4 * 16);  // [tile][16]
    uint8_t* lx = smem + wave * (NCH * 1024 + 256);
#pragma unroll
    for (int c = 0; c < NCH; c++) {
        // item i = ((u * 4 + t) * 4 + s') * 2 + plane
        const int i = min(c * 64 + lane, NI - 1);
        const int pl = i & 1, q = i >> 1, sp = q & 3, t = (q >> 2) & 3, u = q >> 4;
        const int tg = min(t0 + u, ntg - 1);
        __builtin_amdgcn_global_load_lds((const void*)((pl ? lo : hi) + ((size_t)(tg * 4 + t) * 4 + sp) * 16),
                                         (__attribute__((address_space(3))) void*)(lx + c * 1024), 16, 0, 0);
    }
    // the tile biases of the slice (entries [tile][0], hi plane, and
    // [tile][8], lo plane, of the table), one 4-byte direct load per lane
    // after the planes
    {
        const int tb = min((t0 + (lane >> 3)) * 4 + ((lane >> 1) & 3), ntg * 4 - 1);
        __builtin_amdgcn_global_load_lds((const void*)(btab + (size_t)tb * 16 + 8 * (lane & 1)),
                                         (__attribute__((address_space(3))) void*)(lx + NCH * 1024), 4, 0, 0);
    }
    __builtin_amdgcn_sched_barrier(0);
    uint4 wv[RB][SPW];
    uint2 sv[RB][SPW];
#pragma unroll
    for (int q = 0; q < RB; q++) {
        const size_t wbase = (size_t)min(a.rb0 + rb + q, a.rb0 + a.nrb - 1) * ntg;
#pragma unroll
        for (int u = 0; u < SPW; u++) {
            const size_t t = wbase + min(t0 + u, ntg - 1);
            wv[q][u] = ld_stream((const uint4*)a.w + t * 64 + lane);
            const uint64_t sw = ldg((const uint64_t*)a.scale + t * 16 + r);
            sv[q][u] = make_uint2((uint32_t)sw, (uint32_t)(sw >> 32));
        }
    }
    __builtin_amdgcn_sched_barrier(0);
    wait_vmcnt<2 * SPW * RB>();  // this wave's slice is in
    const uint4* X = (const uint4*)lx;
    const float* bias = (const float*)(lx + NCH * 1024);
    float acc[RB];
#pragma unroll
    for (int q = 0; q < RB; q++) acc[q] = 0.f;
#pragma unroll
    for (int u = 0; u < SPW; u++) {
        // steps past the row (clamped loads) get a zero scale: a select, not
        // a branch (see k_gemv_q8_m1)
        const bool in = t0 + u < ntg;
#pragma unroll
        for (int t = 0; t < 4; t++) {
            const half8 xa = __builtin_bit_cast(half8, X[((u * 4 + t) * 4 + s) * 2 + p]);
            const float bt = bias[(u * 4 + t) * 2 + (s >> 1)];  // s >= 2: the lo rows
#pragma unroll
            for (int q = 0; q < RB; q++) {
                const uint32_t wq = t == 0 ? wv[q][u].x : t == 1 ? wv[q][u].y : t == 2 ? wv[q][u].z : wv[q][u].w;
                const float4v z = {0.f, 0.f, 0.f, 0.f};
                const float4v d = __builtin_amdgcn_mfma_f32_16x16x32_f16(xa, dq_nib_word(wq), z, 0, 0, 0);
                const uint32_t sw = t < 2 ? sv[q][u].x : sv[q][u].y;
                const float sc = in ? f16_bits_to_f32((t & 1) ? sw >> 16 : sw & 0xFFFFu) : 0.f;
                acc[q] += (d[0] + bt) * sc;
            }
        }
    }
    // the KS partials in wave order (as m1_reduce), RB row blocks side by side
#pragma unroll
    for (int q = 0; q < RB; q++) part[wave][q * 64 + lane] = acc[q];
    __syncthreads();
    if (wave == 0) {
#pragma unroll
        for (int q = 0; q < RB; q++) {
            float o = part[0][q * 64 + lane];
#pragma unroll
            for (int w = 1; w < KS; w++) o += part[w][q * 64 + lane];
            o += __shfl_xor(o, 32);  // hi rows (lanes s = 0, 1) + lo rows (s = 2, 3)
            const int row = (a.rb0 + rb + q) * 16 + r;
            if (s == 0 && row >= a.row_lo && row < a.row_hi && rb + q < a.nrb) {
                const float val = o * xs * 16777216.0f;  // 2^24: denormal nibbles
                a.y[row - a.row_lo] = RESID ? yold[q] + val : val;
            }
        }
    }
}

// q4t, M = 1, from the f32 operand row itself (XS_ROWS): the workgroup
// needs no producer launch.  Wave w reads the SPW * 128 columns of its own
// steps, one 8-column k-slot item per lane and step group, then the
// workgroup agrees on the row's max |x| (one LDS exchange: the fixed-point
// unit 2^(e - 11) of q4_fix_scale needs the whole row), and each wave writes
// its slice's hi / lo planes and tile biases (exactly what the producer
// would have written) into its own LDS region and runs the MFMA loop of
// k_gemv_q4t_m1.  Columns past the row (steps past ntg, tiles past K) are
// zero: their planes and biases vanish.
template <int KS, int SPW, bool RESID>
__global__ __launch_bounds__(64 * KS) void k_gemv_q4t_m1x(GemvArgs a) {
    constexpr int NIT = SPW / 4;           // 8-column items per lane (16 SPW items per wave)
    static_assert(SPW % 4 == 0 && SPW * 8 <= 64, "items per lane");
    __shared__ float part[KS][64];
    __shared__ float wmax[KS];
    __shared__ __align__(16) uint4 slice[KS][SPW * 32];  // [item][plane] 16 B, item = (u * 4 + t) * 4 + s'
    __shared__ float sbias[KS][SPW * 8];                 // [(u * 4 + t) * 2 + plane]
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int r = lane & 15, s = lane >> 4, p = r < 8 ? 0 : 1;
    const int ntg = a.nk, rb = blockIdx.x, K = a.src.K;
    const int t0 = wave * SPW;
    const int row = (a.rb0 + rb) * 16 + r;
    const int rowc = max(a.row_lo, min(row, a.row_hi - 1));
    const float yold = RESID ? ldg(a.y + (rowc - a.row_lo)) : 0.f;
    // this lane's items: item q = lane + 64 i = (u * 4 + t) * 4 + s', columns
    // 32 ((t0 + u) * 4 + t) + 8 s' .. + 7 (clamped loads, zero by select)
    float4v xv[NIT][2];
    bool on[NIT];
#pragma unroll
    for (int i = 0; i < NIT; i++) {
        const int q = lane + 64 * i, u = q >> 4, t = (q >> 2) & 3, sp = q & 3;
        const int c0 = ((t0 + u) * 4 + t) * 32 + 8 * sp;
        on[i] = t0 + u < ntg && c0 + 8 <= K;
        const float* src = a.src.x + (on[i] ? c0 : 0);
        xv[i][0] = ldg((const float4v*)src);
        xv[i][1] = ldg((const float4v*)(src + 4));
    }
    __builtin_amdgcn_sched_barrier(0);
    uint4 wv[SPW];
    uint2 sv[SPW];
    const size_t wbase = (size_t)(a.rb0 + rb) * ntg;
#pragma unroll
    for (int u = 0; u < SPW; u++) {
        const size_t t = wbase + min(t0 + u, ntg - 1);
        wv[u] = ld_stream((const uint4*)a.w + t * 64 + lane);
        const uint64_t sw = ldg((const uint64_t*)a.scale + t * 16 + r);
        sv[u] = make_uint2((uint32_t)sw, (uint32_t)(sw >> 32));
    }
    __builtin_amdgcn_sched_barrier(0);
    wait_vmcnt<2 * SPW>();  // this wave's operand columns are in
    float am = 0.f;
#pragma unroll
    for (int i = 0; i < NIT; i++)
#pragma unroll
        for (int h = 0; h < 2; h++)
#pragma unroll
            for (int k = 0; k < 4; k++) am = fmaxf(am, on[i] ? fabsf(xv[i][h][k]) : 0.f);
    am = wave_max(am);
    if (lane == 0) wmax[wave] = am;
    // LDS-only barrier: the weights stay in flight
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    am = wmax[0];
#pragma unroll
    for (int w = 1; w < KS; w++) am = fmaxf(am, wmax[w]);
    float scale, xs;
    q4_fix_scale(am, scale, xs);
    const int ord[8] = {0, 4, 2, 6, 1, 5, 3, 7};
#pragma unroll
    for (int i = 0; i < NIT; i++) {
        const int q = lane + 64 * i;
        float v[8];
#pragma unroll
        for (int k = 0; k < 8; k++) v[k] = on[i] ? xv[i][k >> 2][k & 3] : 0.f;
        uint16_t hv[8], lv[8];
        float sh = 0.f, sl = 0.f;  // (exact: integers and multiples of 2^-11)
#pragma unroll
        for (int j = 0; j < 8; j++) {
            _Float16 h, l;
            q4_fix_split(v[ord[j]] * scale, h, l);
            hv[j] = __builtin_bit_cast(uint16_t, h);
            lv[j] = __builtin_bit_cast(uint16_t, l);
            sh += (float)h;
            sl += (float)l;
        }
        sh += __shfl_xor(sh, 1);
        sh += __shfl_xor(sh, 2);
        sl += __shfl_xor(sl, 1);
        sl += __shfl_xor(sl, 2);
        slice[wave][q * 2] = make_uint4(hv[0] | (hv[1] << 16), hv[2] | (hv[3] << 16), hv[4] | (hv[5] << 16),
                                        hv[6] | (hv[7] << 16));
        slice[wave][q * 2 + 1] = make_uint4(lv[0] | (lv[1] << 16), lv[2] | (lv[3] << 16), lv[4] | (lv[5] << 16),
                                            lv[6] | (lv[7] << 16));
        if ((q & 3) == 0) {
            sbias[wave][(q >> 2) * 2] = sh * Q4_BIAS;
            sbias[wave][(q >> 2) * 2 + 1] = sl * Q4_BIAS;
        }
    }
    // the wave reads back what its own lanes wrote (LDS operations of a
    // wave complete in order; the barrier keeps the compiler from moving
    // the reads up)
    __builtin_amdgcn_wave_barrier();
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    const uint4* X = slice[wave];
    const float* bias = sbias[wave];
    float acc = 0.f;
#pragma unroll
    for (int u = 0; u < SPW; u++) {
        const bool in = t0 + u < ntg;
#pragma unroll
        for (int t = 0; t < 4; t++) {
            const half8 xa = __builtin_bit_cast(half8, X[((u * 4 + t) * 4 + s) * 2 + p]);
            const uint32_t wq = t == 0 ? wv[u].x : t == 1 ? wv[u].y : t == 2 ? wv[u].z : wv[u].w;
            const float4v z = {0.f, 0.f, 0.f, 0.f};
            const float4v d = __builtin_amdgcn_mfma_f32_16x16x32_f16(xa, dq_nib_word(wq), z, 0, 0, 0);
            const uint32_t sw = t < 2 ? sv[u].x : sv[u].y;
            const float sc = in ? f16_bits_to_f32((t & 1) ? sw >> 16 : sw & 0xFFFFu) : 0.f;
            acc += (d[0] + bias[(u * 4 + t) * 2 + (s >> 1)]) * sc;  // s >= 2: the lo rows
        }
    }
    float o = m1_reduce<KS>(part, acc, wave, lane);
    o += __shfl_xor(o, 32);  // hi rows (lanes s = 0, 1) + lo rows (s = 2, 3)
    if (wave == 0 && s == 0 && row >= a.row_lo && row < a.row_hi && rb < a.nrb) {
        const float val = o * xs * 16777216.0f;  // 2^24: denormal nibbles
        a.y[row - a.row_lo] = RESID ? yold + val : val;
    }
}

// Instance of the M = 1 kernels for rows of nk 1 KiB steps (nullptr: none);
// *ks = its waves per workgroup, *lds = its dynamic LDS bytes.
template <int KS, int SPW>
inline GemvKernel q8_m1_inst(bool resid, int* ks, size_t* lds) {
    *ks = KS;
    *lds = (size_t)KS * ((SPW * 12 + 63) / 64) * 1024;
    return resid ? k_gemv_q8_m1<KS, SPW, true> : k_gemv_q8_m1<KS, SPW, false>;
}
template <int KS, int SPW>
inline GemvKernel q4t_m1_inst(bool resid, int* ks, size_t* lds) {
    *ks = KS;
    *lds = (size_t)KS * (((SPW * 32 + 63) / 64) * 1024 + 256);
    return resid ? k_gemv_q4t_m1<KS, SPW, true> : k_gemv_q4t_m1<KS, SPW, false>;
}
inline GemvKernel q8_m1_pick(int nk, bool resid, int* ks, size_t* lds) {
    // (measured on MI355X, 10 weight copies rotating: more waves with fewer
    // steps each pay up to 64 steps: 4096x1024 (16 steps) 2.71 -> 2.44 us
    // at 8 x 2, the 151936x1024 lm_head 25.7 -> 24.9 us, 1024x2048 2.46 ->
    // 2.16 us at 8 x 4, 4096x4096 4.72 -> 4.42 us at 16 x 4; for q4t the
    // table below was already the fastest of the shapes tried)
    if (nk <= 8) return q8_m1_inst<1, 8>(resid, ks, lds);
    if (nk <= 16) return q8_m1_inst<8, 2>(resid, ks, lds);
    if (nk <= 32) return q8_m1_inst<8, 4>(resid, ks, lds);
    if (nk <= 64) return q8_m1_inst<16, 4>(resid, ks, lds);
    if (nk <= 128) return q8_m1_inst<16, 8>(resid, ks, lds);
    if (nk <= 192) return q8_m1_inst<16, 12>(resid, ks, lds);
    return nullptr;
}
template <int KS, int SPW>
inline GemvKernel q4t_m1x_inst(bool resid, int* ks) {
    *ks = KS;
    return resid ? k_gemv_q4t_m1x<KS, SPW, true> : k_gemv_q4t_m1x<KS, SPW, false>;
}
// the staged-from-rows kernel: SPW a multiple of 4 (whole items per lane)
inline GemvKernel q4t_m1x_pick(int nk, bool resid, int* ks) {
    if (nk <= 4) return q4t_m1x_inst<1, 4>(resid, ks);
    if (nk <= 8) return q4t_m1x_inst<2, 4>(resid, ks);
    if (nk <= 16) return q4t_m1x_inst<4, 4>(resid, ks);
    if (nk <= 32) return q4t_m1x_inst<8, 4>(resid, ks);
    if (nk <= 64) return q4t_m1x_inst<8, 8>(resid, ks);
    return nullptr;  // (16 waves x 8 steps of slices would pass the 64 KiB of static LDS)
}
inline GemvKernel q4t_m1_pick(int nk, bool resid, int* ks, size_t* lds) {
    if (nk <= 4) return q4t_m1_inst<1, 4>(resid, ks, lds);
    if (nk <= 8) return q4t_m1_inst<2, 4>(resid, ks, lds);
    if (nk <= 16) return q4t_m1_inst<4, 4>(resid, ks, lds);
    if (nk <= 32) return q4t_m1_inst<8, 4>(resid, ks, lds);
    if (nk <= 64) return q4t_m1_inst<8, 8>(resid, ks, lds);
    if (nk <= 96) return q4t_m1_inst<16, 6>(resid, ks, lds);
    if (nk <= 128) return q4t_m1_inst<16, 8>(resid, ks, lds);
    return nullptr;
}

// ---------------------------------------------------------------------------
// Kernel instance tables (one translation unit per weight codec).
// ---------------------------------------------------------------------------
template <int FMT, int NV, bool HL, int XM, int RB>
GemvKernel q4_by_ks(int ks) {
    switch (ks) {
        case 1:  // (RB > 1 spills at one wave)
            if constexpr (RB == 1) return k_gemv_q4<FMT, NV, 1, HL, XM, RB>;
            return nullptr;
        case 2: return k_gemv_q4<FMT, NV, 2, HL, XM, RB>;
        case 4: return k_gemv_q4<FMT, NV, 4, HL, XM, RB>;
        case 8: return k_gemv_q4<FMT, NV, 8, HL, XM, RB>;
    }
    // two MFMAs per tile (or three row blocks) need more than the 128
    // registers a 16-wave workgroup leaves each wave
    if constexpr (HL && RB < 3)
        if (ks == 16) return k_gemv_q4<FMT, NV, 16, HL, XM, RB>;
    return nullptr;
}
// RB > 1 only for the LDS-staged one-MFMA-per-tile kernels (m <= 8)
template <int FMT, int NV, bool HL>
GemvKernel q4_by_xm(int xm, int ks, int rb) {
    if (xm == XM_GLOBAL) {
        if (rb == 1) return q4_by_ks<FMT, NV, HL, XM_GLOBAL, 1>(ks);
        // m > 8 reads the operand in place: RB row blocks share each read
        if constexpr (!HL) {
            if (rb == 2) return q4_by_ks<FMT, NV, HL, XM_GLOBAL, 2>(ks);
            if (rb == 3) return q4_by_ks<FMT, NV, HL, XM_GLOBAL, 3>(ks);
        }
        return nullptr;
    }
    if constexpr (HL)
        if (xm == XM_FUSED) return rb == 1 ? q4_by_ks<FMT, NV, HL, XM_FUSED, 1>(ks) : nullptr;
    if (xm != XM_PREP) return nullptr;
    if constexpr (HL) {
        switch (rb) {
            case 1: return q4_by_ks<FMT, NV, HL, XM_PREP, 1>(ks);
            case 2: return q4_by_ks<FMT, NV, HL, XM_PREP, 2>(ks);
            case 3: return q4_by_ks<FMT, NV, HL, XM_PREP, 3>(ks);
        }
        return nullptr;
    } else {
        return rb == 1 ? q4_by_ks<FMT, NV, HL, XM_PREP, 1>(ks) : nullptr;
    }
}
// Grouped workgroups (G = 3 groups of 4 waves x 8 steps: three row blocks of
// K <= 4096 share one operand copy in LDS), m <= 8
template <int FMT>
GemvKernel q4_pick_g3(int m, int xm, bool one) {
    if (xm != XM_PREP || m > 8) return nullptr;
    if (one)
        return m == 1 ? k_gemv_q4<FMT, 1, 4, true, XM_PREP, 1, 3, 8, true>
                      : k_gemv_q4<FMT, 4, 4, true, XM_PREP, 1, 3, 8, true>;
    return m == 1 ? k_gemv_q4<FMT, 1, 4, true, XM_PREP, 1, 3, 8> : k_gemv_q4<FMT, 4, 4, true, XM_PREP, 1, 3, 8>;
}
// 16 waves x 6 steps: rows of 65..96 steps (K <= 12288) in one K part
template <int FMT>
GemvKernel q4_pick_s6(int m, int xm) {
    if (m > 8) return nullptr;
    if (xm == XM_PREP) return m == 1 ? k_gemv_q4<FMT, 1, 16, true, XM_PREP, 1, 1, 6> : k_gemv_q4<FMT, 4, 16, true, XM_PREP, 1, 1, 6>;
    if (xm != XM_GLOBAL) return nullptr;
    if (m == 1) return k_gemv_q4<FMT, 1, 16, true, XM_GLOBAL, 1, 1, 6>;
    // (q4tp's in-place instance for m > 1 needs more than 128 registers)
    if constexpr (FMT == DT_Q4T) return k_gemv_q4<FMT, 4, 16, true, XM_GLOBAL, 1, 1, 6>;
    return nullptr;
}
template <int FMT>
GemvKernel q4_pick(int m, int xm, int ks, int rb) {
    if (m == 1) return q4_by_xm<FMT, 1, true>(xm, ks, rb);
    if (m <= 8) return q4_by_xm<FMT, 4, true>(xm, ks, rb);
    return q4_by_xm<FMT, 4, false>(xm, ks, rb);
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
        case XM_PREPC: return q8_by_ks<PK, XM_PREPC>(ks);
    }
    return nullptr;
}

}  // namespace cmf
