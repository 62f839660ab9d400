// Dequant GEMV / skinny GEMM kernels for gfx950 (MI355X).
//
// y[b][r] = sum_k W[r][k] * x[b][k] for b < M <= 16 and the three weight
// codecs of the engine (q8 per-row, q4_tiled, q4tp).  Work split:
//   - a workgroup of KS waves owns one block of 16 weight rows at a time and
//     walks row blocks with a grid stride (persistent); its waves split K
//     and reduce in LDS in a fixed order (deterministic);
//   - every wave streams 1 KiB of packed weights per step with one 128-bit
//     load per lane, a whole K share in flight before the first MFMA;
//   - the activations are the MFMA A operand (16 batch rows, zero-padded),
//     the weights the B operand (16 weight rows):
//       q8  : v_mfma_i32_16x16x64_i8 on the raw int8 weights; x is carried
//             as three int8 planes, x ~= sx*(q0 + q1/128 + q2/16384)
//             (|error| <= 2^-22 max|x|), each summed exactly in int32;
//       q4* : v_mfma_f32_16x16x32_f16, one tile (32 columns, one scale) per
//             MFMA; nibbles become exact f16 (n - 8) in registers and x is
//             carried as f16 hi + lo of x*2^e (22-bit significand).  Each
//             tile's product is scaled by its tile scale and accumulated in
//             f32, as q4t_row_exact does (qtensor.rs:4418-4432).
//   - the activation operand is built once per workgroup into LDS from its
//     producer (RMSNorm of the residual rows, SwiGLU of the gate/up rows,
//     plain rows, the MTP [enorm(embed); hnorm(h)] concat, or a prepared
//     buffer), so the producer needs no kernel of its own; when it does not
//     fit in LDS the prepared planes are read from global memory (L2).
//   - optional residual epilogue: y is added into the output (h += W x).
#include "common.h"
#include "gemv.h"

namespace cmf {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float float4v __attribute__((ext_vector_type(4)));
typedef int int4v __attribute__((ext_vector_type(4)));

constexpr int PF = 8;            // weight steps in flight per wave
constexpr int LDSX_MAX = 128 * 1024;  // largest LDS-staged activation operand (+ scratch)

// Four nibble bytes (8 weights: elements 8s..8s+7 of a tile) to exact f16
// (n - 8) in the in-slot order {0,2,4,6,1,3,5,7}.
__device__ __forceinline__ half8 dq_nib_word(uint32_t w) {
    const uint32_t lo = w & 0x0F0F0F0Fu, hi = (w >> 4) & 0x0F0F0F0Fu;
    const uint32_t p0 = (lo & 0xFFu) | ((lo & 0xFF00u) << 8) | 0x64006400u;
    const uint32_t p1 = ((lo >> 16) & 0xFFu) | ((lo >> 8) & 0xFF0000u) | 0x64006400u;
    const uint32_t p2 = (hi & 0xFFu) | ((hi & 0xFF00u) << 8) | 0x64006400u;
    const uint32_t p3 = ((hi >> 16) & 0xFFu) | ((hi >> 8) & 0xFF0000u) | 0x64006400u;
    const half2v off = {(_Float16)1032.0f, (_Float16)1032.0f};
    half2v a = __builtin_bit_cast(half2v, p0) - off;
    half2v b = __builtin_bit_cast(half2v, p1) - off;
    half2v c = __builtin_bit_cast(half2v, p2) - off;
    half2v d = __builtin_bit_cast(half2v, p3) - off;
    half8 r;
    r[0] = a[0]; r[1] = a[1]; r[2] = b[0]; r[3] = b[1];
    r[4] = c[0]; r[5] = c[1]; r[6] = d[0]; r[7] = d[1];
    return r;
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
//     q4: hi plane then lo plane, [tile*4 + s][b] x 16 B; lxs[b] = 2^-e
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
            // in-slot order {0,2,4,6,1,3,5,7}
            const float xo[8] = {xa.x, xa.z, xb.x, xb.z, xa.y, xa.w, xb.y, xb.w};
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
}

// Operand staging of a whole workgroup; XS_GLOBAL planes are copied into the
// LDS layout.
__device__ __forceinline__ void stage_x(const XSrc& s, int M, int fmt, int nk, uint8_t* lx, float* lxs) {
    if (s.mode == XS_GLOBAL) {
        // global [item/4][16*s + b] x 16 B  ->  LDS [item][b] x 16 B
        const int npl = fmt == DT_Q8ROW ? 3 : 2;
        const size_t gpl = (size_t)nk * 64, lpl = (size_t)nk * 4 * M;
        const uint4* g = (const uint4*)s.planes;
        uint4* l = (uint4*)lx;
        const int n = nk * 4 * M;
        for (int i = threadIdx.x; i < n * npl; i += blockDim.x) {
            const int p = i / n, e = i % n, item = e / M, b = e % M;
            l[p * lpl + e] = g[p * gpl + (size_t)(item >> 2) * 64 + 16 * (item & 3) + b];
        }
        if (threadIdx.x < 16) lxs[threadIdx.x] = s.xs[threadIdx.x];
    } else {
        const size_t pbytes = (size_t)nk * 4 * M * 16 * (fmt == DT_Q8ROW ? 3 : 2);
        stage_fused(s, M, fmt, nk, lx, lxs, (float*)(lx + pbytes));
    }
    __syncthreads();
}

// ---------------------------------------------------------------------------
// q4t / q4tp
// ---------------------------------------------------------------------------
template <int FMT, int NV, int KS>
__global__ __launch_bounds__(64 * KS) void k_gemv_q4(GemvArgs a) {
    extern __shared__ __align__(16) uint8_t smem[];
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int r = lane & 15, s = lane >> 4;
    const int M = a.m, ntg = a.nk;  // nk = groups of 4 tiles
    __shared__ float lad[FMT == DT_Q4TP ? 16 * 33 : 1];
    __shared__ float4v part[KS][64];
    __shared__ float lxs[16];
    const int tg0 = (ntg * wave) / KS, tg1 = (ntg * (wave + 1)) / KS;
    // the first weight steps are requested before the operand staging so
    // the HBM latency overlaps it
    uint4 wv[PF];
    uint32_t sv[PF][2];
    auto load_w = [&](size_t wbase, int it0) {
#pragma unroll
        for (int u = 0; u < PF; u++) {
            if (it0 + u < tg1) {
                wv[u] = ((const uint4*)a.w)[(wbase + it0 + u) * 64 + lane];
                if constexpr (FMT == DT_Q4T) {
                    const uint2 v = ((const uint2*)a.scale)[(wbase + it0 + u) * 16 + r];
                    sv[u][0] = v.x;
                    sv[u][1] = v.y;
                } else {
                    sv[u][0] = ((const uint32_t*)a.scale)[(wbase + it0 + u) * 16 + r];
                    sv[u][1] = 0;
                }
            }
        }
    };
    if ((int)blockIdx.x < a.nrb) load_w((size_t)(a.rb0 + blockIdx.x) * ntg, tg0);
    const bool in_lds = a.lds != 0;
    if (in_lds) stage_x(a.src, M, FMT, ntg * 4, smem, lxs);
    else if (threadIdx.x < 16) lxs[threadIdx.x] = a.src.xs[threadIdx.x];
    __syncthreads();
    const uint4* XH = (const uint4*)a.src.planes;
    const uint4* XL = XH + (size_t)ntg * 4 * 64;
    const uint4* LH = (const uint4*)smem;
    const uint4* LL = LH + (size_t)ntg * 4 * 4 * M;
    const bool xload = r < M;
    const float4v zero = {0.f, 0.f, 0.f, 0.f};
    bool have = true;
    for (int rb = blockIdx.x; rb < a.nrb; rb += gridDim.x) {
        const size_t wbase = (size_t)(a.rb0 + rb) * ntg;
        if constexpr (FMT == DT_Q4TP) {
            __syncthreads();
            if (threadIdx.x < 16) {
                const float2 p = a.rowp[(a.rb0 + rb) * 16 + threadIdx.x];
                float tv = p.x;
                lad[threadIdx.x * 33] = tv;
                for (int c = 1; c < 32; c++) {
                    tv = tv * p.y;
                    lad[threadIdx.x * 33 + c] = tv;
                }
            }
            __syncthreads();
        }
        float4v acc = {0.f, 0.f, 0.f, 0.f};
        for (int it0 = tg0; it0 < tg1; it0 += PF) {
            if (!have) load_w(wbase, it0);
            have = false;
#pragma unroll
            for (int u = 0; u < PF; u++) {
                if (it0 + u >= tg1) break;
                const int tg = it0 + u;
                float sc[4];
                if constexpr (FMT == DT_Q4T) {
                    sc[0] = f16_bits_to_f32(sv[u][0] & 0xFFFFu);
                    sc[1] = f16_bits_to_f32(sv[u][0] >> 16);
                    sc[2] = f16_bits_to_f32(sv[u][1] & 0xFFFFu);
                    sc[3] = f16_bits_to_f32(sv[u][1] >> 16);
                } else {
                    const uint32_t cw = sv[u][0];
                    sc[0] = lad[r * 33 + (cw & 31)];
                    sc[1] = lad[r * 33 + ((cw >> 5) & 31)];
                    sc[2] = lad[r * 33 + ((cw >> 10) & 31)];
                    sc[3] = lad[r * 33 + ((cw >> 15) & 31)];
                }
                const uint32_t ww[4] = {wv[u].x, wv[u].y, wv[u].z, wv[u].w};
#pragma unroll
                for (int t = 0; t < 4; t++) {
                    const int tile = tg * 4 + t;
                    half8 xh = {}, xl = {};
                    if (xload) {
                        if (in_lds) {
                            xh = __builtin_bit_cast(half8, LH[(size_t)(tile * 4 + s) * M + r]);
                            xl = __builtin_bit_cast(half8, LL[(size_t)(tile * 4 + s) * M + r]);
                        } else {
                            xh = __builtin_bit_cast(half8, XH[(size_t)tile * 64 + lane]);
                            xl = __builtin_bit_cast(half8, XL[(size_t)tile * 64 + lane]);
                        }
                    }
                    const half8 bq = dq_nib_word(ww[t]);
                    float4v d = __builtin_amdgcn_mfma_f32_16x16x32_f16(xh, bq, zero, 0, 0, 0);
                    d = __builtin_amdgcn_mfma_f32_16x16x32_f16(xl, bq, d, 0, 0, 0);
#pragma unroll
                    for (int v = 0; v < NV; v++) acc[v] += d[v] * sc[t];
                }
            }
        }
        if constexpr (KS > 1) {
            part[wave][lane] = acc;
            __syncthreads();
            if (wave == 0) {
                for (int q = 1; q < KS; q++) {
                    const float4v o = part[q][lane];
#pragma unroll
                    for (int v = 0; v < NV; v++) acc[v] += o[v];
                }
            }
            __syncthreads();
        }
        if (wave == 0) {
            const int row = (a.rb0 + rb) * 16 + r;
            if (row >= a.row_lo && row < a.row_hi) {
#pragma unroll
                for (int v = 0; v < NV; v++) {
                    const int b = 4 * s + v;
                    if (b < M) {
                        float* yp = a.y + (size_t)b * a.ldy + (row - a.row_lo);
                        const float val = acc[v] * lxs[b];
                        *yp = a.resid ? *yp + val : val;
                    }
                }
            }
        }
    }
}

// ---------------------------------------------------------------------------
// q8
// ---------------------------------------------------------------------------
template <int KS>
__global__ __launch_bounds__(64 * KS) void k_gemv_q8(GemvArgs a) {
    extern __shared__ __align__(16) uint8_t smem[];
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int r = lane & 15, s = lane >> 4;
    const int M = a.m, nkc = a.nk;
    __shared__ int4v part[KS > 1 ? KS : 1][3][64];
    __shared__ float lxs[16];
    const int k0 = (nkc * wave) / KS, k1 = (nkc * (wave + 1)) / KS;
    int4v wv[PF];
    auto load_w = [&](size_t wbase, int it0) {
#pragma unroll
        for (int u = 0; u < PF; u++)
            if (it0 + u < k1) wv[u] = ((const int4v*)a.w)[(wbase + it0 + u) * 64 + lane];
    };
    if ((int)blockIdx.x < a.nrb) load_w((size_t)(a.rb0 + blockIdx.x) * nkc, k0);
    const bool in_lds = a.lds != 0;
    if (in_lds) stage_x(a.src, M, DT_Q8ROW, nkc, smem, lxs);
    else if (threadIdx.x < 16) lxs[threadIdx.x] = a.src.xs[threadIdx.x];
    __syncthreads();
    const int4v* X0 = (const int4v*)a.src.planes;
    const size_t gpl = (size_t)nkc * 64, lpl = (size_t)nkc * 4 * M;
    const int4v* L0 = (const int4v*)smem;
    const bool xload = r < M;
    bool have = true;
    for (int rb = blockIdx.x; rb < a.nrb; rb += gridDim.x) {
        const size_t wbase = (size_t)(a.rb0 + rb) * nkc;
        int4v a0 = {0, 0, 0, 0}, a1 = {0, 0, 0, 0}, a2 = {0, 0, 0, 0};
        for (int it0 = k0; it0 < k1; it0 += PF) {
            if (!have) load_w(wbase, it0);
            have = false;
#pragma unroll
            for (int u = 0; u < PF; u++) {
                if (it0 + u >= k1) break;
                const int kc = it0 + u;
                int4v x0 = {0, 0, 0, 0}, x1 = {0, 0, 0, 0}, x2 = {0, 0, 0, 0};
                if (xload) {
                    if (in_lds) {
                        const size_t o = (size_t)(kc * 4 + s) * M + r;
                        x0 = L0[o];
                        x1 = L0[lpl + o];
                        x2 = L0[2 * lpl + o];
                    } else {
                        x0 = X0[(size_t)kc * 64 + lane];
                        x1 = X0[gpl + (size_t)kc * 64 + lane];
                        x2 = X0[2 * gpl + (size_t)kc * 64 + lane];
                    }
                }
                a0 = __builtin_amdgcn_mfma_i32_16x16x64_i8(x0, wv[u], a0, 0, 0, 0);
                a1 = __builtin_amdgcn_mfma_i32_16x16x64_i8(x1, wv[u], a1, 0, 0, 0);
                a2 = __builtin_amdgcn_mfma_i32_16x16x64_i8(x2, wv[u], a2, 0, 0, 0);
            }
        }
        if constexpr (KS > 1) {
            part[wave][0][lane] = a0;
            part[wave][1][lane] = a1;
            part[wave][2][lane] = a2;
            __syncthreads();
            if (wave == 0) {
                for (int q = 1; q < KS; q++) {
                    a0 += part[q][0][lane];
                    a1 += part[q][1][lane];
                    a2 += part[q][2][lane];
                }
            }
            __syncthreads();
        }
        if (wave == 0) {
            const int row = (a.rb0 + rb) * 16 + r;
            if (row >= a.row_lo && row < a.row_hi) {
                const float rs = ((const float*)a.scale)[row];
#pragma unroll
                for (int v = 0; v < 4; v++) {
                    const int b = 4 * s + v;
                    if (b < M) {
                        const float tt = (float)a0[v] + (float)a1[v] * 0.0078125f + (float)a2[v] * 6.103515625e-05f;
                        float* yp = a.y + (size_t)b * a.ldy + (row - a.row_lo);
                        const float val = (tt * lxs[b]) * rs;
                        *yp = a.resid ? *yp + val : val;
                    }
                }
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Activation preparation into global planes (standalone GEMV calls and the
// operands too large for LDS).  One workgroup per batch row.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_prep(const float* __restrict__ X, int ldx, int K, int kind,
                                              int nk, uint8_t* __restrict__ planes,
                                              float* __restrict__ xs) {
    const int b = blockIdx.x;
    const float* x = X + (size_t)b * ldx;
    __shared__ float red[256];
    float m = 0.f;
    for (int i = threadIdx.x; i < K; i += 256) m = fmaxf(m, fabsf(x[i]));
    red[threadIdx.x] = m;
    __syncthreads();
    for (int o = 128; o > 0; o >>= 1) {
        if (threadIdx.x < o) red[threadIdx.x] = fmaxf(red[threadIdx.x], red[threadIdx.x + o]);
        __syncthreads();
    }
    const float amax = red[0];
    if (kind == 8) prep8_row(x, K, amax, nk, b, planes, xs, threadIdx.x, 256);
    else prep16_row(x, K, amax, nk, b, planes, xs, threadIdx.x, 256);
}

// ---------------------------------------------------------------------------
// Host launchers.
// ---------------------------------------------------------------------------
size_t prep_bytes(const DevWeight& w) {
    // q8: 3 planes of nk*1 KiB ; q4: 2 planes of ntiles*1 KiB
    return w.dtype == DT_Q8ROW ? (size_t)w.kchunks * 1024 * 3 : (size_t)w.kchunks * 4 * 1024 * 2;
}

int launch_prep(const DevWeight& w, const float* x, int ldx, int m, uint8_t* planes, float* xs,
                hipStream_t st) {
    const int kind = w.dtype == DT_Q8ROW ? 8 : 16;
    const int nk = w.dtype == DT_Q8ROW ? w.kchunks : w.kchunks * 4;
    hipLaunchKernelGGL(k_prep, dim3(m), dim3(256), 0, st, x, ldx, w.cols, kind, nk, planes, xs);
    return CMF_OK;
}

static size_t lds_bytes(const DevWeight& w, int m) {
    return w.dtype == DT_Q8ROW ? (size_t)w.kchunks * 64 * 3 * m : (size_t)w.kchunks * 128 * 4 * m;
}
// plus the f32 scratch of the in-kernel producers: the m raw rows and the
// norm weights
static size_t lds_scratch(const DevWeight& w, int m) {
    return (size_t)(w.dtype == DT_Q8ROW ? w.kchunks * 64 : w.kchunks * 128) * 4 * (m + 1);
}

template <int FMT, int NV, int KS>
static void set_lds_q4() {
    static bool done = false;
    if (!done) {
        (void)hipFuncSetAttribute((const void*)k_gemv_q4<FMT, NV, KS>,
                                  hipFuncAttributeMaxDynamicSharedMemorySize, LDSX_MAX);
        done = true;
    }
}
template <int KS>
static void set_lds_q8() {
    static bool done = false;
    if (!done) {
        (void)hipFuncSetAttribute((const void*)k_gemv_q8<KS>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                  LDSX_MAX);
        done = true;
    }
}

template <int FMT, int NV>
static void launch_q4_nv(const GemvArgs& a, int ks, int grid, size_t lds, hipStream_t st) {
#define CMF_Q4(KS)                                                                             \
    set_lds_q4<FMT, NV, KS>();                                                                 \
    hipLaunchKernelGGL((k_gemv_q4<FMT, NV, KS>), dim3(grid), dim3(64 * KS), lds, st, a)
    switch (ks) {
        case 1: CMF_Q4(1); break;
        case 2: CMF_Q4(2); break;
        case 4: CMF_Q4(4); break;
        default: CMF_Q4(8); break;
    }
#undef CMF_Q4
}

// K split (waves per workgroup) and persistent grid for nrb row blocks of nk
// K steps: enough waves to fill 256 CUs, at least two steps per wave, and
// few enough workgroups that the per-workgroup staging stays cheap.
static void pick_shape(int nrb, int nk, int* ks, int* grid) {
    int k = 1;
    while (k < 8 && (long)nrb * k < 4096 && nk / (k * 2) >= 2) k *= 2;
    *ks = k;
    const int maxg = std::max(256, 2048 / k);
    *grid = std::min(nrb, maxg);
}

int gemv(const DevWeight& w, const XSrc& src, float* y, int ldy, int m, int row_lo, int row_hi,
         bool resid, hipStream_t st, int ks_override, int grid_override) {
    if (m < 1 || m > MAXB) return fail("gemv: batch must be 1..16");
    if (row_lo < 0 || row_hi > w.rows || row_lo >= row_hi) return fail("gemv: bad row range");
    GemvArgs a;
    a.w = w.w;
    a.scale = w.scale;
    a.rowp = w.rowp;
    a.y = y;
    a.ldy = ldy;
    a.m = m;
    a.nk = w.kchunks;
    a.rb0 = row_lo / 16;
    a.nrb = (row_hi + 15) / 16 - a.rb0;
    a.row_lo = row_lo;
    a.row_hi = row_hi;
    a.resid = resid ? 1 : 0;
    a.src = src;
    if (a.src.K == 0) a.src.K = w.cols;
    int ks, grid;
    pick_shape(a.nrb, w.kchunks, &ks, &grid);
    if (ks_override > 0) ks = ks_override;
    size_t lds = lds_bytes(w, m);
    if (src.mode != XS_GLOBAL) {
        const int kpad = w.dtype == DT_Q8ROW ? w.kchunks * 64 : w.kchunks * 128;
        if (a.src.K % 4 || (src.mode != XS_CAT && src.ldx % 4) || (src.mode == XS_CAT && (src.H % 4 || src.ldx % 4)) ||
            ((uintptr_t)src.x & 15) || kpad > 4 * SEG4 * SEGMAX)
            return fail("gemv: fused operand needs K, H, ldx multiples of 4, a 16-byte aligned row base and K <= 16384");
        lds += lds_scratch(w, m);
    }
    if (lds > LDSX_MAX) {
        if (src.mode != XS_GLOBAL) return fail("gemv: activation operand exceeds LDS; prepare it globally");
        lds = 0;  // planes read from global memory per step
    }
    a.lds = lds ? 1 : 0;
    if (grid_override > 0) grid = std::min(grid_override, a.nrb);
    if (w.dtype == DT_Q8ROW) {
#define CMF_Q8(KS) \
    set_lds_q8<KS>(); \
    hipLaunchKernelGGL((k_gemv_q8<KS>), dim3(grid), dim3(64 * KS), lds, st, a)
        switch (ks) {
            case 1: CMF_Q8(1); break;
            case 2: CMF_Q8(2); break;
            case 4: CMF_Q8(4); break;
            default: CMF_Q8(8); break;
        }
#undef CMF_Q8
        return CMF_OK;
    }
    const int nv = m >= 4 ? 4 : m;
#define CMF_Q4F(FMT)                                                        \
    switch (nv) {                                                           \
        case 1: launch_q4_nv<FMT, 1>(a, ks, grid, lds, st); break;          \
        case 2: launch_q4_nv<FMT, 2>(a, ks, grid, lds, st); break;          \
        case 3: launch_q4_nv<FMT, 3>(a, ks, grid, lds, st); break;          \
        default: launch_q4_nv<FMT, 4>(a, ks, grid, lds, st); break;         \
    }
    if (w.dtype == DT_Q4T) {
        CMF_Q4F(DT_Q4T)
    } else {
        CMF_Q4F(DT_Q4TP)
    }
#undef CMF_Q4F
    return CMF_OK;
}

bool fits_lds(const DevWeight& w, int m) { return lds_bytes(w, m) + lds_scratch(w, m) <= LDSX_MAX; }

int launch_gemv(const DevWeight& w, const uint8_t* planes, const float* xs, float* y, int ldy,
                int m, int row_lo, int row_hi, hipStream_t st, int ks_override) {
    XSrc s{};
    s.mode = XS_GLOBAL;
    s.planes = planes;
    s.xs = xs;
    return gemv(w, s, y, ldy, m, row_lo, row_hi, false, st, ks_override, 0);
}

}  // namespace cmf
