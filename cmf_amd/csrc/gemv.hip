// Dequant GEMV / skinny GEMM kernels for gfx950 (MI355X).
//
// y[b][r] = sum_k W[r][k] * x[b][k] for b < M <= 16 and the three weight
// codecs of the engine (q8 per-row, q4_tiled, q4tp).  One workgroup owns one
// block of 16 weight rows; its KS waves split the K range and reduce in LDS
// in a fixed order (deterministic).  Every wave streams 1 KiB of packed
// weights per step with one 128-bit load per lane and feeds them to the
// matrix cores with the activations as the MFMA A operand (16 batch rows,
// zero-padded) and the weights as the B operand (16 weight rows):
//
//   q8   : v_mfma_i32_16x16x64_i8 on the raw int8 weights; x is carried as
//          three int8 planes, x ~= sx*(q0 + q1/128 + q2/16384) (|error| <=
//          2^-22 max|x|), each accumulated exactly in int32 over all of K.
//   q4*  : v_mfma_f32_16x16x32_f16, one tile (32 columns = one scale) per
//          MFMA; nibbles become exact f16 (n - 8) in registers and x is
//          carried as f16 hi + lo of x*2^e (22-bit significand).  Each
//          tile's f32 product is scaled by its tile scale and accumulated in
//          f32, as q4t_row_exact does (qtensor.rs:4418-4432).
#include "common.h"
#include "gemv.h"

namespace cmf {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float float4v __attribute__((ext_vector_type(4)));
typedef int int4v __attribute__((ext_vector_type(4)));

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

template <int FMT, int NV, int KS>
__global__ __launch_bounds__(64 * KS) void k_gemv_q4(
    const uint4* __restrict__ W, const void* __restrict__ S, const float2* __restrict__ RP,
    const uint4* __restrict__ XH, const uint4* __restrict__ XL, const float* __restrict__ XS,
    float* __restrict__ Y, int ldy, int ntg, int M, int row_lo, int row_hi) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int rb = blockIdx.x;
    const int r = lane & 15, s = lane >> 4;
    __shared__ float lad[FMT == DT_Q4TP ? 16 * 33 : 1];
    __shared__ float4v part[KS][64];
    if constexpr (FMT == DT_Q4TP) {
        if (threadIdx.x < 16) {
            const float2 p = RP[rb * 16 + threadIdx.x];
            float t = p.x;
            lad[threadIdx.x * 33] = t;
            for (int c = 1; c < 32; c++) {
                t = t * p.y;
                lad[threadIdx.x * 33 + c] = t;
            }
        }
        __syncthreads();
    }
    const bool xload = r < M;
    const int tg0 = (ntg * wave) / KS, tg1 = (ntg * (wave + 1)) / KS;
    const size_t wbase = (size_t)rb * ntg;
    float4v acc = {0.f, 0.f, 0.f, 0.f};
    const float4v zero = {0.f, 0.f, 0.f, 0.f};
    for (int tg = tg0; tg < tg1; ++tg) {
        const uint4 w = W[(wbase + tg) * 64 + lane];
        float sc[4];
        if constexpr (FMT == DT_Q4T) {
            const uint2 sv = ((const uint2*)S)[(wbase + tg) * 16 + r];
            sc[0] = f16_bits_to_f32(sv.x & 0xFFFFu);
            sc[1] = f16_bits_to_f32(sv.x >> 16);
            sc[2] = f16_bits_to_f32(sv.y & 0xFFFFu);
            sc[3] = f16_bits_to_f32(sv.y >> 16);
        } else {
            const uint32_t cw = ((const uint32_t*)S)[(wbase + tg) * 16 + r];
            sc[0] = lad[r * 33 + (cw & 31)];
            sc[1] = lad[r * 33 + ((cw >> 5) & 31)];
            sc[2] = lad[r * 33 + ((cw >> 10) & 31)];
            sc[3] = lad[r * 33 + ((cw >> 15) & 31)];
        }
        const uint32_t wv[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
        for (int t = 0; t < 4; t++) {
            const int tile = tg * 4 + t;
            half8 xh = {}, xl = {};
            if (xload) {
                xh = __builtin_bit_cast(half8, XH[(size_t)tile * 64 + lane]);
                xl = __builtin_bit_cast(half8, XL[(size_t)tile * 64 + lane]);
            }
            const half8 b = dq_nib_word(wv[t]);
            float4v d = __builtin_amdgcn_mfma_f32_16x16x32_f16(xh, b, zero, 0, 0, 0);
            d = __builtin_amdgcn_mfma_f32_16x16x32_f16(xl, b, d, 0, 0, 0);
#pragma unroll
            for (int v = 0; v < NV; v++) acc[v] += d[v] * sc[t];
        }
    }
    if constexpr (KS > 1) {
        part[wave][lane] = acc;
        __syncthreads();
        if (wave != 0) return;
        for (int q = 1; q < KS; q++) {
            const float4v o = part[q][lane];
#pragma unroll
            for (int v = 0; v < NV; v++) acc[v] += o[v];
        }
    }
    const int row = rb * 16 + r;
    if (row < row_lo || row >= row_hi) return;
#pragma unroll
    for (int v = 0; v < NV; v++) {
        const int b = 4 * s + v;
        if (b < M) Y[(size_t)b * ldy + (row - row_lo)] = acc[v] * XS[b];
    }
    if constexpr (NV == 4) {
        (void)0;
    }
}

template <int KS>
__global__ __launch_bounds__(64 * KS) void k_gemv_q8(
    const int4v* __restrict__ W, const float* __restrict__ RS, const int4v* __restrict__ X0,
    const int4v* __restrict__ X1, const int4v* __restrict__ X2, const float* __restrict__ XS,
    float* __restrict__ Y, int ldy, int nkc, int M, int row_lo, int row_hi) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int rb = blockIdx.x;
    const int r = lane & 15, s = lane >> 4;
    __shared__ int4v part[KS > 1 ? KS : 1][3][64];
    const bool xload = r < M;
    const int k0 = (nkc * wave) / KS, k1 = (nkc * (wave + 1)) / KS;
    const size_t wbase = (size_t)rb * nkc;
    int4v a0 = {0, 0, 0, 0}, a1 = {0, 0, 0, 0}, a2 = {0, 0, 0, 0};
    for (int kc = k0; kc < k1; ++kc) {
        const int4v w = W[(wbase + kc) * 64 + lane];
        int4v x0 = {0, 0, 0, 0}, x1 = {0, 0, 0, 0}, x2 = {0, 0, 0, 0};
        if (xload) {
            x0 = X0[(size_t)kc * 64 + lane];
            x1 = X1[(size_t)kc * 64 + lane];
            x2 = X2[(size_t)kc * 64 + lane];
        }
        a0 = __builtin_amdgcn_mfma_i32_16x16x64_i8(x0, w, a0, 0, 0, 0);
        a1 = __builtin_amdgcn_mfma_i32_16x16x64_i8(x1, w, a1, 0, 0, 0);
        a2 = __builtin_amdgcn_mfma_i32_16x16x64_i8(x2, w, a2, 0, 0, 0);
    }
    if constexpr (KS > 1) {
        part[wave][0][lane] = a0;
        part[wave][1][lane] = a1;
        part[wave][2][lane] = a2;
        __syncthreads();
        if (wave != 0) return;
        for (int q = 1; q < KS; q++) {
            a0 += part[q][0][lane];
            a1 += part[q][1][lane];
            a2 += part[q][2][lane];
        }
    }
    const int row = rb * 16 + r;
    if (row < row_lo || row >= row_hi) return;
    const float rs = RS[row];
#pragma unroll
    for (int v = 0; v < 4; v++) {
        const int b = 4 * s + v;
        if (b < M) {
            const float t = (float)a0[v] + (float)a1[v] * 0.0078125f + (float)a2[v] * 6.103515625e-05f;
            Y[(size_t)b * ldy + (row - row_lo)] = (t * XS[b]) * rs;
        }
    }
}

// ---------------------------------------------------------------------------
// Activation preparation from f32 x[M][ldx] (standalone GEMV calls).  One
// workgroup per batch row; the fused producers of the model path write the
// same layouts through the device helpers in prep.h.
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
static int pick_ks(int nrb, int nk) {
    int ks = 1;
    while (ks < 8 && nrb * ks < 3072 && nk / (ks * 2) >= 2) ks *= 2;
    return ks;
}

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

template <int FMT, int NV>
static void launch_q4_nv(const DevWeight& w, const uint8_t* planes, const float* xs, float* y,
                         int ldy, int m, int rb0, int nrb, int row_lo, int row_hi, int ks,
                         hipStream_t st) {
    const uint4* W = (const uint4*)w.w + (size_t)rb0 * w.kchunks * 64;
    const uint8_t* S = (const uint8_t*)w.scale + (size_t)rb0 * w.kchunks * (FMT == DT_Q4T ? 128 : 64);
    const float2* RP = w.rowp ? w.rowp + (size_t)rb0 * 16 : nullptr;
    const uint4* XH = (const uint4*)planes;
    const uint4* XL = (const uint4*)(planes + (size_t)w.kchunks * 4 * 1024);
    const int lo = row_lo - rb0 * 16, hi = row_hi - rb0 * 16;
#define CMF_Q4(KS)                                                                       \
    hipLaunchKernelGGL((k_gemv_q4<FMT, NV, KS>), dim3(nrb), dim3(64 * KS), 0, st, W, S, RP, \
                       XH, XL, xs, y, ldy, w.kchunks, m, lo, hi)
    switch (ks) {
        case 1: CMF_Q4(1); break;
        case 2: CMF_Q4(2); break;
        case 4: CMF_Q4(4); break;
        default: CMF_Q4(8); break;
    }
#undef CMF_Q4
}

int launch_gemv(const DevWeight& w, const uint8_t* planes, const float* xs, float* y, int ldy,
                int m, int row_lo, int row_hi, hipStream_t st, int ks_override) {
    if (m < 1 || m > MAXB) return fail("gemv: batch must be 1..16");
    if (row_lo < 0 || row_hi > w.rows || row_lo >= row_hi) return fail("gemv: bad row range");
    const int rb0 = row_lo / 16, rb1 = (row_hi + 15) / 16, nrb = rb1 - rb0;
    const int ks = ks_override > 0 ? ks_override : pick_ks(nrb, w.kchunks);
    if (w.dtype == DT_Q8ROW) {
        const int4v* W = (const int4v*)w.w + (size_t)rb0 * w.kchunks * 64;
        const float* RS = (const float*)w.scale + (size_t)rb0 * 16;
        const int4v* X0 = (const int4v*)planes;
        const int4v* X1 = X0 + (size_t)w.kchunks * 64;
        const int4v* X2 = X1 + (size_t)w.kchunks * 64;
        const int lo = row_lo - rb0 * 16, hi = row_hi - rb0 * 16;
#define CMF_Q8(KS)                                                                                 \
    hipLaunchKernelGGL((k_gemv_q8<KS>), dim3(nrb), dim3(64 * KS), 0, st, W, RS, X0, X1, X2, xs, y, \
                       ldy, w.kchunks, m, lo, hi)
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
#define CMF_Q4F(FMT)                                                                                 \
    switch (nv) {                                                                                    \
        case 1: launch_q4_nv<FMT, 1>(w, planes, xs, y, ldy, m, rb0, nrb, row_lo, row_hi, ks, st); break; \
        case 2: launch_q4_nv<FMT, 2>(w, planes, xs, y, ldy, m, rb0, nrb, row_lo, row_hi, ks, st); break; \
        case 3: launch_q4_nv<FMT, 3>(w, planes, xs, y, ldy, m, rb0, nrb, row_lo, row_hi, ks, st); break; \
        default: launch_q4_nv<FMT, 4>(w, planes, xs, y, ldy, m, rb0, nrb, row_lo, row_hi, ks, st); break; \
    }
    if (w.dtype == DT_Q4T) {
        CMF_Q4F(DT_Q4T)
    } else {
        CMF_Q4F(DT_Q4TP)
    }
#undef CMF_Q4F
    return CMF_OK;
}

}  // namespace cmf
