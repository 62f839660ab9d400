// The operand producer of one prepared-plane row (k_prep_src's body), as an
// inline device function so that other kernels can run it in their own
// workgroups (the MoE routing launch prepares the token rows beside it).
#pragma once

#include "gemv.h"

namespace cmf {

// Row b of m (the planes' row count for GEMV operands) of the producer s
// by the whole workgroup (up to 16 waves); vals: K floats of LDS.
__device__ inline void prep_src_row(XSrc s, int K, int fmt, int nk, uint8_t* __restrict__ planes, float* __restrict__ xs,
                             int mstride, int b, int m, float* vals) {
    __shared__ double red1[16], red2[16];
    __shared__ float redm[16];
    const int tid = threadIdx.x, nt = blockDim.x, lane = tid & 63, wave = tid >> 6;
    const int nw = nt >> 6;
    const bool nrm = s.mode == XS_NORM || s.mode == XS_CAT;
    const int H = s.mode == XS_CAT ? s.H : K;
    const float* row = s.x + (size_t)b * s.ldx;
    int tok = 0, rb = 0, r = 0;
    float rs = 0.f;
    bool tv = false;
    if (s.mode == XS_CAT) {
        tok = s.toks[b];
        tv = tok >= 0 && tok < s.emb.rows;
        rb = tok >> 4;
        r = tok & 15;
        rs = tv ? s.emb.rs[tok] : 0.f;
    }
    auto raw = [&](int i) -> float {
        if (s.mode == XS_SILU) {
            const float g = row[i], u = row[s.K + i];
            return (g / (1.0f + expf(-g))) * u;
        }
        if (s.mode == XS_SILU8) {
            const int o = 16 * (i >> 3) + (i & 7);
            const float g = row[o], u = row[o + 8];
            return (g / (1.0f + expf(-g))) * u;
        }
        if (s.mode == XS_CAT) {
            if (i < H) {
                // int8 of the token's row in the q8 device layout, times its row scale
                const int kc = i >> 6, sl = (i >> 4) & 3, jj = i & 15;
                const int8_t q = tv ? s.emb.w[(((size_t)rb * s.emb.nkc + kc) * 64 + 16 * sl + r) * 16 + jj] : 0;
                return (float)q * rs;
            }
            return row[i - H];
        }
        return row[i];
    };
    // four columns per thread at a time, their loads issued together (one
    // round trip per four instead of one per column); the sums of squares
    // still add the thread's columns in increasing order
    double s1 = 0.0, s2 = 0.0;
    for (int i0 = tid; i0 < K; i0 += 4 * nt) {
        float v[4];
#pragma unroll
        for (int u = 0; u < 4; u++) v[u] = raw(min(i0 + u * nt, K - 1));
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const int i = i0 + u * nt;
            if (i < K) {
                vals[i] = v[u];
                if (nrm) {
                    if (i < H) s1 += (double)v[u] * (double)v[u];
                    else s2 += (double)v[u] * (double)v[u];
                }
            }
        }
    }
    if (nrm) {
        for (int o = 32; o > 0; o >>= 1) {
            s1 += __shfl_xor(s1, o);
            s2 += __shfl_xor(s2, o);
        }
        if (lane == 0) {
            red1[wave] = s1;
            red2[wave] = s2;
        }
    }
    __syncthreads();
    float am = 0.f;
    if (nrm) {
        double t1 = 0.0, t2 = 0.0;
        for (int q = 0; q < nw; q++) {
            t1 += red1[q];
            t2 += red2[q];
        }
        const float inv1 = 1.0f / (float)sqrt(t1 / (double)H + s.eps);
        const float inv2 = s.mode == XS_CAT ? 1.0f / (float)sqrt(t2 / (double)(K - H) + s.eps) : 1.f;
        for (int i0 = tid; i0 < K; i0 += 4 * nt) {
            float wv[4];
#pragma unroll
            for (int u = 0; u < 4; u++) {
                const int i = min(i0 + u * nt, K - 1);
                wv[u] = i < H ? s.w[i] : s.w2[i - H];
            }
#pragma unroll
            for (int u = 0; u < 4; u++) {
                const int i = i0 + u * nt;
                if (i < K) {
                    const float y = vals[i] * (i < H ? inv1 : inv2) * wv[u];
                    vals[i] = y;
                    am = fmaxf(am, fabsf(y));
                }
            }
        }
    } else {
        for (int i = tid; i < K; i += nt) am = fmaxf(am, fabsf(vals[i]));
    }
    for (int o = 32; o > 0; o >>= 1) am = fmaxf(am, __shfl_xor(am, o));
    if (lane == 0) redm[wave] = am;
    __syncthreads();
    am = 0.f;
    for (int q = 0; q < nw; q++) am = fmaxf(am, redm[q]);
    // row stride of the planes: the batch (GEMV operands) or a padded row
    // count (GEMM operands, whose tile biases share that stride)
    const int ms = mstride ? mstride : m;
    if (fmt == DT_Q8ROW) prep8_row(vals, K, am, nk, b, ms, planes, xs, tid, nt);
    else prep16_row(vals, K, am, nk, b, ms, planes, xs, tid, nt, mstride ? mstride : 16);
}

}  // namespace cmf
