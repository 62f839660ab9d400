// GEMV launchers and the activation-preparation helpers shared by the
// standalone preparation kernel and the fused producers (norms, SwiGLU,
// attention merge) of the model path.
#pragma once

#include "common.h"

namespace cmf {

// The tied q8 embedding table in its device layout.
struct EmbedSrc {
    const int8_t* w;
    const float* rs;
    int rows;
    int nkc;
};

// Producer of a GEMV's activation operand (launch_prep_src evaluates it into
// prepared planes; the GEMV itself takes XS_GLOBAL = prepared planes):
//   XS_NORM : x = rms_norm(x_row) * w                  (inference.rs:33-50)
//   XS_SILU : x = silu(g) * u, g/u at [0, K) / [K, 2K)  (inference.rs:14-16)
//   XS_ROWS : x = x_row
//   XS_CAT  : x = [rms_norm(embed(tok), w) ; rms_norm(x_row, w2)]  (H each,
//             the MTP input, pipeline.rs:3085-3094)
//   XS_SILU8: x[i] = silu(g) * u of a gate|up row whose 16-column blocks
//             hold 8 gate then the 8 matching up values (the interleaved
//             gate|up weight's output): g = row[16 (i/8) + i%8], u = g's + 8
enum { XS_GLOBAL = 0, XS_NORM = 2, XS_SILU = 3, XS_ROWS = 4, XS_CAT = 5, XS_SILU8 = 6 };
struct XSrc {
    int mode;
    const float* x;
    int ldx;
    const float* w;
    const float* w2;
    const int* toks;
    EmbedSrc emb;
    int K;   // logical length of the operand (0: the weight's cols)
    int H;   // XS_CAT: length of each half
    double eps;
    const uint8_t* planes;  // XS_GLOBAL
    const float* xs;
    // XS_GLOBAL, q8 only: chunk-scaled planes (x of batch row b in 64-column
    // chunk c ~= cs[b * cs_ld + c] (q0 + q1/128 + q2/16384)) instead of one
    // scale per row (xs); written by a producer that owns whole chunks
    const float* cs;
    int cs_ld;
};

// One weight of a group (an MoE expert): its device blocks.
struct GemvDesc {
    const void* w;
    const void* scale;
    const float2* rowp;
};

// split_act outliers of the a8w8 operand: cnt[b] of them for batch row b at
// idx/val[b * cap ..] (index order).
struct A8Out {
    int* cnt;
    int* idx;
    float* val;
    int cap;
};

struct GemvArgs {
    const void* w;
    const void* scale;
    const float2* rowp;
    float* y;
    int ldy, m, nk, rb0, nrb, row_lo, row_hi, resid, lds;
    int epi;  // EPI_SWIGLU: rows interleaved 8 gate / 8 up per block, y = silu(g) * u [m][rows / 2]
    XSrc src;
    // grouped launch (grid.y = job): jobs = [njobs, weight index of job 0,
    // ...] on the device; job j multiplies desc[jobs[1 + j]] with the
    // operand at planes + j * planes_stride (xs + 16 j; planes_stride 0: one
    // operand, one xs for all jobs) into y + j * y_stride.
    const int* jobs;
    const GemvDesc* desc;
    size_t planes_stride, y_stride;
};

// Kernel instance for m batch rows, operand source xm (0: prepared planes
// staged in LDS, 1: fused producer staged in LDS, 2: prepared planes read in
// place) and ks waves per workgroup (nullptr: none).
typedef void (*GemvKernel)(GemvArgs);
GemvKernel q4t_kernel(int m, int xm, int ks, int rb);
GemvKernel q4tp_kernel(int m, int xm, int ks, int rb);
// three groups of 4 waves per workgroup (k_gemv_q4<..., G = 3, SPW = 8>)
// (one: the single-unit instance, for grids where every workgroup serves one unit)
GemvKernel q4t_kernel_g3(int m, int xm, bool one = false);
GemvKernel q4tp_kernel_g3(int m, int xm, bool one = false);
// 16 waves x 6 steps (k_gemv_q4<..., KS = 16, HL, ..., SPW = 6>), m <= 8
GemvKernel q4t_kernel_s6(int m, int xm);
GemvKernel q4tp_kernel_s6(int m, int xm);
GemvKernel q8_kernel(int m, int xm, int ks);
// M = 1 over a prepared operand, rows of nk 1 KiB steps (k_gemv_q8_m1 /
// k_gemv_q4t_m1): the instance, its waves per workgroup (*ks) and dynamic
// LDS bytes (*lds), or nullptr
GemvKernel q8_kernel_m1(int nk, bool resid, int* ks, size_t* lds);
GemvKernel q4t_kernel_m1(int nk, bool resid, int* ks, size_t* lds);
// q4t, M = 1, the operand staged from its f32 row inside the kernel (XS_ROWS)
GemvKernel q4t_kernel_m1x(int nk, bool resid, int* ks);

enum { EPI_NONE = 0, EPI_SWIGLU = 1 };

// y[b*ldy + (r - row_lo)] (+)= W x for rows [row_lo, row_hi), b < m, from a
// prepared operand (XS_GLOBAL; launch_prep_src writes it) or from XS_NORM /
// XS_ROWS rows that every workgroup prepares itself (fused_lds_bytes > 0).
// LDS bytes of a GEMV whose workgroups evaluate src (XS_NORM / XS_ROWS)
// themselves, 0 when src must be prepared by launch_prep_src first.
size_t fused_lds_bytes(const DevWeight& w, const XSrc& src, int m);
// Whether that path is the faster one for m rows of w.
bool gemv_fuse_pays(const DevWeight& w, int m);
int gemv(const DevWeight& w, const XSrc& src, float* y, int ldy, int m, int row_lo, int row_hi,
         bool resid, hipStream_t st, int ks_override = 0, int grid_override = 0, int epi = EPI_NONE);
// Grouped GEMV: up to max_jobs jobs (the device list `jobs`, see GemvArgs),
// every weight of the group shaped and typed like `proto`; job j reads the
// prepared operand planes + j * planes_stride (xs + 16 j; stride 0: one
// operand for all jobs) and writes y + j * y_stride ([m][ldy] each).
int gemv_grouped(const DevWeight& proto, const GemvDesc* desc, const int* jobs, int max_jobs,
                 const uint8_t* planes, size_t planes_stride, const float* xs, float* y, size_t y_stride,
                 int ldy, int m, hipStream_t st);

size_t prep_bytes(const DevWeight& w);
// Prepared planes (prep_bytes, the layout of prep8_row / prep16_row) and
// xs[16] of the operand producer src for m batch rows of w.
int launch_prep_src(const DevWeight& w, const XSrc& src, int m, uint8_t* planes, float* xs, hipStream_t st);
// Prepared GEMM operand of m rows of the producer src: planes with row
// stride mstride (a multiple of 64; q4: and tile biases [tile][mstride]).
int launch_prep_src_gemm(const DevWeight& w, const XSrc& src, int m, int mstride, uint8_t* planes, float* xs,
                         hipStream_t st);
int launch_prep_rows_gemm(const DevWeight& w, const float* x, int ldx, int m, int mstride, uint8_t* planes,
                          float* xs, hipStream_t st);
// y[b][n] (ldy) (+)= W x[b] for b < m, any m, q8 / q4t / q4tp weights: the
// large-batch MFMA GEMM (gemm.hip) over the operand of the producer src
// (XS_ROWS, XS_NORM, XS_SILU8, XS_CAT; resid: y += W x).
int gemm(const DevWeight& w, const XSrc& src, int m, float* y, int ldy, bool resid, hipStream_t st);
// the same over plain device rows x [m][ldx]
int gemm_q4(const DevWeight& w, const float* x, int ldx, int m, float* y, int ldy, hipStream_t st);
// The same for up to max_jobs jobs of a device job list (GemvArgs::jobs):
// job j reads rows at src.x + j * x_stride and writes planes + j *
// planes_stride, xs + 16 j.
int launch_prep_src_grouped(const DevWeight& w, const XSrc& src, int m, const int* jobs, int max_jobs,
                            size_t x_stride, uint8_t* planes, size_t planes_stride, float* xs, hipStream_t st);
int launch_prep(const DevWeight& w, const float* x, int ldx, int m, uint8_t* planes, float* xs,
                hipStream_t st);
// The a8w8 operand (split_act) of m rows of x: planes / xs as launch_prep,
// plus the outlier lists in o (cap >= w.cols).
int launch_prep_a8(const DevWeight& w, const float* x, int ldx, int m, uint8_t* planes, float* xs, const A8Out& o,
                   hipStream_t st);
// y = W x under the a8w8 contract from launch_prep_a8's operand (the GEMV,
// then the outlier terms).
int gemv_a8(const DevWeight& w, const uint8_t* planes, const float* xs, const A8Out& o, float* y, int ldy, int m,
            hipStream_t st);
// y[b*ldy + (r - row_lo)] for rows [row_lo, row_hi) and b < m.
int launch_gemv(const DevWeight& w, const uint8_t* planes, const float* xs, float* y, int ldy,
                int m, int row_lo, int row_hi, hipStream_t st, int ks_override = 0);

// x ~= q0 + q1/128 + q2/16384 (each int8, |error| <= 2^-22 * 127), the
// three bytes or-ed into byte j of a, b, c.  v = x / (amax / 127) lies
// within 127 * (1 + 2^-22) of zero, so rint(v) is in [-127, 127] and the
// remainders (v - q0) * 128 and (r1 - q1) * 128 in [-64, 64]: no clamps.
__device__ __forceinline__ void q8_split(float v, int j, uint32_t& a, uint32_t& b, uint32_t& c) {
    const float q0 = rintf(v);
    const float r1 = (v - q0) * 128.0f;
    const float q1 = rintf(r1);
    const float r2 = (r1 - q1) * 128.0f;
    const float q2 = rintf(r2);
    a |= (uint32_t)(uint8_t)(int8_t)q0 << (8 * j);
    b |= (uint32_t)(uint8_t)(int8_t)q1 << (8 * j);
    c |= (uint32_t)(uint8_t)(int8_t)q2 << (8 * j);
}

// Writes batch row b (of M) of the q8 activation planes: three int8 planes
// with x ~= sx * (q0 + q1/128 + q2/16384), sx = max|x|/127, each plane
// [item = 4*chunk + s][b] x 16 bytes of columns 64*chunk + 16*s ...
__device__ inline void prep8_row(const float* x, int K, float amax, int nk, int b, int M,
                                 uint8_t* planes, float* xs, int tid, int nthr) {
    const float sx = amax > 0.f ? amax / 127.0f : 1.0f;
    const float inv = 1.0f / sx;
    if (tid == 0) xs[b] = sx;
    uint8_t* p0 = planes;
    uint8_t* p1 = planes + (size_t)nk * 64 * M;
    uint8_t* p2 = planes + (size_t)nk * 128 * M;
    for (int idx = tid; idx < nk * 4; idx += nthr) {
        const int kc = idx >> 2, s = idx & 3, c0 = kc * 64 + 16 * s;
        uint32_t w0[4], w1[4], w2[4];
#pragma unroll
        for (int q = 0; q < 4; q++) {
            uint32_t a = 0, bb = 0, c = 0;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int col = c0 + 4 * q + j;
                q8_split(col < K ? x[col] * inv : 0.f, j, a, bb, c);
            }
            w0[q] = a;
            w1[q] = bb;
            w2[q] = c;
        }
        const size_t off = ((size_t)idx * M + b) * 16;
        *(uint4*)(p0 + off) = make_uint4(w0[0], w0[1], w0[2], w0[3]);
        *(uint4*)(p1 + off) = make_uint4(w1[0], w1[1], w1[2], w1[3]);
        *(uint4*)(p2 + off) = make_uint4(w2[0], w2[1], w2[2], w2[3]);
    }
}

// hi + lo of one split value as f32 (exact: 22 significant bits), by one
// mixed-precision FMA lo * 1.0 + hi on the f16 registers instead of two
// conversions and an add.
__device__ __forceinline__ float f16_pair_sum(_Float16 hi, _Float16 lo) {
#if defined(__HIP_DEVICE_COMPILE__)
    float r;
    asm("v_fma_mix_f32 %0, %1, 1.0, %2 op_sel_hi:[1,0,1]" : "=v"(r) : "v"(lo), "v"(hi));
    return r;
#else
    return (float)hi + (float)lo;
#endif
}

// The q4 activation operand in fixed point: x ~= xs * (a + k / 2048) with
// xs = 2^(e - 11) for max|x| in [2^(e-1), 2^e), a = rint(x / xs) (|a| <=
// 2048) and k = rint((x / xs - a) * 2048) (|k| <= 1024): hi = a and lo =
// k * 2^-11 are exact f16 values (error <= max|x| * 2^-23).  Against the
// nibbles as f16 denormals n * 2^-24, every product of a tile's MFMA is then
// a multiple of 2^-24 (hi) or 2^-35 (lo), and a tile's sum, bias included,
// stays below 2^-3: the MFMA adds exactly.  (With x * 2^e split into
// floating f16 hi + lo the MFMA's internal sums are not exact: measured on
// MI355X, 1e-6 relative per tile, biased, so that a q4t matvec drifted
// 2e-5..5e-5 from an exact product where the reference's f32 loop stays at
// 1e-7.)  The tiles' products are then scaled and summed in f32.
constexpr float Q4_LO_UNIT = 0.00048828125f;  // 2^-11
__device__ __forceinline__ void q4_fix_scale(float amax, float& inv_xs, float& xs) {
    int ex = 0;
    if (amax > 0.f) frexpf(amax, &ex);
    inv_xs = amax > 0.f ? ldexpf(1.0f, 11 - ex) : 1.0f;
    xs = amax > 0.f ? ldexpf(1.0f, ex - 11) : 1.0f;
}
// hi / lo of v = x / xs (|v| < 2048)
__device__ __forceinline__ void q4_fix_split(float v, _Float16& hi, _Float16& lo) {
    const float a = rintf(v);
    hi = (_Float16)a;
    lo = (_Float16)(rintf((v - a) * 2048.0f) * Q4_LO_UNIT);
}
constexpr float Q4_BIAS = -4.76837158203125e-07f;  // -8 * 2^-24: the format's nibble offset

// Writes batch row b (of M) of the q4 activation operand: the fixed-point
// hi / lo planes of x (q4_fix_split), xs[b] = 2^(e - 11), planes [item =
// 4*tile + s][b] x 8 halves of columns 32*tile + 8*s + {0,4,2,6,1,5,3,7} (hi
// plane, then lo plane), then two tables of tile biases [tile][bstride] f32:
// T1[t][b] = -8 * 2^-24 * sum(hi) and T2[t][b] = -8 * 2^-24 * sum(lo) of the
// tile (T2 right after T1), zero for rows in [M, bstride).  With bstride ==
// 16 and M <= 8 (the GEMVs whose A rows 8 + b carry the lo plane of batch
// row b) T1[t][8 + b] holds the lo bias as well.  M is the planes' row
// stride (the batch of a GEMV; the padded row count of a GEMM, with bstride
// = M).  The q4 kernels multiply by the nibbles as f16 denormals n * 2^-24
// and start each tile's accumulator at the bias of its plane, so that
// D = 2^-24 * sum((n - 8) * x) / xs exactly.  nthr must be a multiple of 64:
// the four items of a tile sit in lanes 4t..4t+3 of one wave, which add
// their partial sums for the biases.
__device__ __forceinline__ void q4_put_bias(float* bias, int ntiles, int bstride, int M, int t, int b, float sh,
                                            float sl) {
    float* t1 = bias + (size_t)t * bstride;
    float* t2 = bias + (size_t)ntiles * bstride + (size_t)t * bstride;
    const bool hl = bstride == 16 && M <= 8;
    t1[b] = sh * Q4_BIAS;
    t2[b] = sl * Q4_BIAS;
    if (hl) t1[8 + b] = sl * Q4_BIAS;
    if (b == 0)
        for (int r = M; r < bstride; r++) {
            if (!(hl && r >= 8 && r - 8 < M)) t1[r] = 0.f;
            t2[r] = 0.f;
        }
}
__device__ inline void prep16_row(const float* x, int K, float amax, int ntiles, int b, int M,
                                  uint8_t* planes, float* xs, int tid, int nthr, int bstride = 16) {
    float scale, xsv;
    q4_fix_scale(amax, scale, xsv);
    if (tid == 0) xs[b] = xsv;
    uint8_t* ph = planes;
    uint8_t* pl = planes + (size_t)ntiles * 64 * M;
    float* bias = (float*)(planes + (size_t)ntiles * 128 * M);
    const int ord[8] = {0, 4, 2, 6, 1, 5, 3, 7};
    for (int i0 = 0; i0 < ntiles * 4; i0 += nthr) {  // uniform trip count (shuffles below)
        const int idx = i0 + tid;
        const bool on = idx < ntiles * 4;
        const int t = idx >> 2, s = idx & 3, c0 = t * 32 + 8 * s;
        uint16_t hv[8], lv[8];
        float sh = 0.f, sl = 0.f;  // (exact: integers and multiples of 2^-11)
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const int col = c0 + ord[j];
            const float v = on && col < K ? x[col] * scale : 0.f;
            _Float16 h, l;
            q4_fix_split(v, h, l);
            hv[j] = __builtin_bit_cast(uint16_t, h);
            lv[j] = __builtin_bit_cast(uint16_t, l);
            sh += (float)h;
            sl += (float)l;
        }
        sh += __shfl_xor(sh, 1);
        sh += __shfl_xor(sh, 2);
        sl += __shfl_xor(sl, 1);
        sl += __shfl_xor(sl, 2);
        if (!on) continue;
        const size_t off = ((size_t)idx * M + b) * 16;
        *(uint4*)(ph + off) = make_uint4(hv[0] | (hv[1] << 16), hv[2] | (hv[3] << 16),
                                         hv[4] | (hv[5] << 16), hv[6] | (hv[7] << 16));
        *(uint4*)(pl + off) = make_uint4(lv[0] | (lv[1] << 16), lv[2] | (lv[3] << 16),
                                         lv[4] | (lv[5] << 16), lv[6] | (lv[7] << 16));
        if (s == 0) q4_put_bias(bias, ntiles, bstride, M, t, b, sh, sl);
    }
}

// The planes of rows b < m at raw + b*K (prep8_row / prep16_row layout, M =
// m) by the whole workgroup at once, the work of all rows spread over its
// threads; amv[b] = max|x| of row b.  Work per thread: q8 4 columns when the
// rows give fewer than 3 such units per thread, else 16 (one 16-byte word of
// each plane, the row's scale computed once); q4 one 8-column item when a
// single pass covers the rows, else a pair of items (16 columns), halving
// the passes.  Measured on MI355X: m = 5 down 1024x3072 9.5 -> 8.2 us.
__device__ inline void prep8_rows(const float* raw, int K, const float* amv, int nk, int m,
                                  uint8_t* planes, float* xs, int tid, int nthr) {
    const int items = nk * 4;
    uint8_t* p0 = planes;
    uint8_t* p1 = planes + (size_t)nk * 64 * m;
    uint8_t* p2 = planes + (size_t)nk * 128 * m;
    if (m * items * 4 < 3 * nthr) {
        // few columns per thread: one thread per 4 columns (one byte lane of
        // a word in each plane), more threads busy
        const int units = items * 4;
        for (int j = tid; j < m * units; j += nthr) {
            const int b = j / units, u = j - b * units;
            const float amax = amv[b];
            const float sx = amax > 0.f ? amax / 127.0f : 1.0f;
            const float inv = 1.0f / sx;
            if (u == 0) xs[b] = sx;
            const int idx = u >> 2, q4 = u & 3;
            const int c0 = (idx >> 2) * 64 + 16 * (idx & 3) + 4 * q4;
            // K % 4 == 0: a unit is all inside or all past the row
            const float4 xv = c0 < K ? *(const float4*)(raw + (size_t)b * K + c0) : make_float4(0.f, 0.f, 0.f, 0.f);
            uint32_t a = 0, bb = 0, c = 0;
            q8_split(xv.x * inv, 0, a, bb, c);
            q8_split(xv.y * inv, 1, a, bb, c);
            q8_split(xv.z * inv, 2, a, bb, c);
            q8_split(xv.w * inv, 3, a, bb, c);
            const size_t off = ((size_t)idx * m + b) * 16 + 4 * q4;
            *(uint32_t*)(p0 + off) = a;
            *(uint32_t*)(p1 + off) = bb;
            *(uint32_t*)(p2 + off) = c;
        }
        return;
    }
    // one thread per item (16 columns): the row's scale and reciprocal once
    // for its four 4-column units
    for (int j = tid; j < m * items; j += nthr) {
        const int b = j / items, idx = j - b * items;
        const float amax = amv[b];
        const float sx = amax > 0.f ? amax / 127.0f : 1.0f;
        const float inv = 1.0f / sx;
        if (idx == 0) xs[b] = sx;
        const int c0 = (idx >> 2) * 64 + 16 * (idx & 3);
        const size_t off = ((size_t)idx * m + b) * 16;
#pragma unroll
        for (int q4 = 0; q4 < 4; q4++) {
            const int c = c0 + 4 * q4;
            const float4 xv = c < K ? *(const float4*)(raw + (size_t)b * K + c) : make_float4(0.f, 0.f, 0.f, 0.f);
            uint32_t a = 0, bb = 0, cc = 0;
            q8_split(xv.x * inv, 0, a, bb, cc);
            q8_split(xv.y * inv, 1, a, bb, cc);
            q8_split(xv.z * inv, 2, a, bb, cc);
            q8_split(xv.w * inv, 3, a, bb, cc);
            *(uint32_t*)(p0 + off + 4 * q4) = a;
            *(uint32_t*)(p1 + off + 4 * q4) = bb;
            *(uint32_t*)(p2 + off + 4 * q4) = cc;
        }
    }
}
__device__ inline void prep16_rows(const float* raw, int K, const float* amv, int ntiles, int m,
                                   uint8_t* planes, float* xs, int tid, int nthr) {
    constexpr int bstride = 16;
    uint8_t* ph = planes;
    uint8_t* pl = planes + (size_t)ntiles * 64 * m;
    float* bias = (float*)(planes + (size_t)ntiles * 128 * m);
    if (m * ntiles * 4 <= nthr) {
        // one pass with one item (8 columns) per thread: the tile's four
        // items are the lanes of one quad
        const int per = ntiles * 4;
        const int jx = tid;
        const bool on = jx < m * per;
        const int b = on ? jx / per : 0, idx = jx - b * per;
        float scale, xsv;
        q4_fix_scale(amv[b], scale, xsv);
        if (on && idx == 0) xs[b] = xsv;
        const int t = idx >> 2, s = idx & 3, c0 = t * 32 + 8 * s;
        const bool in = on && c0 < K;
        const float* x = raw + (size_t)b * K + min(c0, K - 8);
        const float4 xa0 = *(const float4*)x, xb0 = *(const float4*)(x + 4);
        const float4 z4 = make_float4(0.f, 0.f, 0.f, 0.f);
        const float4 xa = in ? xa0 : z4, xb = in ? xb0 : z4;
        const float xv[8] = {xa.x, xb.x, xa.z, xb.z, xa.y, xb.y, xa.w, xb.w};  // columns {0,4,2,6,1,5,3,7}
        uint16_t hv[8], lv[8];
        float sh = 0.f, sl = 0.f;  // (exact: integers and multiples of 2^-11)
#pragma unroll
        for (int j = 0; j < 8; j++) {
            _Float16 h, l;
            q4_fix_split(xv[j] * scale, h, l);
            hv[j] = __builtin_bit_cast(uint16_t, h);
            lv[j] = __builtin_bit_cast(uint16_t, l);
            sh += (float)h;
            sl += (float)l;
        }
        sh += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, sh), 0xb1, 0xf, 0xf, false));
        sh += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, sh), 0x4e, 0xf, 0xf, false));
        sl += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, sl), 0xb1, 0xf, 0xf, false));
        sl += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, sl), 0x4e, 0xf, 0xf, false));
        if (!on) return;
        const size_t off = ((size_t)idx * m + b) * 16;
        *(uint4*)(ph + off) = make_uint4(hv[0] | (hv[1] << 16), hv[2] | (hv[3] << 16),
                                         hv[4] | (hv[5] << 16), hv[6] | (hv[7] << 16));
        *(uint4*)(pl + off) = make_uint4(lv[0] | (lv[1] << 16), lv[2] | (lv[3] << 16),
                                         lv[4] | (lv[5] << 16), lv[6] | (lv[7] << 16));
        if (s == 0) q4_put_bias(bias, ntiles, bstride, m, t, b, sh, sl);
        return;
    }
    // otherwise one thread per pair of items (s = 2p, 2p + 1) of a tile: 16
    // columns, half the passes; the tile's two pairs sit in lanes 2k, 2k + 1
    // (per2 is even)
    const int per2 = ntiles * 2;
    for (int i0 = 0; i0 < m * per2; i0 += nthr) {  // uniform trip count (shuffles below)
        const int jx = i0 + tid;
        const bool on = jx < m * per2;
        const int b = on ? jx / per2 : 0, ip = jx - b * per2;
        float scale, xsv;
        q4_fix_scale(amv[b], scale, xsv);
        if (on && ip == 0) xs[b] = xsv;
        const int t = ip >> 1, s0 = (ip & 1) * 2, c0 = t * 32 + 8 * s0;
        // K % 32 == 0 (q4 rows are whole tiles) and c0 % 16 == 0: the pair
        // is all inside or all past the row.  Unconditional 16-byte reads at
        // a clamped address, the values selected.
        const bool in = on && c0 < K;
        const float* x = raw + (size_t)b * K + min(c0, K - 16);
        const float4 z4 = make_float4(0.f, 0.f, 0.f, 0.f);
        float4 q[4];
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const float4 r = *(const float4*)(x + 4 * k);
            q[k] = in ? r : z4;
        }
        uint4 hq[2], lq[2];
        float ph_[2], pl_[2];
#pragma unroll
        for (int u = 0; u < 2; u++) {
            const float4 xa = q[2 * u], xb = q[2 * u + 1];
            const float xv[8] = {xa.x, xb.x, xa.z, xb.z, xa.y, xb.y, xa.w, xb.w};  // columns {0,4,2,6,1,5,3,7}
            uint16_t hv[8], lv[8];
            float sh = 0.f, sl = 0.f;
#pragma unroll
            for (int j = 0; j < 8; j++) {
                _Float16 h, l;
                q4_fix_split(xv[j] * scale, h, l);
                hv[j] = __builtin_bit_cast(uint16_t, h);
                lv[j] = __builtin_bit_cast(uint16_t, l);
                sh += (float)h;
                sl += (float)l;
            }
            ph_[u] = sh;
            pl_[u] = sl;
            hq[u] = make_uint4(hv[0] | (hv[1] << 16), hv[2] | (hv[3] << 16), hv[4] | (hv[5] << 16),
                               hv[6] | (hv[7] << 16));
            lq[u] = make_uint4(lv[0] | (lv[1] << 16), lv[2] | (lv[3] << 16), lv[4] | (lv[5] << 16),
                               lv[6] | (lv[7] << 16));
        }
        // tile sums (p0 + p1) + (p2 + p3), the pairs' partners one lane apart
        float sh = ph_[0] + ph_[1], sl = pl_[0] + pl_[1];
        sh += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, sh), 0xb1, 0xf, 0xf, false));
        sl += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, sl), 0xb1, 0xf, 0xf, false));
        if (!on) continue;
        const int idx = 4 * t + s0;
        const size_t off = ((size_t)idx * m + b) * 16;
        *(uint4*)(ph + off) = hq[0];
        *(uint4*)(pl + off) = lq[0];
        *(uint4*)(ph + off + (size_t)m * 16) = hq[1];
        *(uint4*)(pl + off + (size_t)m * 16) = lq[1];
        if (s0 == 0) q4_put_bias(bias, ntiles, bstride, m, t, b, sh, sl);
    }
}

}  // namespace cmf
