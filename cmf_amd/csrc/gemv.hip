// GEMV host side: operand preparation kernel, kernel choice and launch.
#include <map>
#include <mutex>

#include "gemv_kern.h"
#include "prep_src.h"

namespace cmf {

// ---------------------------------------------------------------------------
// Operand producers into prepared planes, one workgroup per batch row: the
// producer (XSrc) is evaluated into LDS in f32, reduced (f64 sums of squares
// for the RMSNorm producers, max|x|) and written as the planes of a weight
// of format fmt (prep8_row / prep16_row), which the GEMV then copies to LDS.
//   XS_ROWS: x          XS_NORM: rms_norm(x) * w (inference.rs:33-50)
//   XS_SILU: silu(g) * u with g/u at [0, K) / [K, 2K) of the row (inference.rs:14-16)
//   XS_CAT : [rms_norm(embed(tok)) * w ; rms_norm(x) * w2], H each (pipeline.rs:3085-3094)
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(512) void k_prep_src(XSrc s, int K, int fmt, int nk, uint8_t* __restrict__ planes,
                                                  float* __restrict__ xs, const int* __restrict__ jobs,
                                                  size_t x_stride, size_t planes_stride, int mstride, int m) {
    extern __shared__ float vals[];  // K
    if (jobs) {  // grouped: blockIdx.y = job
        const int j = blockIdx.y;
        if (j >= jobs[0]) return;
        s.x += j * x_stride;
        planes += j * planes_stride;
        xs += 16 * j;
    }
    int b = blockIdx.x;
    if (mstride) {
        // GEMM operands: row b's 16-byte items sit 16 mstride bytes apart,
        // so one 128-byte line of a plane holds 8 consecutive rows (and one
        // of the q4 bias tables 32): rows 32 (x + 8 k) .. + 31 go to the
        // workgroups of XCD x (the dispatcher deals workgroups to the 8
        // XCDs in turn), so that each line is written from one XCD's L2
        // instead of in pieces from several (the grid is padded to 256)
        const int x = b & 7, j = b >> 3;
        b = 32 * (x + 8 * (j >> 5)) + (j & 31);
        if (b >= m) return;
    }
    prep_src_row(s, K, fmt, nk, planes, xs, mstride, b, mstride ? m : gridDim.x, vals);
}

// The a8w8 operand (split_act, qtensor.rs:9237-9281) of row b of x: rms =
// sqrt(sum(x*x) / n) (f32 products, f64 sum), outliers |x| > 8 rms listed
// exactly in index order (idx/val, count), sx = max|x| of the rest / 127
// (1 if 0), xq = clamp(round half away(x / sx), +-127) and 0 at outliers.
// xq (small integers) is written as the prepared planes: q8 plane 0 = xq,
// planes 1, 2 = 0; q4 hi = xq * 2^4 exactly (the fixed-point operand of
// max|x| = 127), lo = 0.  xs[b] = sx (q8) or sx * 2^-4 (q4), so the GEMVs'
// integer tile dots and scales reproduce the contract; the outliers are
// added in their epilogue.  grid (m), 512.
__global__ __launch_bounds__(512) void k_prep_a8(const float* __restrict__ x, int ldx, int K, int fmt, int nk,
                                                 uint8_t* __restrict__ planes, float* __restrict__ xs,
                                                 int* __restrict__ ocnt, int* __restrict__ oidx,
                                                 float* __restrict__ oval, int ocap) {
    extern __shared__ float vals[];  // K
    __shared__ double red[8];
    __shared__ float redm[8];
    __shared__ int wcnt[8], cnt_thr[512];
    const int b = blockIdx.x, tid = threadIdx.x, nt = blockDim.x, lane = tid & 63, wave = tid >> 6;
    const int nw = nt >> 6;
    const float* row = x + (size_t)b * ldx;
    double ss = 0.0;
    for (int i = tid; i < K; i += nt) {
        const float v = row[i];
        vals[i] = v;
        ss += (double)(v * v);
    }
    for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o);
    if (lane == 0) red[wave] = ss;
    __syncthreads();
    double t = 0.0;
    for (int q = 0; q < nw; q++) t += red[q];
    const float thr = 8.0f * (float)sqrt(t / (double)(K > 1 ? K : 1));
    // thread tid owns the contiguous columns [c0, c1): outliers keep index order
    const int per = (K + nt - 1) / nt, c0 = min(K, tid * per), c1 = min(K, c0 + per);
    int n_out = 0;
    float am = 0.f;
    for (int i = c0; i < c1; i++) {
        const float a = fabsf(vals[i]);
        if (a > thr) n_out++;
        else am = fmaxf(am, a);
    }
    cnt_thr[tid] = n_out;
    for (int o = 32; o > 0; o >>= 1) am = fmaxf(am, __shfl_xor(am, o));
    if (lane == 0) redm[wave] = am;
    __syncthreads();
    if (tid == 0) {  // exclusive scan of the per-thread counts
        int acc = 0;
        for (int q = 0; q < nt; q++) {
            const int c = cnt_thr[q];
            cnt_thr[q] = acc;
            acc += c;
        }
        ocnt[b] = acc;
        wcnt[0] = acc;
    }
    __syncthreads();
    am = 0.f;
    for (int q = 0; q < nw; q++) am = fmaxf(am, redm[q]);
    const float sx = am > 0.f ? am / 127.0f : 1.0f;
    const float inv = 1.0f / sx;
    const bool any = wcnt[0] > 0;
    int o = cnt_thr[tid];
    for (int i = c0; i < c1; i++) {
        const float v = vals[i];
        float q;
        if (any && fabsf(v) > thr) {
            oidx[(size_t)b * ocap + o] = i;
            oval[(size_t)b * ocap + o] = v;
            o++;
            q = 0.f;
        } else {
            q = fminf(127.f, fmaxf(-127.f, roundf(v * inv)));
        }
        vals[i] = q;
    }
    __syncthreads();
    if (fmt == DT_Q8ROW) prep8_row(vals, K, 127.0f, nk, b, gridDim.x, planes, xs, tid, nt);
    else prep16_row(vals, K, 127.0f, nk, b, gridDim.x, planes, xs, tid, nt);
    __syncthreads();
    if (tid == 0) xs[b] = fmt == DT_Q8ROW ? sx : ldexpf(sx, -4);  // (127 < 2^7: the operand unit 2^(7 - 11))
}

// The split_act outlier terms of the a8w8 contract, after the GEMV (grid
// (rows / 256, m)): q4t / q4tp y += ((nib - 8) * tile scale) * x per outlier
// in index order, as q4t_outlier / q4tp_outlier add them after the tile sum
// (qtensor.rs:4405-4413, 4666-4671); q8 y += (sum of w * x) * row scale (the
// reference adds w * x before its row-scale multiply, qtensor.rs:9094-9101:
// one rounding apart).  The weight is read from the device layout (row block
// row / 16, lane 16 s + row % 16).
__global__ __launch_bounds__(256) void k_a8_outliers(const void* __restrict__ wv, const void* __restrict__ scale,
                                                     const float2* __restrict__ rowp, int fmt, int rows, int nk,
                                                     A8Out o, float* __restrict__ y, int ldy) {
    const int row = blockIdx.x * blockDim.x + threadIdx.x, b = blockIdx.y;
    if (row >= rows) return;
    const int n = o.cnt[b];
    if (n == 0) return;
    const int rb = row >> 4, r = row & 15;
    float* yp = y + (size_t)b * ldy + row;
    if (fmt == DT_Q8ROW) {
        const int8_t* wq = (const int8_t*)wv;
        float acc = 0.f;
        for (int i = 0; i < n; i++) {
            const int j = o.idx[(size_t)b * o.cap + i];
            const int c = j >> 6, sl = (j >> 4) & 3, jj = j & 15;
            acc += (float)wq[(((size_t)rb * nk + c) * 64 + 16 * sl + r) * 16 + jj] * o.val[(size_t)b * o.cap + i];
        }
        *yp += acc * ((const float*)scale)[row];
        return;
    }
    const uint8_t* wb = (const uint8_t*)wv;
    float acc = *yp;
    for (int i = 0; i < n; i++) {
        const int j = o.idx[(size_t)b * o.cap + i];
        const int g = j >> 7, t = (j >> 5) & 3, sl = (j >> 3) & 3, q = j & 7;  // column 128 g + 32 t + 8 sl + q
        const size_t step = (size_t)rb * nk + g;
        const uint8_t by = wb[(step * 64 + 16 * sl + r) * 16 + 4 * t + (q >> 1)];
        const int nib = (by >> (4 * (q & 1))) & 15;
        float sc;
        if (fmt == DT_Q4T) {
            const uint16_t h = ((const uint16_t*)scale)[(step * 16 + r) * 4 + t];
            sc = (float)__builtin_bit_cast(_Float16, h);
        } else {
            const uint32_t cw = ((const uint32_t*)scale)[step * 16 + r];
            const int code = (cw >> (5 * t)) & 31;
            const float2 pr = rowp[row];
            float tv = pr.x;  // the ladder t[c] = t[c-1] * ratio
            for (int c = 1; c <= code; c++) tv = tv * pr.y;
            sc = tv;
        }
        acc += ((float)(nib - 8) * sc) * o.val[(size_t)b * o.cap + i];
    }
    *yp = acc;
}

// ---------------------------------------------------------------------------
// Host launchers.
// ---------------------------------------------------------------------------
int launch_prep_src(const DevWeight& w, const XSrc& src, int m, uint8_t* planes, float* xs, hipStream_t st) {
    const int K = src.K ? src.K : w.cols;
    if (m < 1 || m > MAXB) return fail("prep: batch must be 1..16");
    if (K < 1 || K > w.cols || K > 16384) return fail("prep: operand length must be 1..min(cols, 16384)");
    if (src.mode == XS_CAT && (src.H < 1 || src.H >= K)) return fail("prep: bad concat split");
    const int nk = w.dtype == DT_Q8ROW ? w.kchunks : w.kchunks * 4;
    hipLaunchKernelGGL(k_prep_src, dim3(m), dim3(512), (size_t)K * sizeof(float), st, src, K, w.dtype, nk, planes,
                       xs, (const int*)nullptr, (size_t)0, (size_t)0, 0, m);
    return CMF_OK;
}

int launch_prep_src_gemm(const DevWeight& w, const XSrc& src, int m, int mstride, uint8_t* planes, float* xs,
                         hipStream_t st) {
    const int K = src.K ? src.K : w.cols;
    if (m < 1 || m > mstride || mstride % 64) return fail("prep: GEMM rows must be 1..mstride, mstride % 64 == 0");
    if (m > 65535) return fail("prep: at most 65535 GEMM rows per launch");
    if (K < 1 || K > w.cols || K > 16384) return fail("prep: operand length must be 1..min(cols, 16384)");
    if (src.mode == XS_CAT && (src.H < 1 || src.H >= K)) return fail("prep: bad concat split");
    const int nk = w.dtype == DT_Q8ROW ? w.kchunks : w.kchunks * 4;
    // (256 threads a row: all of a 2048-row chunk's workgroups resident at
    // once; measured on MI355X, the 2048-position prefill 12.45 -> 12.21 ms
    // against 512, 12.5 ms at 128)
    hipLaunchKernelGGL(k_prep_src, dim3((m + 255) / 256 * 256), dim3(256), (size_t)K * sizeof(float), st, src, K,
                       w.dtype, nk, planes, xs, (const int*)nullptr, (size_t)0, (size_t)0, mstride, m);
    return CMF_OK;
}

int launch_prep_rows_gemm(const DevWeight& w, const float* x, int ldx, int m, int mstride, uint8_t* planes,
                          float* xs, hipStream_t st) {
    XSrc r{};
    r.mode = XS_ROWS;
    r.x = x;
    r.ldx = ldx;
    return launch_prep_src_gemm(w, r, m, mstride, planes, xs, st);
}

int launch_prep_src_grouped(const DevWeight& w, const XSrc& src, int m, const int* jobs, int max_jobs,
                            size_t x_stride, uint8_t* planes, size_t planes_stride, float* xs, hipStream_t st) {
    const int K = src.K ? src.K : w.cols;
    if (m < 1 || m > MAXB) return fail("prep: batch must be 1..16");
    if (K < 1 || K > w.cols || K > 16384) return fail("prep: operand length must be 1..min(cols, 16384)");
    if (src.mode == XS_CAT) return fail("prep: no grouped concat producer");
    if (max_jobs < 1 || max_jobs > 65535 || !jobs) return fail("prep: bad job list");
    const int nk = w.dtype == DT_Q8ROW ? w.kchunks : w.kchunks * 4;
    hipLaunchKernelGGL(k_prep_src, dim3(m, max_jobs), dim3(512), (size_t)K * sizeof(float), st, src, K, w.dtype, nk,
                       planes, xs, jobs, x_stride, planes_stride, 0, m);
    return CMF_OK;
}

size_t prep_bytes(const DevWeight& w) {
    // at most 16 batch rows: q8 3 planes of nk*64*16 B ; q4 2 planes of ntiles*64*16 B
    // (+ the q4 hi and lo tile-bias tables [tile][16] f32)
    return w.dtype == DT_Q8ROW ? (size_t)w.kchunks * 1024 * 3 : (size_t)w.kchunks * 4 * (1024 * 2 + 128);
}

int launch_prep_a8(const DevWeight& w, const float* x, int ldx, int m, uint8_t* planes, float* xs, const A8Out& o,
                   hipStream_t st) {
    if (m < 1 || m > MAXB || o.cap < w.cols) return fail("prep_a8: batch 1..16 and an outlier capacity of cols");
    const int nk = w.dtype == DT_Q8ROW ? w.kchunks : w.kchunks * 4;
    hipLaunchKernelGGL(k_prep_a8, dim3(m), dim3(512), (size_t)w.cols * sizeof(float), st, x, ldx, w.cols, w.dtype,
                       nk, planes, xs, o.cnt, o.idx, o.val, o.cap);
    return CMF_OK;
}

int launch_prep(const DevWeight& w, const float* x, int ldx, int m, uint8_t* planes, float* xs,
                hipStream_t st) {
    XSrc r{};
    r.mode = XS_ROWS;
    r.x = x;
    r.ldx = ldx;
    return launch_prep_src(w, r, m, planes, xs, st);
}

static size_t lds_bytes(const DevWeight& w, int m) {
    // q4: hi + lo planes and the tile biases [tile][16] f32 (m > 8: both tables)
    return w.dtype == DT_Q8ROW ? (size_t)w.kchunks * 64 * 3 * m
                               : (size_t)w.kchunks * 4 * (128 * m + (m > 8 ? 128 : 64));
}
// LDS of a GEMV that evaluates the producer of src itself (XM_FUSED): the
// planes (1 KiB aligned), then the raw rows and the norm weight; 0 when that
// path does not apply (other producers, the f16 operand of m > 8 rows,
// unaligned rows, more than the LDS budget).
size_t fused_lds_bytes(const DevWeight& w, const XSrc& src, int m) {
    if (src.mode != XS_NORM && src.mode != XS_ROWS && src.mode != XS_CAT) return 0;
    if (w.dtype != DT_Q8ROW && m > 8) return 0;
    const int K = src.K ? src.K : w.cols;
    if (K != w.cols || K % 4 || src.ldx % 4 || (uintptr_t)src.x % 16) return 0;
    if (src.mode == XS_NORM && (!src.w || (uintptr_t)src.w % 16)) return 0;
    const size_t planes = (lds_bytes(w, m) + 1023) & ~(size_t)1023;
    size_t raw = ((size_t)(m + (src.mode == XS_NORM ? 1 : 0)) * K * 4 + 1023) & ~(size_t)1023;
    if (src.mode == XS_CAT) {
        const int H = src.H;
        if (2 * H != K || H % 256 || !src.toks || !src.emb.w || !src.emb.rs || !src.w || !src.w2 ||
            (uintptr_t)src.w % 16 || (uintptr_t)src.w2 % 16)
            return 0;
        // rows x, w, w2 (f32), the int8 embedding rows (1 KiB each), their scales
        const size_t eh = ((size_t)H + 1023) & ~(size_t)1023;
        raw += ((size_t)(m + 2) * H * 4 + (size_t)m * eh + 4 * (size_t)m + 1023) & ~(size_t)1023;
    }
    return planes + raw <= (size_t)LDSX_MAX ? planes + raw : 0;
}

static int env_int(const char* name, int dflt) {
    const char* v = getenv(name);
    return v && *v ? atoi(v) : dflt;
}

static int num_cus() {
    static int n = 0;
    if (n == 0) {
        int dev = 0, c = 0;
        (void)hipGetDevice(&dev);
        if (hipDeviceGetAttribute(&c, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || c < 1) c = 256;
        n = c;
    }
    return n;
}

// Workgroups of kernel k (threads, dyn LDS) resident per CU, once per
// (kernel, threads, LDS); the kernel is also allowed the dynamic LDS the
// CU's 160 KiB leave beside its static LDS.
static int resident_per_cu(GemvKernel k, int threads, size_t lds) {
    static std::mutex mu;
    static std::map<std::tuple<const void*, int, size_t>, int> cache;
    std::lock_guard<std::mutex> g(mu);
    const auto key = std::make_tuple((const void*)k, threads, lds);
    auto it = cache.find(key);
    if (it != cache.end()) return it->second;
    hipFuncAttributes fa{};
    size_t st = 0;
    if (hipFuncGetAttributes(&fa, (const void*)k) == hipSuccess) st = fa.sharedSizeBytes;
    const size_t cap = 160 * 1024 > st ? 160 * 1024 - st : 0;
    (void)hipFuncSetAttribute((const void*)k, hipFuncAttributeMaxDynamicSharedMemorySize,
                              (int)cap);
    int occ = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, (const void*)k, threads, lds) != hipSuccess) occ = 0;
    (void)hipGetLastError();
    cache[key] = occ;
    return occ;
}

// Waves per workgroup for nk K steps of SP per wave: the power of two that
// covers nk in one K part, at most 16 (longer rows take several K parts).
static int pick_ks(int nk) {
    static const int cap = std::min(16, std::max(1, env_int("CMF_GEMV_MAXKS", 16)));
    int k = 1;
    while (k < cap && k * SP < nk) k *= 2;
    return k;
}

constexpr int FUSED_MIN_KS = 8;  // waves of a workgroup that stages m > 2 rows

// Whether evaluating the producer inside the GEMV workgroups beats a
// producer launch: measured on MI355X (decode-layer shapes, m = 1, 2, 5) it
// does while every wave of a workgroup stages at most two operand rows
// (the staging is spread over the workgroup's threads), except on
// matrices much taller than one wave of workgroups for m > 2 (the lm_head:
// there the raw rows' LDS halves the occupancy that hides the weight
// stream's latency, 40.7 vs 32.2 us at m = 5).
bool gemv_fuse_pays(const DevWeight& w, int m) {
    int ks = pick_ks(w.kchunks);
    if (w.dtype != DT_Q8ROW && m > 8) ks = std::min(ks, 8);
    if (m > 2 && w.rows_pad / 16 > 8 * num_cus()) return false;
    return m <= 8 && m <= 2 * std::max(ks, FUSED_MIN_KS);  // (measured up to the m = 5 verify batch)
}

// Kernel choice and launch of a filled GemvArgs (grid.y = gridy jobs).
static int launch_args(const DevWeight& w, GemvArgs& a, int ks_override, int grid_override, int gridy,
                       hipStream_t st) {
    const int m = a.m;
    if (a.src.K == 0) a.src.K = w.cols;
    // K steps of 1 KiB per row block: q8 chunks of 64 columns, q4 groups of
    // 4 tiles (128 columns)
    int ks = ks_override > 0 ? ks_override : pick_ks(w.kchunks);
    if (w.dtype != DT_Q8ROW && m > 8) ks = std::min(ks, 8);  // no 16-wave instance (registers)
    // a workgroup that stages m > 2 rows itself gets at least 8 waves (those
    // past the row's K steps only help with the staging, which is VALU
    // bound; measured on MI355X 8 beats 4 and 16: K=4 round 1.80 ms vs 1.86
    // and 1.88)
    if (a.src.mode != XS_GLOBAL && m > 2 && ks_override <= 0) ks = std::max(ks, FUSED_MIN_KS);
    size_t lds = 0;
    int xm = XM_GLOBAL;
    if (a.src.mode == XS_GLOBAL && a.src.cs) {
        // chunk-scaled q8 planes: the planes (1 KiB aligned) then the chunk
        // scales, rounded to whole 1 KiB direct-load chunks
        if (w.dtype != DT_Q8ROW || a.src.cs_ld != w.kchunks || gridy > 1)
            return fail("gemv: chunk-scaled operands are q8, contiguous, ungrouped");
        lds = ((lds_bytes(w, m) + 1023) & ~(size_t)1023) + (((size_t)m * w.kchunks * 4 + 1023) & ~(size_t)1023);
        if (lds > LDSX_MAX) return fail("gemv: chunk-scaled operand too large for LDS");
        xm = XM_PREPC;
    } else if (a.src.mode == XS_GLOBAL) {
        lds = lds_bytes(w, m);
        if (lds > LDSX_MAX) lds = 0;  // planes read in place from global memory
        xm = lds ? XM_PREP : XM_GLOBAL;
    } else {
        lds = fused_lds_bytes(w, a.src, m);
        if (!lds || gridy > 1) return fail("gemv: this operand must be prepared (launch_prep_src)");
        xm = XM_FUSED;
    }
    // M = 1 over a prepared operand: the per-wave operand-slice kernels
    // (k_gemv_q8_m1, k_gemv_q4t_m1), one workgroup per row block
    // (CMF_GEMV_M1=0 keeps the general kernel)
    static const int m1_env = env_int("CMF_GEMV_M1", 1);
    if (m1_env && m == 1 && xm == XM_PREP && gridy == 1 && grid_override <= 0 && ks_override <= 0 &&
        a.epi == EPI_NONE && (w.dtype == DT_Q8ROW || w.dtype == DT_Q4T)) {
        int ks1 = 0;
        size_t l1 = 0;
        GemvKernel k1 = w.dtype == DT_Q8ROW ? q8_kernel_m1(w.kchunks, a.resid, &ks1, &l1)
                                            : q4t_kernel_m1(w.kchunks, a.resid, &ks1, &l1);
        // (resident_per_cu also allows the kernel its dynamic LDS above the default limit)
        if (k1 && resident_per_cu(k1, 64 * ks1, l1) >= 1) {
            void* args[] = {&a};
            CMF_HIP(hipLaunchKernel((const void*)k1, dim3(a.nrb), dim3(64 * ks1), args, l1, st));
            return CMF_OK;
        }
    }
    // q4t M = 1 from the f32 row (XS_ROWS): the kernel that stages its own
    // operand slices (CMF_GEMV_M1X=0 keeps the general fused kernel)
    static const int m1x_env = env_int("CMF_GEMV_M1X", 1);
    if (m1x_env && m == 1 && xm == XM_FUSED && a.src.mode == XS_ROWS && w.dtype == DT_Q4T && gridy == 1 &&
        grid_override <= 0 && ks_override <= 0 && a.epi == EPI_NONE && a.src.K % 8 == 0) {
        int ks1 = 0;
        GemvKernel k1 = q4t_kernel_m1x(w.kchunks, a.resid, &ks1);
        if (k1 && resident_per_cu(k1, 64 * ks1, 0) >= 1) {
            void* args[] = {&a};
            CMF_HIP(hipLaunchKernel((const void*)k1, dim3(a.nrb), dim3(64 * ks1), args, 0, st));
            return CMF_OK;
        }
    }
    // Two more q4 shapes of the prepared-operand GEMV, chosen by what
    // measured faster on MI355X (GEMV alone, 10 weight copies rotating;
    // CMF_GEMV_G=0/3 and CMF_GEMV_S6=0/1 force either):
    //  - three groups of 4 waves x 8 steps per workgroup, one workgroup per
    //    CU sharing one operand copy, for K <= 4096 and 4 <= m <= 8 (the
    //    per-workgroup operand, 16 KiB per batch row, was read three times
    //    per CU): 12288x4096 m=4 10.3 -> 9.4 us, m=8 12.5 -> 10.1 us; q4tp
    //    m=5 11.0 -> 10.7 us (m=1 8.2 vs 7.5 us, m=2 8.9 vs 8.4: 12 waves per
    //    CU hide the stream's latency worse than 24);
    //  - 16 waves x 6 steps for rows of 65..96 steps (K <= 12288), one K part
    //    instead of two walked one after the other: 4096x12288 m=1 9.0 ->
    //    8.8 us, m=8 12.9 -> 12.6 us (m=2 9.6 vs 10.0 us: not used there;
    //    q4tp at m > 1 keeps the 16 x 4 kernel, whose in-place variant
    //    would spill).
    static const int g_env = env_int("CMF_GEMV_G", -1), s6_env = env_int("CMF_GEMV_S6", -1);
    const bool alt_ok = w.dtype != DT_Q8ROW && gridy == 1 && grid_override <= 0 && ks_override <= 0 &&
                        a.src.mode == XS_GLOBAL && !a.src.cs;
    const bool g3 = alt_ok && w.kchunks <= 32 && a.nrb >= 3 * num_cus() &&
                    (g_env == 3 || (g_env < 0 && m >= 4 && m <= 8));
    if (g3) {
        const size_t lg = lds_bytes(w, m);  // (K <= 4096, m <= 8: at most 139 KiB)
        GemvKernel kg = lg <= (size_t)LDSX_MAX_G3 ? (w.dtype == DT_Q4T ? q4t_kernel_g3(m, XM_PREP)
                                                                    : q4tp_kernel_g3(m, XM_PREP))
                                                  : nullptr;
        const int og = kg ? resident_per_cu(kg, 64 * 4 * 3, lg) : 0;
        if (og >= 1) {
            a.lds = 1;
            const int units = (a.nrb + 2) / 3;
            const int grid = std::min(units, og * num_cus());
            // every workgroup one unit (K <= 4096 is one K part): the loop-free
            // instance, if the CUs hold as many of it
            static const int one_env = env_int("CMF_GEMV_ONE", 1);
            if (one_env && grid == units) {
                GemvKernel k1 = w.dtype == DT_Q4T ? q4t_kernel_g3(m, XM_PREP, true) : q4tp_kernel_g3(m, XM_PREP, true);
                if (k1 && resident_per_cu(k1, 64 * 4 * 3, lg) * num_cus() >= grid) kg = k1;
            }
            void* args[] = {&a};
            CMF_HIP(hipLaunchKernel((const void*)kg, dim3(grid), dim3(64 * 4 * 3), args, lg, st));
            return CMF_OK;
        }
    }
    const bool s6 = alt_ok && w.kchunks > 64 && w.kchunks <= 96 && m <= 8 &&
                    (s6_env == 1 || (s6_env < 0 && (m == 1 || m >= 5)));
    if (s6) {
        GemvKernel k6 = w.dtype == DT_Q4T ? q4t_kernel_s6(m, xm) : q4tp_kernel_s6(m, xm);
        const int o6 = k6 ? resident_per_cu(k6, 1024, lds) : 0;
        if (o6 >= 1) {
            a.lds = lds ? 1 : 0;
            const int grid = std::min(a.nrb, o6 * num_cus());
            void* args[] = {&a};
            CMF_HIP(hipLaunchKernel((const void*)k6, dim3(grid), dim3(1024), args, lds, st));
            return CMF_OK;
        }
    }
    a.lds = lds ? 1 : 0;
    const int threads = 64 * ks;
    auto pick = [&](int rb) -> GemvKernel {
        return w.dtype == DT_Q8ROW ? (rb == 1 ? q8_kernel(m, xm, ks) : nullptr)
               : w.dtype == DT_Q4T ? q4t_kernel(m, xm, ks, rb)
                                   : q4tp_kernel(m, xm, ks, rb);
    };
    // row blocks per workgroup (q4, LDS-staged operand): the smallest RB
    // whose grid the CUs hold at once, so that no workgroup walks its row
    // blocks one after another (CMF_GEMV_RB forces one)
    static const int rb_env = env_int("CMF_GEMV_RB", 0);
    int rb = 1;
    GemvKernel k = pick(1);
    if (!k) return fail("gemv: no kernel instance for this shape");
    int occ = resident_per_cu(k, threads, lds);
    if (occ < 1) return fail("gemv: kernel does not fit a CU (LDS or registers)");
    // m > 8 with the operand read in place (XM_GLOBAL): RB row blocks share
    // each operand read while the grid still covers every CU (the operand,
    // 2 x 16 rows of f16 planes, is read by every workgroup: q4t
    // 12288x4096 m = 16 20.0 -> 13.0 us at RB = 3; 4096x12288, 256 row
    // blocks, 19.8 -> 25.9 us, so not there)
    const bool share_rb = xm == XM_GLOBAL && m > 8;
    if (gridy == 1 && grid_override <= 0 && pick(2)) {
        for (int c = 2; c <= 3; c++) {
            const bool want = rb_env > 0 ? c == rb_env
                              : share_rb ? a.nrb >= c * num_cus()
                                         : (a.nrb + rb - 1) / rb > occ * num_cus();
            if (!want) continue;
            GemvKernel kc = pick(c);
            const int oc = kc ? resident_per_cu(kc, threads, lds) : 0;
            if (oc < 1) break;
            k = kc;
            occ = oc;
            rb = c;
        }
    }
    // grouped launches (MoE experts): two row blocks per workgroup share one
    // operand copy; measured on MI355X for the config-5 layer 56.6 -> 53.0 us
    // (3: 54.8 us).  CMF_GEMV_GRB overrides.
    static const int grb_env = env_int("CMF_GEMV_GRB", 2);
    if (gridy > 1 && grb_env > 1 && pick(grb_env)) {
        GemvKernel kc = pick(grb_env);
        const int oc = resident_per_cu(kc, threads, lds);
        if (oc >= 1) {
            k = kc;
            occ = oc;
            rb = grb_env;
        }
    }
    // one workgroup per RB row blocks while the CUs hold them all at once;
    // grouped launches always give every job its full set
    const int units = (a.nrb + rb - 1) / rb;
    int grid = gridy > 1 ? units : std::min(units, occ * num_cus());
    if (grid_override > 0) grid = std::min(grid_override, a.nrb);
    void* args[] = {&a};
    CMF_HIP(hipLaunchKernel((const void*)k, dim3(grid, gridy), dim3(threads), args, lds, st));
    return CMF_OK;
}

static GemvArgs base_args(const DevWeight& w, const XSrc& src, float* y, int ldy, int m, int row_lo, int row_hi,
                          bool resid, int epi = EPI_NONE) {
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
    a.lds = 0;
    a.src = src;
    a.jobs = nullptr;
    a.desc = nullptr;
    a.planes_stride = a.y_stride = 0;
    a.epi = epi;
    return a;
}

int gemv(const DevWeight& w, const XSrc& src, float* y, int ldy, int m, int row_lo, int row_hi,
         bool resid, hipStream_t st, int ks_override, int grid_override, int epi) {
    if (m < 1 || m > MAXB) return fail("gemv: batch must be 1..16");
    if (row_lo < 0 || row_hi > w.rows || row_lo >= row_hi) return fail("gemv: bad row range");
    if (epi == EPI_SWIGLU && (row_lo != 0 || row_hi != w.rows || w.rows % 16 || resid))
        return fail("gemv: the SwiGLU epilogue needs the whole interleaved gate/up weight, no residual");
    GemvArgs a = base_args(w, src, y, ldy, m, row_lo, row_hi, resid, epi);
    return launch_args(w, a, ks_override, grid_override, 1, st);
}

int gemv_grouped(const DevWeight& proto, const GemvDesc* desc, const int* jobs, int max_jobs,
                 const uint8_t* planes, size_t planes_stride, const float* xs, float* y, size_t y_stride,
                 int ldy, int m, hipStream_t st) {
    if (m < 1 || m > MAXB) return fail("gemv: batch must be 1..16");
    if (!desc || !jobs || max_jobs < 1 || max_jobs > 65535) return fail("gemv: bad job list");
    XSrc src{};
    src.mode = XS_GLOBAL;
    src.planes = planes;
    src.xs = xs;
    GemvArgs a = base_args(proto, src, y, ldy, m, 0, proto.rows, false);
    a.jobs = jobs;
    a.desc = desc;
    a.planes_stride = planes_stride;
    a.y_stride = y_stride;
    return launch_args(proto, a, 0, 0, max_jobs, st);
}


int gemv_a8(const DevWeight& w, const uint8_t* planes, const float* xs, const A8Out& o, float* y, int ldy, int m,
            hipStream_t st) {
    if (m < 1 || m > MAXB) return fail("gemv: batch must be 1..16");
    XSrc src{};
    src.mode = XS_GLOBAL;
    src.planes = planes;
    src.xs = xs;
    GemvArgs a = base_args(w, src, y, ldy, m, 0, w.rows, false);
    if (launch_args(w, a, 0, 0, 1, st) != CMF_OK) return CMF_ERR;
    hipLaunchKernelGGL(k_a8_outliers, dim3((w.rows + 255) / 256, m), dim3(256), 0, st, w.w, w.scale, w.rowp,
                       w.dtype, w.rows, w.kchunks, o, y, ldy);
    return CMF_OK;
}

int launch_gemv(const DevWeight& w, const uint8_t* planes, const float* xs, float* y, int ldy,
                int m, int row_lo, int row_hi, hipStream_t st, int ks_override) {
    XSrc s{};
    s.mode = XS_GLOBAL;
    s.planes = planes;
    s.xs = xs;
    return gemv(w, s, y, ldy, m, row_lo, row_hi, false, st, ks_override, 0);
}

}  // namespace cmf
