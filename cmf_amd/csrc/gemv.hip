// GEMV host side: operand preparation kernel, kernel choice and launch.
#include <map>
#include <mutex>

#include "gemv_kern.h"

namespace cmf {

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
    if (kind == 8) prep8_row(x, K, amax, nk, b, gridDim.x, planes, xs, threadIdx.x, 256);
    else prep16_row(x, K, amax, nk, b, gridDim.x, planes, xs, threadIdx.x, 256);
}

// ---------------------------------------------------------------------------
// Host launchers.
// ---------------------------------------------------------------------------
size_t prep_bytes(const DevWeight& w) {
    // at most 16 batch rows: q8 3 planes of nk*64*16 B ; q4 2 planes of ntiles*64*16 B
    // (+ q4 tile biases [tile][16] f32)
    return w.dtype == DT_Q8ROW ? (size_t)w.kchunks * 1024 * 3 : (size_t)w.kchunks * 4 * (1024 * 2 + 64);
}

int launch_prep(const DevWeight& w, const float* x, int ldx, int m, uint8_t* planes, float* xs,
                hipStream_t st) {
    const int kind = w.dtype == DT_Q8ROW ? 8 : 16;
    const int nk = w.dtype == DT_Q8ROW ? w.kchunks : w.kchunks * 4;
    hipLaunchKernelGGL(k_prep, dim3(m), dim3(256), 0, st, x, ldx, w.cols, kind, nk, planes, xs);
    return CMF_OK;
}

static size_t lds_bytes(const DevWeight& w, int m) {
    // q4: hi + lo planes and the tile biases [tile][16] f32
    return w.dtype == DT_Q8ROW ? (size_t)w.kchunks * 64 * 3 * m : (size_t)w.kchunks * 4 * (128 * m + 64);
}
// plus the f32 scratch of the in-kernel producers: the m raw rows and the
// norm weights
static size_t lds_scratch(const DevWeight& w, int m) {
    return (size_t)(w.dtype == DT_Q8ROW ? w.kchunks * 64 : w.kchunks * 128) * 4 * (m + 1);
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
                              (int)std::min<size_t>(cap, LDSX_MAX));
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
    // K steps of 1 KiB per row block: q8 chunks of 64 columns, q4 groups of
    // 4 tiles (128 columns)
    int ks = ks_override > 0 ? ks_override : pick_ks(w.kchunks);
    if (w.dtype != DT_Q8ROW && m > 8) ks = std::min(ks, 8);  // no 16-wave instance (registers)
    const bool fu = src.mode != XS_GLOBAL;
    size_t lds = lds_bytes(w, m);
    if (fu) {
        const int kpad = w.dtype == DT_Q8ROW ? w.kchunks * 64 : w.kchunks * 128;
        if (a.src.K % 4 || (src.mode != XS_CAT && src.ldx % 4) || (src.mode == XS_CAT && (src.H % 4 || src.ldx % 4)) ||
            ((uintptr_t)src.x & 15) || kpad > 4 * SEG4 * SEGMAX)
            return fail("gemv: fused operand needs K, H, ldx multiples of 4, a 16-byte aligned row base and K <= 16384");
        lds += lds_scratch(w, m);
    }
    if (lds > LDSX_MAX) {
        if (fu) return fail("gemv: activation operand exceeds LDS; prepare it globally");
        lds = 0;  // planes read in place from global memory
    }
    a.lds = lds ? 1 : 0;
    const int xm = fu ? XM_FUSED : lds ? XM_PREP : XM_GLOBAL;
    GemvKernel k = w.dtype == DT_Q8ROW ? q8_kernel(m, xm, ks)
                   : w.dtype == DT_Q4T ? q4t_kernel(m, xm, ks)
                                       : q4tp_kernel(m, xm, ks);
    if (!k) return fail("gemv: no kernel instance for this shape");
    const int threads = 64 * ks;
    const int occ = resident_per_cu(k, threads, lds);
    if (occ < 1) return fail("gemv: kernel does not fit a CU (LDS or registers)");
    int grid = std::min(a.nrb, occ * num_cus());
    if (grid_override > 0) grid = std::min(grid_override, a.nrb);
    void* args[] = {&a};
    CMF_HIP(hipLaunchKernel((const void*)k, dim3(grid), dim3(threads), args, lds, st));
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
