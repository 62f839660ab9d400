// Library runtime: errors, device/stream, weight residency (upload + repack
// into the device layouts of common.h) and the matmul seam entry points.
#include <math.h>
#include <string.h>

#include <mutex>
#include <string>
#include <vector>

#include "../../include/cmf_hip.h"
#include "common.h"
#include "gemv.h"
#include "layers.h"
#include "runtime.h"

namespace cmf {

static thread_local std::string g_err;
void set_error(const std::string& m) { g_err = m; }
int fail(const std::string& m) {
    g_err = m;
    return CMF_ERR;
}

// Workspace of cmf_gemv_dev_noalloc: the prepared operand planes of one
// GEMV (prep_bytes of a weight with cols <= 16384: q4 128 KiB-tile groups
// 1 114 112 B, q8 786 432 B) followed by the 16 per-row operand scales.
// Each device the library initialises holds its own copy until the process
// ends; calls on one device share it (the last call's contents stay).
constexpr size_t NOALLOC_PLANES_MAX = 1310720;
constexpr size_t NOALLOC_BYTES = NOALLOC_PLANES_MAX + 256;
constexpr int NOALLOC_MAX_DEV = 64;
static __device__ __align__(256) uint8_t scratch[NOALLOC_BYTES];
// device address of `scratch` per device (the host-side name is a stand-in,
// never a device address)
static uint8_t* g_scratch_ptr[NOALLOC_MAX_DEV] = {};

static std::mutex g_mu;
static bool g_init = false;
static int g_dev = 0;

// One HIP stream per host thread (the reference's GPU gate is thread-local,
// gpu.rs:18-46, 978-1000): a thread's first call makes the library's device
// current on it and creates its stream (default priority); calls of
// different threads run on their own streams with their own seam and GEMM
// scratch, and the calls on one model handle are the caller's to serialise
// (as the reference FFI's per handle).  A thread's stream and scratch stay
// until the process ends.
static thread_local hipStream_t t_stream = nullptr;
hipStream_t stream() {
    if (!t_stream && g_init) {
        if (hipSetDevice(g_dev) != hipSuccess || hipStreamCreateWithFlags(&t_stream, hipStreamNonBlocking) != hipSuccess)
            t_stream = nullptr;
    }
    return t_stream;
}
int device() { return g_dev; }

int ensure_init() {
    if (!g_init && cmf_init(0) != CMF_OK) return CMF_ERR;
    if (!stream()) return fail("no HIP stream for this thread");
    return CMF_OK;
}

static float f16_to_f32_host(uint16_t h) {
    uint32_t sign = h >> 15, exp = (h >> 10) & 0x1F, mant = h & 0x3FF, bits;
    if (exp == 0) {
        if (mant == 0) {
            bits = sign << 31;
        } else {
            uint32_t e = 0, m = mant;
            while (!(m & 0x400)) {
                m <<= 1;
                e++;
            }
            bits = (sign << 31) | ((113 - e) << 23) | ((m & 0x3FF) << 13);
        }
    } else if (exp == 0x1F) {
        bits = (sign << 31) | (0xFFu << 23) | (mant << 13);
    } else {
        bits = (sign << 31) | ((exp + 112) << 23) | (mant << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

// ---------------------------------------------------------------------------
// Repack on the host, then one upload.
// ---------------------------------------------------------------------------
static int upload_blocks(DevWeight& w, const std::vector<uint8_t>& wb, const void* sc, size_t scb,
                         const std::vector<float2>* rp) {
    CMF_HIP(hipMalloc(&w.w, wb.size()));
    CMF_HIP(hipMemcpy(w.w, wb.data(), wb.size(), hipMemcpyHostToDevice));
    CMF_HIP(hipMalloc(&w.scale, scb));
    CMF_HIP(hipMemcpy(w.scale, sc, scb, hipMemcpyHostToDevice));
    w.bytes = wb.size() + scb;
    if (rp) {
        CMF_HIP(hipMalloc(&w.rowp, rp->size() * sizeof(float2)));
        CMF_HIP(hipMemcpy(w.rowp, rp->data(), rp->size() * sizeof(float2), hipMemcpyHostToDevice));
        w.bytes += rp->size() * sizeof(float2);
    }
    w.device = g_dev;
    return CMF_OK;
}

// q8: rows of int8 (stride `cols`) + f32 row scales.  row_of(i) maps device
// row i to a source row pointer (concatenation support).
int build_q8(DevWeight& w, int rows, int cols, const int8_t* const* rowptr, const float* rs) {
    w.dtype = DT_Q8ROW;
    w.rows = rows;
    w.cols = cols;
    w.rows_pad = (rows + 15) / 16 * 16;
    w.cols_pad = (cols + 63) / 64 * 64;
    w.kchunks = w.cols_pad / 64;
    const int nrb = w.rows_pad / 16;
    std::vector<uint8_t> wb((size_t)nrb * w.kchunks * 1024, 0);
    for (int rb = 0; rb < nrb; rb++)
        for (int kc = 0; kc < w.kchunks; kc++)
            for (int s = 0; s < 4; s++)
                for (int r = 0; r < 16; r++) {
                    const int row = rb * 16 + r;
                    if (row >= rows) continue;
                    uint8_t* dst = wb.data() + (((size_t)rb * w.kchunks + kc) * 64 + 16 * s + r) * 16;
                    const int c0 = kc * 64 + 16 * s;
                    const int n = std::max(0, std::min(16, cols - c0));
                    if (n > 0) memcpy(dst, rowptr[row] + c0, n);
                }
    std::vector<float> scl(w.rows_pad, 0.f);
    memcpy(scl.data(), rs, sizeof(float) * rows);
    return upload_blocks(w, wb, scl.data(), scl.size() * sizeof(float), nullptr);
}

static int code_at(const uint8_t* codes, size_t stride, size_t g) {
    size_t bit = g * 5, b = bit / 8, sh = bit % 8;
    uint16_t lo = codes[b];
    uint16_t hi = (sh > 3 && b + 1 < stride) ? codes[b + 1] : 0;
    return (int)(((lo | (hi << 8)) >> sh) & 0x1F);
}

int build_q4(DevWeight& w, const Q4Src& src) {
    const int rows = src.rows, cols = src.cols;
    if (cols % 32) return fail("q4 tensors need cols % 32 == 0");
    w.dtype = src.dtype;
    w.rows = rows;
    w.cols = cols;
    w.rows_pad = (rows + 15) / 16 * 16;
    w.cols_pad = (cols + 127) / 128 * 128;
    w.kchunks = w.cols_pad / 128;  // groups of 4 tiles
    const int gpr = cols / 32, nrb = w.rows_pad / 16, ntg = w.kchunks;
    const bool tp = src.dtype == DT_Q4TP;
    const int tstride = tp ? 16 : 18, toff = tp ? 0 : 2;
    std::vector<uint8_t> wb((size_t)nrb * ntg * 1024, 0);
    std::vector<uint8_t> scl((size_t)nrb * ntg * (tp ? 64 : 128), 0);
    std::vector<float2> rp;
    if (tp) rp.assign(w.rows_pad, make_float2(0.f, 0.f));
    for (int row = 0; row < rows; row++) {
        const int rb = row / 16, r = row % 16;
        const uint8_t* base = src.rowbase[row];
        for (int tg = 0; tg < ntg; tg++) {
            uint32_t cw = 0;
            for (int t = 0; t < 4; t++) {
                const int tile = tg * 4 + t;
                if (tile >= gpr) continue;
                const uint8_t* tb = base + (size_t)tile * tstride;
                for (int s = 0; s < 4; s++) {
                    uint8_t* dst = wb.data() + (((size_t)rb * ntg + tg) * 64 + 16 * s + r) * 16 + 4 * t;
                    memcpy(dst, tb + toff + 4 * s, 4);
                }
                if (!tp) {
                    uint8_t* sd = scl.data() + (((size_t)rb * ntg + tg) * 16 + r) * 8 + 2 * t;
                    sd[0] = tb[0];
                    sd[1] = tb[1];
                } else {
                    cw |= (uint32_t)code_at(src.codes[row], src.code_stride, tile) << (5 * t);
                }
            }
            if (tp) memcpy(scl.data() + (((size_t)rb * ntg + tg) * 16 + r) * 4, &cw, 4);
        }
        if (tp) {
            // 2^lo and 2^step with the host libm, as q4tp_ladder (quant.rs:399-410)
            const uint8_t* p = src.params[row];
            const float lo = f16_to_f32_host((uint16_t)(p[0] | (p[1] << 8)));
            const float st = f16_to_f32_host((uint16_t)(p[2] | (p[3] << 8)));
            rp[row] = make_float2(exp2f(lo), exp2f(st));
        }
    }
    return upload_blocks(w, wb, scl.data(), scl.size(), tp ? &rp : nullptr);
}

int fill_q4src(Q4Src& s, int dtype, int rows, int cols, const uint8_t* payload, int row_offset) {
    // appends rows of one payload to s (concatenation support)
    const size_t gpr = cols / 32;
    s.dtype = dtype;
    s.cols = cols;
    if (dtype == DT_Q4T) {
        for (int r = 0; r < rows; r++) s.rowbase.push_back(payload + (size_t)r * gpr * 18);
    } else {
        const size_t nib = (size_t)rows * gpr * 16, stride = (gpr * 5 + 7) / 8;
        s.code_stride = stride;
        for (int r = 0; r < rows; r++) {
            s.rowbase.push_back(payload + (size_t)r * gpr * 16);
            s.params.push_back(payload + nib + (size_t)r * 4);
            s.codes.push_back(payload + nib + (size_t)rows * 4 + (size_t)r * stride);
        }
    }
    s.rows += rows;
    (void)row_offset;
    return CMF_OK;
}

// gate and up as one weight whose row blocks hold 8 gate rows then the 8
// matching up rows, so that the GEMV's SwiGLU epilogue sees g and u of the
// same index in one row block.
int build_swiglu(DevWeight& w, const cmf_tensor* g, const cmf_tensor* u) {
    const int dt = g->dtype, cols = g->cols, I = g->rows;
    if (u->dtype != dt || u->cols != cols || u->rows != I) return fail("gate/up must share dtype and shape");
    if (I % 8) return fail("gate/up rows must be a multiple of 8");
    if (dt == DT_Q8ROW) {
        std::vector<const int8_t*> rp;
        std::vector<float> rs;
        for (int r0 = 0; r0 < I; r0 += 8)
            for (const cmf_tensor* t : {g, u})
                for (int r = r0; r < r0 + 8; r++) {
                    rp.push_back(t->q + (size_t)r * cols);
                    rs.push_back(t->row_scale[r]);
                }
        return build_q8(w, 2 * I, cols, rp.data(), rs.data());
    }
    Q4Src sg, su, s;
    fill_q4src(sg, dt, I, cols, g->bytes, 0);
    fill_q4src(su, dt, I, cols, u->bytes, 0);
    s.dtype = dt;
    s.cols = cols;
    s.code_stride = sg.code_stride;
    for (int r0 = 0; r0 < I; r0 += 8)
        for (const Q4Src* t : {&sg, &su})
            for (int r = r0; r < r0 + 8; r++) {
                s.rowbase.push_back(t->rowbase[r]);
                if (dt == DT_Q4TP) {
                    s.codes.push_back(t->codes[r]);
                    s.params.push_back(t->params[r]);
                }
            }
    s.rows = 2 * I;
    return build_q4(w, s);
}

void free_weight(DevWeight& w) {
    if (w.w) (void)hipFree(w.w);
    if (w.scale) (void)hipFree(w.scale);
    if (w.rowp) (void)hipFree(w.rowp);
    w.w = nullptr;
    w.scale = nullptr;
    w.rowp = nullptr;
}

// Device scratch for the host-slice seam ops (grown on demand).
struct SeamScratch {
    uint8_t* planes = nullptr;
    size_t planes_cap = 0;
    float* xs = nullptr;
    float* x = nullptr;
    size_t x_cap = 0;
    float* y = nullptr;
    size_t y_cap = 0;
    float* rs = nullptr;   // caller q8 row scales [rows_pad]
    size_t rs_cap = 0;
    int* a8cnt = nullptr;  // split_act outliers of the a8w8 ops: [MAXB], [MAXB][cols]
    int* a8idx = nullptr;
    float* a8val = nullptr;
    size_t a8_cap = 0;
    float* gu = nullptr;   // cmf_ffn / cmf_moe_block_jobs: gate | up rows
    size_t gu_cap = 0;
    float* d = nullptr;    // cmf_moe_block_jobs: the jobs' down outputs
    size_t d_cap = 0;
    float* w = nullptr;    // ... their blend weights
    size_t w_cap = 0;
};
static thread_local SeamScratch g_ss;  // (per host thread, as the stream)

static int grow(void** p, size_t* cap, size_t need) {
    if (*cap >= need) return CMF_OK;
    if (*p) (void)hipFree(*p);
    *p = nullptr;
    CMF_HIP(hipMalloc(p, need));
    *cap = need;
    return CMF_OK;
}

// y (host) = w rows [row0, row0+rows) * x (host), x [b][cols].  q8 only:
// row_scale (host, rows entries for rows row0..; NULL = the upload-time
// scales) replaces the stored per-row scales, as the reference seam passes
// them with every call (gpu.rs:1104, 1155).
int seam_matmat(const DevWeight& w_in, int row0, const float* xs, int b, int rows, float* out,
                const float* row_scale) {
    if (ensure_init() != CMF_OK) return CMF_ERR;
    if (row0 < 0 || rows < 1 || row0 + rows > w_in.rows) return fail("row range outside the tensor");
    DevWeight w = w_in;
    if (row_scale) {
        if (w.dtype != DT_Q8ROW) return fail("row_scale applies to q8 weights only");
        if (grow((void**)&g_ss.rs, &g_ss.rs_cap, (size_t)w.rows_pad * sizeof(float)) != CMF_OK) return CMF_ERR;
        CMF_HIP(hipMemcpyAsync(g_ss.rs + row0, row_scale, (size_t)rows * sizeof(float), hipMemcpyHostToDevice,
                               stream()));
        w.scale = g_ss.rs;
    }
    if (grow((void**)&g_ss.planes, &g_ss.planes_cap, prep_bytes(w)) != CMF_OK) return CMF_ERR;
    if (!g_ss.xs) CMF_HIP(hipMalloc(&g_ss.xs, 64 * sizeof(float)));
    const size_t xb = (size_t)std::min(b, MAXB) * w.cols * sizeof(float);
    const size_t yb = (size_t)std::min(b, MAXB) * rows * sizeof(float);
    if (grow((void**)&g_ss.x, &g_ss.x_cap, xb) != CMF_OK) return CMF_ERR;
    if (grow((void**)&g_ss.y, &g_ss.y_cap, yb) != CMF_OK) return CMF_ERR;
    hipStream_t st = stream();
    if (b > MAXB && row0 == 0 && rows == w.rows) {
        // large batch: one MFMA GEMM pass over the weights
        const size_t xb_all = (size_t)b * w.cols * sizeof(float), yb_all = (size_t)b * rows * sizeof(float);
        if (grow((void**)&g_ss.x, &g_ss.x_cap, xb_all) != CMF_OK) return CMF_ERR;
        if (grow((void**)&g_ss.y, &g_ss.y_cap, yb_all) != CMF_OK) return CMF_ERR;
        CMF_HIP(hipMemcpyAsync(g_ss.x, xs, xb_all, hipMemcpyHostToDevice, st));
        if (gemm_q4(w, g_ss.x, w.cols, b, g_ss.y, rows, st) != CMF_OK) return CMF_ERR;
        CMF_HIP(hipMemcpyAsync(out, g_ss.y, yb_all, hipMemcpyDeviceToHost, st));
        CMF_HIP(hipStreamSynchronize(st));
        CMF_HIP(hipGetLastError());
        return CMF_OK;
    }
    for (int b0 = 0; b0 < b; b0 += MAXB) {
        const int m = std::min(MAXB, b - b0);
        CMF_HIP(hipMemcpyAsync(g_ss.x, xs + (size_t)b0 * w.cols, (size_t)m * w.cols * sizeof(float),
                               hipMemcpyHostToDevice, st));
        int ks1 = 0;
        if (m == 1 && w.dtype == DT_Q4T && q4t_kernel_m1x(w.kchunks, false, &ks1)) {
            // one launch: the kernel stages its operand from the f32 row
            XSrc src{};
            src.mode = XS_ROWS;
            src.x = g_ss.x;
            src.ldx = w.cols;
            if (gemv(w, src, g_ss.y, rows, 1, row0, row0 + rows, false, st) != CMF_OK) return CMF_ERR;
        } else {
            launch_prep(w, g_ss.x, w.cols, m, g_ss.planes, g_ss.xs, st);
            if (launch_gemv(w, g_ss.planes, g_ss.xs, g_ss.y, rows, m, row0, row0 + rows, st) != CMF_OK)
                return CMF_ERR;
        }
        CMF_HIP(hipMemcpyAsync(out + (size_t)b0 * rows, g_ss.y, (size_t)m * rows * sizeof(float),
                               hipMemcpyDeviceToHost, st));
    }
    CMF_HIP(hipStreamSynchronize(st));
    CMF_HIP(hipGetLastError());
    return CMF_OK;
}

}  // namespace cmf

using namespace cmf;

struct cmf_weight_s {
    DevWeight w;
};

extern "C" {

const char* cmf_last_error(void) { return g_err.c_str(); }

int cmf_device_count(void) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) return 0;
    return n;
}

int cmf_init(int dev) {
    std::lock_guard<std::mutex> lk(g_mu);
    if (g_init) return CMF_OK;
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n == 0) return fail("no HIP device visible");
    if (dev < 0 || dev >= n) return fail("device index out of range");
    CMF_HIP(hipSetDevice(dev));
    hipDeviceProp_t p;
    CMF_HIP(hipGetDeviceProperties(&p, dev));
    if (strncmp(p.gcnArchName, "gfx950", 6) != 0)
        return fail(std::string("libcmfhip is built for gfx950, device is ") + p.gcnArchName);
    if (dev < NOALLOC_MAX_DEV) {
        // this device's copy of the no-allocation workspace (device current)
        const hipError_t e = hipGetSymbolAddress((void**)&g_scratch_ptr[dev], HIP_SYMBOL(scratch));
        if (e != hipSuccess) {
            g_scratch_ptr[dev] = nullptr;
            return fail(std::string("hipGetSymbolAddress(scratch): ") + hipGetErrorString(e));
        }
    }
    g_dev = dev;
    g_init = true;
    if (!stream()) return fail("cmf_init: stream creation failed");
    return CMF_OK;
}

int cmf_sync(void) {
    if (!g_init) return fail("cmf_init not called");
    CMF_HIP(hipStreamSynchronize(stream()));
    return CMF_OK;
}

int cmf_weight_upload(const uint8_t* payload, size_t nbytes, int dtype, int rows, int cols,
                      cmf_weight* out) {
    if (ensure_init() != CMF_OK) return CMF_ERR;
    if (!payload || !out || rows < 1 || cols < 1) return fail("weight_upload: bad arguments");
    auto* h = new cmf_weight_s();
    int rc;
    if (dtype == DT_Q8ROW) {
        if (nbytes < (size_t)rows * cols + (size_t)rows * 2) {
            delete h;
            return fail("q8 payload too short");
        }
        std::vector<const int8_t*> rp(rows);
        std::vector<float> rs(rows);
        for (int r = 0; r < rows; r++) {
            rp[r] = (const int8_t*)payload + (size_t)r * cols;
            const uint8_t* s = payload + (size_t)rows * cols + 2 * (size_t)r;
            rs[r] = f16_to_f32_host((uint16_t)(s[0] | (s[1] << 8)));
        }
        rc = build_q8(h->w, rows, cols, rp.data(), rs.data());
    } else if (dtype == DT_Q4T || dtype == DT_Q4TP) {
        if (cols % 32) {
            delete h;
            return fail("q4 tensors need cols % 32 == 0");
        }
        const size_t gpr = cols / 32;
        const size_t need = dtype == DT_Q4T ? (size_t)rows * gpr * 18
                                            : (size_t)rows * gpr * 16 + (size_t)rows * 4 +
                                                  (size_t)rows * ((gpr * 5 + 7) / 8);
        if (nbytes < need) {
            delete h;
            return fail("q4 payload too short");
        }
        Q4Src s;
        s.rows = 0;
        fill_q4src(s, dtype, rows, cols, payload, 0);
        rc = build_q4(h->w, s);
    } else {
        delete h;
        return CMF_DECLINED;
    }
    if (rc != CMF_OK) {
        free_weight(h->w);
        delete h;
        return rc;
    }
    *out = h;
    return CMF_OK;
}

int cmf_weight_upload_q8(const int8_t* q, const float* rs, int rows, int cols, cmf_weight* out) {
    if (ensure_init() != CMF_OK) return CMF_ERR;
    if (!q || !rs || !out || rows < 1 || cols < 1) return fail("weight_upload_q8: bad arguments");
    auto* h = new cmf_weight_s();
    std::vector<const int8_t*> rp(rows);
    for (int r = 0; r < rows; r++) rp[r] = q + (size_t)r * cols;
    int rc = build_q8(h->w, rows, cols, rp.data(), rs);
    if (rc != CMF_OK) {
        free_weight(h->w);
        delete h;
        return rc;
    }
    *out = h;
    return CMF_OK;
}

int cmf_weight_free(cmf_weight w) {
    if (!w) return CMF_OK;
    free_weight(w->w);
    delete w;
    return CMF_OK;
}

size_t cmf_weight_device_bytes(cmf_weight w) { return w ? w->w.bytes : 0; }

// y[b][rows] = W x[b] under the a8w8 contract (split_act operand, integer
// tile dots, outliers exact), batches of 16.
static int seam_matmat_a8(const DevWeight& w, const float* xs, int b, float* out) {
    if (ensure_init() != CMF_OK) return CMF_ERR;
    const int rows = w.rows, cols = w.cols;
    if (grow((void**)&g_ss.planes, &g_ss.planes_cap, prep_bytes(w)) != CMF_OK) return CMF_ERR;
    if (!g_ss.xs) CMF_HIP(hipMalloc(&g_ss.xs, 64 * sizeof(float)));
    if (grow((void**)&g_ss.x, &g_ss.x_cap, (size_t)MAXB * cols * sizeof(float)) != CMF_OK) return CMF_ERR;
    if (grow((void**)&g_ss.y, &g_ss.y_cap, (size_t)MAXB * rows * sizeof(float)) != CMF_OK) return CMF_ERR;
    if (!g_ss.a8cnt) CMF_HIP(hipMalloc(&g_ss.a8cnt, MAXB * sizeof(int)));
    if ((size_t)cols > g_ss.a8_cap) {
        if (g_ss.a8idx) (void)hipFree(g_ss.a8idx);
        if (g_ss.a8val) (void)hipFree(g_ss.a8val);
        g_ss.a8idx = nullptr;
        g_ss.a8val = nullptr;
        g_ss.a8_cap = 0;
        CMF_HIP(hipMalloc(&g_ss.a8idx, (size_t)MAXB * cols * sizeof(int)));
        CMF_HIP(hipMalloc(&g_ss.a8val, (size_t)MAXB * cols * sizeof(float)));
        g_ss.a8_cap = cols;
    }
    const A8Out o{g_ss.a8cnt, g_ss.a8idx, g_ss.a8val, (int)g_ss.a8_cap};
    hipStream_t st = stream();
    for (int b0 = 0; b0 < b; b0 += MAXB) {
        const int m = std::min(MAXB, b - b0);
        CMF_HIP(hipMemcpyAsync(g_ss.x, xs + (size_t)b0 * cols, (size_t)m * cols * sizeof(float), hipMemcpyHostToDevice,
                               st));
        if (launch_prep_a8(w, g_ss.x, cols, m, g_ss.planes, g_ss.xs, o, st) != CMF_OK) return CMF_ERR;
        if (gemv_a8(w, g_ss.planes, g_ss.xs, o, g_ss.y, rows, m, st) != CMF_OK) return CMF_ERR;
        CMF_HIP(hipMemcpyAsync(out + (size_t)b0 * rows, g_ss.y, (size_t)m * rows * sizeof(float),
                               hipMemcpyDeviceToHost, st));
    }
    CMF_HIP(hipStreamSynchronize(st));
    CMF_HIP(hipGetLastError());
    return CMF_OK;
}

static int seam(cmf_weight w, int dt, int row0, const float* xs, int b, int rows, int cols,
                float* out, const float* row_scale = nullptr) {
    if (!w || !xs || !out) return fail("null argument");
    if (w->w.dtype != dt) return CMF_DECLINED;  // not this codec: caller's CPU path
    if (cols != w->w.cols) return fail("cols mismatch");
    return seam_matmat(w->w, row0, xs, b, rows, out, row_scale);
}

int cmf_matmat_a8w8(cmf_weight w, const float* xs, int b, float* out) {
    if (!w || !xs || !out || b < 1) return fail("null argument or empty batch");
    return seam_matmat_a8(w->w, xs, b, out);
}

int cmf_q8_matvec_range(cmf_weight w, int row0, const float* row_scale, const float* xs, int rows, int cols,
                        float* out) {
    return seam(w, DT_Q8ROW, row0, xs, 1, rows, cols, out, row_scale);
}
int cmf_q8_matmat(cmf_weight w, const float* row_scale, const float* xs, int b, int rows, int cols, float* out) {
    return seam(w, DT_Q8ROW, 0, xs, b, rows, cols, out, row_scale);
}
int cmf_q4t_matvec(cmf_weight w, const float* xs, int rows, int cols, float* out) {
    return seam(w, DT_Q4T, 0, xs, 1, rows, cols, out);
}
int cmf_q4t_matmat(cmf_weight w, const float* xs, int b, int rows, int cols, float* out) {
    return seam(w, DT_Q4T, 0, xs, b, rows, cols, out);
}
int cmf_q4tp_matvec(cmf_weight w, const float* xs, int rows, int cols, float* out) {
    return seam(w, DT_Q4TP, 0, xs, 1, rows, cols, out);
}
int cmf_q4tp_matmat(cmf_weight w, const float* xs, int b, int rows, int cols, float* out) {
    return seam(w, DT_Q4TP, 0, xs, b, rows, cols, out);
}

int cmf_ffn(cmf_weight w1, cmf_weight w3, cmf_weight w2, const float* xs, int b, int hidden,
            int inter, float* out) {
    if (ensure_init() != CMF_OK) return CMF_ERR;
    if (!w1 || !w3 || !w2 || !xs || !out) return fail("null argument");
    if (w1->w.rows != inter || w3->w.rows != inter || w1->w.cols != hidden || w3->w.cols != hidden ||
        w2->w.rows != hidden || w2->w.cols != inter)
        return fail("ffn: shape mismatch");
    if (w1->w.dtype != w3->w.dtype) return CMF_DECLINED;
    hipStream_t st = stream();
    // device buffers (the thread's grow-only seam scratch): x [m][hidden],
    // g/u [m][2*inter], planes, out [m][hidden]
    const size_t pb = std::max(prep_bytes(w1->w), prep_bytes(w2->w));
    if (grow((void**)&g_ss.x, &g_ss.x_cap, (size_t)MAXB * hidden * sizeof(float)) != CMF_OK ||
        grow((void**)&g_ss.gu, &g_ss.gu_cap, (size_t)MAXB * 2 * inter * sizeof(float)) != CMF_OK ||
        grow((void**)&g_ss.y, &g_ss.y_cap, (size_t)MAXB * hidden * sizeof(float)) != CMF_OK ||
        grow((void**)&g_ss.planes, &g_ss.planes_cap, pb) != CMF_OK)
        return CMF_ERR;
    if (!g_ss.xs) CMF_HIP(hipMalloc(&g_ss.xs, 64 * sizeof(float)));
    float *dx = g_ss.x, *dgu = g_ss.gu, *dy = g_ss.y, *dxs = g_ss.xs;
    uint8_t* pl = g_ss.planes;
    int rc = CMF_OK;
    for (int b0 = 0; b0 < b && rc == CMF_OK; b0 += MAXB) {
        const int m = std::min(MAXB, b - b0);
        CMF_HIP(hipMemcpyAsync(dx, xs + (size_t)b0 * hidden, (size_t)m * hidden * 4, hipMemcpyHostToDevice, st));
        launch_prep(w1->w, dx, hidden, m, pl, dxs, st);
        rc = launch_gemv(w1->w, pl, dxs, dgu, 2 * inter, m, 0, inter, st);
        if (rc == CMF_OK) rc = launch_gemv(w3->w, pl, dxs, dgu + inter, 2 * inter, m, 0, inter, st);
        if (rc != CMF_OK) break;
        XSrc sg{};
        sg.mode = XS_SILU;
        sg.x = dgu;
        sg.ldx = 2 * inter;
        sg.K = inter;
        rc = launch_prep_src(w2->w, sg, m, pl, dxs, st);
        if (rc != CMF_OK) break;
        rc = launch_gemv(w2->w, pl, dxs, dy, hidden, m, 0, hidden, st);
        if (rc != CMF_OK) break;
        CMF_HIP(hipMemcpyAsync(out + (size_t)b0 * hidden, dy, (size_t)m * hidden * 4, hipMemcpyDeviceToHost, st));
    }
    CMF_HIP(hipStreamSynchronize(st));
    if (rc == CMF_OK) CMF_HIP(hipGetLastError());
    return rc;
}

}  // extern "C"

namespace cmf {
// y[i] = sum_j w_j d_j[i] over the jobs in order, from 0, one rounded
// multiply and one rounded add per term (acc += w * d of moe_ffn_cpu,
// pipeline.rs:11017-11030, and of the device block's y += w * d).
__global__ void k_combine_jobs(const float* __restrict__ d, const float* __restrict__ w, int njobs, int n,
                               float* __restrict__ y) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    float acc = 0.f;
    for (int j = 0; j < njobs; j++) acc = __fadd_rn(acc, __fmul_rn(w[j], d[(size_t)j * n + i]));
    y[i] = acc;
}

// q8 weights with caller scales: a view whose scale array holds them (rows
// [0, rows) of a [rows_pad] buffer).
static int with_scales(DevWeight& v, const float* row_scale, float* dbuf, hipStream_t st) {
    if (!row_scale) return CMF_OK;
    if (v.dtype != DT_Q8ROW) return fail("row_scale applies to q8 weights only");
    CMF_HIP(hipMemcpyAsync(dbuf, row_scale, (size_t)v.rows * sizeof(float), hipMemcpyHostToDevice, st));
    v.scale = dbuf;
    return CMF_OK;
}
}  // namespace cmf

extern "C" {

int cmf_moe_block_jobs(const cmf_moe_job* jobs, int njobs, float* out) {
    if (ensure_init() != CMF_OK) return CMF_ERR;
    if (!jobs || !out || njobs < 1) return fail("moe_block_jobs: null argument or no jobs");
    // refusals of gpu.rs:814-841 / gpu_wgpu.rs moe_block: the whole block
    // goes back to the caller's CPU path, nothing written
    const int kind = jobs[0].q4tp ? 2 : (jobs[0].q4t ? 1 : 0);
    for (int j = 0; j < njobs; j++) {
        const cmf_moe_job& J = jobs[j];
        if (J.q1 || J.gu_q2 || J.swiglu_limit != 0.0f || J.down_col) return CMF_DECLINED;
        if (J.q4t && J.q4tp) return CMF_DECLINED;
        if ((J.q4tp ? 2 : (J.q4t ? 1 : 0)) != kind) return CMF_DECLINED;
        if (!J.gate || !J.up || !J.down || !J.xs_gate || !J.xs_up) return fail("moe_block_jobs: null job field");
        const int want = kind == 2 ? DT_Q4TP : (kind == 1 ? DT_Q4T : DT_Q8ROW);
        if (J.gate->w.dtype != want || J.up->w.dtype != want || J.down->w.dtype != want) return CMF_DECLINED;
    }
    const int inter = jobs[0].gate->w.rows, hidden = jobs[0].down->w.rows, cols = jobs[0].gate->w.cols;
    for (int j = 0; j < njobs; j++) {
        const cmf_moe_job& J = jobs[j];
        if (J.gate->w.rows != inter || J.up->w.rows != inter || J.gate->w.cols != cols || J.up->w.cols != cols ||
            J.down->w.cols != inter || J.down->w.rows != hidden)
            return fail("moe_block_jobs: every trio must share gate/up [inter x cols] and down [hidden x inter]");
    }
    hipStream_t st = stream();
    // device staging: xs [2 njobs][cols], gate|up [2 inter], d [njobs][hidden],
    // weights, y, caller scales (3 x rows_pad), planes, xs scales
    const size_t pb = std::max(prep_bytes(jobs[0].gate->w), prep_bytes(jobs[0].down->w));
    const size_t rsn = (size_t)std::max(jobs[0].gate->w.rows_pad, jobs[0].down->w.rows_pad);
    // (the thread's grow-only seam scratch)
    if (grow((void**)&g_ss.x, &g_ss.x_cap, (size_t)2 * njobs * cols * 4) != CMF_OK ||
        grow((void**)&g_ss.gu, &g_ss.gu_cap, (size_t)2 * inter * 4) != CMF_OK ||
        grow((void**)&g_ss.d, &g_ss.d_cap, (size_t)njobs * hidden * 4) != CMF_OK ||
        grow((void**)&g_ss.w, &g_ss.w_cap, (size_t)njobs * 4) != CMF_OK ||
        grow((void**)&g_ss.y, &g_ss.y_cap, (size_t)hidden * 4) != CMF_OK ||
        grow((void**)&g_ss.rs, &g_ss.rs_cap, 3 * rsn * 4) != CMF_OK ||
        grow((void**)&g_ss.planes, &g_ss.planes_cap, pb) != CMF_OK)
        return CMF_ERR;
    if (!g_ss.xs) CMF_HIP(hipMalloc(&g_ss.xs, 64 * sizeof(float)));
    float *dx = g_ss.x, *dgu = g_ss.gu, *dd = g_ss.d, *dw = g_ss.w, *dy = g_ss.y, *drs = g_ss.rs, *dxs = g_ss.xs;
    uint8_t* pl = g_ss.planes;
    int rc = CMF_OK;
    std::vector<float> ws(njobs);
    for (int j = 0; j < njobs && rc == CMF_OK; j++) {
        const cmf_moe_job& J = jobs[j];
        ws[j] = J.w;
        if (hipMemcpyAsync(dx + (size_t)(2 * j) * cols, J.xs_gate, (size_t)cols * 4, hipMemcpyHostToDevice, st) ||
            hipMemcpyAsync(dx + (size_t)(2 * j + 1) * cols, J.xs_up, (size_t)cols * 4, hipMemcpyHostToDevice, st))
            rc = fail("moe_block_jobs: upload failed");
        DevWeight g = J.gate->w, u = J.up->w, d = J.down->w;
        if (rc == CMF_OK) rc = with_scales(g, J.gate_row_scale, drs, st);
        if (rc == CMF_OK) rc = with_scales(u, J.up_row_scale, drs + rsn, st);
        if (rc == CMF_OK) rc = with_scales(d, J.down_row_scale, drs + 2 * rsn, st);
        if (rc != CMF_OK) break;
        // g = W_g xs_gate, u = W_u xs_up, a = silu(g) * u, d_j = W_d a
        launch_prep(g, dx + (size_t)(2 * j) * cols, cols, 1, pl, dxs, st);
        rc = launch_gemv(g, pl, dxs, dgu, inter, 1, 0, inter, st);
        if (rc != CMF_OK) break;
        launch_prep(u, dx + (size_t)(2 * j + 1) * cols, cols, 1, pl, dxs, st);
        rc = launch_gemv(u, pl, dxs, dgu + inter, inter, 1, 0, inter, st);
        if (rc != CMF_OK) break;
        XSrc sg{};
        sg.mode = XS_SILU;
        sg.x = dgu;
        sg.ldx = 2 * inter;
        sg.K = inter;
        rc = launch_prep_src(d, sg, 1, pl, dxs, st);
        if (rc == CMF_OK) rc = launch_gemv(d, pl, dxs, dd + (size_t)j * hidden, hidden, 1, 0, hidden, st);
        // the scale staging is reused by the next job: wait for this one
        if (rc == CMF_OK && (J.gate_row_scale || J.up_row_scale || J.down_row_scale) &&
            hipStreamSynchronize(st) != hipSuccess)
            rc = fail("moe_block_jobs: stream error");
    }
    if (rc == CMF_OK) {
        if (hipMemcpyAsync(dw, ws.data(), (size_t)njobs * 4, hipMemcpyHostToDevice, st) != hipSuccess)
            rc = fail("moe_block_jobs: upload failed");
        hipLaunchKernelGGL(k_combine_jobs, dim3((hidden + 255) / 256), dim3(256), 0, st, dd, dw, njobs, hidden, dy);
        if (rc == CMF_OK &&
            hipMemcpyAsync(out, dy, (size_t)hidden * 4, hipMemcpyDeviceToHost, st) != hipSuccess)
            rc = fail("moe_block_jobs: download failed");
    }
    (void)hipStreamSynchronize(st);
    if (rc == CMF_OK) CMF_HIP(hipGetLastError());
    return rc;
}

int cmf_matvec_batch(const cmf_batch_job* jobs, int njobs, float* const* outs) {
    if (ensure_init() != CMF_OK) return CMF_ERR;
    if (!jobs || !outs || njobs < 1) return fail("matvec_batch: null argument or no jobs");
    // validate every job first: a refusal writes nothing (gpu.rs:1-12)
    size_t pb = 0, ymax = 0, xmax = 0;
    for (int j = 0; j < njobs; j++) {
        const cmf_batch_job& J = jobs[j];
        if (!J.w || !J.xs || !outs[j]) return fail("matvec_batch: null job field");
        if (J.layout != DT_Q8ROW && J.layout != DT_Q4T && J.layout != DT_Q4TP) return CMF_DECLINED;  // Q1
        if (J.w->w.dtype != J.layout) return CMF_DECLINED;
        if (J.rows != J.w->w.rows || J.cols != J.w->w.cols) return fail("matvec_batch: job shape != weight shape");
        if (J.row_scale && J.layout != DT_Q8ROW) return fail("matvec_batch: row_scale applies to q8 jobs only");
        pb = std::max(pb, prep_bytes(J.w->w));
        ymax = std::max(ymax, (size_t)J.w->w.rows_pad);
        xmax = std::max(xmax, (size_t)J.cols);
    }
    hipStream_t st = stream();
    if (grow((void**)&g_ss.planes, &g_ss.planes_cap, pb) != CMF_OK) return CMF_ERR;
    if (!g_ss.xs) CMF_HIP(hipMalloc(&g_ss.xs, 64 * sizeof(float)));
    if (grow((void**)&g_ss.x, &g_ss.x_cap, xmax * 4) != CMF_OK) return CMF_ERR;
    if (grow((void**)&g_ss.y, &g_ss.y_cap, ymax * 4) != CMF_OK) return CMF_ERR;
    if (grow((void**)&g_ss.rs, &g_ss.rs_cap, ymax * 4) != CMF_OK) return CMF_ERR;
    for (int j = 0; j < njobs; j++) {
        const cmf_batch_job& J = jobs[j];
        DevWeight w = J.w->w;
        if (with_scales(w, J.row_scale, g_ss.rs, st) != CMF_OK) return CMF_ERR;
        CMF_HIP(hipMemcpyAsync(g_ss.x, J.xs, (size_t)J.cols * 4, hipMemcpyHostToDevice, st));
        launch_prep(w, g_ss.x, J.cols, 1, g_ss.planes, g_ss.xs, st);
        const int rc = launch_gemv(w, g_ss.planes, g_ss.xs, g_ss.y, J.rows, 1, 0, J.rows, st);
        if (rc != CMF_OK) return rc;
        CMF_HIP(hipMemcpyAsync(outs[j], g_ss.y, (size_t)J.rows * 4, hipMemcpyDeviceToHost, st));
        CMF_HIP(hipStreamSynchronize(st));  // the staging is reused by the next job
    }
    CMF_HIP(hipGetLastError());
    return CMF_OK;
}

void* cmf_dev_alloc(size_t bytes) {
    if (ensure_init() != CMF_OK) return nullptr;
    void* p = nullptr;
    if (hipMalloc(&p, bytes) != hipSuccess) {
        set_error("hipMalloc failed");
        return nullptr;
    }
    return p;
}
int cmf_dev_free(void* p) {
    if (p) CMF_HIP(hipFree(p));
    return CMF_OK;
}
int cmf_h2d(void* d, const void* s, size_t n) {
    CMF_HIP(hipMemcpy(d, s, n, hipMemcpyHostToDevice));
    return CMF_OK;
}
int cmf_d2h(void* d, const void* s, size_t n) {
    CMF_HIP(hipMemcpy(d, s, n, hipMemcpyDeviceToHost));
    return CMF_OK;
}

size_t cmf_prep_bytes(cmf_weight w) { return w ? prep_bytes(w->w) : 0; }

int cmf_prep_dev(cmf_weight w, const float* d_x, int ldx, int b, void* d_planes, float* d_xs) {
    if (ensure_init() != CMF_OK) return CMF_ERR;
    if (!w || b < 1 || b > MAXB) return fail("prep_dev: bad arguments");
    launch_prep(w->w, d_x, ldx, b, (uint8_t*)d_planes, d_xs, stream());
    CMF_HIP(hipGetLastError());
    return CMF_OK;
}

int cmf_gemv_dev_noalloc(cmf_weight w, const float* d_x, int ldx, int b, float* d_y, int ldy) {
    if (!g_init) return fail("gemv_dev_noalloc: call cmf_init first");
    if (!w || !d_x || !d_y) return fail("gemv_dev_noalloc: null argument");
    if (b < 1 || b > MAXB) return fail("gemv_dev_noalloc: batch must be 1..16");
    if (ldx < w->w.cols || ldy < w->w.rows) return fail("gemv_dev_noalloc: ldx < cols or ldy < rows");
    const size_t need = prep_bytes(w->w);
    if (need > NOALLOC_PLANES_MAX)
        return fail("gemv_dev_noalloc: the operand of this weight needs " + std::to_string(need) +
                    " B of workspace, more than the " + std::to_string(NOALLOC_PLANES_MAX) +
                    " B the library holds (cols <= 16384)");
    uint8_t* base = g_dev < NOALLOC_MAX_DEV ? g_scratch_ptr[g_dev] : nullptr;
    if (!base) return fail("gemv_dev_noalloc: no workspace on this device");
    float* xs = (float*)(base + NOALLOC_PLANES_MAX);
    hipStream_t st = stream();
    int rc = launch_prep(w->w, d_x, ldx, b, base, xs, st);
    if (rc != CMF_OK) return rc;
    rc = launch_gemv(w->w, base, xs, d_y, ldy, b, 0, w->w.rows, st);
    if (rc != CMF_OK) return rc;
    CMF_HIP(hipGetLastError());
    return CMF_OK;
}

int cmf_gemv_prepared(cmf_weight w, const void* d_planes, const float* d_xs, int b, float* d_y,
                      int ldy, int ks) {
    if (ensure_init() != CMF_OK) return CMF_ERR;
    if (!w) return fail("null weight");
    int rc = launch_gemv(w->w, (const uint8_t*)d_planes, d_xs, d_y, ldy, b, 0, w->w.rows, stream(), ks);
    if (rc != CMF_OK) return rc;
    CMF_HIP(hipGetLastError());
    return CMF_OK;
}

}  // extern "C"

namespace cmf {
typedef int int4v_rt __attribute__((ext_vector_type(4)));
// Busy-wait ~`ticks` of the constant-rate wall clock (bounded: also exits
// after `max_iter` polls), so that launches enqueued behind it leave the
// device queue full and back-to-back timing sees no host gaps.
__global__ void k_spin(unsigned long long ticks, int max_iter) {
    const unsigned long long t0 = wall_clock64();
    for (int i = 0; i < max_iter; i++) {
        if (wall_clock64() - t0 >= ticks) break;
        __builtin_amdgcn_s_sleep(2);
    }
}
// Plain copy, 16 bytes per lane per step (the calibration kernel of the
// HBM traffic counters).
__global__ __launch_bounds__(256) void k_copy16(const uint4* __restrict__ src, uint4* __restrict__ dst, size_t n) {
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) dst[i] = src[i];
}
// Plain read with the M = 1 GEMV's structure: workgroups of 8 waves, each
// wave requesting 4 KiB (four 1 KiB steps, 16 bytes per lane) at once; the
// words are folded so that the loads cannot be dropped.
__global__ __launch_bounds__(512) void k_read32k(const int4v_rt* __restrict__ src, uint32_t* __restrict__ sink) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const size_t base = ((size_t)blockIdx.x * 8 + wave) * 4 * 64 + lane;
    int4v_rt v[4];
#pragma unroll
    for (int u = 0; u < 4; u++) v[u] = __builtin_nontemporal_load(src + base + u * 64);
    uint32_t x = 0;
#pragma unroll
    for (int u = 0; u < 4; u++) x ^= (uint32_t)(v[u].x ^ v[u].y ^ v[u].z ^ v[u].w);
    if (x == 0x9E3779B9u) sink[0] = x;  // (practically never: keeps the loads)
}
}  // namespace cmf

extern "C" {

int cmf_time_read(size_t bytes, int nbuf, int iters, float* avg_ms) {
    if (ensure_init() != CMF_OK) return CMF_ERR;
    if (bytes < 32768 || bytes % 32768 || nbuf < 1 || nbuf > 64 || iters < 1 || !avg_ms)
        return fail("time_read: bytes must be a positive multiple of 32768, 1 <= nbuf <= 64, iters >= 1");
    hipStream_t st = stream();
    std::vector<void*> src(nbuf, nullptr);
    uint32_t* sink = nullptr;
    int rc = CMF_OK;
    for (auto& p : src)
        if (hipMalloc(&p, bytes) != hipSuccess || hipMemsetAsync(p, 1, bytes, st) != hipSuccess) rc = fail("time_read: allocation failed");
    if (rc == CMF_OK && hipMalloc(&sink, 64) != hipSuccess) rc = fail("time_read: allocation failed");
    hipEvent_t e0 = nullptr, e1 = nullptr;
    if (rc == CMF_OK && (hipEventCreate(&e0) != hipSuccess || hipEventCreate(&e1) != hipSuccess)) rc = fail("time_read: event");
    if (rc == CMF_OK) {
        const int grid = (int)(bytes / 32768);
        for (int i = 0; i < 20; i++)
            hipLaunchKernelGGL(k_read32k, dim3(grid), dim3(512), 0, st, (const int4v_rt*)src[i % nbuf], sink);
        int rate_khz = 100000;
        (void)hipDeviceGetAttribute(&rate_khz, hipDeviceAttributeWallClockRate, g_dev);
        hipLaunchKernelGGL(k_spin, dim3(1), dim3(64), 0, st, (unsigned long long)rate_khz * 5, 1 << 22);
        (void)hipEventRecord(e0, st);
        for (int i = 0; i < iters; i++)
            hipLaunchKernelGGL(k_read32k, dim3(grid), dim3(512), 0, st, (const int4v_rt*)src[i % nbuf], sink);
        (void)hipEventRecord(e1, st);
        float ms = 0.f;
        if (hipEventSynchronize(e1) != hipSuccess || hipEventElapsedTime(&ms, e0, e1) != hipSuccess) rc = fail("time_read: timing");
        *avg_ms = ms / iters;
    }
    if (e0) (void)hipEventDestroy(e0);
    if (e1) (void)hipEventDestroy(e1);
    (void)hipStreamSynchronize(st);
    for (auto p : src)
        if (p) (void)hipFree(p);
    if (sink) (void)hipFree(sink);
    if (rc == CMF_OK) CMF_HIP(hipGetLastError());
    return rc;
}

int cmf_time_copy(size_t bytes, int nbuf, int iters, float* avg_ms) {
    if (ensure_init() != CMF_OK) return CMF_ERR;
    if (bytes < 16 || bytes % 16 || nbuf < 1 || nbuf > 64 || iters < 1 || !avg_ms)
        return fail("time_copy: bytes must be a positive multiple of 16, 1 <= nbuf <= 64, iters >= 1");
    hipStream_t st = stream();
    std::vector<void*> src(nbuf, nullptr);
    void* dst = nullptr;
    int rc = CMF_OK;
    for (auto& p : src)
        if (hipMalloc(&p, bytes) != hipSuccess || hipMemsetAsync(p, 1, bytes, st) != hipSuccess) rc = fail("time_copy: allocation failed");
    if (rc == CMF_OK && hipMalloc(&dst, bytes) != hipSuccess) rc = fail("time_copy: allocation failed");
    hipEvent_t e0 = nullptr, e1 = nullptr;
    if (rc == CMF_OK && (hipEventCreate(&e0) != hipSuccess || hipEventCreate(&e1) != hipSuccess)) rc = fail("time_copy: event");
    if (rc == CMF_OK) {
        const size_t n = bytes / 16;
        const int grid = (int)std::min<size_t>((n + 255) / 256, 8192);
        for (int i = 0; i < std::min(iters, 4); i++)
            hipLaunchKernelGGL(k_copy16, dim3(grid), dim3(256), 0, st, (const uint4*)src[i % nbuf], (uint4*)dst, n);
        (void)hipEventRecord(e0, st);
        for (int i = 0; i < iters; i++)
            hipLaunchKernelGGL(k_copy16, dim3(grid), dim3(256), 0, st, (const uint4*)src[i % nbuf], (uint4*)dst, n);
        (void)hipEventRecord(e1, st);
        float ms = 0.f;
        if (hipEventSynchronize(e1) != hipSuccess || hipEventElapsedTime(&ms, e0, e1) != hipSuccess) rc = fail("time_copy: timing");
        *avg_ms = ms / iters;
    }
    if (e0) (void)hipEventDestroy(e0);
    if (e1) (void)hipEventDestroy(e1);
    (void)hipStreamSynchronize(st);
    for (auto p : src)
        if (p) (void)hipFree(p);
    if (dst) (void)hipFree(dst);
    if (rc == CMF_OK) CMF_HIP(hipGetLastError());
    return rc;
}

int cmf_time_gemm(cmf_weight w, const float* d_x, int m, float* d_y, int warmup, int iters, float* avg_ms) {
    if (ensure_init() != CMF_OK) return CMF_ERR;
    if (!w || !d_x || !d_y || m < 1 || iters < 1 || warmup < 0 || !avg_ms) return fail("time_gemm: bad arguments");
    hipStream_t st = stream();
    for (int i = 0; i < warmup; i++)
        if (gemm_q4(w->w, d_x, w->w.cols, m, d_y, w->w.rows, st) != CMF_OK) return CMF_ERR;
    hipEvent_t e0, e1;
    CMF_HIP(hipEventCreate(&e0));
    CMF_HIP(hipEventCreate(&e1));
    CMF_HIP(hipEventRecord(e0, st));
    int rc = CMF_OK;
    for (int i = 0; i < iters && rc == CMF_OK; i++) rc = gemm_q4(w->w, d_x, w->w.cols, m, d_y, w->w.rows, st);
    CMF_HIP(hipEventRecord(e1, st));
    CMF_HIP(hipEventSynchronize(e1));
    float ms = 0.f;
    CMF_HIP(hipEventElapsedTime(&ms, e0, e1));
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    *avg_ms = ms / iters;
    return rc;
}

int cmf_time_gemv(const cmf_weight* ws, int nw, const void* d_planes, const float* d_xs, int b,
                  float* d_y, int ldy, int ks, int warmup, int iters, float* avg_ms) {
    if (ensure_init() != CMF_OK) return CMF_ERR;
    if (!ws || nw < 1 || iters < 1) return fail("time_gemv: bad arguments");
    hipStream_t st = stream();
    for (int i = 0; i < warmup; i++)
        if (launch_gemv(ws[i % nw]->w, (const uint8_t*)d_planes, d_xs, d_y, ldy, b, 0, ws[i % nw]->w.rows, st, ks) != CMF_OK)
            return CMF_ERR;
    int rate_khz = 100000;
    (void)hipDeviceGetAttribute(&rate_khz, hipDeviceAttributeWallClockRate, g_dev);
    hipEvent_t e0, e1;
    CMF_HIP(hipEventCreate(&e0));
    CMF_HIP(hipEventCreate(&e1));
    // ~5 ms of queue head start, bounded by an iteration cap
    hipLaunchKernelGGL(k_spin, dim3(1), dim3(64), 0, st, (unsigned long long)rate_khz * 5, 1 << 22);
    CMF_HIP(hipEventRecord(e0, st));
    for (int i = 0; i < iters; i++)
        launch_gemv(ws[i % nw]->w, (const uint8_t*)d_planes, d_xs, d_y, ldy, b, 0, ws[i % nw]->w.rows, st, ks);
    CMF_HIP(hipEventRecord(e1, st));
    CMF_HIP(hipEventSynchronize(e1));
    float ms = 0.f;
    CMF_HIP(hipEventElapsedTime(&ms, e0, e1));
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    *avg_ms = ms / iters;
    CMF_HIP(hipGetLastError());
    return CMF_OK;
}

int cmf_time_gemv_rows(const cmf_weight* ws, int nw, const float* d_x, int ldx, const float* d_norm_w, int b,
                       float* d_y, int ldy, int fused, int warmup, int iters, float* avg_ms) {
    if (ensure_init() != CMF_OK) return CMF_ERR;
    if (!ws || nw < 1 || iters < 1 || b < 1 || b > MAXB || !d_x || !avg_ms) return fail("time_gemv_rows: bad arguments");
    hipStream_t st = stream();
    XSrc src{};
    src.mode = d_norm_w ? XS_NORM : XS_ROWS;
    src.x = d_x;
    src.ldx = ldx;
    src.w = d_norm_w;
    src.eps = 1e-6;
    uint8_t* planes = nullptr;
    float* xs = nullptr;
    size_t pb = 0;
    for (int i = 0; i < nw; i++) pb = std::max(pb, prep_bytes(ws[i]->w));
    if (!fused) {
        CMF_HIP(hipMalloc(&planes, pb));
        CMF_HIP(hipMalloc(&xs, 16 * sizeof(float)));
    }
    auto one = [&](int i) -> int {
        const DevWeight& w = ws[i % nw]->w;
        if (fused) return gemv(w, src, d_y, ldy, b, 0, w.rows, false, st);
        if (launch_prep_src(w, src, b, planes, xs, st) != CMF_OK) return CMF_ERR;
        XSrc g{};
        g.mode = XS_GLOBAL;
        g.planes = planes;
        g.xs = xs;
        return gemv(w, g, d_y, ldy, b, 0, w.rows, false, st);
    };
    int rc = CMF_OK;
    for (int i = 0; i < warmup && rc == CMF_OK; i++) rc = one(i);
    float ms = 0.f;
    if (rc == CMF_OK) {
        int rate_khz = 100000;
        (void)hipDeviceGetAttribute(&rate_khz, hipDeviceAttributeWallClockRate, g_dev);
        hipEvent_t e0, e1;
        CMF_HIP(hipEventCreate(&e0));
        CMF_HIP(hipEventCreate(&e1));
        hipLaunchKernelGGL(k_spin, dim3(1), dim3(64), 0, st, (unsigned long long)rate_khz * 5, 1 << 22);
        CMF_HIP(hipEventRecord(e0, st));
        for (int i = 0; i < iters && rc == CMF_OK; i++) rc = one(i);
        CMF_HIP(hipEventRecord(e1, st));
        CMF_HIP(hipEventSynchronize(e1));
        CMF_HIP(hipEventElapsedTime(&ms, e0, e1));
        (void)hipEventDestroy(e0);
        (void)hipEventDestroy(e1);
    }
    if (planes) (void)hipFree(planes);
    if (xs) (void)hipFree(xs);
    if (rc != CMF_OK) return rc;
    *avg_ms = ms / iters;
    CMF_HIP(hipGetLastError());
    return CMF_OK;
}

}  // extern "C"
