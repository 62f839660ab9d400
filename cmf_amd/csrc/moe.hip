// MoE FFN of a verify batch on the device: routing (moe_route,
// pipeline.rs:10780-10841), the batch's (token, expert) pairs grouped by
// expert, the expert FFNs as grouped GEMVs and the weighted combine in the
// reference's per-token order (moe_ffn_cpu, pipeline.rs:10997-11045).
//
//   1. routing        one wave per token: softmax of the router logits
//                     (max-subtracted, sequential sum), top-k by descending
//                     probability with the lower index first on ties,
//                     w_i = p_i / wsum, wsum = sum of the kept p (norm_topk)
//                     or 1, divided by routed_scaling;
//   2. job numbering  one job per distinct routed expert, in expert order,
//                     and the job of every (token, rank) slot; 1 and 2 are
//                     one launch (k_moe_route_jobs), 2 alone for caller-routed
//                     batches (k_moe_jobs).
//   3. prep x         prepared operand of the b token rows (shared by all jobs).
//   4. gate|up        grouped GEMV: job j = W_gu[e_j] x for all b rows (the
//                     weights are read once per expert; rows of tokens that
//                     did not pick the expert are computed and ignored: they
//                     cost MFMA rows, not bandwidth).
//   5. prep h         grouped: h = silu(g) * u per job.
//   6. down           grouped GEMV: job j = W_down[e_j] h_j.
//   7. k_moe_combine  out[t] = sum over ranks i of w[t][i] * down[job(t, i)][t],
//                     accumulated from 0 in rank order, as the reference does.
#include <vector>

#include "../../include/cmf_hip.h"
#include "common.h"
#include "gemv.h"
#include "prep_src.h"
#include "runtime.h"
#include "wave.h"

namespace cmf {

constexpr int MOE_MAX_EXPERTS = 1024;
constexpr int MOE_MAX_TOPK = 32;

// Routing of token t by wave t (b <= 16 waves, all tokens at once): softmax
// of the router logits (max-subtracted; the sum sequential in expert order,
// as the reference adds), then the top k by k rounds of a wave arg-max over
// the normalised p: the largest p, the lower index among equal p (the
// reference's order), each pick removed before the next round.  w_i = p_i /
// wsum with wsum = the sum of the kept p in rank order (norm_topk) or 1,
// divided by routed_scaling.  The picks also go to sidx (LDS) for the job
// numbering that follows.
__device__ __forceinline__ void moe_route_tokens(const float* __restrict__ logits, int b, int ne, int k,
                                                 int norm_topk, float scaling, int* __restrict__ idx,
                                                 float* __restrict__ w, int* sidx) {
    __shared__ float p[MAXB][MOE_MAX_EXPERTS];
    __shared__ float tot[MAXB];
    const int lane = threadIdx.x & 63, t = threadIdx.x >> 6;
    const bool on = t < b;
    const float* lg = logits + (size_t)(on ? t : 0) * ne;
    float mx = -INFINITY;
    for (int e = lane; e < ne; e += 64) mx = fmaxf(mx, lg[e]);
    mx = wave_max(mx);
    for (int e = lane; e < ne; e += 64) p[t][e] = expf(lg[e] - mx);
    __syncthreads();
    if (lane == 0) {
        float sm = 0.0f;  // in expert order; the reads eight at a time
        int e = 0;
        for (; e + 8 <= ne; e += 8) {
            float v[8];
#pragma unroll
            for (int j = 0; j < 8; j++) v[j] = p[t][e + j];
#pragma unroll
            for (int j = 0; j < 8; j++) sm += v[j];
        }
        for (; e < ne; e++) sm += p[t][e];
        tot[t] = sm;
    }
    __syncthreads();
    const float sm = tot[t];
    for (int e = lane; e < ne; e += 64) p[t][e] = p[t][e] / sm;
    float wsum = 0.0f;
    for (int i = 0; i < k; i++) {
        // the lane's best (largest p, then lowest index) among its experts;
        // picked experts hold -1
        float bv = -1.0f;
        int bi = ne;
        for (int e = lane; e < ne; e += 64) {
            const float pe = p[t][e];
            if (pe > bv) {
                bv = pe;
                bi = e;
            }
        }
        const float v = wave_max(bv);
        const int e = (int)wave_reduce_f32(bv == v ? (float)bi : INFINITY, INFINITY,
                                           [](float x, float y) { return fminf(x, y); });
        const float pv = v;  // p of the pick (every lane)
        if (lane == (e & 63)) p[t][e] = -1.0f;
        if (on && lane == 0) {
            idx[t * k + i] = e;
            sidx[t * k + i] = e;
            w[t * k + i] = pv;  // scaled below
        }
        wsum += pv;
    }
    if (on && lane == 0) {
        const float ws = norm_topk ? wsum / scaling : 1.0f / scaling;
        for (int i = 0; i < k; i++) w[t * k + i] = w[t * k + i] / ws;
    }
    __syncthreads();
}

// jobs = [njobs, expert of job 0, ...] (experts in increasing order);
// slot[t * k + i] = job of token t's rank-i expert.  One workgroup of 256:
// per-wave ballots and popcounts number the used experts.
__device__ __forceinline__ void moe_jobs_body(const int* idx, int b, int k, int ne, int* __restrict__ jobs,
                                              int* __restrict__ slot) {
    __shared__ int job_of[MOE_MAX_EXPERTS];
    __shared__ int used[MOE_MAX_EXPERTS];
    __shared__ int wave_base[MOE_MAX_EXPERTS / 64 + 1];
    const int tid = threadIdx.x, lane = tid & 63;
    for (int e = tid; e < ne; e += blockDim.x) used[e] = 0;
    __syncthreads();
    for (int i = tid; i < b * k; i += blockDim.x) used[idx[i]] = 1;  // benign same-value races
    __syncthreads();
    // expert e sits in chunk e / 64, lane e % 64; chunk c is counted by wave c % 4
    const int nch = (ne + 63) / 64;
    for (int c = tid >> 6; c < nch; c += blockDim.x >> 6) {
        const int e = c * 64 + lane;
        const bool u = e < ne && used[e];
        const unsigned long long bal = __ballot(u);
        if (lane == 0) wave_base[c] = __popcll(bal);
        if (e < ne) job_of[e] = u ? (int)__popcll(bal & ((1ull << lane) - 1ull)) : -1;
    }
    __syncthreads();
    if (tid == 0) {
        int n = 0;
        for (int c = 0; c < nch; c++) {
            const int cnt = wave_base[c];
            wave_base[c] = n;
            n += cnt;
        }
        jobs[0] = n;
    }
    __syncthreads();
    for (int e = tid; e < ne; e += blockDim.x) {
        if (job_of[e] >= 0) {
            job_of[e] += wave_base[e >> 6];
            jobs[1 + job_of[e]] = e;
        }
    }
    __syncthreads();
    for (int i = tid; i < b * k; i += blockDim.x) slot[i] = job_of[idx[i]];
}
__global__ __launch_bounds__(256) void k_moe_jobs(const int* __restrict__ idx, int b, int k, int ne,
                                                  int* __restrict__ jobs, int* __restrict__ slot) {
    moe_jobs_body(idx, b, k, ne, jobs, slot);
}
// Routing of the b tokens and their job numbering in one launch (one
// workgroup, one wave per token slot).
__global__ __launch_bounds__(1024) void k_moe_route_jobs(const float* __restrict__ logits, int b, int ne, int k,
                                                        int norm_topk, float scaling, int* __restrict__ idx,
                                                        float* __restrict__ w, int* __restrict__ jobs,
                                                        int* __restrict__ slot) {
    __shared__ int sidx[MAXB * MOE_MAX_TOPK];
    moe_route_tokens(logits, b, ne, k, norm_topk, scaling, idx, w, sidx);
    moe_jobs_body(sidx, b, k, ne, jobs, slot);
}

// Routing + job numbering (workgroup b) and the gate|up operand of the b
// token rows (workgroups 0 .. b-1, the producer src) in one launch: the two
// are independent, and each was a launch of its own in the chain before the
// expert GEMVs.  1024 threads (one wave per token slot for the routing).
__global__ __launch_bounds__(1024) void k_moe_route_prep(const float* __restrict__ logits, int b, int ne, int k,
                                                        int norm_topk, float scaling, int* __restrict__ idx,
                                                        float* __restrict__ w, int* __restrict__ jobs,
                                                        int* __restrict__ slot, XSrc src, int K, int fmt, int nk,
                                                        uint8_t* __restrict__ planes, float* __restrict__ xs) {
    extern __shared__ float vals[];  // K (the operand workgroups)
    __shared__ int sidx[MAXB * MOE_MAX_TOPK];
    if ((int)blockIdx.x < b) {
        prep_src_row(src, K, fmt, nk, planes, xs, 0, blockIdx.x, b, vals);
        return;
    }
    moe_route_tokens(logits, b, ne, k, norm_topk, scaling, idx, w, sidx);
    moe_jobs_body(sidx, b, k, ne, jobs, slot);
}

// out[t][h] = sum over ranks i (in order, from 0) of w[t][i] * yd[job][t][h];
// grid (hidden / 256, b): the k job rows of a thread are requested together.
__global__ __launch_bounds__(256) void k_moe_combine(const float* __restrict__ yd, size_t y_stride, int ldy,
                                                     const int* __restrict__ slot, const float* __restrict__ w,
                                                     int k, int hidden, float* __restrict__ out, int ldo,
                                                     int resid) {
    __shared__ int js[MOE_MAX_TOPK];
    __shared__ float ws[MOE_MAX_TOPK];
    const int t = blockIdx.y, h = blockIdx.x * blockDim.x + threadIdx.x;
    if (threadIdx.x < k) {
        js[threadIdx.x] = slot[t * k + threadIdx.x];
        ws[threadIdx.x] = w[t * k + threadIdx.x];
    }
    __syncthreads();
    if (h >= hidden) return;
    float v[MOE_MAX_TOPK];
#pragma unroll 8
    for (int i = 0; i < k; i++) v[i] = yd[js[i] * y_stride + (size_t)t * ldy + h];
    float acc = 0.0f;
    for (int i = 0; i < k; i++) acc += ws[i] * v[i];
    // resid: the decoder block's h += moe_ffn(x) (the sum completed first)
    float* o = out + (size_t)t * ldo + h;
    *o = resid ? *o + acc : acc;
}

}  // namespace cmf

using namespace cmf;

struct cmf_moe_s {
    int ne = 0, hidden = 0, inter = 0, top_k = 0, norm_topk = 1, max_jobs = 0;
    float scaling = 1.0f;
    std::vector<DevWeight> gu, down;  // per expert: [gate; up] rows, down
    std::vector<char> set;
    GemvDesc* d_gu = nullptr;  // device descriptor arrays [ne]
    GemvDesc* d_down = nullptr;
    bool desc_ok = false;
    // device scratch
    float *x = nullptr, *logits = nullptr, *w = nullptr, *out = nullptr;
    int *idx = nullptr, *jobs = nullptr, *slot = nullptr;
    uint8_t *px = nullptr, *ph = nullptr;
    float *xsx = nullptr, *xsh = nullptr, *ygu = nullptr, *yd = nullptr;
    size_t ph_stride = 0;
    std::vector<void*> allocs;
};

static int moe_alloc(cmf_moe m, void** p, size_t bytes) {
    if (hipMalloc(p, bytes) != hipSuccess) return fail("moe: hipMalloc failed");
    m->allocs.push_back(*p);
    return CMF_OK;
}

static int moe_ready(cmf_moe m) {
    if (!m) return fail("null moe");
    for (int e = 0; e < m->ne; e++)
        if (!m->set[e]) return fail("moe: expert " + std::to_string(e) + " not set");
    if (!m->desc_ok) {
        std::vector<GemvDesc> a(m->ne), b(m->ne);
        for (int e = 0; e < m->ne; e++) {
            a[e] = GemvDesc{m->gu[e].w, m->gu[e].scale, m->gu[e].rowp};
            b[e] = GemvDesc{m->down[e].w, m->down[e].scale, m->down[e].rowp};
        }
        CMF_HIP(hipMemcpy(m->d_gu, a.data(), sizeof(GemvDesc) * m->ne, hipMemcpyHostToDevice));
        CMF_HIP(hipMemcpy(m->d_down, b.data(), sizeof(GemvDesc) * m->ne, hipMemcpyHostToDevice));
        m->desc_ok = true;
    }
    return CMF_OK;
}

// Steps 3-7 on the routed batch (idx / w already on the device), k experts
// per token.
// x: the operand producer of the token rows (plain rows, or the block's
// RMSNorm of the residual); out rows [b][ldo], resid: out += the FFN.
static int moe_experts(cmf_moe m, const XSrc& x, int b, int k, float* d_out, int ldo, bool resid, hipStream_t s,
                       bool numbered, bool prepared = false) {
    const int H = m->hidden, I = m->inter;
    if (!numbered) hipLaunchKernelGGL(k_moe_jobs, dim3(1), dim3(256), 0, s, m->idx, b, k, m->ne, m->jobs, m->slot);
    int rc = prepared ? CMF_OK : launch_prep_src(m->gu[0], x, b, m->px, m->xsx, s);
    const int mj = std::min(m->max_jobs, b * k);
    const size_t ygu_stride = (size_t)MAXB * 2 * I, yd_stride = (size_t)MAXB * H;
    if (rc == CMF_OK)
        rc = gemv_grouped(m->gu[0], m->d_gu, m->jobs, mj, m->px, 0, m->xsx, m->ygu, ygu_stride, 2 * I, b, s);
    if (rc != CMF_OK) return rc;
    XSrc sg{};
    sg.mode = XS_SILU;
    sg.x = m->ygu;
    sg.ldx = 2 * I;
    sg.K = I;
    rc = launch_prep_src_grouped(m->down[0], sg, b, m->jobs, mj, ygu_stride, m->ph, m->ph_stride, m->xsh, s);
    if (rc == CMF_OK)
        rc = gemv_grouped(m->down[0], m->d_down, m->jobs, mj, m->ph, m->ph_stride, m->xsh, m->yd, yd_stride, H, b, s);
    if (rc != CMF_OK) return rc;
    hipLaunchKernelGGL(k_moe_combine, dim3((H + 255) / 256, b), dim3(256), 0, s, m->yd, yd_stride, H, m->slot, m->w,
                       k, H, d_out, ldo, resid ? 1 : 0);
    return CMF_OK;
}

static XSrc rows_src(const float* d_x, int H) {
    XSrc r{};
    r.mode = XS_ROWS;
    r.x = d_x;
    r.ldx = H;
    return r;
}

int cmf::moe_prepare(cmf_moe m) { return moe_ready(m); }
int cmf::moe_hidden(cmf_moe m) { return m ? m->hidden : 0; }
int cmf::moe_experts_count(cmf_moe m) { return m ? m->ne : 0; }

int cmf::moe_ffn_launch(cmf_moe m, const XSrc& x, const float* d_logits, int b, float* d_out, int ldo, bool resid,
                   hipStream_t s) {
    if (b < 1 || b > MAXB) return fail("moe: batch must be 1..16");
    const DevWeight& g = m->gu[0];
    const int K = x.K ? x.K : g.cols;
    if (K < 1 || K > g.cols || K > 16384 || (x.mode == XS_CAT && (x.H < 1 || x.H >= K)))
        return fail("moe: bad operand producer");
    const int nk = g.dtype == DT_Q8ROW ? g.kchunks : g.kchunks * 4;
    static const bool attr = [] {
        // the routing arrays' static LDS plus the operand row's K floats
        hipFuncAttributes fa{};
        const size_t st = hipFuncGetAttributes(&fa, (const void*)k_moe_route_prep) == hipSuccess ? fa.sharedSizeBytes : 0;
        return hipFuncSetAttribute((const void*)k_moe_route_prep, hipFuncAttributeMaxDynamicSharedMemorySize,
                                   (int)(160 * 1024 - st)) == hipSuccess;
    }();
    (void)attr;
    hipLaunchKernelGGL(k_moe_route_prep, dim3(b + 1), dim3(64 * MAXB), (size_t)K * sizeof(float), s, d_logits, b,
                       m->ne, m->top_k, m->norm_topk, m->scaling, m->idx, m->w, m->jobs, m->slot, x, K, g.dtype, nk,
                       m->px, m->xsx);
    return moe_experts(m, x, b, m->top_k, d_out, ldo, resid, s, true, true);
}

extern "C" {

int cmf_moe_create(int n_experts, int hidden, int inter, int top_k, int norm_topk, float routed_scaling,
                   cmf_moe* out) {
    if (ensure_init() != CMF_OK) return CMF_ERR;
    if (!out) return fail("null output");
    *out = nullptr;
    if (n_experts < 1 || n_experts > MOE_MAX_EXPERTS) return fail("moe: n_experts must be 1..1024");
    if (top_k < 1 || top_k > MOE_MAX_TOPK || top_k > n_experts) return fail("moe: top_k must be 1..min(32, n_experts)");
    if (hidden < 32 || inter < 32 || hidden % 32 || inter % 32 || hidden > 16384 || inter > 16384)
        return fail("moe: hidden and inter must be multiples of 32 in 32..16384");
    if (!(routed_scaling > 0.0f)) return fail("moe: routed_scaling must be > 0");
    cmf_moe m = new cmf_moe_s();
    m->ne = n_experts;
    m->hidden = hidden;
    m->inter = inter;
    m->top_k = top_k;
    m->norm_topk = norm_topk ? 1 : 0;
    m->scaling = routed_scaling;
    m->max_jobs = std::min(n_experts, MAXB * top_k);
    m->gu.resize(n_experts);
    m->down.resize(n_experts);
    m->set.assign(n_experts, 0);
    const int H = hidden, I = inter, mj = m->max_jobs;
    // prepared operand sizes of the widest codec (q8 3 B / q4 4 B per element + the q4 tile-bias tables)
    const size_t px = std::max(((size_t)H + 63) / 64 * 1024 * 3, ((size_t)H + 127) / 128 * 4 * (2048 + 128));
    m->ph_stride = std::max(((size_t)I + 63) / 64 * 1024 * 3, ((size_t)I + 127) / 128 * 4 * (2048 + 128));
    if (moe_alloc(m, (void**)&m->d_gu, sizeof(GemvDesc) * n_experts) ||
        moe_alloc(m, (void**)&m->d_down, sizeof(GemvDesc) * n_experts) ||
        moe_alloc(m, (void**)&m->x, sizeof(float) * MAXB * H) ||
        moe_alloc(m, (void**)&m->logits, sizeof(float) * MAXB * n_experts) ||
        moe_alloc(m, (void**)&m->w, sizeof(float) * MAXB * top_k) ||
        moe_alloc(m, (void**)&m->out, sizeof(float) * MAXB * H) ||
        moe_alloc(m, (void**)&m->idx, sizeof(int) * MAXB * top_k) ||
        moe_alloc(m, (void**)&m->jobs, sizeof(int) * (1 + MAXB * top_k)) ||
        moe_alloc(m, (void**)&m->slot, sizeof(int) * MAXB * top_k) ||
        moe_alloc(m, (void**)&m->px, px) || moe_alloc(m, (void**)&m->xsx, sizeof(float) * 16) ||
        moe_alloc(m, (void**)&m->ph, m->ph_stride * mj) || moe_alloc(m, (void**)&m->xsh, sizeof(float) * 16 * mj) ||
        moe_alloc(m, (void**)&m->ygu, sizeof(float) * MAXB * 2 * I * mj) ||
        moe_alloc(m, (void**)&m->yd, sizeof(float) * MAXB * H * mj)) {
        for (void* p : m->allocs) (void)hipFree(p);
        delete m;
        return CMF_ERR;
    }
    *out = m;
    return CMF_OK;
}

int cmf_moe_free(cmf_moe m) {
    if (!m) return CMF_OK;
    (void)hipDeviceSynchronize();
    for (auto& w : m->gu) free_weight(w);
    for (auto& w : m->down) free_weight(w);
    for (void* p : m->allocs) (void)hipFree(p);
    delete m;
    return CMF_OK;
}

int cmf_moe_set_expert(cmf_moe m, int e, const cmf_tensor* gate, const cmf_tensor* up, const cmf_tensor* down) {
    if (!m) return fail("null moe");
    if (e < 0 || e >= m->ne) return fail("moe: expert index out of range");
    if (!gate || !up || !down) return fail("moe: null tensor");
    const int H = m->hidden, I = m->inter;
    if (gate->rows != I || up->rows != I || gate->cols != H || up->cols != H || down->rows != H || down->cols != I)
        return fail("moe: expert shapes must be gate/up [inter x hidden], down [hidden x inter]");
    if (gate->dtype != up->dtype) return fail("moe: gate and up must share a dtype");
    for (const cmf_tensor* t : {gate, up, down}) {
        if (t->dtype == DT_Q8ROW) {
            if (!t->q || !t->row_scale) return fail("moe: q8 needs q and row_scale");
        } else if (t->dtype == DT_Q4T || t->dtype == DT_Q4TP) {
            if (!t->bytes) return fail("moe: q4 needs bytes");
        } else {
            return CMF_DECLINED;  // codec without a device kernel: the caller keeps its CPU path
        }
    }
    for (int f = 0; f < m->ne; f++)
        if (m->set[f] && f != e && (m->gu[f].dtype != gate->dtype || m->down[f].dtype != down->dtype))
            return fail("moe: every expert must use the same codecs");
    DevWeight gu, dn;
    if (gate->dtype == DT_Q8ROW) {
        std::vector<const int8_t*> rp;
        std::vector<float> rs;
        for (const cmf_tensor* t : {gate, up})
            for (int r = 0; r < t->rows; r++) {
                rp.push_back(t->q + (size_t)r * H);
                rs.push_back(t->row_scale[r]);
            }
        if (build_q8(gu, 2 * I, H, rp.data(), rs.data()) != CMF_OK) return CMF_ERR;
    } else {
        Q4Src s;
        fill_q4src(s, gate->dtype, I, H, gate->bytes, 0);
        fill_q4src(s, up->dtype, I, H, up->bytes, 0);
        if (build_q4(gu, s) != CMF_OK) return CMF_ERR;
    }
    int rc;
    if (down->dtype == DT_Q8ROW) {
        std::vector<const int8_t*> rp;
        for (int r = 0; r < H; r++) rp.push_back(down->q + (size_t)r * I);
        rc = build_q8(dn, H, I, rp.data(), down->row_scale);
    } else {
        Q4Src s;
        fill_q4src(s, down->dtype, H, I, down->bytes, 0);
        rc = build_q4(dn, s);
    }
    if (rc != CMF_OK) {
        free_weight(gu);
        return CMF_ERR;
    }
    if (m->set[e]) {
        (void)hipDeviceSynchronize();
        free_weight(m->gu[e]);
        free_weight(m->down[e]);
    }
    m->gu[e] = gu;
    m->down[e] = dn;
    m->set[e] = 1;
    m->desc_ok = false;
    return CMF_OK;
}

int cmf_moe_ffn_dev(cmf_moe m, const float* d_x, const float* d_logits, int b, float* d_out) {
    if (ensure_init() != CMF_OK) return CMF_ERR;
    if (moe_ready(m) != CMF_OK) return CMF_ERR;
    if (b < 1 || b > MAXB) return fail("moe: batch must be 1..16");
    if (!d_x || !d_logits || !d_out) return fail("moe: null pointer");
    const int rc = moe_ffn_launch(m, rows_src(d_x, m->hidden), d_logits, b, d_out, m->hidden, false, stream());
    if (rc != CMF_OK) return rc;
    CMF_HIP(hipGetLastError());
    return CMF_OK;
}

int cmf_moe_ffn(cmf_moe m, const float* x, const float* router_logits, int b, float* out, int32_t* idx_out,
                float* w_out) {
    if (ensure_init() != CMF_OK) return CMF_ERR;
    if (!m || !x || !router_logits || !out) return fail("moe: null pointer");
    if (b < 1 || b > MAXB) return fail("moe: batch must be 1..16");
    hipStream_t s = stream();
    CMF_HIP(hipMemcpyAsync(m->x, x, sizeof(float) * b * m->hidden, hipMemcpyHostToDevice, s));
    CMF_HIP(hipMemcpyAsync(m->logits, router_logits, sizeof(float) * b * m->ne, hipMemcpyHostToDevice, s));
    const int rc = cmf_moe_ffn_dev(m, m->x, m->logits, b, m->out);
    if (rc != CMF_OK) return rc;
    CMF_HIP(hipMemcpyAsync(out, m->out, sizeof(float) * b * m->hidden, hipMemcpyDeviceToHost, s));
    if (idx_out) CMF_HIP(hipMemcpyAsync(idx_out, m->idx, sizeof(int) * b * m->top_k, hipMemcpyDeviceToHost, s));
    if (w_out) CMF_HIP(hipMemcpyAsync(w_out, m->w, sizeof(float) * b * m->top_k, hipMemcpyDeviceToHost, s));
    CMF_HIP(hipStreamSynchronize(s));
    return CMF_OK;
}

int cmf_time_moe(cmf_moe m, const float* d_x, const float* d_logits, int b, float* d_out, int warmup, int iters,
                 float* avg_ms) {
    if (!avg_ms || iters < 1 || warmup < 0) return fail("time_moe: bad arguments");
    for (int i = 0; i < warmup; i++)
        if (cmf_moe_ffn_dev(m, d_x, d_logits, b, d_out) != CMF_OK) return CMF_ERR;
    hipStream_t s = stream();
    hipEvent_t e0, e1;
    CMF_HIP(hipEventCreate(&e0));
    CMF_HIP(hipEventCreate(&e1));
    CMF_HIP(hipEventRecord(e0, s));
    int rc = CMF_OK;
    for (int i = 0; i < iters && rc == CMF_OK; i++) rc = cmf_moe_ffn_dev(m, d_x, d_logits, b, d_out);
    CMF_HIP(hipEventRecord(e1, s));
    CMF_HIP(hipEventSynchronize(e1));
    float ms = 0.f;
    CMF_HIP(hipEventElapsedTime(&ms, e0, e1));
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    *avg_ms = ms / iters;
    return rc;
}

int cmf_moe_block(cmf_moe m, const float* x, const int32_t* experts, const float* weights, int njobs, float* out) {
    if (ensure_init() != CMF_OK) return CMF_ERR;
    if (moe_ready(m) != CMF_OK) return CMF_ERR;
    if (!x || !experts || !weights || !out) return fail("moe: null pointer");
    if (njobs < 1 || njobs > m->top_k) return fail("moe: njobs must be 1..top_k");
    for (int i = 0; i < njobs; i++)
        if (experts[i] < 0 || experts[i] >= m->ne) return fail("moe: expert index out of range");
    hipStream_t s = stream();
    CMF_HIP(hipMemcpyAsync(m->x, x, sizeof(float) * m->hidden, hipMemcpyHostToDevice, s));
    CMF_HIP(hipMemcpyAsync(m->idx, experts, sizeof(int) * njobs, hipMemcpyHostToDevice, s));
    CMF_HIP(hipMemcpyAsync(m->w, weights, sizeof(float) * njobs, hipMemcpyHostToDevice, s));
    const int rc = moe_experts(m, rows_src(m->x, m->hidden), 1, njobs, m->out, m->hidden, false, s, false);
    if (rc != CMF_OK) return rc;
    CMF_HIP(hipMemcpyAsync(out, m->out, sizeof(float) * m->hidden, hipMemcpyDeviceToHost, s));
    CMF_HIP(hipStreamSynchronize(s));
    CMF_HIP(hipGetLastError());
    return CMF_OK;
}

}  // extern "C"
