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
//                     the job of every (token, rank) slot and each job's
//                     token list; 1 and 2 are one launch with the prepared
//                     operand of the b token rows (k_moe_route_prep), 2 alone
//                     for caller-routed batches (k_moe_jobs).
//   q4t experts, b <= 8 (k_moe_q4t, over each job's own tokens only):
//   3. gate|up        job j: h = silu(g) * u of W_gu[e_j] x for its tokens;
//   4. down           routed batches: per (row block, token), one wave per
//                     rank i: W_down[e_ti] h_ti with the operand made from
//                     the h row in the wave, and 5 in the same launch
//                     (k_moe_down_tok); caller-routed jobs: job j:
//                     W_down[e_j] h, the operand made from the h rows in the
//                     workgroup;
//   other codecs or larger batches (grouped GEMVs over all b rows; rows of
//   tokens that did not pick the expert are computed and ignored):
//   3. gate|up, 3b. the per-job operand h = silu(g) * u, 4. down;
//   5. k_moe_combine  out[t] = sum over ranks i of w[t][i] * down[job(t, i)][t],
//                     accumulated from 0 in rank order, as the reference does.
#include <map>
#include <mutex>
#include <vector>

#include "../../include/cmf_hip.h"
#include "common.h"
#include "gemv.h"
#include "gemv_kern.h"
#include "prep_src.h"
#include "runtime.h"
#include "wave.h"

namespace cmf {

constexpr int MOE_MAX_EXPERTS = 1024;
constexpr int MOE_MAX_TOPK = 32;
constexpr int MOE_JT = 1 + MAXB;  // job token list: count, then the tokens

// Routing of token t by wave t (b <= 16 waves, all tokens at once; no
// barrier: each wave works on its own token): softmax of the router logits
// (max-subtracted; the sum sequential in expert order, as the reference
// adds), then the top k by k rounds of a wave arg-max over the normalised
// p: the largest p, the lower index among equal p (the reference's order),
// each pick removed before the next round.  w_i = p_i / wsum with wsum =
// the sum of the kept p in rank order (norm_topk) or 1, divided by
// routed_scaling.  Lane l holds experts l + 64 c in registers; the
// sequential sum reads the exponentials back from LDS, 32 at a time, in
// every lane (broadcast reads), so the total is wave-uniform.  A round's
// pick: the wave max v of p, then the lowest expert holding v from one
// ballot per register column (experts of column c all precede those of
// c + 1).  The picks also go to sidx (LDS) for the job numbering.
template <int MOE_NC>  // register columns: ne <= 64 MOE_NC
__device__ __forceinline__ void moe_route_tokens(const float* __restrict__ logits, int b, int ne, int k,
                                                 int norm_topk, float scaling, int* __restrict__ idx,
                                                 float* __restrict__ w, int* sidx,
                                                 float (*pe)[MOE_MAX_EXPERTS]) {
    const int lane = threadIdx.x & 63, t = threadIdx.x >> 6;
    if (t >= b) return;  // (uniform per wave; the caller's barrier follows)
    const int nc = (ne + 63) >> 6;
    const float* lg = logits + (size_t)t * ne;
    float p[MOE_NC];
#pragma unroll
    for (int c = 0; c < MOE_NC; c++) {
        const int e = lane + 64 * c;
        p[c] = (c < nc && e < ne) ? lg[e] : -INFINITY;
    }
    float mx = p[0];
#pragma unroll
    for (int c = 1; c < MOE_NC; c++) mx = fmaxf(mx, p[c]);
    mx = wave_max(mx);
#pragma unroll
    for (int c = 0; c < MOE_NC; c++) {
        const int e = lane + 64 * c;
        if (c < nc) {
            const float v = e < ne ? expf(p[c] - mx) : 0.f;
            pe[t][e] = v;
            p[c] = v;
        }
    }
    // the sum in expert order (the wave's own LDS writes precede its reads)
    float sm = 0.0f;
    const float4* row = (const float4*)pe[t];
    for (int e0 = 0; e0 < ne; e0 += 32) {
        float4 v[8];
#pragma unroll
        for (int q = 0; q < 8; q++) v[q] = row[(e0 >> 2) + q];
#pragma unroll
        for (int q = 0; q < 8; q++) {
            if (e0 + 4 * q + 0 < ne) sm += v[q].x;
            if (e0 + 4 * q + 1 < ne) sm += v[q].y;
            if (e0 + 4 * q + 2 < ne) sm += v[q].z;
            if (e0 + 4 * q + 3 < ne) sm += v[q].w;
        }
    }
#pragma unroll
    for (int c = 0; c < MOE_NC; c++) p[c] = (c < nc && lane + 64 * c < ne) ? p[c] / sm : -1.0f;
    float wsum = 0.0f, myw = 0.0f;
    int mye = 0;
    for (int i = 0; i < k; i++) {
        float bv = p[0];
#pragma unroll
        for (int c = 1; c < MOE_NC; c++) bv = fmaxf(bv, p[c]);
        const float v = wave_max(bv);
        int e = ne;
#pragma unroll
        for (int c = 0; c < MOE_NC; c++) {
            const unsigned long long m = __ballot(p[c] == v);
            if (e == ne && m) e = 64 * c + (int)__ffsll((long long)m) - 1;
        }
        e = __builtin_amdgcn_readfirstlane(e);
#pragma unroll
        for (int c = 0; c < MOE_NC; c++)
            if (e == lane + 64 * c) p[c] = -1.0f;
        if (lane == i) {
            mye = e;
            myw = v;  // scaled below
        }
        wsum += v;
    }
    if (lane < k) {
        const float ws = norm_topk ? wsum / scaling : 1.0f / scaling;
        idx[t * k + lane] = mye;
        sidx[t * k + lane] = mye;
        w[t * k + lane] = myw / ws;
    }
}

// jobs = [njobs, expert of job 0, ...] (experts in increasing order);
// slot[t * k + i] = job of token t's rank-i expert.  One workgroup of 256:
// per-wave ballots and popcounts number the used experts.
__device__ __forceinline__ void moe_jobs_body(const int* idx, int b, int k, int ne, int* __restrict__ jobs,
                                              int* __restrict__ slot, int* __restrict__ jt) {
    __shared__ int job_of[MOE_MAX_EXPERTS];
    __shared__ unsigned used[MOE_MAX_EXPERTS];  // bit t: token t picked the expert
    __shared__ int wave_base[MOE_MAX_EXPERTS / 64 + 1];
    const int tid = threadIdx.x, lane = tid & 63;
    for (int e = tid; e < ne; e += blockDim.x) used[e] = 0u;
    __syncthreads();
    for (int i = tid; i < b * k; i += blockDim.x) atomicOr(&used[idx[i]], 1u << (i / k));
    __syncthreads();
    // expert e sits in chunk e / 64, lane e % 64; chunk c is counted by wave c % 4
    const int nch = (ne + 63) / 64;
    for (int c = tid >> 6; c < nch; c += blockDim.x >> 6) {
        const int e = c * 64 + lane;
        const bool u = e < ne && used[e] != 0u;
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
            // the job's tokens in increasing order
            int* l = jt + (size_t)job_of[e] * MOE_JT;
            unsigned msk = used[e];
            l[0] = __popc(msk);
            for (int n = 1; msk; n++) {
                l[n] = __ffs(msk) - 1;
                msk &= msk - 1u;
            }
        }
    }
    __syncthreads();
    for (int i = tid; i < b * k; i += blockDim.x) slot[i] = job_of[idx[i]];
}
__global__ __launch_bounds__(256) void k_moe_jobs(const int* __restrict__ idx, int b, int k, int ne,
                                                  int* __restrict__ jobs, int* __restrict__ slot, int* __restrict__ jt) {
    moe_jobs_body(idx, b, k, ne, jobs, slot, jt);
}

// Routing + job numbering (workgroup b) and the gate|up operand of the b
// token rows (workgroups 0 .. b-1, the producer src) in one launch: the two
// are independent, and each was a launch of its own in the chain before the
// expert GEMVs.  1024 threads (one wave per token slot for the routing).
__global__ __launch_bounds__(1024) void k_moe_route_prep(const float* __restrict__ logits, int b, int ne, int k,
                                                        int norm_topk, float scaling, int* __restrict__ idx,
                                                        float* __restrict__ w, int* __restrict__ jobs,
                                                        int* __restrict__ slot, int* __restrict__ jt, XSrc src, int K,
                                                        int fmt, int nk, uint8_t* __restrict__ planes,
                                                        float* __restrict__ xs) {
    extern __shared__ float vals[];  // K (the operand workgroups)
    __shared__ int sidx[MAXB * MOE_MAX_TOPK];
    __shared__ __align__(16) float pe[MAXB][MOE_MAX_EXPERTS];  // the routing's exponentials
    if ((int)blockIdx.x < b) {
        prep_src_row(src, K, fmt, nk, planes, xs, 0, blockIdx.x, b, vals);
        return;
    }
    if (ne <= 64)
        moe_route_tokens<1>(logits, b, ne, k, norm_topk, scaling, idx, w, sidx, pe);
    else if (ne <= 128)
        moe_route_tokens<2>(logits, b, ne, k, norm_topk, scaling, idx, w, sidx, pe);
    else if (ne <= 256)
        moe_route_tokens<4>(logits, b, ne, k, norm_topk, scaling, idx, w, sidx, pe);
    else
        moe_route_tokens<MOE_MAX_EXPERTS / 64>(logits, b, ne, k, norm_topk, scaling, idx, w, sidx, pe);
    __syncthreads();
    moe_jobs_body(sidx, b, k, ne, jobs, slot, jt);
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

// ---------------------------------------------------------------------------
// q4t expert GEMVs over the job's own tokens.  Job j (grid.y) multiplies
// expert desc[jobs[1 + j]] with the n <= 8 token rows of its list jt[j]
// only: the other tokens of the batch cost no operand traffic and no LDS.
// A workgroup holds RBW row blocks x KP parts of the row (wave = K part x
// RBW + row block, SPW 1 KiB steps each; the parts' partial sums meet in
// LDS in part order).  Its waves share one copy of the job's operand rows
// in LDS ([slot][item][plane], 16-byte items of the fixed-point hi / lo
// f16 planes) and of their tile biases ([tile][16]: A rows 0..7 the hi
// plane of slots 0..7, 8..15 the lo plane).  A rows of slots past n repeat
// slot n - 1 and are never stored.
//   GU: the operand is the prepared planes of all M batch rows (one for
//       all jobs), copied by direct loads; the weight's row blocks hold 8
//       gate rows then the matching 8 up rows (build_swiglu), and
//       y[t][8 rb + r] = silu(g) * u (inference.rs:14-16);
//   else the operand is made from the job's f32 rows hx[t] in the
//       workgroup, exactly as the producer would prepare them, and
//       y[t][16 rb + r] = the row's dot product.
// ---------------------------------------------------------------------------
struct MoeGx {
    const GemvDesc* desc;
    const int* jobs;
    const int* jt;
    const uint8_t* planes;  // GU
    const float* xs;        // GU: xs[t] of the operand
    float* y;         // + j * y_stride, token t's row at t * ldy
    size_t y_stride;
    int ldy, M, nk, nrb, rows, ns;  // ns: token slots of the LDS copy (>= any job's count)
    // !GU: the operand rows themselves, f32: token t of job j at hx + j * hx_stride + t * ldh, K columns
    const float* hx;
    size_t hx_stride;
    int ldh, K;
};

template <int RBW, int KP, int SPW, bool GU>
__global__ __launch_bounds__(64 * RBW * KP, GU && KP > 1 ? 6 : 1) void k_moe_q4t(MoeGx a) {
    constexpr int NW = RBW * KP;
    extern __shared__ __align__(16) uint8_t smem[];
    __shared__ float4v part[KP > 1 ? KP - 1 : 1][RBW][64];
    const int j = blockIdx.y;
    if (j >= a.jobs[0]) return;  // uniform
    const GemvDesc d = a.desc[a.jobs[1 + j]];
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int r = lane & 15, s = lane >> 4, p = r < 8 ? 0 : 1;
    // wave: row block rbi of the workgroup's RBW, K part kp (steps SPW kp ..)
    const int rbi = wave % RBW, kp = wave / RBW, g0 = kp * SPW;
    const int ntg = a.nk, M = a.M, rb = blockIdx.x * RBW + rbi;
    // GU: xs of every batch row (lane t % 16), independent of the token list
    const float xsv = GU ? ldg(a.xs + (lane & 15)) : 0.f;
    // the token list by scalar loads (uniform, in flight with the
    // descriptor's); lane k (mod 8) holds the token of slot min(k, n - 1)
    const int* jl = a.jt + (size_t)j * MOE_JT;
    const int n = min(jl[0], 8);
    int tk[8];
#pragma unroll
    for (int k = 0; k < 8; k++) tk[k] = jl[1 + k];
    const int ls = min(lane & 7, n - 1);
    int tokv = tk[0];
#pragma unroll
    for (int k = 1; k < 8; k++) tokv = ls == k ? tk[k] : tokv;
    const int QI = ntg * 32;  // items of one slot: (step, tile, k-slot) x plane
    float* lb = (float*)(smem + (size_t)a.ns * QI * 16);
    uint4 wv[SPW];
    uint2 sv[SPW];
    // the weights + tile scales of the wave's row block (clamped: every load unconditional)
    auto load_weights = [&]() {
        const size_t wbase = (size_t)min(rb, a.nrb - 1) * ntg;
#pragma unroll
        for (int u = 0; u < SPW; u++) {
            const size_t t = wbase + min(g0 + u, ntg - 1);
            wv[u] = ld_stream((const uint4*)d.w + t * 64 + lane);
            const uint64_t sw = ldg((const uint64_t*)d.scale + t * 16 + r);
            sv[u] = make_uint2((uint32_t)sw, (uint32_t)(sw >> 32));
        }
    };
    __shared__ unsigned smax[8];  // !GU: max |x| of each slot's row (f32 bits)
    __shared__ float sxs[8];      // !GU: the slot's operand unit xs
    if constexpr (GU) {
        // the prepared operand: this wave's share of the copy of the job's
        // rows first, then its weights (the MFMAs wait for the copy, then
        // for each step's weights in turn)
        const uint8_t* hi = a.planes;
        const uint8_t* lo = hi + (size_t)ntg * 4 * 64 * M;
        const float* T1 = (const float*)(hi + (size_t)ntg * 4 * 128 * M);  // tile biases [tile][16]
        const float* T2 = T1 + (size_t)ntg * 4 * 16;
        const int NI = n * QI;
        constexpr int CMAX = (8 * SPW * KP * 32 / 64 + NW - 1) / NW;  // chunks per wave of 8 slots
#pragma unroll
        for (int kc = 0; kc < CMAX; kc++) {
            const int c = wave + NW * kc;
            if (c * 64 >= NI) break;
            const int i = min(c * 64 + lane, NI - 1);
            const int slot = i / QI, rest = i - slot * QI, pl = rest & 1, q = rest >> 1;
            int tok = tk[0];
#pragma unroll
            for (int k = 1; k < 8; k++) tok = slot == k ? tk[k] : tok;
            __builtin_amdgcn_global_load_lds((const void*)((pl ? lo : hi) + ((size_t)q * M + tok) * 16),
                                             (__attribute__((address_space(3))) void*)(smem + c * 1024), 16, 0, 0);
        }
#pragma unroll
        for (int kc = 0; kc < (SPW * KP + NW - 1) / NW; kc++) {
            const int c = wave + NW * kc;
            if (c >= ntg) break;
            const int i = c * 64 + lane, tile = i >> 4, k = i & 15;
            __builtin_amdgcn_global_load_lds((const void*)((k < 8 ? T1 : T2) + (size_t)tile * 16 + tokv),
                                             (__attribute__((address_space(3))) void*)(lb + c * 64), 4, 0, 0);
        }
        __builtin_amdgcn_sched_barrier(0);
        load_weights();
        __builtin_amdgcn_sched_barrier(0);
        wait_vmcnt<2 * SPW>();                   // this wave's share of the copy
        asm volatile("s_barrier" ::: "memory");  // ... and every other wave's
    } else {
        // the operand from the f32 rows: the workgroup's threads take the
        // 8-column items (slot, 4 tile + k-slot) in turn, request them before
        // the weights, agree on each slot's max |x| (LDS atomics), then write
        // the fixed-point hi / lo planes and tile biases that the producer
        // (prep16_row) would write, into the LDS layout of the copy above
        constexpr int NT = 64 * NW;
        constexpr int IPT = (8 * SPW * KP * 16 + NT - 1) / NT;  // items per thread for 8 slots
        const int tid = threadIdx.x, IPS = ntg * 16, NIT = n * IPS;
        const float* hx = a.hx + (size_t)j * a.hx_stride;
        float4v xv[IPT][2] = {};
#pragma unroll
        for (int k = 0; k < IPT; k++) {
            if (NT * k >= NIT) break;  // (uniform)
            if (tid + NT * k >= NIT) continue;
            const int it = tid + NT * k, slot = it / IPS, item = it - slot * IPS;
            const int c0 = 8 * item;  // 32 tile + 8 k-slot
            int tok = tk[0];
#pragma unroll
            for (int q = 1; q < 8; q++) tok = slot == q ? tk[q] : tok;
            const float* src = hx + (size_t)tok * a.ldh + min(c0, a.K - 8);
            xv[k][0] = ldg((const float4v*)src);
            xv[k][1] = ldg((const float4v*)(src + 4));
        }
        __builtin_amdgcn_sched_barrier(0);
        load_weights();
        __builtin_amdgcn_sched_barrier(0);
        if (tid < 8) smax[tid] = 0u;
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
        wait_vmcnt<2 * SPW>();  // the rows' items (requested before the weights)
#pragma unroll
        for (int k = 0; k < IPT; k++) {
            if (NT * k >= NIT) break;  // (uniform)
            const int it = tid + NT * k, slot = it / IPS, c0 = 8 * (it - slot * IPS);
            float am = 0.f;
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const float x = xv[k][e >> 2][e & 3];
                am = fmaxf(am, c0 + e < a.K ? fabsf(x) : 0.f);
            }
            if (it < NIT) atomicMax(&smax[slot], __float_as_uint(am));
        }
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
        const int ord[8] = {0, 4, 2, 6, 1, 5, 3, 7};
#pragma unroll
        for (int k = 0; k < IPT; k++) {
            if (NT * k >= NIT) break;  // (uniform: the shuffles below need whole waves)
            const int it = tid + NT * k, on = it < NIT;
            const int itc = min(it, NIT - 1), slot = itc / IPS, item = itc - slot * IPS, c0 = 8 * item;
            float scale, xsl;
            q4_fix_scale(__uint_as_float(smax[slot]), scale, xsl);
            uint16_t hv[8], lv[8];
            float sh = 0.f, sl = 0.f;  // (exact: integers and multiples of 2^-11)
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const int col = ord[e];
                const float x = xv[k][col >> 2][col & 3];
                _Float16 h, l;
                q4_fix_split(c0 + col < a.K ? x * scale : 0.f, h, l);
                hv[e] = __builtin_bit_cast(uint16_t, h);
                lv[e] = __builtin_bit_cast(uint16_t, l);
                sh += (float)h;
                sl += (float)l;
            }
            sh += __shfl_xor(sh, 1);
            sh += __shfl_xor(sh, 2);
            sl += __shfl_xor(sl, 1);
            sl += __shfl_xor(sl, 2);
            if (on) {
                uint4* dst = (uint4*)smem + slot * QI + item * 2;
                dst[0] = make_uint4(hv[0] | (hv[1] << 16), hv[2] | (hv[3] << 16), hv[4] | (hv[5] << 16),
                                    hv[6] | (hv[7] << 16));
                dst[1] = make_uint4(lv[0] | (lv[1] << 16), lv[2] | (lv[3] << 16), lv[4] | (lv[5] << 16),
                                    lv[6] | (lv[7] << 16));
                if ((item & 3) == 0) {
                    lb[(item >> 2) * 16 + slot] = sh * Q4_BIAS;
                    lb[(item >> 2) * 16 + 8 + slot] = sl * Q4_BIAS;
                }
                if (item == 0) sxs[slot] = xsl;
            }
        }
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    }
    const uint4* X = (const uint4*)smem + ls * QI + p;
    const float4v* LB = (const float4v*)lb;
    float4v acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int u = 0; u < SPW; u++) {
        const bool in = g0 + u < ntg;  // (steps past the row: zero scale, a select)
        const int uc = min(g0 + u, ntg - 1);
#pragma unroll
        for (int t = 0; t < 4; t++) {
            const int q = (uc * 4 + t) * 4 + s;
            const half8 xa = __builtin_bit_cast(half8, X[q * 2]);
            const float4v cb = LB[(uc * 4 + t) * 4 + s];  // A rows 4s..4s+3
            const uint32_t wq = t == 0 ? wv[u].x : t == 1 ? wv[u].y : t == 2 ? wv[u].z : wv[u].w;
            const float4v dd = __builtin_amdgcn_mfma_f32_16x16x32_f16(xa, dq_nib_word(wq), cb, 0, 0, 0);
            const uint32_t sw = t < 2 ? sv[u].x : sv[u].y;
            const float sc = in ? f16_bits_to_f32((t & 1) ? sw >> 16 : sw & 0xFFFFu) : 0.f;
#pragma unroll
            for (int v = 0; v < 4; v++) acc[v] += dd[v] * sc;
        }
    }
    if constexpr (KP > 1) {  // the other K parts' partials through LDS, added in part order
        if (kp > 0) part[kp - 1][rbi][lane] = acc;
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
        if (kp > 0) return;
#pragma unroll
        for (int k = 0; k < KP - 1; k++) {
            const float4v o = part[k][rbi][lane];
#pragma unroll
            for (int v = 0; v < 4; v++) acc[v] += o[v];
        }
    }
    float* y = a.y + (size_t)j * a.y_stride;
#pragma unroll
    for (int v = 0; v < 4; v++) {
        acc[v] += __shfl_xor(acc[v], 32);  // hi rows (lanes s = 0, 1) + lo rows (s = 2, 3)
        const int slot = 4 * (s & 1) + v;
        const int tok = __shfl(tokv, slot);
        const float xsl = GU ? __shfl(xsv, tok) : sxs[min(slot, n - 1)];
        const float val = acc[v] * xsl * 16777216.0f;  // 2^24: denormal nibbles
        if constexpr (GU) {
            const float u = __shfl_xor(val, 8);  // the matching up row
            const int row = 8 * rb + r;
            if (s < 2 && slot < n && r < 8 && rb < a.nrb && row < a.rows / 2)
                y[(size_t)tok * a.ldy + row] = (val / (1.0f + expf(-val))) * u;
        } else {
            const int row = 16 * rb + r;
            if (s < 2 && slot < n && rb < a.nrb && row < a.rows) y[(size_t)tok * a.ldy + row] = val;
        }
    }
}

// Down projection and combine of routed batches in one launch (q4t, K =
// inter <= 1024): workgroup (rb, t) computes rows [16 rb, 16 rb + 16) of
// token t's MoE output; wave i (one per rank, k waves) multiplies expert
// idx[t][i]'s down rows with token t's h row of that job, staged by the
// wave itself exactly as the producer would (row max |x| by a wave
// reduction, the fixed-point hi / lo planes and tile biases into the
// wave's own LDS slice), and the k results meet in LDS, where
// out[t][row] = sum over ranks in order of w[t][i] * down_i[row] (as
// k_moe_combine).  Every routed expert's down rows are read once per token
// that picked it instead of once per job; no per-job down rows are stored.
template <int SPW>
__global__ __launch_bounds__(1024) void k_moe_down_tok(const GemvDesc* __restrict__ desc, const int* __restrict__ idx,
                                                      const int* __restrict__ slot, const float* __restrict__ w,
                                                      int k, const float* __restrict__ hx, size_t hx_stride,
                                                      int ldh, int K, int nrb, int rows, float* __restrict__ out,
                                                      int ldo, int resid) {
    extern __shared__ __align__(16) uint8_t smem[];  // per wave: SPW * 32 items x 16 B + SPW * 4 tiles x 16 biases
    __shared__ float res[16][16];                    // [rank][row] results
    __shared__ float resw[16];                       // the ranks' routing weights
    constexpr int QI = SPW * 32, IPW = (SPW * 16 + 63) / 64;  // items of the row; items per lane
    const int lane = threadIdx.x & 63, i = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int r = lane & 15, s = lane >> 4, p = r < 8 ? 0 : 1;
    const int rb = blockIdx.x, t = blockIdx.y, ntg = SPW;
    const int e = idx[t * k + i], j = slot[t * k + i];
    const float wi = w[t * k + i];
    const GemvDesc d = desc[e];
    // the h row's items first (8 columns per item: 32 tile + 8 k-slot)
    const float* h = hx + (size_t)j * hx_stride + (size_t)t * ldh;
    float4v xv[IPW][2];
#pragma unroll
    for (int q = 0; q < IPW; q++) {
        const int c0 = min(8 * (lane + 64 * q), K - 8);
        xv[q][0] = ldg((const float4v*)(h + c0));
        xv[q][1] = ldg((const float4v*)(h + c0 + 4));
    }
    __builtin_amdgcn_sched_barrier(0);
    uint4 wv[SPW];
    uint2 sv[SPW];
#pragma unroll
    for (int u = 0; u < SPW; u++) {
        const size_t tt = (size_t)rb * ntg + u;
        wv[u] = ld_stream((const uint4*)d.w + tt * 64 + lane);
        const uint64_t sw = ldg((const uint64_t*)d.scale + tt * 16 + r);
        sv[u] = make_uint2((uint32_t)sw, (uint32_t)(sw >> 32));
    }
    __builtin_amdgcn_sched_barrier(0);
    wait_vmcnt<2 * SPW>();  // the row's items
    float am = 0.f;
#pragma unroll
    for (int q = 0; q < IPW; q++) {
        const int c0 = 8 * (lane + 64 * q);
#pragma unroll
        for (int c = 0; c < 8; c++) am = fmaxf(am, c0 + c < K ? fabsf(xv[q][c >> 2][c & 3]) : 0.f);
    }
    am = wave_max(am);
    float scale, xsl;
    q4_fix_scale(am, scale, xsl);
    uint8_t* lw = smem + (size_t)i * (QI * 16 + SPW * 4 * 64);
    float* lb = (float*)(lw + QI * 16);
    const int ord[8] = {0, 4, 2, 6, 1, 5, 3, 7};
#pragma unroll
    for (int q = 0; q < IPW; q++) {
        const int item = lane + 64 * q, c0 = 8 * item;
        uint16_t hv[8], lv[8];
        float sh = 0.f, sl = 0.f;  // (exact: integers and multiples of 2^-11)
#pragma unroll
        for (int c = 0; c < 8; c++) {
            const int col = ord[c];
            _Float16 hh, ll;
            q4_fix_split(c0 + col < K ? xv[q][col >> 2][col & 3] * scale : 0.f, hh, ll);
            hv[c] = __builtin_bit_cast(uint16_t, hh);
            lv[c] = __builtin_bit_cast(uint16_t, ll);
            sh += (float)hh;
            sl += (float)ll;
        }
        sh += __shfl_xor(sh, 1);
        sh += __shfl_xor(sh, 2);
        sl += __shfl_xor(sl, 1);
        sl += __shfl_xor(sl, 2);
        if (item < SPW * 16) {
            uint4* dst = (uint4*)lw + item * 2;
            dst[0] = make_uint4(hv[0] | (hv[1] << 16), hv[2] | (hv[3] << 16), hv[4] | (hv[5] << 16),
                                hv[6] | (hv[7] << 16));
            dst[1] = make_uint4(lv[0] | (lv[1] << 16), lv[2] | (lv[3] << 16), lv[4] | (lv[5] << 16),
                                lv[6] | (lv[7] << 16));
            if ((item & 3) == 0) {  // A rows 0..7: the hi bias, 8..15: the lo bias (every row the same token)
#pragma unroll
                for (int c = 0; c < 8; c++) {
                    lb[(item >> 2) * 16 + c] = sh * Q4_BIAS;
                    lb[(item >> 2) * 16 + 8 + c] = sl * Q4_BIAS;
                }
            }
        }
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // (the wave's own slice: no barrier)
    const uint4* X = (const uint4*)lw + p;
    const float4v* LB = (const float4v*)lb;
    float4v acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int u = 0; u < SPW; u++) {
#pragma unroll
        for (int tq = 0; tq < 4; tq++) {
            const int q = (u * 4 + tq) * 4 + s;
            const half8 xa = __builtin_bit_cast(half8, X[q * 2]);
            const float4v cb = LB[(u * 4 + tq) * 4 + s];
            const uint32_t wq = tq == 0 ? wv[u].x : tq == 1 ? wv[u].y : tq == 2 ? wv[u].z : wv[u].w;
            const float4v dd = __builtin_amdgcn_mfma_f32_16x16x32_f16(xa, dq_nib_word(wq), cb, 0, 0, 0);
            const uint32_t sw = tq < 2 ? sv[u].x : sv[u].y;
            const float sc = f16_bits_to_f32((tq & 1) ? sw >> 16 : sw & 0xFFFFu);
#pragma unroll
            for (int v = 0; v < 4; v++) acc[v] += dd[v] * sc;
        }
    }
    // D row 0 (hi, lanes s = 0) + D row 8 (lo, lanes s = 2)
    const float val = (acc[0] + __shfl_xor(acc[0], 32)) * xsl * 16777216.0f;  // 2^24: denormal nibbles
    if (s == 0) res[i][r] = val;
    if (lane == 0) resw[i] = wi;
    __syncthreads();
    if (i == 0 && lane < 16) {
        const int row = 16 * rb + lane;
        float v[16], ws[16];
        for (int q = 0; q < k; q++) {
            v[q] = res[q][lane];
            ws[q] = resw[q];
        }
        float a2 = 0.0f;
        for (int q = 0; q < k; q++) a2 += ws[q] * v[q];
        if (row < rows) {
            float* o = out + (size_t)t * ldo + row;
            *o = resid ? *o + a2 : a2;
        }
    }
    (void)nrb;
}
typedef void (*MoeDownTok)(const GemvDesc*, const int*, const int*, const float*, int, const float*, size_t, int, int,
                           int, int, float*, int, int);
// the instance for rows of nk 1 KiB steps (nullptr: none), its dynamic LDS
// attribute set once
MoeDownTok moe_down_tok_pick(int nk) {
    static MoeDownTok tab[9] = {nullptr,
                                k_moe_down_tok<1>,
                                k_moe_down_tok<2>,
                                k_moe_down_tok<3>,
                                k_moe_down_tok<4>,
                                k_moe_down_tok<5>,
                                k_moe_down_tok<6>,
                                k_moe_down_tok<7>,
                                k_moe_down_tok<8>};
    static std::once_flag once;
    static bool ok = true;
    std::call_once(once, [] {
        for (int n = 1; n <= 8; n++)
            if (hipFuncSetAttribute((const void*)tab[n], hipFuncAttributeMaxDynamicSharedMemorySize,
                                    16 * (n * 32 * 16 + n * 4 * 64)) != hipSuccess)
                ok = false;
        (void)hipGetLastError();
    });
    return ok && nk >= 1 && nk <= 8 ? tab[nk] : nullptr;
}

typedef void (*MoeKernel)(MoeGx);
template <int RBW, int KP, int SPW>
MoeKernel moe_q4t_inst(bool gu, int* nw, int* rbw) {
    *nw = RBW * KP;
    *rbw = RBW;
    return gu ? k_moe_q4t<RBW, KP, SPW, true> : k_moe_q4t<RBW, KP, SPW, false>;
}
// Whether k may take lds bytes of dynamic LDS (allowed once per kernel up
// to what the CU's 160 KiB leave beside its static LDS).
bool moe_lds_ok(MoeKernel k, size_t lds) {
    static std::mutex mu;
    static std::map<const void*, size_t> cap;
    std::lock_guard<std::mutex> g(mu);
    auto it = cap.find((const void*)k);
    if (it == cap.end()) {
        hipFuncAttributes fa{};
        size_t st = 0;
        if (hipFuncGetAttributes(&fa, (const void*)k) == hipSuccess) st = fa.sharedSizeBytes;
        size_t c = 160 * 1024 > st ? 160 * 1024 - st : 0;
        if (hipFuncSetAttribute((const void*)k, hipFuncAttributeMaxDynamicSharedMemorySize, (int)c) != hipSuccess) c = 0;
        (void)hipGetLastError();
        it = cap.emplace((const void*)k, c).first;
    }
    return lds <= it->second;
}
// the instance for rows of nk 1 KiB steps (nullptr: none); *nw = its waves
// (measured on MI355X, config 5: four row blocks per workgroup, gate|up
// in two K halves of 8 steps: 16.7 us; 8 x 2: 19.2, 2 x 2: 18.2, 4 x 4
// halves of 4: 16.7, 8 row blocks of whole rows: 30.6; down 4 x 1 x 6
// steps: 10.7 us; 8 x 1: 10.9, 4 x 2 x 3: 10.8, 2 x 1: 11.6).  The
// gate|up instances with two K parts are held to 6 waves per SIMD (<= 80
// VGPRs, no spill): three 8-wave workgroups per CU instead of two, so the
// config-5 grid of 840 workgroups takes ~1.1 dispatch rounds instead of
// ~1.6 (gate|up 16.7 -> 16.1 us; the down instances spill at that bound,
// and 4 x 2 x 3 there at 64 VGPRs was no faster)
MoeKernel moe_q4t_pick(int nk, bool gu, int* nw, int* rbw) {
    if (nk <= 2) return moe_q4t_inst<4, 1, 2>(gu, nw, rbw);
    if (nk <= 4) return moe_q4t_inst<4, 1, 4>(gu, nw, rbw);
    if (nk <= 6) return moe_q4t_inst<4, 1, 6>(gu, nw, rbw);
    if (nk <= 8) return moe_q4t_inst<4, 1, 8>(gu, nw, rbw);
    if (nk <= 12) return moe_q4t_inst<4, 2, 6>(gu, nw, rbw);
    if (nk <= 16) return moe_q4t_inst<4, 2, 8>(gu, nw, rbw);
    return nullptr;
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
    int *idx = nullptr, *jobs = nullptr, *slot = nullptr, *jt = nullptr;
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
    if (!numbered)
        hipLaunchKernelGGL(k_moe_jobs, dim3(1), dim3(256), 0, s, m->idx, b, k, m->ne, m->jobs, m->slot, m->jt);
    int rc = prepared ? CMF_OK : launch_prep_src(m->gu[0], x, b, m->px, m->xsx, s);
    const int mj = std::min(m->max_jobs, b * k);
    const size_t ygu_stride = (size_t)MAXB * 2 * I, yd_stride = (size_t)MAXB * H;
    if (rc != CMF_OK) return rc;
    // q4t experts and at most 8 tokens: the GEMVs over each job's own tokens
    // (CMF_MOE_GATHER=0 keeps the all-rows grouped GEMVs)
    static const bool gather_env = [] {
        const char* v = getenv("CMF_MOE_GATHER");
        return !(v && *v == '0');
    }();
    int sp1 = 0, sp2 = 0, rw1 = 1, rw2 = 1;  // waves, row blocks per workgroup
    const DevWeight &gw = m->gu[0], &dw = m->down[0];
    MoeKernel kg = nullptr, kd = nullptr;
    if (gather_env && b <= 8 && gw.dtype == DT_Q4T && dw.dtype == DT_Q4T) {
        kg = moe_q4t_pick(gw.kchunks, true, &sp1, &rw1);
        kd = moe_q4t_pick(dw.kchunks, false, &sp2, &rw2);
    }
    // LDS: the operand rows of up to b tokens + the tile biases
    const size_t lg = (size_t)gw.kchunks * (b * 512 + 256), ld = (size_t)dw.kchunks * (b * 512 + 256);
    if (kg && kd && moe_lds_ok(kg, lg) && moe_lds_ok(kd, ld)) {
        // gate|up -> h = silu(g) * u [job][t][I] (in the ygu area), then
        // down over the listed h rows -> yd [job][t][H]
        MoeGx g{};
        g.desc = m->d_gu;
        g.jobs = m->jobs;
        g.jt = m->jt;
        g.planes = m->px;
        g.xs = m->xsx;
        g.y = m->ygu;
        g.y_stride = (size_t)MAXB * I;
        g.ldy = I;
        g.M = b;
        g.nk = gw.kchunks;
        g.rows = gw.rows;
        g.ns = b;
        g.nrb = gw.rows_pad / 16;
        hipLaunchKernelGGL(kg, dim3((g.nrb + rw1 - 1) / rw1, mj), dim3(64 * sp1), lg, s, g);
        static const bool tok_env = [] {
            const char* v = getenv("CMF_MOE_DOWN_TOK");
            return !(v && *v == '0');
        }();
        MoeDownTok kt = numbered && tok_env && k <= 16 ? moe_down_tok_pick(dw.kchunks) : nullptr;
        if (kt) {
            // routed (no expert twice in a token's picks): down + combine per
            // (row block, token), one wave per rank
            const size_t lt = (size_t)k * (dw.kchunks * 32 * 16 + dw.kchunks * 4 * 64);
            hipLaunchKernelGGL(kt, dim3(dw.rows_pad / 16, b), dim3(64 * k), lt, s, m->d_down, m->idx, m->slot, m->w,
                               k, m->ygu, (size_t)MAXB * I, I, I, dw.rows_pad / 16, dw.rows, d_out, ldo,
                               resid ? 1 : 0);
            return CMF_OK;
        }
        MoeGx d = g;
        d.desc = m->d_down;
        d.planes = nullptr;  // (the operand from the h rows themselves)
        d.xs = nullptr;
        d.hx = m->ygu;
        d.hx_stride = (size_t)MAXB * I;
        d.ldh = I;
        d.K = I;
        d.y = m->yd;
        d.y_stride = yd_stride;
        d.ldy = H;
        d.nk = dw.kchunks;
        d.rows = dw.rows;
        d.nrb = dw.rows_pad / 16;
        hipLaunchKernelGGL(kd, dim3((d.nrb + rw2 - 1) / rw2, mj), dim3(64 * sp2), ld, s, d);
    } else {
        rc = gemv_grouped(gw, m->d_gu, m->jobs, mj, m->px, 0, m->xsx, m->ygu, ygu_stride, 2 * I, b, s);
        if (rc != CMF_OK) return rc;
        XSrc sg{};
        sg.mode = XS_SILU8;  // (gate|up rows interleaved 8 / 8)
        sg.x = m->ygu;
        sg.ldx = 2 * I;
        sg.K = I;
        rc = launch_prep_src_grouped(dw, sg, b, m->jobs, mj, ygu_stride, m->ph, m->ph_stride, m->xsh, s);
        if (rc == CMF_OK)
            rc = gemv_grouped(dw, m->d_down, m->jobs, mj, m->ph, m->ph_stride, m->xsh, m->yd, yd_stride, H, b, s);
        if (rc != CMF_OK) return rc;
    }
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
                       m->ne, m->top_k, m->norm_topk, m->scaling, m->idx, m->w, m->jobs, m->slot, m->jt, x, K,
                       g.dtype, nk, m->px, m->xsx);
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
        moe_alloc(m, (void**)&m->jt, sizeof(int) * MOE_JT * mj) ||
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
    // gate and up interleaved 8 / 8 per row block (the SwiGLU pairs in one block)
    if (build_swiglu(gu, gate, up) != CMF_OK) return CMF_ERR;
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
