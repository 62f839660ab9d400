// XCD-partitioned decoder blocks for gfx950 (MI355X).
//
// One Qwen3-arch block (rms_norm -> q/k/v -> qk-norm + RoPE -> causal
// attention over the KV cache -> output projection -> residual; rms_norm ->
// gate/up -> SwiGLU -> down -> residual: forward_layers_span,
// pipeline.rs:7981-8700) as two launches of 8 x 32 workgroups.  The hardware
// dispatches a launch's workgroups round-robin over the 8 XCDs (workgroup i
// on XCD (c + i) % 8, c depending on the launches before it), so each
// workgroup takes its XCD x from HW_REG_XCC_ID and its index j = i / 8 among
// the XCD's 32; those share one L2 and hand data to each other through it:
// each value is
// written as a 64-bit (tag, value) pair and read with L1-bypassing
// (agent-scope) loads until the tag of this launch appears.  No cache
// writeback or fence is needed inside an XCD, and a hand-off costs about
// one L2 round trip, far less than a kernel boundary.
//
// XCD x owns kv head x (its query heads, k and v rows, its cache), the x-th
// slice of the FFN's intermediate dimension and the matching K slices of the
// output and down projections, so every reduction that crosses XCDs is one
// of the two residual sums, left as eight per-XCD partials that the next
// launch adds while it loads its operand (kernel boundary = visibility).
//
// Attention launch (k_xl_attn), per XCD:
//   0. q|k|v rows of the XCD, split over K: workgroup (row part, 64-column
//      chunk) quantizes its chunk of h * w_norm (int8 planes, its own scale)
//      and writes partial dot products and its share of sum(h^2);
//   1. workgroup j sums the partials of 16 rows in chunk order and applies
//      1 / rms (rms_norm's row factor moves past the matvec);
//   2. attention: workgroup j takes an equal share of 16-position tiles of
//      [0, pos0 + nb); q-norm + RoPE of the queries, k-norm + RoPE and the
//      cache append of new rows, scores on the f16 MFMA from hi / lo halves
//      of q and k (q_h k_h + q_h k_l + q_l k_h, 22-bit operands, f32
//      accumulation; the host keeps layers whose qk-norm weights could take
//      |q|, |k| past the f16 range on the six-launch path), softmax, values
//      on the fp32 MFMA (K and V of its cached positions were requested at
//      kernel start by waves 4-7, so that stream overlaps steps 0-1);
//   3. workgroup j merges 8 output dims over the 32 position shares;
//   4. output projection rows [32 j, 32 j + 32) over the XCD's K slice
//      (weights requested at kernel start) -> partial pa[x].
// FFN launch (k_xl_ffn), per XCD:
//   0. gate|up rows of the XCD's inter slice, split over K (128-column
//      groups, f16 hi/lo planes, q4t tiles on the f16 MFMA);
//   1. sums in group order, 1 / rms, silu(g) * u of 12 inter indices;
//   2. down projection rows [32 j, 32 j + 32) over the slice -> pb[x].
// Every wait is bounded: a wait that gives up sets err and the launch still
// completes (wrong values, reported by the host).  The launch needs all 256
// workgroups resident at once (one per CU, the host checks 256 CUs) and
// dealt to the XCDs in turn: each workgroup first swaps the launch's tag
// into the claim slot of its (XCD, index); finding the tag there already
// (two workgroups on one slot, so another slot has none) sets err bit 8,
// which also ends every wait of the launch early.  The host then switches
// the model to the six-launch blocks and runs the call again.
#include <math.h>

#include "common.h"
#include "gemv.h"
#include "gemv_kern.h"
#include "layers.h"
#include "wave.h"
#include "xlayer.h"

namespace cmf {

namespace {

constexpr int XL_SPIN = 1 << 16;  // polls before a wait gives up (~50 ms)

// Phase timestamps for tuning builds (XL_STAMPS defined before this file is
// compiled: lane 0 of waves 0 and 4 of every workgroup records
// s_memrealtime at the marks into stamps[workgroup][wave / 4][32], the
// buffer a kernel argument so that a mark waits for no memory operation).
#ifdef XL_STAMPS
unsigned long long* xl_stamp_buf = nullptr;  // host: the buffer the launches pass
#define XL_MARK(k)                                                                               \
    do {                                                                                         \
        if ((threadIdx.x & 255) == 0 && a.stamps)                                                \
            a.stamps[(blockIdx.x * 2 + (threadIdx.x >> 8)) * 32 + (k)] = __builtin_amdgcn_s_memrealtime(); \
    } while (0)
#else
#define XL_MARK(k) \
    do {           \
    } while (0)
#endif

__device__ __forceinline__ uint32_t xcc_id() {
    uint32_t v;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID, 0, 4)" : "=s"(v));
    return v;
}

// (tag, value) pair: one aligned 64-bit store (a single global_store_dwordx2,
// written whole), visible to the XCD's other CUs once it reaches the shared L2
// (the L1 writes through).  A plain store: measured on MI355X, an agent-scope
// (sc1) store takes 0.66 us per hand-off against 0.41 us; a volatile one
// waits for its write-through after every store.
__device__ __forceinline__ void xput(uint64_t* p, float v, uint32_t tag) {
    *p = ((uint64_t)tag << 32) | (uint64_t)__float_as_uint(v);
}
// agent-scope load (sc1): misses the CU's L1, so another CU's store is seen
// (a plain or sc0 load can keep returning the L1's stale line)
__device__ __forceinline__ uint64_t xraw(const uint64_t* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// The N values at addr(0..N-1) once each carries tag: all requested at once,
// the missing ones polled again.
template <int N, class F>
__device__ __forceinline__ void xget(F addr, uint32_t tag, float (&out)[N], int* err) {
    uint64_t v[N];
#pragma unroll
    for (int i = 0; i < N; i++) v[i] = xraw(addr(i));
    for (int it = 0;; it++) {
        bool ok = true;
#pragma unroll
        for (int i = 0; i < N; i++) ok = ok && (uint32_t)(v[i] >> 32) == tag;
        if (ok) break;
        if (it >= XL_SPIN) {
            atomicOr(err, 1);
            break;
        }
        // a misplaced launch (err bit 8, set at kernel start) never delivers
        // some of the values: give up at once instead of after XL_SPIN polls
        if ((it & 255) == 255 && (__hip_atomic_load(err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) & 8)) break;
        __builtin_amdgcn_s_sleep(1);
#pragma unroll
        for (int i = 0; i < N; i++)
            if ((uint32_t)(v[i] >> 32) != tag) v[i] = xraw(addr(i));
    }
#pragma unroll
    for (int i = 0; i < N; i++) out[i] = __uint_as_float((uint32_t)v[i]);
}

// Workgroup barrier over LDS only.  The waves of a workgroup share data
// only through LDS here (global memory goes to other workgroups, tagged, or
// to the next launch), so the barrier need not wait for the wave's global
// loads: __syncthreads() would (vmcnt(0)), and waves 4-7 would hold every
// barrier until their K / V / weight prefetch had landed.
// (A workgroup fence restricted to LDS still made the compiler wait for the
// wave's global stores before the barrier.)
__device__ __forceinline__ void lds_barrier() {
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// x ~= sx (q0 + q1/128 + q2/16384): the three int8 digits of v = x / sx
// (|v| <= 127, as q8_split)
__device__ __forceinline__ void q8_digits(float v, int8_t& d0, int8_t& d1, int8_t& d2) {
    const float q0 = rintf(v);
    const float r1 = (v - q0) * 128.0f;
    const float q1 = rintf(r1);
    const float q2 = rintf((r1 - q1) * 128.0f);
    d0 = (int8_t)q0;
    d1 = (int8_t)q1;
    d2 = (int8_t)q2;
}

typedef _Float16 half4 __attribute__((ext_vector_type(4)));
// x = hi + lo in f16 (22 significant bits while |x| < 65504: the score
// operands q and k after their RMS norms, |.| <= sqrt(128) max|norm weight|)
__device__ __forceinline__ void split16(float x, _Float16& hi, _Float16& lo) {
    hi = (_Float16)x;
    lo = (_Float16)(x - (float)hi);
}

// slot of tile element e (0..7 of a k-slot) in the MFMA operand order
// {0,4,2,6,1,5,3,7} (the nibble-pair order of dq_nib_word); an involution
__device__ __forceinline__ int nib_slot(int e) { return ((e & 1) << 2) | (e & 2) | ((e >> 2) & 1); }

// Reductions over a DPP row (16 lanes) or a quad (4 lanes) in registers
// (no LDS permutes): quad swaps, row_shr 4 and 8 (the row's total in lane
// 15), row_newbcast 15 hands it to the row's 16 lanes.
template <int CTRL>
__device__ __forceinline__ float dppf(float v, float ident) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, ident),
                                                                 __builtin_bit_cast(int, v), CTRL, 0xf, 0xf, false));
}
template <int CTRL>
__device__ __forceinline__ double dppd(double v) {
    const uint64_t u = __builtin_bit_cast(uint64_t, v);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)u, CTRL, 0xf, 0xf, false);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)(u >> 32), CTRL, 0xf, 0xf, false);
    return __builtin_bit_cast(double, ((uint64_t)hi << 32) | lo);
}
__device__ __forceinline__ float quad_sum(float v) {
    v += dppf<0xb1>(v, 0.f);
    return v + dppf<0x4e>(v, 0.f);
}
__device__ __forceinline__ float row_sum(float v) {
    v = quad_sum(v);
    v += dppf<0x114>(v, 0.f);
    v += dppf<0x118>(v, 0.f);
    return dppf<0x15F>(v, 0.f);
}
__device__ __forceinline__ double row_sum_d(double v) {
    v += dppd<0xb1>(v);
    v += dppd<0x4e>(v);
    v += dppd<0x114>(v);
    v += dppd<0x118>(v);
    return dppd<0x15F>(v);
}
__device__ __forceinline__ float row_max(float v) {
    v = fmaxf(v, dppf<0xb1>(v, -INFINITY));
    v = fmaxf(v, dppf<0x4e>(v, -INFINITY));
    v = fmaxf(v, dppf<0x114>(v, -INFINITY));
    v = fmaxf(v, dppf<0x118>(v, -INFINITY));
    return dppf<0x15F>(v, -INFINITY);
}

struct XlAArgs {
    const float* hb;     // input rows [nb][H]
    const float* parts;  // previous FFN partials [8][MAXB][H] (nullptr: none)
    float* hout;         // h_in = hb (+ parts) [nb][H]
    const float* nw;     // input norm [H]
    const int4v* wqkv;   // q8 device blocks
    const float* sqkv;
    const int4v* wo;
    const float* so;
    int nkco;            // 64-column chunks of wo
    const float *qn, *kn;
    const float2* rope;
    float *kc, *vc;
    const int* pbase;
    int padd;
    float* pout;         // output projection partials [8][MAXB][H]
    uint64_t *e0, *e1, *e2, *e3;
    int e0s, e1s;
    const uint32_t* gen;
    int call;
    int* err;
    uint32_t* claim;  // [8][32] the launch tag of each (XCD, index) slot
    int nb, H, nh, max_seq;
    double eps;
    unsigned long long* stamps;  // tuning builds only (XL_STAMPS)
};

struct XlBArgs {
    const float* hb;     // h_in [nb][H]
    const float* parts;  // output projection partials [8][MAXB][H]
    float* hout;         // h_mid = hb + parts
    const float* nw;     // post-attention norm
    const uint4* wgu;
    const uint64_t* sgu;
    int ntg_gu;
    const uint4* wdn;
    const uint64_t* sdn;
    int ntg_dn;
    float* pout;         // down projection partials [8][MAXB][H]
    uint64_t *e0, *e1;
    int e0s, e1s;
    const uint32_t* gen;
    int call;
    int* err;
    uint32_t* claim;  // [8][32] the launch tag of each (XCD, index) slot
    int nb, H;
    double eps;
    unsigned long long* stamps;  // tuning builds only (XL_STAMPS)
};

// ---------------------------------------------------------------------------
// attention launch
// ---------------------------------------------------------------------------
// HPK query heads per kv head, NKC = H / 64 (K chunks of the q|k|v rows),
// BT = 16-position tiles a workgroup holds (<= XL_BT; the K / V requests
// cover BT tiles whatever the share, so the host picks the smallest BT the
// call's position bound needs).
template <int HPK, int NKC, int BT>
__global__ __launch_bounds__(XL_T) void k_xl_attn(XlAArgs a) {
    constexpr int HD = 128, NKV = XL_XCD;
    constexpr int RX = (HPK + 2) * HD;         // q|k|v rows of one XCD
    constexpr int RP = XL_WG / NKC;            // row parts of step 0
    constexpr int NRB0 = RX / 16 / RP;         // row blocks per workgroup in step 0
    constexpr int RBW = NRB0 / 4;              // ... per wave (waves 0-3)
    constexpr int ROWS0 = NRB0 * 16;
    constexpr int RW = RX / XL_WG;             // rows reduced per workgroup in step 1
    constexpr int QD = HPK * HD;               // the XCD's query dims (its K slice of wo)
    constexpr int QC = QD / 64;                // ... in 64-column chunks
    constexpr int RBO = NKC / 8;               // wo row blocks per workgroup (H / 512)
    constexpr int WPR = 4 / RBO;               // waves per wo row block (waves 4-7)
    constexpr int CW = QC / WPR;               // wo chunks per wave
    constexpr int DJ = QD / XL_WG;             // merged dims per workgroup
    constexpr int NPOS = BT * 16;
    constexpr int KVN = NPOS * 32 / 256;       // float4 of K (and of V) per thread of waves 4-7
    static_assert(NRB0 % 4 == 0 && RP * NKC == XL_WG && RW <= 16 && WPR * RBO == 4 && DJ >= 1 && BT <= XL_BT, "shape");

    // the XCD this workgroup runs on; workgroups i and i + 8 share one, so
    // blockIdx / 8 numbers the 32 workgroups of each XCD
    const int x = (int)xcc_id() & 7, j = blockIdx.x >> 3;
    const int t = threadIdx.x, lane = t & 63, wave = __builtin_amdgcn_readfirstlane(t >> 6);
    const int r = lane & 15, s = lane >> 4;
    const int nb = a.nb, H = a.H;
    const uint32_t tag = *a.gen * 256u + (uint32_t)a.call;
    int* err = a.err;
    if (t == 0 && atomicExch(a.claim + x * XL_WG + j, tag) == tag) atomicOr(err, 8);

    // LDS: K / V tiles (positions of this workgroup), queries, scores; the
    // step-4 operand and planes overlay the K tiles
    // (K and Q rows as f16 hi / lo planes [row][dim], padded against bank
    // conflicts; V rows f32; scores, then the softmax weights in place)
    constexpr int KS = HD + 8;
    __shared__ __align__(16) _Float16 KHL[2][NPOS][KS];
    __shared__ __align__(16) float VT[NPOS][HD + 4];
    __shared__ __align__(16) _Float16 QHL[2][XL_NQ][KS];
    __shared__ __align__(16) float S[XL_NQ][NPOS + 4];
    __shared__ __align__(16) int8_t P8[3 * 4 * 16 * 16];
    __shared__ float sx0[MAXB], sxo[MAXB];
    __shared__ double ssd[MAXB], ssp[MAXB][NKC];
    static_assert(3 * QC * 1024 + 12 * 64 * 16 <= 2 * NPOS * (HD + 8) * 2, "overlay");

    const int kc = j % NKC, rp = j / NKC;
    const int pos0 = *a.pbase + a.padd;
    const int P = pos0 + nb, T = (P + 15) >> 4;
    // shares rounded up: the extra tiles of T % 32 go to the first
    // workgroups, not to the last one, which also appends the new rows
    const int tlo = (j * T + XL_WG - 1) / XL_WG;
    int thi = ((j + 1) * T + XL_WG - 1) / XL_WG;
    if (thi - tlo > BT) {  // more positions than the host's bound admitted
        if (t == 0) atomicOr(err, 4);
        thi = tlo + BT;
    }
    const int plo = tlo * 16, phi = min(thi * 16, P);
    const int np = max(0, phi - plo), nold = max(0, min(phi, pos0) - plo);
    const int ntile = thi - tlo;
    XL_MARK(0);


    // ---- requests: waves 0-3 the step-0 weights and operand; waves 4-7 the
    // output projection's weights and this workgroup's cached K / V
    int4v wq[RBW];
    float rsq[RBW];
    float4v hv4 = {0.f, 0.f, 0.f, 0.f}, pv4[8], wn4 = hv4;
    int4v wov[CW];
    float rso = 0.f;
    float4v kq[KVN], vq[KVN];
    if (wave < 4) {
        // the weights first (the long HBM round trip), then the operand:
        // thread (b = t / 16, four columns) of the chunk, the row of h and
        // the eight partials as float4
#pragma unroll
        for (int i = 0; i < RBW; i++) {
            const int l = rp * NRB0 + wave + 4 * i;  // XCD row block
            const int g = l < HPK * 8       ? x * HPK * 8 + l
                          : l < HPK * 8 + 8 ? a.nh * 8 + x * 8 + (l - HPK * 8)
                                            : (a.nh + NKV) * 8 + x * 8 + (l - HPK * 8 - 8);
            wq[i] = ld_stream(a.wqkv + ((size_t)g * NKC + kc) * 64 + lane);
            rsq[i] = ldg(a.sqkv + g * 16 + r);
        }
        __builtin_amdgcn_sched_barrier(0);
        const int b = min(t >> 4, nb - 1), c = kc * 64 + 4 * (t & 15);
        hv4 = ldg((const float4v*)(a.hb + (size_t)b * H + c));
        if (a.parts) {
#pragma unroll
            for (int xx = 0; xx < 8; xx++) pv4[xx] = ldg((const float4v*)(a.parts + ((size_t)xx * MAXB + b) * H + c));
        }
        wn4 = ldg((const float4v*)(a.nw + c));
    } else {
        const int w4 = wave - 4, rbl = w4 % RBO, cs = w4 / RBO, g = j * RBO + rbl;
#pragma unroll
        for (int i = 0; i < CW; i++)
            wov[i] = ld_stream(a.wo + ((size_t)g * a.nkco + x * QC + cs + WPR * i) * 64 + lane);
        rso = ldg(a.so + g * 16 + r);
        const int t4 = t - 256;
        const float* kb = a.kc + (size_t)x * a.max_seq * HD;
        const float* vb = a.vc + (size_t)x * a.max_seq * HD;
#pragma unroll
        for (int u = 0; u < KVN; u++) {
            const int f = t4 + 256 * u, sl = f >> 5, c4 = f & 31;
            const size_t off = (size_t)(sl < nold ? plo + sl : 0) * HD + 4 * c4;
            kq[u] = __builtin_nontemporal_load(gptr((const float4v*)(kb + off)));
            vq[u] = __builtin_nontemporal_load(gptr((const float4v*)(vb + off)));
        }
    }

    XL_MARK(1);
    // ---- step 0: this chunk of h_in * w_norm as int8 planes (waves 0-3),
    // thread (b = t / 16, columns 4 (t % 16) ..): the row's statistics over
    // its 16 lanes; h_in written by XCD 0
    if (wave < 4) {
        const int b = t >> 4, c4 = t & 15;
        float4v h = hv4;
        if (a.parts) {
#pragma unroll
            for (int xx = 0; xx < 8; xx++) h += pv4[xx];
        }
        if (b < nb && x == 0 && rp == 0) *(float4v*)(a.hout + (size_t)b * H + kc * 64 + 4 * c4) = h;
        const double ss = row_sum_d((double)h[0] * (double)h[0] + (double)h[1] * (double)h[1] +
                                     (double)h[2] * (double)h[2] + (double)h[3] * (double)h[3]);
        const float4v u = h * wn4;
        const float am = row_max(fmaxf(fmaxf(fabsf(u[0]), fabsf(u[1])), fmaxf(fabsf(u[2]), fabsf(u[3]))));
        const float sx = am > 0.f ? am / 127.0f : 1.0f;
        uint32_t w0 = 0, w1 = 0, w2 = 0;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            int8_t d0, d1, d2;
            q8_digits(u[i] / sx, d0, d1, d2);
            w0 |= (uint32_t)(uint8_t)d0 << (8 * i);
            w1 |= (uint32_t)(uint8_t)d1 << (8 * i);
            w2 |= (uint32_t)(uint8_t)d2 << (8 * i);
        }
        if (b < nb) {
            const int o = ((c4 >> 2) * 16 + b) * 16 + 4 * (c4 & 3);
            *(uint32_t*)&P8[o] = w0;
            *(uint32_t*)&P8[1024 + o] = w1;
            *(uint32_t*)&P8[2048 + o] = w2;
            if (c4 == 0) {
                sx0[b] = sx;
                ssd[b] = ss;
            }
        }
    }
    XL_MARK(13);
    lds_barrier();
    XL_MARK(14);
    uint64_t* e0w = a.e0 + (size_t)(x * XL_WG + j) * MAXB * a.e0s;
    // step 1's thread (row, b1): XCD row R1; its partials and share in pv1
    const bool on1 = t < RW * nb, ss_on = t < NKC * nb;
    const int b1 = min(t / RW, nb - 1), R1 = j * RW + t % RW;
    const int rpp = R1 / ROWS0, lrow = R1 % ROWS0;
    float pv1[NKC + 2];
    if (wave < 4) {
        const int4v* A = (const int4v*)P8;
        const int4v a0 = A[s * 16 + r], a1 = A[64 + s * 16 + r], a2 = A[128 + s * 16 + r];
        const int4v z = {0, 0, 0, 0};
#pragma unroll
        for (int i = 0; i < RBW; i++) {
            const int4v d0 = __builtin_amdgcn_mfma_i32_16x16x64_i8(a0, wq[i], z, 0, 0, 0);
            const int4v d1 = __builtin_amdgcn_mfma_i32_16x16x64_i8(a1, wq[i], z, 0, 0, 0);
            const int4v d2 = __builtin_amdgcn_mfma_i32_16x16x64_i8(a2, wq[i], z, 0, 0, 0);
            const int lrow = (wave + 4 * i) * 16 + r;
#pragma unroll
            for (int v = 0; v < 4; v++) {
                const int b = 4 * s + v;
                if (b < nb) {
                    const float val = ((float)d0[v] + (float)d1[v] * 0.0078125f + (float)d2[v] * 6.103515625e-05f) *
                                      sx0[b] * rsq[i];
                    xput(e0w + (size_t)b * a.e0s + lrow, val, tag);
                }
            }
        }
        if (t < nb) {
            const double ss = ssd[t];
            const float hi = (float)ss, lo = (float)(ss - (double)hi);
            xput(e0w + (size_t)t * a.e0s + ROWS0, hi, tag);
            xput(e0w + (size_t)t * a.e0s + ROWS0 + 1, lo, tag);
        }
        XL_MARK(2);
        // ---- step 1: rows [RW j, RW j + RW) of the XCD: thread (row, b)
        // waits for its NKC chunk partials and, at once, for one of the
        // sum(h^2) shares (chunk t % NKC, row t / NKC; row part 0)
        const int ks = ss_on ? t % NKC : 0, bs = ss_on ? t / NKC : 0;
        const uint64_t* pss = a.e0 + ((size_t)(x * XL_WG + ks) * MAXB + bs) * a.e0s + ROWS0;
        if (on1 || ss_on) {  // (only the threads that own a row or a share poll)
            xget<NKC + 2>(
                [&](int k) {
                    return k < NKC ? a.e0 + ((size_t)(x * XL_WG + rpp * NKC + k) * MAXB + b1) * a.e0s + lrow
                                   : pss + (k - NKC);
                },
                tag, pv1, err);
            if (ss_on) ssp[bs][ks] = (double)pv1[NKC] + (double)pv1[NKC + 1];
        }
    } else {
        // waves 4-7: the cached K (as f16 hi / lo) and V of this workgroup's
        // positions into LDS; V rows past its share zeroed (their weights
        // are 0)
        const int t4 = t - 256;
#pragma unroll
        for (int u = 0; u < KVN; u++) {
            const int f = t4 + 256 * u, sl = f >> 5, c4 = f & 31;
            if (sl < nold) {
                half4 kh, kl;
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    _Float16 h, l;
                    split16(kq[u][i], h, l);
                    kh[i] = h;
                    kl[i] = l;
                }
                *(half4*)&KHL[0][sl][4 * c4] = kh;
                *(half4*)&KHL[1][sl][4 * c4] = kl;
                *(float4v*)&VT[sl][4 * c4] = vq[u];
            } else if (sl >= np) {
                *(float4v*)&VT[sl][4 * c4] = float4v{0.f, 0.f, 0.f, 0.f};
            }
        }
    }
    XL_MARK(3);
    lds_barrier();
    if (wave < 4) {
        // the partials in chunk order, times 1 / rms (inference.rs:33-50: f64
        // mean of squares)
        if (on1) {
            double ss = 0.0;
#pragma unroll
            for (int k = 0; k < NKC; k++) ss += ssp[b1][k];
            const float inv = (float)(1.0 / sqrt(ss / (double)H + a.eps));
            float acc = 0.f;
#pragma unroll
            for (int k = 0; k < NKC; k++) acc += pv1[k];
            xput(a.e1 + ((size_t)x * MAXB + b1) * a.e1s + R1, acc * inv, tag);
        }
    }

    XL_MARK(4);
    // ---- step 2a: queries (q-norm + RoPE, attention.rs:606-624, 818-890)
    // and the new rows of this workgroup's positions (k-norm + RoPE, appended
    // to the cache), one wave per row, lane = rotation pair (lane, lane + 64)
    const int nq = HPK * nb;
    const uint64_t* e1x = a.e1 + (size_t)x * MAXB * a.e1s;
    for (int qi = wave; qi < nq; qi += 8) {
        const int b = qi / HPK, hh = qi % HPK;
        float v2[2];
        xget<2>([&](int i) { return e1x + (size_t)b * a.e1s + hh * HD + lane + 64 * i; }, tag, v2, err);
        const float2 o = norm_rope(v2[0], v2[1], a.qn[lane], a.qn[lane + 64], a.rope[(size_t)(pos0 + b) * 64 + lane],
                                   a.eps);
        split16(o.x, QHL[0][qi][lane], QHL[1][qi][lane]);
        split16(o.y, QHL[0][qi][lane + 64], QHL[1][qi][lane + 64]);
    }
    {
        const int blo = max(0, plo - pos0), bhi = min(nb, phi - pos0);
        for (int b = blo + wave; b < bhi; b += 8) {
            float v4[4];
            xget<4>([&](int i) { return e1x + (size_t)b * a.e1s + QD + (i >> 1) * HD + lane + 64 * (i & 1); }, tag, v4,
                    err);
            const int pos = pos0 + b, sl = pos - plo;
            const float2 k = norm_rope(v4[0], v4[1], a.kn[lane], a.kn[lane + 64], a.rope[(size_t)pos * 64 + lane],
                                       a.eps);
            split16(k.x, KHL[0][sl][lane], KHL[1][sl][lane]);
            split16(k.y, KHL[0][sl][lane + 64], KHL[1][sl][lane + 64]);
            VT[sl][lane] = v4[2];
            VT[sl][lane + 64] = v4[3];
            float* kd = a.kc + ((size_t)x * a.max_seq + pos) * HD;
            float* vd = a.vc + ((size_t)x * a.max_seq + pos) * HD;
            kd[lane] = k.x;
            kd[lane + 64] = k.y;
            vd[lane] = v4[2];
            vd[lane + 64] = v4[3];
        }
    }
    XL_MARK(5);
    lds_barrier();
    // ---- step 2b: scores on the f16 MFMA (16x16x32) from hi / lo planes,
    // q.k = qh.kh + qh.kl + ql.kh (22 significant bits), one (tile, query
    // block) per wave: A = 16 queries, B = the tile's 16 positions; causal
    // limit pos0 + b (kv_cache.rs:521-690)
    const int nqb = (nq + 15) >> 4;
    const float scale = 1.0f / sqrtf((float)HD);
    for (int it = wave; it < ntile * nqb; it += 8) {
        const int tt = it % ntile, qb = it / ntile;
        const int qr = min(qb * 16 + r, XL_NQ - 1);
        float4v d = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < HD / 32; ks++) {
            const int o = 32 * ks + 8 * s;
            const half8 qh = *(const half8*)&QHL[0][qr][o], ql = *(const half8*)&QHL[1][qr][o];
            const half8 kh = *(const half8*)&KHL[0][tt * 16 + r][o], kl = *(const half8*)&KHL[1][tt * 16 + r][o];
            d = __builtin_amdgcn_mfma_f32_16x16x32_f16(qh, kh, d, 0, 0, 0);
            d = __builtin_amdgcn_mfma_f32_16x16x32_f16(qh, kl, d, 0, 0, 0);
            d = __builtin_amdgcn_mfma_f32_16x16x32_f16(ql, kh, d, 0, 0, 0);
        }
        const int p = plo + tt * 16 + r;
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const int q = qb * 16 + 4 * s + e;
            if (q < nq) {
                const bool see = p < phi && p <= pos0 + q / HPK;
                S[q][tt * 16 + r] = see ? d[e] * scale : -INFINITY;
            }
        }
    }
    XL_MARK(6);
    lds_barrier();
    // ---- step 2c: softmax over this workgroup's positions, one wave per
    // query: m, l to the partial, the weights e = exp(s - m) over the scores
    uint64_t* e2w = a.e2 + (size_t)(x * XL_WG + j) * XL_NQ * XL_E2S;
    const int npr = ntile * 16;
    for (int q = wave; q < nq; q += 8) {
        const float s0 = lane < npr ? S[q][lane] : -INFINITY;
        const float s1 = lane + 64 < npr ? S[q][lane + 64] : -INFINITY;
        const float m = wave_max(fmaxf(s0, s1));
        const float x0 = m == -INFINITY ? 0.f : expf(s0 - m);
        const float x1 = m == -INFINITY ? 0.f : expf(s1 - m);
        const float l = wave_sum(x0 + x1);
        if (lane < npr) S[q][lane] = x0;
        if (lane + 64 < npr) S[q][lane + 64] = x1;
        if (lane == 0) {
            xput(e2w + (size_t)q * XL_E2S, m, tag);
            xput(e2w + (size_t)q * XL_E2S + 1, l, tag);
        }
        if (npr == 0) {  // no positions: an empty share
            xput(e2w + (size_t)q * XL_E2S + 2 + lane, 0.f, tag);
            xput(e2w + (size_t)q * XL_E2S + 66 + lane, 0.f, tag);
        }
    }
    XL_MARK(7);
    lds_barrier();
    // ---- step 2d: values by fp32 MFMA (16x16x4), wave w dims 16 w .. 16 w +
    // 15: o[q][d] = sum_p e[q][p] V[p][d], two accumulators over the k steps
    // (on the f16 MFMA this pass would need V transposed in LDS: slower)
    if (npr > 0) {
        const int d0 = 16 * wave;
        for (int qb = 0; qb < nqb; qb++) {
            const float* erow = S[min(qb * 16 + r, XL_NQ - 1)];
            float4v acc[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
            for (int k = 0; k < npr / 4; k++) {
                const int p = 4 * k + s;
                acc[k & 1] = __builtin_amdgcn_mfma_f32_16x16x4f32(erow[p], VT[p][d0 + r], acc[k & 1], 0, 0, 0);
            }
            const float4v o = acc[0] + acc[1];
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const int q = qb * 16 + 4 * s + e;
                if (q < nq) xput(e2w + (size_t)q * XL_E2S + 2 + d0 + r, o[e], tag);
            }
        }
    }
    XL_MARK(8);
    // ---- step 3: merge of dims [DJ j, DJ j + DJ) over the 32 shares:
    // out = sum_c w_c o_c / sum_c w_c l_c, w_c = exp(m_c - M) (lanes = shares)
    {
        // thread (share pair js, js + 16; batch row b = t / 16): one DPP row
        // per batch row reduces the 32 shares in registers
        const int dbase = j * DJ, hh = dbase / HD, dd = dbase % HD;
        const int js = t & 15, b = t >> 4, bq = min(b, nb - 1), q = bq * HPK + hh;
        const uint64_t* s0 = a.e2 + ((size_t)(x * XL_WG + js) * XL_NQ + q) * XL_E2S;
        const uint64_t* s1 = s0 + (size_t)16 * XL_NQ * XL_E2S;
        float v[2 * (DJ + 2)];
        if (b < nb) {
            xget<2 * (DJ + 2)>(
                [&](int i) {
                    const uint64_t* sp = i < DJ + 2 ? s0 : s1;
                    const int k = i < DJ + 2 ? i : i - (DJ + 2);
                    return k < 2 ? sp + k : sp + 2 + dd + (k - 2);
                },
                tag, v, err);
        } else {
#pragma unroll
            for (int i = 0; i < 2 * (DJ + 2); i++) v[i] = i == 0 || i == DJ + 2 ? -INFINITY : 0.f;
        }
        const float* v0 = v;
        const float* v1 = v + DJ + 2;
        const float M = row_max(fmaxf(v0[0], v1[0]));
        const float w0 = v0[0] == -INFINITY ? 0.f : expf(v0[0] - M);
        const float w1 = v1[0] == -INFINITY ? 0.f : expf(v1[0] - M);
        const float L = row_sum(w0 * v0[1] + w1 * v1[1]);
        float O[DJ];
#pragma unroll
        for (int i = 0; i < DJ; i++) O[i] = row_sum(w0 * v0[2 + i] + w1 * v1[2 + i]);
        if (js == 0 && b < nb) {
            const float inv = L > 0.f ? 1.0f / L : 0.f;
#pragma unroll
            for (int i = 0; i < DJ; i++)
                xput(a.e3 + ((size_t)x * MAXB + b) * QD + dbase + i, O[i] * inv, tag);
        }
    }
    XL_MARK(9);
    // ---- step 4: output projection rows of this workgroup over the XCD's
    // K slice: the merged rows (all of them) as int8 planes with one scale
    // per row, then the MFMAs of waves 4-7 on the weights requested at start
    float* Xo = (float*)&KHL[0][0][0];
    int8_t* P8o = (int8_t*)(Xo + MAXB * QD);
    int4v* red = (int4v*)(P8o + 3 * QC * 1024);
    {
        // the nb * QD values, 4 per thread (one wait for each thread's share)
        const int n = nb * QD;
        const uint64_t* e3x = a.e3 + (size_t)x * MAXB * QD;
        for (int i0 = 4 * t; i0 < n; i0 += 4 * XL_T) {
            float ov[4];
            xget<4>([&](int i) { return e3x + i0 + i; }, tag, ov, err);
#pragma unroll
            for (int i = 0; i < 4; i++) Xo[i0 + i] = ov[i];
        }
    }
    XL_MARK(10);
    lds_barrier();
    for (int b = wave; b < nb; b += 8) {
        float vv[QC];
        float am = 0.f;
#pragma unroll
        for (int c = 0; c < QC; c++) {
            vv[c] = Xo[b * QD + 64 * c + lane];
            am = fmaxf(am, fabsf(vv[c]));
        }
        am = wave_max(am);
        const float sx = am > 0.f ? am / 127.0f : 1.0f;
        if (lane == 0) sxo[b] = sx;
#pragma unroll
        for (int c = 0; c < QC; c++) {
            int8_t d0, d1, d2;
            q8_digits(vv[c] / sx, d0, d1, d2);
            const int o = ((c * 4 + (lane >> 4)) * 16 + b) * 16 + (lane & 15);
            P8o[o] = d0;
            P8o[QC * 1024 + o] = d1;
            P8o[2 * QC * 1024 + o] = d2;
        }
    }
    XL_MARK(11);
    lds_barrier();
    const int w4 = wave - 4, rbl = w4 % RBO, cs = w4 / RBO;
    if (wave >= 4) {
        int4v c0 = {0, 0, 0, 0}, c1 = c0, c2 = c0;
        const int4v* A = (const int4v*)P8o;
#pragma unroll
        for (int i = 0; i < CW; i++) {
            const int c = cs + WPR * i;
            c0 = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[(c * 4 + s) * 16 + r], wov[i], c0, 0, 0, 0);
            c1 = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[QC * 64 + (c * 4 + s) * 16 + r], wov[i], c1, 0, 0, 0);
            c2 = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[2 * QC * 64 + (c * 4 + s) * 16 + r], wov[i], c2, 0, 0, 0);
        }
        red[(w4 * 3 + 0) * 64 + lane] = c0;
        red[(w4 * 3 + 1) * 64 + lane] = c1;
        red[(w4 * 3 + 2) * 64 + lane] = c2;
    }
    lds_barrier();
    if (wave >= 4 && cs == 0) {
        int4v c0 = {0, 0, 0, 0}, c1 = c0, c2 = c0;
#pragma unroll
        for (int k = 0; k < WPR; k++) {  // the row block's waves, exact int32 sums
            const int ww = rbl + RBO * k;
            c0 += red[(ww * 3 + 0) * 64 + lane];
            c1 += red[(ww * 3 + 1) * 64 + lane];
            c2 += red[(ww * 3 + 2) * 64 + lane];
        }
        const int row = (j * RBO + rbl) * 16 + r;
#pragma unroll
        for (int v = 0; v < 4; v++) {
            const int b = 4 * s + v;
            if (b < nb) {
                const float val = ((float)c0[v] + (float)c1[v] * 0.0078125f + (float)c2[v] * 6.103515625e-05f) *
                                  sxo[b] * rso;
                a.pout[((size_t)x * MAXB + b) * H + row] = val;
            }
        }
    }
    XL_MARK(12);
}

// ---------------------------------------------------------------------------
// FFN launch
// ---------------------------------------------------------------------------
// Eight operand columns 8 s .. 8 s + 7 of tile tt, batch row b (already
// divided by the row's operand unit xs), as the fixed-point f16 hi / lo of
// q4_fix_split in the MFMA A layout [tile][k-slot][row][8] (the nibble-pair
// order {0,4,2,6,1,5,3,7} within the slot); HL: hi in row b, lo in row 8 + b
// of one plane, otherwise hi and lo planes (lo at +lo_off halves), row b.
// The quad sums of hi and of lo over the tile's four slots come back (the
// two tile biases; exact).
template <bool HL>
__device__ __forceinline__ float2 put8(_Float16* ap, int lo_off, int tt, int s, int b, const float (&v)[8], bool on) {
    half8 h8, l8;
    float sh = 0.f, sl = 0.f;
#pragma unroll
    for (int k = 0; k < 8; k++) {
        _Float16 hi, lo;
        q4_fix_split(v[nib_slot(k)], hi, lo);
        h8[k] = hi;
        l8[k] = lo;
        sh += (float)hi;
        sl += (float)lo;
    }
    const int o = ((tt * 4 + s) * 16 + b) * 8;
    if (on) {
        *(half8*)(ap + o) = h8;
        if constexpr (HL) *(half8*)(ap + o + 64) = l8;  // row 8 + b
        else *(half8*)(ap + lo_off + o) = l8;
    }
    return make_float2(quad_sum(sh), quad_sum(sl));
}
// One tile's MFMA: A rows of the operand, B the 8 nibbles of the lane's word
// as f16 denormals, C the tile's bias rows 4 s .. 4 s + 3 (HL: the hi rows'
// and the lo rows' biases); !HL: the lo plane in an MFMA of its own started
// at its biases cl (a tile's sum is exact within one plane).
template <bool HL>
__device__ __forceinline__ float4v tile_mfma(const _Float16* ap, int lo_off, int tt, int s, int r, uint32_t word,
                                             float4v c, float4v cl) {
    const half8 bq = dq_nib_word(word);
    const int o = ((tt * 4 + s) * 16 + r) * 8;
    float4v d = __builtin_amdgcn_mfma_f32_16x16x32_f16(*(const half8*)(ap + o), bq, c, 0, 0, 0);
    if constexpr (!HL) d += __builtin_amdgcn_mfma_f32_16x16x32_f16(*(const half8*)(ap + lo_off + o), bq, cl, 0, 0, 0);
    return d;
}
__device__ __forceinline__ uint32_t word_of(const uint4& w, int tt) {
    return tt == 0 ? w.x : tt == 1 ? w.y : tt == 2 ? w.z : w.w;
}
__device__ __forceinline__ float tile_scale(uint64_t sw, int tt) {
    return f16_bits_to_f32((uint32_t)(sw >> (16 * tt)) & 0xFFFFu);
}

// NKG = H / 128 (K groups of gate|up), I8 = I / 8 (the XCD's inter slice),
// HL: nb <= 8 (hi and lo rows in one MFMA).
template <int NKG, int I8, bool HL>
__global__ __launch_bounds__(XL_T) void k_xl_ffn(XlBArgs a) {
    constexpr int RPB = XL_WG / NKG;        // row parts of step 0
    constexpr int NRBX = I8 / 8;            // gate|up row blocks of one XCD (8 gate + 8 up rows each)
    constexpr int NRB0 = NRBX / RPB;        // ... per workgroup in step 0
    constexpr int RBW = NRB0 / 4;           // ... per wave (waves 0-3)
    constexpr int ROWS0 = NRB0 * 16;
    constexpr int IW = I8 / XL_WG;          // inter indices finished per workgroup in step 1
    constexpr int RBD = NKG / 4;            // down row blocks per workgroup (H / 512)
    constexpr int G8 = I8 / 128;            // down K groups of the slice
    constexpr int NPAIR = RBD * G8, PW = (NPAIR + 3) / 4;
    constexpr int NT2 = I8 / 32;            // tiles of the down operand
    constexpr int LO0 = HL ? 0 : 4 * 4 * 16 * 8, LO2 = HL ? 0 : NT2 * 4 * 16 * 8;
    static_assert(NRB0 % 4 == 0 && RPB * NKG == XL_WG && IW <= 16 && I8 % 128 == 0 && I8 <= 512,
                  "shape");

    // the XCD this workgroup runs on; workgroups i and i + 8 share one, so
    // blockIdx / 8 numbers the 32 workgroups of each XCD
    const int x = (int)xcc_id() & 7, j = blockIdx.x >> 3;
    const int t = threadIdx.x, lane = t & 63, wave = __builtin_amdgcn_readfirstlane(t >> 6);
    const int r = lane & 15, s = lane >> 4;
    const int nb = a.nb, H = a.H;
    const uint32_t tag = *a.gen * 256u + (uint32_t)a.call;
    int* err = a.err;
    if (t == 0 && atomicExch(a.claim + x * XL_WG + j, tag) == tag) atomicOr(err, 8);

    __shared__ __align__(16) _Float16 AP[(HL ? 1 : 2) * 4 * 4 * 16 * 8];
    // tile biases [tile][16 rows]: HL rows b the hi plane's, rows 8 + b the
    // lo plane's; !HL the lo plane's in LBL / LB2L
    __shared__ __align__(16) float LB[4 * 16];
    __shared__ __align__(16) float LBL[HL ? 1 : 4 * 16];
    __shared__ __align__(16) _Float16 AP2[(HL ? 1 : 2) * NT2 * 4 * 16 * 8];
    __shared__ __align__(16) float LB2[NT2 * 16];
    __shared__ __align__(16) float LB2L[HL ? 1 : NT2 * 16];
    __shared__ __align__(16) float Xd[MAXB * I8];
    __shared__ __align__(16) float4v red2[NPAIR * 64];
    __shared__ float GU[2 * MAXB * IW];
    __shared__ float xs0[MAXB], xs2[MAXB];
    __shared__ double ssd[MAXB], ssp[MAXB][NKG];

    const int kg = j % NKG, rp = j / NKG;
    XL_MARK(16);
    const int w4 = wave - 4;
    uint4 wg[RBW];
    uint64_t sg[RBW];
    // step-0 operand: thread (b = t / 16, columns 8 (t % 16) .. + 7) of the
    // group, i.e. one DPP row per batch row and one quad per 32-column tile
    float4v hv4[2], pv4[2][8], wn4[2];
    uint4 wd[PW];
    uint64_t sd[PW];
    const int cg = kg * 128 + 8 * (t & 15);
    if (wave < 4) {
        // the weights first (the long HBM round trip), then the operand
#pragma unroll
        for (int i = 0; i < RBW; i++) {
            const int g = x * NRBX + rp * NRB0 + wave + 4 * i;
            wg[i] = ld_stream(a.wgu + ((size_t)g * a.ntg_gu + kg) * 64 + lane);
            sg[i] = ldg(a.sgu + ((size_t)g * a.ntg_gu + kg) * 16 + r);
        }
        __builtin_amdgcn_sched_barrier(0);
        const int b = min(t >> 4, nb - 1);
#pragma unroll
        for (int hf = 0; hf < 2; hf++) {
            hv4[hf] = ldg((const float4v*)(a.hb + (size_t)b * H + cg + 4 * hf));
#pragma unroll
            for (int xx = 0; xx < 8; xx++)
                pv4[hf][xx] = ldg((const float4v*)(a.parts + ((size_t)xx * MAXB + b) * H + cg + 4 * hf));
            wn4[hf] = ldg((const float4v*)(a.nw + cg + 4 * hf));
        }
    } else {
#pragma unroll
        for (int k = 0; k < PW; k++) {
            const int p = min(w4 + 4 * k, NPAIR - 1), rbl = p / G8, gl = p % G8;
            const size_t u = (size_t)(j * RBD + rbl) * a.ntg_dn + x * G8 + gl;
            wd[k] = ld_stream(a.wdn + u * 64 + lane);
            sd[k] = ldg(a.sdn + u * 16 + r);
        }
        // bias rows nobody writes (batch rows past nb; HL: rows r and 8 + r)
        const int t4 = t - 256;
        auto dead = [&](int i) { return HL ? (i & 7) >= nb : (i & 15) >= nb; };
        if (t4 < 64 && dead(t4)) {
            LB[t4] = 0.f;
            if constexpr (!HL) LBL[t4] = 0.f;
        }
        for (int i = t4; i < NT2 * 16; i += 256)
            if (dead(i)) {
                LB2[i] = 0.f;
                if constexpr (!HL) LB2L[i] = 0.f;
            }
    }

    XL_MARK(17);
    // ---- step 0: this 128-column group of h_mid * w_norm as f16 hi/lo
    // (waves 0-3), h_mid written by XCD 0
    if (wave < 4) {
        const int b = t >> 4, c8 = t & 15;
        float4v h[2];
        float u[8];
        double ss = 0.0;
        float am = 0.f;
#pragma unroll
        for (int hf = 0; hf < 2; hf++) {
            h[hf] = hv4[hf];
#pragma unroll
            for (int xx = 0; xx < 8; xx++) h[hf] += pv4[hf][xx];
            if (b < nb && x == 0 && rp == 0) *(float4v*)(a.hout + (size_t)b * H + cg + 4 * hf) = h[hf];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                ss += (double)h[hf][i] * (double)h[hf][i];
                u[4 * hf + i] = h[hf][i] * wn4[hf][i];
                am = fmaxf(am, fabsf(u[4 * hf + i]));
            }
        }
        ss = row_sum_d(ss);
        am = row_max(am);
        float sc, xs;
        q4_fix_scale(am, sc, xs);
#pragma unroll
        for (int i = 0; i < 8; i++) u[i] *= sc;
        const int tt = c8 >> 2;
        const float2 ts = put8<HL>(AP, LO0, tt, c8 & 3, b, u, b < nb);
        if (b < nb) {
            if ((c8 & 3) == 0) {
                LB[tt * 16 + b] = ts.x * Q4_BIAS;
                if constexpr (HL) LB[tt * 16 + 8 + b] = ts.y * Q4_BIAS;
                else LBL[tt * 16 + b] = ts.y * Q4_BIAS;
            }
            if (c8 == 0) {
                xs0[b] = xs;
                ssd[b] = ss;
            }
        }
    }
    XL_MARK(26);
    lds_barrier();
    XL_MARK(27);
    uint64_t* e0w = a.e0 + (size_t)(x * XL_WG + j) * MAXB * a.e0s;
    // step 1's items t and t + 256: row part, row within it, batch row; the
    // partials (and a sum(h^2) share) in pg
    const bool ss_on = t < NKG * nb;
    int rpi[2], lri[2], bi[2];
#pragma unroll
    for (int u = 0; u < 2; u++) {
        const int id = min(t + 256 * u, 2 * IW * nb - 1);
        const int il = id % IW, gu = (id / IW) & 1;
        const int i = IW * j + il, R = 16 * (i >> 3) + (i & 7) + 8 * gu;
        rpi[u] = R / ROWS0;
        lri[u] = R % ROWS0;
        bi[u] = id / (2 * IW);
    }
    float pg[2 * NKG + 2];
    if (wave < 4) {
#pragma unroll
        for (int i = 0; i < RBW; i++) {
            float4v acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int tt = 0; tt < 4; tt++) {
                const float4v d = tile_mfma<HL>(AP, LO0, tt, s, r, word_of(wg[i], tt), *(const float4v*)&LB[tt * 16 + 4 * s],
                                                *(const float4v*)&LBL[HL ? 0 : tt * 16 + 4 * s]);
                acc += d * tile_scale(sg[i], tt);
            }
            if constexpr (HL) {
#pragma unroll
                for (int v = 0; v < 4; v++) acc[v] += __shfl_xor(acc[v], 32);
            }
            const int lrow = (wave + 4 * i) * 16 + r;
#pragma unroll
            for (int v = 0; v < 4; v++) {
                const int b = 4 * s + v;
                if (b < nb && (!HL || s < 2)) xput(e0w + (size_t)b * a.e0s + lrow, acc[v] * xs0[b] * 16777216.0f, tag);
            }
        }
        if (t < nb) {
            const double ss = ssd[t];
            const float hi = (float)ss, lo = (float)(ss - (double)hi);
            xput(e0w + (size_t)t * a.e0s + ROWS0, hi, tag);
            xput(e0w + (size_t)t * a.e0s + ROWS0 + 1, lo, tag);
        }
        XL_MARK(18);
        // ---- step 1: thread t waits for the group partials of the gate / up
        // rows of items t and t + 256 (item = (inter index IW j + il, gate or
        // up, b)) and, at once, for one sum(h^2) share (group t % NKG, row
        // t / NKG; row part 0)
        const int ks = ss_on ? t % NKG : 0, bs = ss_on ? t / NKG : 0;
        const uint64_t* pss = a.e0 + ((size_t)(x * XL_WG + ks) * MAXB + bs) * a.e0s + ROWS0;
        if (t < 2 * IW * nb || ss_on) {  // (only the threads that own an item or a share poll)
            xget<2 * NKG + 2>(
                [&](int k) {
                    return k < 2 * NKG
                               ? a.e0 + ((size_t)(x * XL_WG + rpi[k / NKG] * NKG + k % NKG) * MAXB + bi[k / NKG]) *
                                            a.e0s +
                                     lri[k / NKG]
                               : pss + (k - 2 * NKG);
                },
                tag, pg, err);
            if (ss_on) ssp[bs][ks] = (double)pg[2 * NKG] + (double)pg[2 * NKG + 1];
        }
    }
    XL_MARK(19);
    lds_barrier();
    // the partials in group order, times 1 / rms
    if (wave < 4) {
#pragma unroll
        for (int u = 0; u < 2; u++) {
            const int id = t + 256 * u;
            if (id < 2 * IW * nb) {
                const int il = id % IW, gu = (id / IW) & 1, b = bi[u];
                double ss = 0.0;
#pragma unroll
                for (int k = 0; k < NKG; k++) ss += ssp[b][k];
                const float inv = (float)(1.0 / sqrt(ss / (double)H + a.eps));
                float acc = 0.f;
#pragma unroll
                for (int k = 0; k < NKG; k++) acc += pg[u * NKG + k];
                GU[(gu * MAXB + b) * IW + il] = acc * inv;
            }
        }
    }
    XL_MARK(20);
    lds_barrier();
    // ---- step 1c: silu(g) * u (inference.rs:14-16) of this workgroup's indices
    const uint64_t* e1x = a.e1 + (size_t)x * MAXB * a.e1s;
    if (t < IW * nb) {
        const int il = t % IW, b = t / IW;
        const float g = GU[b * IW + il], u = GU[(MAXB + b) * IW + il];
        xput(a.e1 + ((size_t)x * MAXB + b) * a.e1s + IW * j + il, (g / (1.0f + expf(-g))) * u, tag);
    }
    XL_MARK(21);
    // ---- step 2: the down projection rows of this workgroup over the slice
    {
        // the nb * I8 values, 4 consecutive per thread
        const int n = nb * I8;
        for (int i0 = 4 * t; i0 < n; i0 += 4 * XL_T) {
            const int b = i0 / I8, c = i0 - b * I8;
            float ov[4];
            xget<4>([&](int i) { return e1x + (size_t)b * a.e1s + c + i; }, tag, ov, err);
#pragma unroll
            for (int i = 0; i < 4; i++) Xd[i0 + i] = ov[i];
        }
    }
    XL_MARK(22);
    lds_barrier();
    for (int b = wave; b < nb; b += 8) {
        // lane l < I8 / 8: columns 8 l .. 8 l + 7 (tile l / 4, k-slot l % 4)
        constexpr int NL = I8 / 8;
        const int l = min(lane, NL - 1);
        const float4v v0 = *(const float4v*)&Xd[b * I8 + 8 * l], v1 = *(const float4v*)&Xd[b * I8 + 8 * l + 4];
        float u[8] = {v0[0], v0[1], v0[2], v0[3], v1[0], v1[1], v1[2], v1[3]};
        float am = 0.f;
#pragma unroll
        for (int i = 0; i < 8; i++) am = fmaxf(am, fabsf(u[i]));
        am = wave_max(am);
        float sc, xs;
        q4_fix_scale(am, sc, xs);
        if (lane == 0) xs2[b] = xs;
#pragma unroll
        for (int i = 0; i < 8; i++) u[i] *= sc;
        const float2 ts = put8<HL>(AP2, LO2, l >> 2, l & 3, b, u, lane < NL);
        if (lane < NL && (lane & 3) == 0) {
            LB2[(l >> 2) * 16 + b] = ts.x * Q4_BIAS;
            if constexpr (HL) LB2[(l >> 2) * 16 + 8 + b] = ts.y * Q4_BIAS;
            else LB2L[(l >> 2) * 16 + b] = ts.y * Q4_BIAS;
        }
    }
    XL_MARK(23);
    lds_barrier();
    if (wave >= 4) {
#pragma unroll
        for (int k = 0; k < PW; k++) {
            const int p = w4 + 4 * k;
            if (p < NPAIR) {
                const int gl = p % G8;
                float4v acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int tt = 0; tt < 4; tt++) {
                    const int tile = 4 * gl + tt;
                    const float4v d = tile_mfma<HL>(AP2, LO2, tile, s, r, word_of(wd[k], tt),
                                                    *(const float4v*)&LB2[tile * 16 + 4 * s],
                                                    *(const float4v*)&LB2L[HL ? 0 : tile * 16 + 4 * s]);
                    acc += d * tile_scale(sd[k], tt);
                }
                if constexpr (HL) {
#pragma unroll
                    for (int v = 0; v < 4; v++) acc[v] += __shfl_xor(acc[v], 32);
                }
                red2[p * 64 + lane] = acc;
            }
        }
    }
    XL_MARK(24);
    lds_barrier();
    if (wave >= 4 && w4 < RBD) {
        float4v f = red2[(w4 * G8) * 64 + lane];
#pragma unroll
        for (int gl = 1; gl < G8; gl++) f += red2[(w4 * G8 + gl) * 64 + lane];
        const int row = (j * RBD + w4) * 16 + r;
#pragma unroll
        for (int v = 0; v < 4; v++) {
            const int b = 4 * s + v;
            if (b < nb && (!HL || s < 2)) a.pout[((size_t)x * MAXB + b) * H + row] = f[v] * xs2[b] * 16777216.0f;
        }
    }
    XL_MARK(25);
}

// hout = hb + sum over XCDs of parts (XCD order); the generation advances
__global__ __launch_bounds__(256) void k_xl_finish(const float* __restrict__ hb, const float* __restrict__ parts,
                                                   float* __restrict__ hout, int n, int H, uint32_t* gen) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i < n) {
        const int b = i / H, c = i - b * H;
        float v = hb[i];
#pragma unroll
        for (int xx = 0; xx < 8; xx++) v += parts[((size_t)xx * MAXB + b) * H + c];
        hout[i] = v;
    }
    if (blockIdx.x == 0 && threadIdx.x == 0) *gen = *gen + 1u;
}

}  // namespace

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------
bool xl_device_fits() {
    static int ok = -1;
    if (ok < 0) {
        int dev = 0;
        hipDeviceProp_t p{};
        ok = hipGetDevice(&dev) == hipSuccess && hipGetDeviceProperties(&p, dev) == hipSuccess &&
             p.multiProcessorCount == XL_XCD * XL_WG && std::string(p.gcnArchName).rfind("gfx950", 0) == 0;
    }
    return ok;
}

bool xl_shape_ok(const XlShape& s, int nb, int max_len) {
    if (!xl_device_fits()) return false;
    if (s.H != 1024 || s.I != 3072 || s.nkv != XL_XCD || s.hd != 128 || s.nh != 2 * XL_XCD) return false;
    if (nb < 1 || nb > MAXB || 2 * nb > XL_NQ) return false;
    const int tiles = (max_len + 15) / 16;
    return (tiles + XL_WG - 1) / XL_WG <= XL_BT && max_len <= s.max_seq;
}

static size_t e0_stride() { return 260; }
static size_t e1_stride() { return 512; }

size_t xl_bytes(const XlShape& s) {
    const size_t pairs = (size_t)XL_XCD * XL_WG * MAXB * e0_stride() + (size_t)XL_XCD * MAXB * e1_stride() +
                         (size_t)XL_XCD * XL_WG * XL_NQ * XL_E2S + (size_t)XL_XCD * MAXB * 2 * 128 * 2;
    return pairs * 8 + ((size_t)2 * XL_XCD * MAXB * s.H + (size_t)2 * MAXB * s.H) * 4 + 256;
}

int xl_alloc(XlBufs& b, const XlShape& s, void* (*alloc)(void*, size_t), void* ctx) {
    auto get = [&](size_t n) { return alloc(ctx, n); };
    b.e0s = (int)e0_stride();
    b.e1s = (int)e1_stride();
    b.e0 = (uint64_t*)get((size_t)XL_XCD * XL_WG * MAXB * b.e0s * 8);
    b.e1 = (uint64_t*)get((size_t)XL_XCD * MAXB * b.e1s * 8);
    b.e2 = (uint64_t*)get((size_t)XL_XCD * XL_WG * XL_NQ * XL_E2S * 8);
    b.e3 = (uint64_t*)get((size_t)XL_XCD * MAXB * 2 * 128 * 2 * 8);
    b.pa = (float*)get((size_t)XL_XCD * MAXB * s.H * 4);
    b.pb = (float*)get((size_t)XL_XCD * MAXB * s.H * 4);
    b.ha = (float*)get((size_t)MAXB * s.H * 4);
    b.hb = (float*)get((size_t)MAXB * s.H * 4);
    b.gen = (uint32_t*)get(256);
    b.err = (int*)(b.gen + 16);
    b.claim = (uint32_t*)get((size_t)XL_XCD * XL_WG * 4);
    if (!b.e0 || !b.e1 || !b.e2 || !b.e3 || !b.pa || !b.pb || !b.ha || !b.hb || !b.gen || !b.claim)
        return fail("xl: allocation");
    // tags start at generation 1 (memory starts zeroed)
    const uint32_t one = 1;
    CMF_HIP(hipMemcpy(b.gen, &one, 4, hipMemcpyHostToDevice));
    return CMF_OK;
}

int xl_block(const XlBufs& b, const XlShape& s, const XlAttnW& aw, const XlFfnW& fw, const float* h0, int nb,
             const int* pbase, int padd, int max_len, const float2* rope, int li, hipStream_t st) {
    XlAArgs A{};
    A.hb = li == 0 ? h0 : b.hb;
    A.parts = li == 0 ? nullptr : b.pb;
    A.hout = b.ha;
    A.nw = aw.in_norm;
    A.wqkv = (const int4v*)aw.wqkv;
    A.sqkv = (const float*)aw.sqkv;
    A.wo = (const int4v*)aw.wo;
    A.so = (const float*)aw.so;
    A.nkco = aw.nkc_o;
    A.qn = aw.qn;
    A.kn = aw.kn;
    A.rope = rope;
    A.kc = aw.kc;
    A.vc = aw.vc;
    A.pbase = pbase;
    A.padd = padd;
    A.pout = b.pa;
    A.e0 = b.e0;
    A.e1 = b.e1;
    A.e2 = b.e2;
    A.e3 = b.e3;
    A.e0s = b.e0s;
    A.e1s = b.e1s;
    A.gen = b.gen;
    A.call = 2 * li;
    A.err = b.err;
    A.claim = b.claim;
    A.nb = nb;
    A.H = s.H;
    A.nh = s.nh;
    A.max_seq = s.max_seq;
    A.eps = s.eps;
#ifdef XL_STAMPS
    A.stamps = xl_stamp_buf;
#endif
    if (li > 127) return fail("xl: too many blocks in one sequence");
    // tiles per workgroup for the bound (measured: 5 instead of 6 tiles at
    // context 2048 took the K = 4 round 1.133 -> 1.122 ms)
    const int bt = ((max_len + 15) / 16 + XL_WG - 1) / XL_WG;
    if (bt <= 4)
        hipLaunchKernelGGL((k_xl_attn<2, 16, 4>), dim3(XL_XCD * XL_WG), dim3(XL_T), 0, st, A);
    else if (bt == 5)
        hipLaunchKernelGGL((k_xl_attn<2, 16, 5>), dim3(XL_XCD * XL_WG), dim3(XL_T), 0, st, A);
    else
        hipLaunchKernelGGL((k_xl_attn<2, 16, 6>), dim3(XL_XCD * XL_WG), dim3(XL_T), 0, st, A);
    XlBArgs B{};
    B.hb = b.ha;
    B.parts = b.pa;
    B.hout = b.hb;
    B.nw = fw.post_norm;
    B.wgu = (const uint4*)fw.wgu;
    B.sgu = (const uint64_t*)fw.sgu;
    B.ntg_gu = fw.ntg_gu;
    B.wdn = (const uint4*)fw.wdn;
    B.sdn = (const uint64_t*)fw.sdn;
    B.ntg_dn = fw.ntg_dn;
    B.pout = b.pb;
    B.e0 = b.e0;
    B.e1 = b.e1;
    B.e0s = b.e0s;
    B.e1s = b.e1s;
    B.gen = b.gen;
    B.call = 2 * li + 1;
    B.err = b.err;
    B.claim = b.claim;
    B.nb = nb;
    B.H = s.H;
    B.eps = s.eps;
#ifdef XL_STAMPS
    B.stamps = xl_stamp_buf;
#endif
    if (nb <= 8) hipLaunchKernelGGL((k_xl_ffn<8, 384, true>), dim3(XL_XCD * XL_WG), dim3(XL_T), 0, st, B);
    else hipLaunchKernelGGL((k_xl_ffn<8, 384, false>), dim3(XL_XCD * XL_WG), dim3(XL_T), 0, st, B);
    return CMF_OK;
}

// Zeroes the exchange areas and the claim slots and sets the generation back
// to 1 (stream-ordered; the tags of later launches start over).
__global__ void k_xl_zero(uint64_t* p, size_t n) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) p[i] = 0;
}
__global__ void k_xl_regen(uint32_t* claim, int nclaim, uint32_t* gen) {
    for (int i = threadIdx.x; i < nclaim; i += blockDim.x) claim[i] = 0;
    if (threadIdx.x == 0) *gen = 1u;
}
void xl_reset(const XlBufs& b, hipStream_t st) {
    const size_t n0 = (size_t)XL_XCD * XL_WG * MAXB * b.e0s, n1 = (size_t)XL_XCD * MAXB * b.e1s,
                 n2 = (size_t)XL_XCD * XL_WG * XL_NQ * XL_E2S, n3 = (size_t)XL_XCD * MAXB * 2 * 128 * 2;
    hipLaunchKernelGGL(k_xl_zero, dim3(1024), dim3(256), 0, st, b.e0, n0);
    hipLaunchKernelGGL(k_xl_zero, dim3(256), dim3(256), 0, st, b.e1, n1);
    hipLaunchKernelGGL(k_xl_zero, dim3(1024), dim3(256), 0, st, b.e2, n2);
    hipLaunchKernelGGL(k_xl_zero, dim3(256), dim3(256), 0, st, b.e3, n3);
    hipLaunchKernelGGL(k_xl_regen, dim3(1), dim3(256), 0, st, b.claim, XL_XCD * XL_WG, b.gen);
}

void xl_finish(const XlBufs& b, const XlShape& s, float* hout, int nb, hipStream_t st) {
    const int n = nb * s.H;
    hipLaunchKernelGGL(k_xl_finish, dim3((n + 255) / 256), dim3(256), 0, st, b.hb, b.pb, hout, n, s.H, b.gen);
}

}  // namespace cmf
