// Causal attention of a prefill chunk (head_dim 128) for gfx950.
//
// The chunk's rows sit at positions p0 .. p0 + cnt - 1 (p0 known to the
// host).  Three launches per chunk and layer:
//   - k_prefill_qk: q-norm + RoPE of the queries (into a scratch buffer),
//     k-norm + RoPE of the new K rows, K and V appended to the cache
//     (attention.rs:606-624, 818-890; kv_cache.rs:366-505), as the decode
//     kernels do it;
//   - k_prefill_fakv: the cache's K / V rows [0, p0 + cnt) rearranged into
//     32-key tiles of the attention's MFMA fragments (f16 hi / lo halves);
//   - k_prefill_fa: 64 query rows per block of four waves, two blocks per
//     workgroup sharing each tile through LDS, with a running (online)
//     softmax: scores on the f16 MFMA (q.k = qh.kh + qh.kl + ql.kh, 22-bit
//     operands, f32 sums), causal limit the row's position
//     (kv_cache.rs:521-690), values ph.vh + ph.vl + pl.vh on the f16 MFMA.
// Rows of a block past the chunk see no keys and write nothing.
#include <math.h>

#include "common.h"
#include "layers.h"
#include "wave.h"
#include "xlayer.h"

namespace cmf {

namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef float float4v __attribute__((ext_vector_type(4)));
typedef int int4v __attribute__((ext_vector_type(4)));

constexpr int HD = 128;
constexpr int KT2 = 128;      // the K / V scratch's padding unit (keys)

__device__ __forceinline__ void wait_vmcnt0() { __builtin_amdgcn_s_waitcnt((7 << 4) | (15 << 8)); }  // vmcnt(0) only
__device__ __forceinline__ void wait_vmcnt4() { __builtin_amdgcn_s_waitcnt(4 | (7 << 4) | (15 << 8)); }  // vmcnt(4) only

__device__ __forceinline__ uint32_t xcc_id() {
    uint32_t v;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID, 0, 4)" : "=s"(v));
    return v;
}

// max / sum over the four lanes l, l ^ 16, l ^ 32, l ^ 48 (one MFMA output
// column) by the gfx950 row-swap permutes: each returns the value and its
// partner's, so op(first, second) is the pairwise result in every lane
__device__ __forceinline__ float lanes4_max(float v) {
    auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
    auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ __forceinline__ float lanes4_sum(float v) {
    auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = __uint_as_float(a[0]) + __uint_as_float(a[1]);
    auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

__device__ __forceinline__ void split16(float x, _Float16& hi, _Float16& lo) {
    hi = (_Float16)x;
    lo = (_Float16)(x - (float)hi);
}

// grid (cnt, hq + nkv), 64 threads: block y < hq: query head y of chunk row
// x into qbuf [cnt][nh][128]; else kv head y - hq: K (normed, rotated) and V
// of the row appended at position p0 + x.
__global__ __launch_bounds__(64) void k_prefill_qk(const float* __restrict__ qkv, int ldq,
                                                   const float* __restrict__ qn, const float* __restrict__ kn,
                                                   const float2* __restrict__ rope, float* __restrict__ kc,
                                                   float* __restrict__ vc, int max_seq, int p0, int nh, int nkv,
                                                   double eps, float* __restrict__ qbuf, int hq) {
    const int i = blockIdx.x, h = blockIdx.y, lane = threadIdx.x;
    const int pos = p0 + i;
    const float* row = qkv + (size_t)i * ldq;
    const float2 cs = rope[(size_t)pos * 64 + lane];
    if (h < hq) {
        const float* qr = row + (size_t)h * HD;
        const float2 o = norm_rope(qr[lane], qr[lane + 64], qn[lane], qn[lane + 64], cs, eps);
        float* q = qbuf + ((size_t)i * nh + h) * HD;
        q[lane] = o.x;
        q[lane + 64] = o.y;
    } else {
        const int g = h - hq;
        const float* kr = row + (size_t)(nh + g) * HD;
        const float* vr = row + (size_t)(nh + nkv + g) * HD;
        const float2 k = norm_rope(kr[lane], kr[lane + 64], kn[lane], kn[lane + 64], cs, eps);
        float* kd = kc + ((size_t)g * max_seq + pos) * HD;
        float* vd = vc + ((size_t)g * max_seq + pos) * HD;
        kd[lane] = k.x;
        kd[lane + 64] = k.y;
        vd[lane] = vr[lane];
        vd[lane + 64] = vr[lane + 64];
    }
}

// ---------------------------------------------------------------------------
// 64 query rows per block share each 32-key tile of K / V through LDS.
// Scores are computed transposed, S^T = K Q^T, so that each lane (query r,
// k-slot s) ends up holding the weights of its own query for the keys
// {4s..4s+3, 16+4s..16+4s+3}: exactly the B operand of O^T = V^T P^T when
// the V tile's k-slot s holds the same eight keys, so the weights never go
// through LDS, and the output's lanes hold their own query's dims.  q.k =
// qh.kh + qh.kl + ql.kh (f16 hi / lo halves, f32 sums), exp2 of log2-scaled
// scores with a running maximum, values ph.vh + ph.vl + pl.vh.
// ---------------------------------------------------------------------------
constexpr int FT = 32;                // keys per tile
constexpr int FT_BYTES = 32 * 1024;   // one tile of one kv head: K then V fragments

// The cached K / V rows [0, n) of every kv head as 32-key tiles of MFMA
// fragments, [nkv][npad / 32][32 fragments][64 lanes] x 16 B (keys past n
// zero):
//   K fragment (kb, ks, plane) = 4 kb... index 8 kb + 2 ks + plane: lane
//     16 s + r holds dims 32 ks + 8 s .. + 7 of key 16 kb + r (A operand of
//     S^T, f16 hi / lo);
//   V fragment 16 + 2 db + plane: lane 16 s + r holds dim 16 db + r of the
//     keys 4 s + j (j < 4) and 16 + 4 s + j - 4 (j >= 4) (A operand of
//     O^T = V^T P^T).
// grid (npad / 32, nkv), 256 threads.
__global__ __launch_bounds__(256) void k_prefill_fakv(const float* __restrict__ kc, const float* __restrict__ vc,
                                                      int max_seq, int n, int npad, int4v* __restrict__ op) {
    const int t = threadIdx.x, tile = blockIdx.x, g = blockIdx.y;
    __shared__ float KS[FT][HD + 4], VS[FT][HD + 1];
    for (int e = t; e < FT * 32; e += 256) {
        const int k = e >> 5, c4 = 4 * (e & 31), key = FT * tile + k;
        float4v kv = {0.f, 0.f, 0.f, 0.f}, vv = kv;
        if (key < n) {
            kv = *(const float4v*)(kc + ((size_t)g * max_seq + key) * HD + c4);
            vv = *(const float4v*)(vc + ((size_t)g * max_seq + key) * HD + c4);
        }
        *(float4v*)&KS[k][c4] = kv;
#pragma unroll
        for (int i = 0; i < 4; i++) VS[k][c4 + i] = vv[i];
    }
    __syncthreads();
    int4v* dst = op + ((size_t)g * (npad / FT) + tile) * (FT_BYTES / 16);
    for (int e = t; e < 32 * 64; e += 256) {
        const int l = e & 63, f = e >> 6, r = l & 15, sl = l >> 4, plane = f & 1;
        half8 h;
        if (f < 16) {
            const int kb = f >> 3, ks = (f >> 1) & 3, k = 16 * kb + r;
#pragma unroll
            for (int j = 0; j < 8; j++) {
                _Float16 hh, ll;
                split16(KS[k][32 * ks + 8 * sl + j], hh, ll);
                h[j] = plane ? ll : hh;
            }
        } else {
            const int db = (f - 16) >> 1;
#pragma unroll
            for (int j = 0; j < 8; j++) {
                const int k = j < 4 ? 4 * sl + j : 16 + 4 * sl + (j - 4);
                _Float16 hh, ll;
                split16(VS[k][16 * db + r], hh, ll);
                h[j] = plane ? ll : hh;
            }
        }
        dst[f * 64 + l] = __builtin_bit_cast(int4v, h);
    }
}

// grid (8 np) (XCD: kv head = the workgroup's XCD, pair index i =
// blockIdx / 8) or (np, nkv), np = ceil(nqb / 2); 512 threads.  The
// workgroup serves two 64-row query blocks that see about as many keys
// together as any other pair: waves 0-3 block i, waves 4-7 block nqb - 1 -
// i (none when that is block i again), sharing one fetch of every K / V
// tile the short block needs.  Wave w of a block holds 16 query rows, PPW =
// 16 / HPK positions times the HPK query heads of kv head g (row q: chunk
// row PPW (4 qb + w % 4) + q % PPW, query head g HPK + q / PPW).  XCD: the
// kv head is the XCD the workgroup runs on (its K / V stays in that XCD's
// L2), which covers each (query block, head) once only while the
// dispatcher deals workgroups to the 8 XCDs in turn; each workgroup
// therefore swaps the launch's tag into its blocks' cells [qb][g] first,
// and finding the tag already there sets *perr: the host then re-runs the
// prefill on the grid-indexed variant.
template <int HPK, bool XCD>
__global__ __launch_bounds__(512) void k_prefill_fa(const float* __restrict__ qbuf, const int4v* __restrict__ op,
                                                    int npad, int cnt, int p0, int nh, int nqb, float* __restrict__ out,
                                                    unsigned long long* cells, int* perr, unsigned long long tag) {
    constexpr int PPW = 16 / HPK;
    extern __shared__ __align__(16) uint8_t fsm[];  // three tiles (direct-load targets)
    const int pi = XCD ? (int)(blockIdx.x >> 3) : (int)blockIdx.x;
    const int g = XCD ? (int)(xcc_id() & 7) : (int)blockIdx.y;
    const int qa = pi, qz = nqb - 1 - pi;  // the pair (qz == qa: one block)
    if constexpr (XCD) {
        if (threadIdx.x == 0 && atomicExch(cells + qa * 8 + g, tag) == tag) atomicOr(perr, 1);
        if (threadIdx.x == 64 && qz != qa && atomicExch(cells + qz * 8 + g, tag) == tag) atomicOr(perr, 1);
    }
    const int t = threadIdx.x, lane = t & 63, wave = __builtin_amdgcn_readfirstlane(t >> 6);
    const int r = lane & 15, s = lane >> 4;
    const bool second = wave >= 4;
    const bool live = !second || qz != qa;                 // (uniform per wave)
    const int qb = second ? qz : qa;
    const int i0 = (4 * qb + (wave & 3)) * PPW;           // this wave's first chunk row
    const int lastrow = min((4 * qb + 4) * PPW, cnt) - 1; // its block's last chunk row
    const int lastz = min((4 * max(qa, qz) + 4) * PPW, cnt) - 1;  // the pair's
    // the queries of column r (the B operand of S^T), f16 hi / lo
    const bool qv = live && i0 + r % PPW < cnt;
    const int qpos = p0 + i0 + r % PPW;                 // position of query r
    half8 qh[HD / 32], ql[HD / 32];
    {
        const float* qrow = qbuf + ((size_t)(qv ? i0 + r % PPW : 0) * nh + g * HPK + r / PPW) * HD;
#pragma unroll
        for (int ks = 0; ks < HD / 32; ks++) {
            const float4v a0 = *(const float4v*)(qrow + 32 * ks + 8 * s);
            const float4v a1 = *(const float4v*)(qrow + 32 * ks + 8 * s + 4);
#pragma unroll
            for (int j = 0; j < 8; j++) {
                _Float16 hh, ll;
                split16(qv ? (j < 4 ? a0[j] : a1[j - 4]) : 0.f, hh, ll);
                qh[ks][j] = hh;
                ql[ks][j] = ll;
            }
        }
    }
    // tiles of the pair (the fetch loop) and of this wave's block
    const int ntiles = lastz < 0 ? 0 : (p0 + lastz) / FT + 1;
    const int mytiles = !live || lastrow < 0 ? 0 : (p0 + lastrow) / FT + 1;
    const uint8_t* src = (const uint8_t*)(op + (size_t)g * (npad / FT) * (FT_BYTES / 16));
    // tile tt into buffer b: 32 KiB as 32 chunks of 1 KiB, 4 per wave
    auto fetch = [&](int tt, int b) {
#pragma unroll
        for (int c = 0; c < 4; c++) {
            const int ch = 4 * wave + c;
            __builtin_amdgcn_global_load_lds((const void*)(src + (size_t)tt * FT_BYTES + ch * 1024 + lane * 16),
                                             (__attribute__((address_space(3))) void*)(fsm + b * FT_BYTES + ch * 1024),
                                             16, 0, 0);
        }
    };
    const float scale = 1.4426950408889634f / sqrtf((float)HD);
    float m = -INFINITY, l = 0.f;   // of query r (the same in the four lanes of column r)
    float4v o[8];                   // rows 4 s + e, dims 16 db + r
#pragma unroll
    for (int db = 0; db < 8; db++) o[db] = float4v{0.f, 0.f, 0.f, 0.f};
    // three buffers: tile tt + 2 is requested while tile tt is used
    if (ntiles > 0) fetch(0, 0);
    if (ntiles > 1) fetch(1, 1);
    for (int tt = 0; tt < ntiles; tt++) {
        const int b = tt % 3;
        if (tt + 1 < ntiles) wait_vmcnt4();  // tile tt's share is in (tile tt + 1's may not be)
        else wait_vmcnt0();
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");  // every wave's share is in; tile tt - 1's buffer is free
        if (tt + 2 < ntiles) fetch(tt + 2, (tt + 2) % 3);
        if (tt >= mytiles) continue;  // (uniform per wave: past this block's keys)
        const int4v* F = (const int4v*)(fsm + b * FT_BYTES) + lane;
        // S^T for the two key blocks: d[kb][e] = key 16 kb + 4 s + e, query r
        float4v d[2];
#pragma unroll
        for (int kb = 0; kb < 2; kb++) {
            float4v d0 = {0.f, 0.f, 0.f, 0.f}, d1 = d0, d2 = d0;
#pragma unroll
            for (int ks = 0; ks < HD / 32; ks++) {
                const half8 kh = __builtin_bit_cast(half8, F[(8 * kb + 2 * ks) * 64]);
                const half8 kl = __builtin_bit_cast(half8, F[(8 * kb + 2 * ks + 1) * 64]);
                d0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(kh, qh[ks], d0, 0, 0, 0);
                d1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(kl, qh[ks], d1, 0, 0, 0);
                d2 = __builtin_amdgcn_mfma_f32_16x16x32_f16(kh, ql[ks], d2, 0, 0, 0);
            }
            d[kb] = d0 + (d1 + d2);
        }
        // causal mask, log2 scale, the running softmax of query r
        float sv[8];
        float mt = -INFINITY;
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const int key = FT * tt + (j < 4 ? 4 * s + j : 16 + 4 * s + (j - 4));
            const float x = j < 4 ? d[0][j] : d[1][j - 4];
            sv[j] = qv && key <= qpos ? x * scale : -INFINITY;
            mt = fmaxf(mt, sv[j]);
        }
        mt = lanes4_max(mt);
        const float mn = fmaxf(m, mt);
        const float al = m == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m - mn);
        float ps = 0.f;
        half8 ph, pl;
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const float pv = mn == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(sv[j] - mn);
            ps += pv;
            _Float16 hh, ll;
            split16(pv, hh, ll);
            ph[j] = hh;
            pl[j] = ll;
        }
        ps = lanes4_sum(ps);
        l = l * al + ps;
        m = mn;
        // O^T += V^T P^T (the same registers as operands the other way
        // round): lane (query r, s) holds dims 16 db + 4 s + e of its own
        // query, so the rescale needs no exchange
#pragma unroll
        for (int db = 0; db < 8; db++) {
            float4v acc = o[db] * al;
            const half8 vh = __builtin_bit_cast(half8, F[(16 + 2 * db) * 64]);
            const half8 vl = __builtin_bit_cast(half8, F[(16 + 2 * db + 1) * 64]);
            acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(vh, ph, acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(vl, ph, acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(vh, pl, acc, 0, 0, 0);
            o[db] = acc;
        }
    }
    // out = o / l of query r: dims 16 db + 4 s .. + 3
    const int row = i0 + r % PPW, head = g * HPK + r / PPW;
    if (live && row < cnt) {
        float* dst = out + (size_t)row * nh * HD + (size_t)head * HD + 4 * s;
#pragma unroll
        for (int db = 0; db < 8; db++) *(float4v*)(dst + 16 * db) = o[db] / l;
    }
}

}  // namespace

bool prefill_attention_fits(int nh, int nkv, int hd) {
    if (hd != HD || nkv < 1 || nh % nkv) return false;
    const int hpk = nh / nkv;
    return hpk == 1 || hpk == 2 || hpk == 4 || hpk == 8 || hpk == 16;
}

int launch_prefill_attention(const PrefillAttnArgs& a, hipStream_t st) {
    if (!prefill_attention_fits(a.nh, a.nkv, HD) || a.cnt < 1 || a.p0 < 0 || a.p0 + a.cnt > a.max_seq)
        return fail("prefill attention: head_dim 128, query heads a power-of-two multiple (<= 16) of kv heads");
    const int hq = a.out ? a.nh : 0;
    hipLaunchKernelGGL(k_prefill_qk, dim3(a.cnt, hq + a.nkv), dim3(64), 0, st, a.qkv, a.ldq, a.qn, a.kn, a.rope,
                       a.kc, a.vc, a.max_seq, a.p0, a.nh, a.nkv, a.eps, a.qbuf, hq);
    if (!a.out) return CMF_OK;
    const int hpk = a.nh / a.nkv, ppw = 16 / hpk;
    const int n = a.p0 + a.cnt, npad = (n + KT2 - 1) / KT2 * KT2;
    const int nqb = (a.cnt + 4 * ppw - 1) / (4 * ppw);  // 64-row query blocks, paired
    const int np = (nqb + 1) / 2;
    const bool xcd = a.nkv == 8 && xl_device_fits() && a.allow_xcd && a.cells && a.perr &&
                     8 * nqb <= PREFILL_XCD_CELLS;
    typedef void (*KernF)(const float*, const int4v*, int, int, int, int, int, float*, unsigned long long*, int*,
                          unsigned long long);
    KernF k;
    switch (hpk) {
        case 1: k = xcd ? k_prefill_fa<1, true> : k_prefill_fa<1, false>; break;
        case 2: k = xcd ? k_prefill_fa<2, true> : k_prefill_fa<2, false>; break;
        case 4: k = xcd ? k_prefill_fa<4, true> : k_prefill_fa<4, false>; break;
        case 8: k = xcd ? k_prefill_fa<8, true> : k_prefill_fa<8, false>; break;
        default: k = xcd ? k_prefill_fa<16, true> : k_prefill_fa<16, false>; break;
    }
    int4v* op = (int4v*)a.khl;  // nkv x npad x 1 KiB
    hipLaunchKernelGGL(k_prefill_fakv, dim3(npad / FT, a.nkv), dim3(256), 0, st, a.kc, a.vc, a.max_seq, n, npad, op);
    const dim3 grid = xcd ? dim3(8 * np) : dim3(np, a.nkv);
    static const bool attr = [] {  // (96 KiB: above the default dynamic LDS limit)
        bool ok = true;
        for (KernF f : {k_prefill_fa<1, true>, k_prefill_fa<1, false>, k_prefill_fa<2, true>, k_prefill_fa<2, false>,
                        k_prefill_fa<4, true>, k_prefill_fa<4, false>, k_prefill_fa<8, true>, k_prefill_fa<8, false>,
                        k_prefill_fa<16, true>, k_prefill_fa<16, false>})
            ok &= hipFuncSetAttribute((const void*)f, hipFuncAttributeMaxDynamicSharedMemorySize, 3 * FT_BYTES) ==
                  hipSuccess;
        return ok;
    }();
    if (!attr) return fail("prefill attention: dynamic LDS attribute");
    hipLaunchKernelGGL(k, grid, dim3(512), 3 * FT_BYTES, st, a.qbuf, op, npad, a.cnt, a.p0, a.nh, nqb, a.out,
                       a.cells, a.perr, a.tag);
    return CMF_OK;
}

}  // namespace cmf
