// Causal attention of a prefill chunk (head_dim 128) for gfx950.
//
// The chunk's rows sit at positions p0 .. p0 + cnt - 1 (p0 known to the
// host).  Three launches per chunk and layer:
//   - k_prefill_qk: q-norm + RoPE of the queries (into a scratch buffer),
//     k-norm + RoPE of the new K rows, K and V appended to the cache
//     (attention.rs:606-624, 818-890; kv_cache.rs:366-505), as the decode
//     kernels do it;
//   - k_prefill_kv: the cache's K / V rows [0, p0 + cnt) rearranged into
//     the attention's MFMA operand layout (K as f16 hi / lo halves);
//   - k_prefill_attn: 16 query rows per workgroup — 16 / HPK positions times
//     the HPK query heads of one kv head, which share its K / V — over
//     128-key tiles with a running (online) softmax: scores on the f16 MFMA
//     (q.k = qh.kh + qh.kl + ql.kh, 22-bit operands, f32 sums), causal
//     limit the row's position (kv_cache.rs:521-690), values on the fp32
//     MFMA (16x16x4).
// Rows of a workgroup past the chunk see no keys and write nothing.
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
constexpr int KT = 64;        // key rows per scratch padding unit
constexpr int KT2 = 128;      // keys per attention tile (two groups of 64)
constexpr int PST = KT + 4;   // f32 row stride of the scores / weights (64 keys a group)

// Workgroup barrier over LDS only: __syncthreads also waits for every
// global load in flight (vmcnt(0)), which would wait for the next tile's
// K / V requests; uses of those registers get the compiler's own waits.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }
__device__ __forceinline__ void wait_vmcnt0() { __builtin_amdgcn_s_waitcnt((7 << 4) | (15 << 8)); }  // vmcnt(0) only
__device__ __forceinline__ void wait_vmcnt4() { __builtin_amdgcn_s_waitcnt(4 | (7 << 4) | (15 << 8)); }  // vmcnt(4) only

// Four f32 reductions over the wave at once (each DPP step applied to all
// four before the next, so the chains overlap), with the DPP pattern of
// wave_reduce_f32; the results are wave-uniform.
template <typename Op>
__device__ __forceinline__ void wave_reduce4(float (&v)[4], float ident, Op op) {
    const uint32_t iu = __builtin_bit_cast(uint32_t, ident);
    auto step = [&](auto ctrl, auto rows) {
        constexpr int C = decltype(ctrl)::value, R = decltype(rows)::value;
        float w[4];
#pragma unroll
        for (int i = 0; i < 4; i++) w[i] = __builtin_bit_cast(float, dpp_u32<C, R>(__builtin_bit_cast(uint32_t, v[i]), iu));
#pragma unroll
        for (int i = 0; i < 4; i++) v[i] = op(v[i], w[i]);
    };
    step(std::integral_constant<int, 0xb1>{}, std::integral_constant<int, 0xf>{});
    step(std::integral_constant<int, 0x4e>{}, std::integral_constant<int, 0xf>{});
    step(std::integral_constant<int, 0x114>{}, std::integral_constant<int, 0xf>{});
    step(std::integral_constant<int, 0x118>{}, std::integral_constant<int, 0xf>{});
    step(std::integral_constant<int, 0x142>{}, std::integral_constant<int, 0xa>{});
    step(std::integral_constant<int, 0x143>{}, std::integral_constant<int, 0xc>{});
#pragma unroll
    for (int i = 0; i < 4; i++) v[i] = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v[i]), 63));
}

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

// The cached K / V rows [0, n) of every kv head rearranged once per chunk
// as the attention's MFMA operands, so that each wave load (16 B a lane)
// reads 1 KiB in register order (rows [n, npad) zero):
//   kop [nkv][npad / 16][8 chunks][64 lanes] x 16 B: key block kb (keys
//       16 kb + r), chunk ch = 2 ks + plane (f16 hi / lo), lane 16 s + r:
//       dims 32 ks + 8 s .. + 7 of key 16 kb + r;
//   vop [nkv][npad / 64][8 dim blocks][2 k-steps][2 planes][64 lanes] x
//       16 B: key block kb (keys 64 kb ..), dim block db, k-step ks, plane
//       (f16 hi / lo), lane 16 s + r: keys 64 kb + 32 ks + 8 s .. + 7 of
//       dim 16 db + r (the B operand of the values' f16 MFMA).
// grid (npad / 64, nkv), 256 threads: 64 keys through LDS.
__global__ __launch_bounds__(256) void k_prefill_kv(const float* __restrict__ kc, const float* __restrict__ vc,
                                                    int max_seq, int n, int npad, int4v* __restrict__ kop,
                                                    float4v* __restrict__ vop) {
    const int t = threadIdx.x, kb64 = blockIdx.x, g = blockIdx.y;
    __shared__ float KS[64][HD + 4], VS[64][HD + 1];
    for (int e = t; e < 64 * 32; e += 256) {
        const int k = e >> 5, c4 = 4 * (e & 31), key = 64 * kb64 + k;
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
    const int nkb = npad / 16, nvb = npad / 64;
    // K: 4 key blocks x 8 chunks x 64 lanes
    for (int e = t; e < 4 * 8 * 64; e += 256) {
        const int l = e & 63, ch = (e >> 6) & 7, kb = e >> 9, r = l & 15, sl = l >> 4;
        const int ks = ch >> 1, plane = ch & 1, k = 16 * kb + r;
        half8 h;
#pragma unroll
        for (int j = 0; j < 8; j++) {
            _Float16 hh, ll;
            split16(KS[k][32 * ks + 8 * sl + j], hh, ll);
            h[j] = plane ? ll : hh;
        }
        kop[(((size_t)g * nkb + 4 * kb64 + kb) * 8 + ch) * 64 + l] = __builtin_bit_cast(int4v, h);
    }
    // V: 8 dim blocks x (2 k-steps x 2 planes) x 64 lanes
    for (int e = t; e < 8 * 4 * 64; e += 256) {
        const int l = e & 63, i = (e >> 6) & 3, db = e >> 8, r = l & 15, sl = l >> 4;
        const int ks = i >> 1, plane = i & 1;
        half8 h;
#pragma unroll
        for (int j = 0; j < 8; j++) {
            _Float16 hh, ll;
            split16(VS[32 * ks + 8 * sl + j][16 * db + r], hh, ll);
            h[j] = plane ? ll : hh;
        }
        vop[(((size_t)g * nvb + kb64) * 8 + db) * 4 * 64 + i * 64 + l] = __builtin_bit_cast(float4v, h);
    }
}

// grid (ceil(cnt / (16 / HPK)), nkv), 512 threads.  Row q (0..15) of block
// qb: chunk row qb * PPW + q % PPW, query head g * HPK + q / PPW.  XCD (8 kv
// heads on an MI355X): grid (8 ceil(cnt / PPW)), kv head g = the XCD the
// workgroup runs on, qb = blockIdx / 8 (the dispatcher deals workgroups to
// the 8 XCDs in turn), so one head's K / V serves all of its query blocks
// from that XCD's L2.  That covers each (query block, head) once only while
// the workgroups go to the XCDs strictly in turn; each workgroup therefore
// swaps the launch's tag into its cell [qb][g] first, and finding the tag
// already there (two workgroups on one cell, so some other cell has none)
// sets *perr: the host then re-runs the prefill on the grid-indexed variant.
// The 8 waves form two groups: group G takes keys 64 G .. 64 G + 63 of each
// 128-key tile with a running softmax of its own, wave wl of the group the
// scores of keys 16 wl .. + 15 and the values of dims 32 wl .. + 31; its K
// and V operands come from the rearranged scratch straight into registers
// (the next tile's requested while the current one is used), the queries
// stay in registers, and LDS holds only the weights and row statistics.
// The groups' (m, l, o) are merged at the end.
template <int HPK, bool XCD>
__global__ __launch_bounds__(512) void k_prefill_attn(const float* __restrict__ qbuf, const int4v* __restrict__ kop,
                                                      const float4v* __restrict__ vop, int npad, int cnt, int p0,
                                                      int nh, float* __restrict__ out, unsigned long long* cells,
                                                      int* perr, unsigned long long tag) {
    constexpr int PPW = 16 / HPK;  // positions per workgroup
    constexpr int GK = KT2 / 2;    // keys per group and tile
    const int qb = XCD ? (int)(blockIdx.x >> 3) : (int)blockIdx.x;
    const int g = XCD ? (int)(xcc_id() & 7) : (int)blockIdx.y;
    const int t = threadIdx.x, lane = t & 63;
    if constexpr (XCD) {
        if (t == 0 && atomicExch(cells + qb * 8 + g, tag) == tag) atomicOr(perr, 1);
    }
    const int wave = __builtin_amdgcn_readfirstlane(t >> 6), G = wave >> 2, wl = wave & 3;
    const int r = lane & 15, s = lane >> 4;
    __shared__ __align__(16) float P[2][16][PST];
    __shared__ __align__(16) float O1[16][HD];
    __shared__ float s_m[2][16], s_l[2][16], s_al[2][16];
    const int i0 = qb * PPW;
    const int npos = min(PPW, cnt - i0);
    // the score operand's queries (row r, dims 32 ks + 8 s ..) as f16 hi / lo
    half8 qh[HD / 32], ql[HD / 32];
    {
        const bool qv = r % PPW < npos;
        const float* qrow = qbuf + ((size_t)(i0 + (qv ? r % PPW : 0)) * nh + g * HPK + r / PPW) * HD;
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
    if (t < 32) {
        s_m[t >> 4][t & 15] = -INFINITY;
        s_l[t >> 4][t & 15] = 0.f;
    }
    const int plast = p0 + i0 + npos - 1;  // the block's last query position
    const int ntiles = plast / KT2 + 1;
    const int nkb = npad / 16, nvb = npad / 64;
    const int4v* kw = kop + ((size_t)g * nkb + 4 * G + wl) * 8 * 64 + lane;          // + tile * 8 key blocks
    const float4v* vw = vop + (((size_t)g * nvb + G) * 8 + 2 * wl) * 4 * 64 + lane;  // + tile * 2 key blocks
    int4v ka[8], kn[8];
    float4v va[8], vn[8];
    auto load = [&](int tile, int4v (&k)[8], float4v (&v)[8]) {
#pragma unroll
        for (int ch = 0; ch < 8; ch++) k[ch] = kw[(size_t)tile * 8 * 8 * 64 + ch * 64];
#pragma unroll
        for (int i = 0; i < 8; i++) v[i] = vw[(size_t)tile * 2 * 8 * 4 * 64 + i * 64];
    };
    // scores in log2 units: exp(x - m) = exp2(x log2e - m log2e)
    const float scale = 1.4426950408889634f / sqrtf((float)HD);
    float4v o[4] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
    auto step = [&](int tile, const int4v (&k)[8], const float4v (&v)[8]) {
        // scores of keys GK G + 16 wl .. + 15 of the tile
        {
            float4v d0 = {0.f, 0.f, 0.f, 0.f}, d1 = d0, d2 = d0;
#pragma unroll
            for (int ks = 0; ks < HD / 32; ks++) {
                const half8 kh = __builtin_bit_cast(half8, k[2 * ks]), kl = __builtin_bit_cast(half8, k[2 * ks + 1]);
                d0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(qh[ks], kh, d0, 0, 0, 0);
                d1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(qh[ks], kl, d1, 0, 0, 0);
                d2 = __builtin_amdgcn_mfma_f32_16x16x32_f16(ql[ks], kh, d2, 0, 0, 0);
            }
            const float4v d = d0 + (d1 + d2);
            const int key = tile * KT2 + GK * G + 16 * wl + r;
            lds_barrier();  // the previous tile's weights are read
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const int q = 4 * s + e;
                const bool see = q % PPW < npos && key <= p0 + i0 + q % PPW;
                P[G][q][16 * wl + r] = see ? d[e] * scale : -INFINITY;
            }
        }
        lds_barrier();
        // running softmax of the group: wave wl rows 4 wl .. 4 wl + 3, lane =
        // key (the four rows' reductions interleaved)
        {
            float sv[4], mo[4], mt[4], p[4];
#pragma unroll
            for (int qq = 0; qq < 4; qq++) {
                sv[qq] = P[G][4 * wl + qq][lane];
                mo[qq] = s_m[G][4 * wl + qq];
                mt[qq] = sv[qq];
            }
            wave_reduce4(mt, -INFINITY, [](float x, float y) { return fmaxf(x, y); });
            float mn[4];
#pragma unroll
            for (int qq = 0; qq < 4; qq++) {
                mn[qq] = fmaxf(mo[qq], mt[qq]);
                p[qq] = mn[qq] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(sv[qq] - mn[qq]);
                mt[qq] = p[qq];
            }
            wave_reduce4(mt, 0.f, [](float x, float y) { return x + y; });
#pragma unroll
            for (int qq = 0; qq < 4; qq++) {
                const int q = 4 * wl + qq;
                const float al = mo[qq] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mo[qq] - mn[qq]);
                P[G][q][lane] = p[qq];
                if (lane == 0) {
                    s_m[G][q] = mn[qq];
                    s_l[G][q] = s_l[G][q] * al + mt[qq];
                    s_al[G][q] = al;
                }
            }
        }
        lds_barrier();
        // values: output dims 32 wl + 16 tt + r, rows 4 s + e, on the f16
        // MFMA (16x16x32) in two k-steps of 32 keys: the weights p of row r,
        // keys 32 ks + 8 s .., and V split into f16 hi / lo halves, three
        // products ph vh + ph vl + pl vh (22-bit operands, f32 sums) into
        // o[tt + 2 ks] (v[tt * 4 + ks * 2 + plane], the operand layout)
        {
            float al[4];
#pragma unroll
            for (int e = 0; e < 4; e++) al[e] = s_al[G][4 * s + e];
#pragma unroll
            for (int tt = 0; tt < 4; tt++)
#pragma unroll
                for (int e = 0; e < 4; e++) o[tt][e] *= al[e];
#pragma unroll
            for (int ks = 0; ks < GK / 32; ks++) {
                const float4v p0 = *(const float4v*)&P[G][r][32 * ks + 8 * s];
                const float4v p1 = *(const float4v*)&P[G][r][32 * ks + 8 * s + 4];
                half8 ph, pl;
#pragma unroll
                for (int j = 0; j < 8; j++) {
                    _Float16 hh, ll;
                    split16(j < 4 ? p0[j] : p1[j - 4], hh, ll);
                    ph[j] = hh;
                    pl[j] = ll;
                }
#pragma unroll
                for (int tt = 0; tt < 2; tt++) {
                    const half8 vh = __builtin_bit_cast(half8, v[tt * 4 + ks * 2]);
                    const half8 vl = __builtin_bit_cast(half8, v[tt * 4 + ks * 2 + 1]);
                    float4v& acc = o[tt + 2 * ks];
                    acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(ph, vh, acc, 0, 0, 0);
                    acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(ph, vl, acc, 0, 0, 0);
                    acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(pl, vh, acc, 0, 0, 0);
                }
            }
        }
    };
    load(0, ka, va);
    for (int tile = 0; tile < ntiles; tile += 2) {
        if (tile + 1 < ntiles) load(tile + 1, kn, vn);
        step(tile, ka, va);
        if (tile + 1 >= ntiles) break;
        if (tile + 2 < ntiles) load(tile + 2, ka, va);
        step(tile + 1, kn, vn);
    }
    lds_barrier();
    // merge: group 1 leaves its outputs in LDS, group 0 combines
    // (m = max(m0, m1), w_G = exp2(m_G - m), out = sum_G w_G o_G / sum_G w_G l_G)
    if (G == 1) {
#pragma unroll
        for (int tt = 0; tt < 2; tt++)
#pragma unroll
            for (int e = 0; e < 4; e++) O1[4 * s + e][32 * wl + 16 * tt + r] = o[tt][e] + o[tt + 2][e];
    }
    lds_barrier();
    if (G == 0) {
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const int q = 4 * s + e;
            if (q % PPW >= npos) continue;
            const float m0 = s_m[0][q], m1 = s_m[1][q], m = fmaxf(m0, m1);
            const float w0 = m0 == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m0 - m);
            const float w1 = m1 == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m1 - m);
            const float l = s_l[0][q] * w0 + s_l[1][q] * w1;
            const int row = i0 + q % PPW, head = g * HPK + q / PPW;
#pragma unroll
            for (int tt = 0; tt < 2; tt++) {
                const int dd = 32 * wl + 16 * tt + r;
                out[(size_t)row * nh * HD + (size_t)head * HD + dd] =
                    ((o[tt][e] + o[tt + 2][e]) * w0 + O1[q][dd] * w1) / l;
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Flash form: 64 query rows per workgroup share each 32-key tile of K / V
// through LDS (the 16-row blocks above read every tile from L2 once per 16
// rows).  Scores are computed transposed, S^T = K Q^T, so that each lane
// (query r, k-slot s) ends up holding the weights of its own query for the
// keys {4s..4s+3, 16+4s..16+4s+3}: exactly the B operand of O^T = V^T P^T
// when the V tile's k-slot s holds the same eight keys, so the weights never
// go through LDS, and the output's lanes hold their own query's dims.  Same arithmetic as k_prefill_attn: q.k = qh.kh +
// qh.kl + ql.kh (f16 hi / lo halves, f32 sums), exp2 of log2-scaled scores
// with a running maximum, values ph.vh + ph.vl + pl.vh.
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
// tile the short block needs.  Wave w of a block holds 16 query rows: the
// 16-row block 4 qb + (w % 4) of k_prefill_attn (row q: chunk row PPW (4 qb
// + w % 4) + q % PPW, query head g HPK + q / PPW).  The placement check is
// k_prefill_attn's, on the pair's cells.
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
    // (CMF_PREFILL_FA=0: the 16-row blocks of k_prefill_attn)
    static const bool fa = !(getenv("CMF_PREFILL_FA") && getenv("CMF_PREFILL_FA")[0] == '0');
    if (fa) {
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
        int4v* op = (int4v*)a.khl;  // nkv x npad x 1 KiB, the same bytes as the K / V operands below
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
    const int nqb = (a.cnt + ppw - 1) / ppw;
    const bool xcd = a.nkv == 8 && xl_device_fits() && a.allow_xcd && a.cells && a.perr &&
                     8 * nqb <= PREFILL_XCD_CELLS;
    const dim3 grid = xcd ? dim3(8 * nqb) : dim3(nqb, a.nkv);
    typedef void (*Kern)(const float*, const int4v*, const float4v*, int, int, int, int, float*, unsigned long long*,
                         int*, unsigned long long);
    Kern k;
    switch (hpk) {
        case 1: k = xcd ? k_prefill_attn<1, true> : k_prefill_attn<1, false>; break;
        case 2: k = xcd ? k_prefill_attn<2, true> : k_prefill_attn<2, false>; break;
        case 4: k = xcd ? k_prefill_attn<4, true> : k_prefill_attn<4, false>; break;
        case 8: k = xcd ? k_prefill_attn<8, true> : k_prefill_attn<8, false>; break;
        default: k = xcd ? k_prefill_attn<16, true> : k_prefill_attn<16, false>; break;
    }
    int4v* kop = (int4v*)a.khl;
    float4v* vop = (float4v*)(a.khl + (size_t)a.nkv * npad * 2 * HD);
    hipLaunchKernelGGL(k_prefill_kv, dim3(npad / 64, a.nkv), dim3(256), 0, st, a.kc, a.vc, a.max_seq, n, npad, kop,
                       vop);
    hipLaunchKernelGGL(k, grid, dim3(512), 0, st, a.qbuf, kop, vop, npad, a.cnt, a.p0, a.nh, a.out, a.cells, a.perr,
                       a.tag);
    return CMF_OK;
}

}  // namespace cmf
