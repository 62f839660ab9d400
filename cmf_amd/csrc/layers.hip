// Decode-layer kernels around the GEMVs: qk-norm + RoPE + KV append, split-K
// decode attention over the appended KV (causal inside the verify block),
// merge, embedding gather and argmax.
//
// Semantics follow the reference CPU path:
//   rms_norm_into / add_rmsnorm_fused_into   inference.rs:33-86
//   rmsnorm_head (qk-norm), rope_rotate       attention.rs:606-624, 71-81
//   finish_projection order (norm then RoPE)  attention.rs:818-890
//   attend_group (scale 1/sqrt(hd), softmax)  kv_cache.rs:521-690
//   silu(g) * u                               inference.rs:14-16
//   argmax, ties to the highest index         sampler.rs:832-867
#include "common.h"
#include "gemv.h"
#include "layers.h"
#include "wave.h"

namespace cmf {

typedef float float4v __attribute__((ext_vector_type(4)));

// --------------------------------------------------------------------------
// block reductions (256 threads)
// --------------------------------------------------------------------------
__device__ inline double block_sum_d(double v, double* red) {
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    const int w = threadIdx.x >> 6, l = threadIdx.x & 63;
    __syncthreads();
    if (l == 0) red[w] = v;
    __syncthreads();
    double t = 0.0;
    const int nw = blockDim.x >> 6;
    for (int i = 0; i < nw; i++) t += red[i];
    return t;
}

__device__ inline float block_max_f(float v, float* red) {
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
    const int w = threadIdx.x >> 6, l = threadIdx.x & 63;
    __syncthreads();
    if (l == 0) red[w] = v;
    __syncthreads();
    float t = red[0];
    const int nw = blockDim.x >> 6;
    for (int i = 1; i < nw; i++) t = fmaxf(t, red[i]);
    return t;
}


// Embedding rows from the (tied) q8 lm_head: out[b] = q8 row * row_scale
// (pipeline.rs:5568-5575).  grid (nb), block 256.  With tok0, row 0 embeds
// *tok0 and row b > 0 toks[b - 1] (the verify rows [t_next, drafts...]).
__global__ __launch_bounds__(256) void k_embed(const int* __restrict__ toks, const int* __restrict__ tok0,
                                               EmbedSrc emb, int H, float* __restrict__ out, int ldo) {
    const int b = blockIdx.x;
    const int tok = tok0 ? (b == 0 ? *tok0 : toks[b - 1]) : toks[b];
    const bool ok = tok >= 0 && tok < emb.rows;
    const float rs = ok ? emb.rs[tok] : 0.f;
    const int rb = tok >> 4, r = tok & 15;
    for (int i = threadIdx.x; i < H; i += blockDim.x) {
        float e = 0.f;
        if (ok) {
            const int kc = i >> 6, s = (i >> 4) & 3, j = i & 15;
            e = (float)emb.w[(((size_t)rb * emb.nkc + kc) * 64 + 16 * s + r) * 16 + j] * rs;
        }
        out[(size_t)b * ldo + i] = e;
    }
}

// N head rows at once, as norm_rope with its own weights per row: the f64
// wave reductions of the N rows interleaved.
template <int N>
__device__ __forceinline__ void norm_rope_n(float (&x0)[N], float (&x1)[N], const float2 (&cs)[N], const float (&w0)[N],
                                            const float (&w1)[N], double eps) {
    double ss[N];
#pragma unroll
    for (int i = 0; i < N; i++) ss[i] = (double)x0[i] * (double)x0[i] + (double)x1[i] * (double)x1[i];
    wave_sum_n<N>(ss);
#pragma unroll
    for (int i = 0; i < N; i++) {
        const float inv = (float)(1.0 / sqrt(ss[i] / 128.0 + eps));
        const float a = x0[i] * inv * w0[i], b = x1[i] * inv * w1[i];
        x0[i] = a * cs[i].x - b * cs[i].y;
        x1[i] = a * cs[i].y + b * cs[i].x;
    }
}
__device__ __forceinline__ float2 head_norm_rope(float x0, float x1, const float* w, const float2* rope, int pos,
                                                 double eps, int lane) {
    return norm_rope(x0, x1, w[lane], w[lane + 64], rope[(size_t)pos * 64 + lane], eps);
}

// Chunk softmax and value pass of the n <= NQ queries qi = w + 4i owned by
// one wave: lane = key position for the softmax (max, exp, sum by wave
// reductions; the weights overwrite the scores), lane = dim pair for the
// values, o[qi][d] = sum_p e[qi][p] * V[p][d] in position order.
template <int NQ>
__device__ __forceinline__ void attn_values(float (*S)[ATT_C], const float (*V)[128 + 4], int w, int lane, int hpk,
                                            int nh, int g, int c, int nch, int n, float* pm, float* pl, float* po) {
    constexpr int C = ATT_C, HD = 128;
    float m[NQ], l[NQ], e[NQ];
#pragma unroll
    for (int i = 0; i < NQ; i++) m[i] = wave_max(S[w + 4 * i][lane]);
#pragma unroll
    for (int i = 0; i < NQ; i++) {
        e[i] = m[i] == -INFINITY ? 0.f : expf(S[w + 4 * i][lane] - m[i]);
        l[i] = e[i];
        S[w + 4 * i][lane] = e[i];
    }
#pragma unroll
    for (int i = 0; i < NQ; i++) l[i] = wave_sum(l[i]);
    if (lane == 0) {
#pragma unroll
        for (int i = 0; i < NQ; i++) {
            const int qi = w + 4 * i;
            const size_t row = (size_t)(qi / hpk) * nh + g * hpk + qi % hpk;
            if (i < n) {
                pm[row * nch + c] = m[i];
                pl[row * nch + c] = l[i];
            }
        }
    }
    float2 o[NQ];
#pragma unroll
    for (int i = 0; i < NQ; i++) o[i] = make_float2(0.f, 0.f);
#pragma unroll 2
    for (int p0 = 0; p0 < C; p0 += 4) {
        float2 vd[4];
#pragma unroll
        for (int j = 0; j < 4; j++) vd[j] = *(const float2*)&V[p0 + j][2 * lane];
#pragma unroll
        for (int i = 0; i < NQ; i++) {
            const float4 ew = *(const float4*)&S[w + 4 * i][p0];
            o[i].x += ew.x * vd[0].x;
            o[i].y += ew.x * vd[0].y;
            o[i].x += ew.y * vd[1].x;
            o[i].y += ew.y * vd[1].y;
            o[i].x += ew.z * vd[2].x;
            o[i].y += ew.z * vd[2].y;
            o[i].x += ew.w * vd[3].x;
            o[i].y += ew.w * vd[3].y;
        }
    }
#pragma unroll
    for (int i = 0; i < NQ; i++) {
        const int qi = w + 4 * i;
        const size_t row = (size_t)(qi / hpk) * nh + g * hpk + qi % hpk;
        if (i < n) ((float2*)(po + (row * nch + c) * HD))[lane] = o[i];
    }
}

// Chunk softmax (as attn_values) and then the values of all nq queries of
// the kv head, 16 at a time, by fp32 MFMA (16x16x4): D[q][d] = sum_p E[q][p] V[p][d],
// A = the weights E (query q = lane % 16, position 4k + lane / 16, rows of S
// past nq are never stored), B = V (position x dim), wave w producing dims
// 32w .. 32w+31 (two 16-column blocks).  S rows are SC floats apart and V rows
// VC floats (both padded so that the 16 A rows and the 4 B rows of one MFMA
// fall in distinct LDS banks).
template <int SC, int VC>
__device__ __forceinline__ void attn_values_mfma(float (*S)[SC], const float (*V)[VC], int w, int lane, int nq,
                                                 int hpk, int nh, int g, int c, int nch, float* pm, float* pl,
                                                 float* po) {
    constexpr int C = ATT_C, HD = 128;
    for (int qi = w; qi < nq; qi += 4) {
        const float mx = wave_max(S[qi][lane]);
        const float e = mx == -INFINITY ? 0.f : expf(S[qi][lane] - mx);
        S[qi][lane] = e;
        const float l = wave_sum(e);
        if (lane == 0) {
            const size_t row = (size_t)(qi / hpk) * nh + g * hpk + qi % hpk;
            pm[row * nch + c] = mx;
            pl[row * nch + c] = l;
        }
    }
    __syncthreads();
    const int d0 = 32 * w, q = lane & 15, kq = lane >> 4;
    for (int qb = 0; qb < nq; qb += 16) {  // blocks of 16 queries
        float4v acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = acc0;
#pragma unroll 4
        for (int k = 0; k < C / 4; k++) {
            const int p = 4 * k + kq;
            const float a = S[qb + q][p];
            acc0 = __builtin_amdgcn_mfma_f32_16x16x4f32(a, V[p][d0 + q], acc0, 0, 0, 0);
            acc1 = __builtin_amdgcn_mfma_f32_16x16x4f32(a, V[p][d0 + 16 + q], acc1, 0, 0, 0);
        }
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const int qi = qb + 4 * kq + e;
            if (qi < nq) {
                const size_t row = (size_t)(qi / hpk) * nh + g * hpk + qi % hpk;
                float* o = po + (row * nch + c) * HD + d0 + q;
                o[0] = acc0[e];
                o[16] = acc1[e];
            }
        }
    }
}

// Merge of the chunk partials of one (batch row b, head h) by one wave:
// out = sum_c w_c o_c / sum_c w_c l_c with w_c = exp(m_c - M), M = max_c m_c.
// The chunk maxima, sums and the first CB chunks' outputs (lane = dim pair)
// are requested together, so a merge over <= CB chunks costs one memory
// round trip (chunk indices clamped; chunks past `used` weigh 0).
template <int CB>
__device__ __forceinline__ float2 attn_merge_row(const float* pm, const float* pl, const float* po, int nch,
                                                 size_t row, int used, float* out) {
    constexpr int HD = 128;
    static_assert(64 % CB == 0, "chunk batch");
    const int lane = threadIdx.x & 63;
    const float* pmr = pm + row * nch;
    const float* plr = pl + row * nch;
    const float2* por = (const float2*)(po + row * nch * HD);
    float2 ov[CB];
#pragma unroll
    for (int j = 0; j < CB; j++) ov[j] = por[(size_t)min(j, used - 1) * (HD / 2) + lane];
    const float m_first = pmr[min(lane, used - 1)], l_first = plr[min(lane, used - 1)];
    float M = lane < used ? m_first : -INFINITY;
    for (int c = lane + 64; c < used; c += 64) M = fmaxf(M, pmr[c]);
    M = wave_max(M);
    float L = 0.f;
    float2 O = make_float2(0.f, 0.f);
    for (int c1 = 0; c1 < used; c1 += 64) {
        const int c = c1 + lane;
        const float mc = c1 == 0 ? (lane < used ? m_first : -INFINITY) : (c < used ? pmr[c] : -INFINITY);
        const float lc = c1 == 0 ? l_first : (c < used ? plr[c] : 0.f);
        const float wgt = mc == -INFINITY ? 0.f : expf(mc - M);
        L += wave_sum(c < used ? lc * wgt : 0.f);
        const int c_end = min(used, c1 + 64);
        for (int c0 = c1; c0 < c_end; c0 += CB) {
            if (c0 > 0) {
#pragma unroll
                for (int j = 0; j < CB; j++) ov[j] = por[(size_t)min(c0 + j, used - 1) * (HD / 2) + lane];
            }
#pragma unroll
            for (int j = 0; j < CB; j++) {
                const float wj = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(wgt), c0 - c1 + j));
                O.x += wj * ov[j].x;
                O.y += wj * ov[j].y;
            }
        }
    }
    const float inv = L > 0.f ? 1.0f / L : 0.f;
    const float2 res = make_float2(O.x * inv, O.y * inv);
    ((float2*)out)[lane] = res;
    return res;
}

// Merge of the chunk partials, one wave per (row, head): grid nb * nh.
// With a.wop the wave also writes its head's 128 values as two 64-column
// chunks of the output projection's q8 operand: x ~= cs (q0 + q1/128 +
// q2/16384), cs = max|x| of the chunk / 127 (the layout and split of
// prep8_row with one scale per chunk instead of per row).
__global__ __launch_bounds__(64) void k_attn_merge(AttnArgs a) {
    const int rh = blockIdx.x, b = rh / a.nh;
    const int used = (*a.pbase + a.padd + b + ATT_C) / ATT_C;
    const float2 o = attn_merge_row<32>(a.pm, a.pl, a.po, a.nch, (size_t)rh, used, a.out + (size_t)rh * 128);
    if (!a.wop) return;
    const int lane = threadIdx.x & 63, h = rh - b * a.nh, br = a.wop_b0 + b, nk = 2 * a.nh, M = a.wop_M;
    float am = fmaxf(fabsf(o.x), fabsf(o.y));
#pragma unroll
    for (int off = 16; off > 0; off >>= 1) am = fmaxf(am, __shfl_xor(am, off));  // each 32-lane half: one chunk
    const float sx = am > 0.f ? am / 127.0f : 1.0f;
    const float inv = 1.0f / sx;
    uint32_t p0 = 0, p1 = 0, p2 = 0;
    q8_split(o.x * inv, 0, p0, p1, p2);
    q8_split(o.y * inv, 1, p0, p1, p2);
    const int cc = 2 * h + (lane >> 5), j = (2 * lane) & 63;
    const size_t off = ((size_t)(4 * cc + (j >> 4)) * M + br) * 16 + (j & 15);
    *(uint16_t*)(a.wop + off) = (uint16_t)p0;
    *(uint16_t*)(a.wop + (size_t)nk * 64 * M + off) = (uint16_t)p1;
    *(uint16_t*)(a.wop + (size_t)nk * 128 * M + off) = (uint16_t)p2;
    if ((lane & 31) == 0) a.wop_cs[(size_t)br * nk + cc] = sx;
}

// KV append only (the MTP warm-up, attend = 0): row b of kv head g, one wave
// per (b, g): k-norm + RoPE of K, V as projected (finish_projection +
// append, attention.rs:818-890).  grid (nb, nkv), block 64.
__global__ __launch_bounds__(64) void k_kv_append(AttnArgs a) {
    constexpr int HD = 128;
    const int b = blockIdx.x, g = blockIdx.y, lane = threadIdx.x;
    const int pos = *a.pbase + a.padd + b;
    const float* xk = a.qkv + (size_t)b * a.ldq + (size_t)(a.nh + g) * HD;
    const float* xv = a.qkv + (size_t)b * a.ldq + (size_t)(a.nh + a.nkv + g) * HD;
    const float v0 = xv[lane], v1 = xv[lane + 64];
    const float2 k = head_norm_rope(xk[lane], xk[lane + 64], a.kn, a.rope, pos, a.eps, lane);
    float* kd = a.kc + ((size_t)g * a.max_seq + pos) * HD;
    float* vd = a.vc + ((size_t)g * a.max_seq + pos) * HD;
    kd[lane] = k.x;
    kd[lane + 64] = k.y;
    vd[lane] = v0;
    vd[lane + 64] = v1;
}

// Decode attention of one layer for the nb rows at positions pos0 .. pos0+nb-1
// (pos0 = *pbase + padd), one workgroup per (kv head g, 64-position chunk c),
// NQW = queries per wave (the hpk * nb queries of g, query qi on wave qi % 4):
//   - loads in the order they are needed, so that the short ones do not
//     wait behind the KV stream (a wave's loads complete in order): the
//     query rows, the new K/V rows that fall in the chunk, then the chunk's
//     cached K (registers) and V;
//   - q-norm + RoPE of the queries (Q in LDS) and, in the chunk that holds
//     new positions, k-norm + RoPE of their K rows, appended to the cache
//     and used from LDS with their V rows (finish_projection + append);
//   - scores with the causal limit pos0 + b (lanes = position x dim
//     quarter, the quarters summed by quad DPP), chunk softmax and values
//     (partials m, l, o per row/head/chunk).
template <int NQW>
__global__ __launch_bounds__(256) void k_attention(AttnArgs a) {
    constexpr int HD = 128, C = ATT_C, NR = MAXB / 4;  // NR: new rows per wave
    // the highest chunks (the new positions) first: past 256 workgroups the
    // last ones share a CU, and the new-row chunk has the longest chain
    const int g = blockIdx.x, c = gridDim.y - 1 - blockIdx.y, t = threadIdx.x;
    const int lane = t & 63, wave = __builtin_amdgcn_readfirstlane(t >> 6);
    const int nh = a.nh, hpk = nh / a.nkv, nq = a.nb * hpk;
    const int pos0 = *a.pbase + a.padd;
    const int stored = pos0 + a.nb;
    const int p0 = c * C;
    constexpr int QR = 4 * NQW < 16 ? 16 : 4 * NQW;  // Q rows: whole MFMA query blocks
    __shared__ __align__(16) float Q[QR][HD + 4];  // rows padded: the MFMA A reads take 16 rows at once
    // VM: values by MFMA (at least 9 queries); padded rows for its bank pattern
    constexpr bool VM = NQW >= 3;
    constexpr int VC = VM ? HD + 16 : HD + 4, SC = VM ? C + 4 : C, SR = VM ? (4 * NQW + 15) / 16 * 16 : 4 * NQW;
    __shared__ __align__(16) float V[C][VC];
    __shared__ __align__(16) float S[SR][SC];
    __shared__ __align__(16) float Kn[MAXB][HD + 4];
    if (p0 >= stored) return;
    const int np = min(C, stored - p0);
    const int nold = min(np, max(0, pos0 - p0));  // cached positions of this chunk
    // 1. query rows (indices clamped: every lane loads, extra rows unused)
    float qx0[NQW], qx1[NQW];
    float2 qcs[NQW];
#pragma unroll
    for (int i = 0; i < NQW; i++) {
        const int qi = min(wave + 4 * i, nq - 1), b = qi / hpk, h = g * hpk + qi % hpk;
        const float* x = a.qkv + (size_t)b * a.ldq + (size_t)h * HD;
        qx0[i] = x[lane];
        qx1[i] = x[lane + 64];
        qcs[i] = a.rope[(size_t)(pos0 + b) * 64 + lane];
    }
    const float qw0 = a.qn[lane], qw1 = a.qn[lane + 64];
    // 2. new rows b of this chunk (pos0 + b in [p0, p0 + C)): wave w takes
    // b_lo + w + 4j
    const int b_lo = max(0, p0 - pos0), b_hi = min(a.nb, p0 + C - pos0);
    float kx0[NR], kx1[NR], vx0[NR], vx1[NR];
    float2 kcs[NR];
#pragma unroll
    for (int j = 0; j < NR; j++) {
        const int b = min(b_lo + wave + 4 * j, a.nb - 1);
        const float* xk = a.qkv + (size_t)b * a.ldq + (size_t)(nh + g) * HD;
        const float* xv = a.qkv + (size_t)b * a.ldq + (size_t)(nh + a.nkv + g) * HD;
        kx0[j] = xk[lane];
        kx1[j] = xk[lane + 64];
        vx0[j] = xv[lane];
        vx1[j] = xv[lane + 64];
        kcs[j] = a.rope[(size_t)(pos0 + b) * 64 + lane];
    }
    const float kw0 = a.kn[lane], kw1 = a.kn[lane + 64];
    // 3. cached K: lane = (position pk, dim group dq), float4 j at dims 16 j
    // + 4 dq.  MF (several queries per wave): pk = 16 wave + lane % 16, dq =
    // lane / 16, the B operand of the score MFMAs (k step 4 j + c <-> dim
    // 16 j + 4 dq + c); otherwise pk = 16 wave + lane / 4, dq = lane % 4 and
    // the four dim groups of a position are one quad (VALU dots, quad sums).
    constexpr bool MF = NQW > 1;
    const int pk = wave * 16 + (MF ? (lane & 15) : (lane >> 2)), dq = MF ? lane >> 4 : lane & 3;
    const bool kvalid = pk < np;
    const float4* Kp = (const float4*)(a.kc + ((size_t)g * a.max_seq + p0 + (pk < nold ? pk : 0)) * HD) + dq;
    float4 kv[8];
#pragma unroll
    for (int j = 0; j < 8; j++) kv[j] = Kp[4 * j];
    // cached V: thread t loads float4 column t % 32 of rows t/32 + 8u
    const float4* Vg = (const float4*)(a.vc + ((size_t)g * a.max_seq + p0) * HD);
    float4 vv[8];
#pragma unroll
    for (int u = 0; u < 8; u++) {
        const int r = (t >> 5) + 8 * u;
        vv[u] = Vg[(size_t)(r < nold ? r : 0) * (HD / 4) + (t & 31)];
    }
    // every load is issued before any of them is waited for
    __builtin_amdgcn_sched_barrier(0);
    // queries: q-norm + RoPE and, in the chunk that holds new positions, the
    // new rows' k-norm + RoPE, their wave reductions interleaved (x[NQW + j]:
    // new row b_lo + wave + 4 j)
    float x0[NQW + NR], x1[NQW + NR], w0[NQW + NR], w1[NQW + NR];
    float2 cs[NQW + NR];
#pragma unroll
    for (int i = 0; i < NQW; i++) {
        x0[i] = qx0[i];
        x1[i] = qx1[i];
        w0[i] = qw0;
        w1[i] = qw1;
        cs[i] = qcs[i];
    }
#pragma unroll
    for (int j = 0; j < NR; j++) {
        x0[NQW + j] = kx0[j];
        x1[NQW + j] = kx1[j];
        w0[NQW + j] = kw0;
        w1[NQW + j] = kw1;
        cs[NQW + j] = kcs[j];
    }
    if (b_lo < b_hi) {
        norm_rope_n<NQW + NR>(x0, x1, cs, w0, w1, a.eps);
    } else {
        float (&y0)[NQW] = *reinterpret_cast<float (*)[NQW]>(x0);
        float (&y1)[NQW] = *reinterpret_cast<float (*)[NQW]>(x1);
        const float2 (&c2)[NQW] = *reinterpret_cast<const float2 (*)[NQW]>(cs);
        const float (&v0)[NQW] = *reinterpret_cast<const float (*)[NQW]>(w0);
        const float (&v1)[NQW] = *reinterpret_cast<const float (*)[NQW]>(w1);
        norm_rope_n<NQW>(y0, y1, c2, v0, v1, a.eps);
    }
#pragma unroll
    for (int i = 0; i < NQW; i++) {
        const int qi = wave + 4 * i;
        if (qi < nq) {
            Q[qi][lane] = x0[i];
            Q[qi][lane + 64] = x1[i];
        }
    }
    // new rows: appended to the cache, kept in LDS
#pragma unroll
    for (int j = 0; j < NR; j++) {
        const int b = b_lo + wave + 4 * j;
        if (b < b_hi) {
            const int pos = pos0 + b;
            Kn[b][lane] = x0[NQW + j];
            Kn[b][lane + 64] = x1[NQW + j];
            V[pos - p0][lane] = vx0[j];
            V[pos - p0][lane + 64] = vx1[j];
            float* kd = a.kc + ((size_t)g * a.max_seq + pos) * HD;
            float* vd = a.vc + ((size_t)g * a.max_seq + pos) * HD;
            kd[lane] = x0[NQW + j];
            kd[lane + 64] = x1[NQW + j];
            vd[lane] = vx0[j];
            vd[lane + 64] = vx1[j];
        }
    }
#pragma unroll
    for (int u = 0; u < 8; u++) {
        const int r = (t >> 5) + 8 * u;
        if (r < nold || r >= np) *(float4*)&V[r][4 * (t & 31)] = r < nold ? vv[u] : make_float4(0.f, 0.f, 0.f, 0.f);
    }
    __syncthreads();
    if (kvalid && pk >= nold) {
        const int b = p0 + pk - pos0;
#pragma unroll
        for (int j = 0; j < 8; j++) kv[j] = *(const float4*)&Kn[b][16 * j + 4 * dq];
    }
    // scores (MF) by fp32 MFMA (16x16x4): A = 16 queries (lane % 16) x the dims
    // of group lane / 16, B = K (positions of this wave x the same dims),
    // 32 k steps cover the 128 dims; D row 4 (lane / 16) + e = query, column
    // lane % 16 = position.  Query rows past nq are never stored.
    const float scale = 1.0f / sqrtf((float)HD);
    if constexpr (!MF) {
        // at most 4 queries: VALU dots of the lane's 32 dims, quad DPP sums
        float acc[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            float sv = 0.f;
            if (i < nq) {
#pragma unroll
                for (int j = 0; j < 8; j++) {
                    const float4 qq = *(const float4*)&Q[i][16 * j + 4 * dq];
                    sv += kv[j].x * qq.x + kv[j].y * qq.y + kv[j].z * qq.z + kv[j].w * qq.w;
                }
                sv += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, sv), 0xb1, 0xf, 0xf, false));
                sv += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, sv), 0x4e, 0xf, 0xf, false));
            }
            acc[i] = sv;
        }
        if (dq == 0) {
#pragma unroll
            for (int i = 0; i < 4; i++) {
                if (i < nq) {
                    const bool see = kvalid && p0 + pk <= pos0 + i / hpk;
                    S[i][pk] = see ? acc[i] * scale : -INFINITY;
                }
            }
        }
    }
    for (int qb = 0; MF && qb < nq; qb += 16) {
        const float* qrow = Q[min(qb + (lane & 15), QR - 1)];
        float4v d = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const float4 qa = *(const float4*)&qrow[16 * j + 4 * dq];
            d = __builtin_amdgcn_mfma_f32_16x16x4f32(qa.x, kv[j].x, d, 0, 0, 0);
            d = __builtin_amdgcn_mfma_f32_16x16x4f32(qa.y, kv[j].y, d, 0, 0, 0);
            d = __builtin_amdgcn_mfma_f32_16x16x4f32(qa.z, kv[j].z, d, 0, 0, 0);
            d = __builtin_amdgcn_mfma_f32_16x16x4f32(qa.w, kv[j].w, d, 0, 0, 0);
        }
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const int qi = qb + 4 * dq + e;
            if (qi < nq) {
                const bool see = kvalid && p0 + pk <= pos0 + qi / hpk;
                S[qi][pk] = see ? d[e] * scale : -INFINITY;
            }
        }
    }
    __syncthreads();
    const int nqw = (nq - wave + 3) >> 2;  // queries of this wave
    if constexpr (VM) {
        attn_values_mfma<SC, VC>(S, V, wave, lane, nq, hpk, nh, g, c, a.nch, a.pm, a.pl, a.po);
    } else if (nqw > 0) {
        attn_values<NQW>(S, V, wave, lane, hpk, nh, g, c, a.nch, nqw, a.pm, a.pl, a.po);
    }
}

// Argmax per row, ties to the highest index.  Pass 1: grid (nslices, nrows).
__global__ __launch_bounds__(256) void k_argmax_part(const float* __restrict__ x, int ld, int n,
                                                     int slice, float* __restrict__ pv,
                                                     int* __restrict__ pi) {
    const int s = blockIdx.x, r = blockIdx.y;
    const float* row = x + (size_t)r * ld;
    const int lo = s * slice, hi = min(n, lo + slice);
    float bv = -INFINITY;
    int bi = lo;
    constexpr int PER = 16;  // slice / 256, loads in flight together
    float vals[PER];
#pragma unroll
    for (int j = 0; j < PER; j++) {
        const int i = lo + threadIdx.x + j * 256;
        vals[j] = i < hi ? row[i] : -INFINITY;
    }
#pragma unroll
    for (int j = 0; j < PER; j++) {
        const int i = lo + threadIdx.x + j * 256;
        if (i < hi && (vals[j] > bv || (vals[j] == bv && i > bi))) {
            bv = vals[j];
            bi = i;
        }
    }
    // the same lexicographic (value, index) maximum: butterfly in each wave,
    // then the four waves' winners
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const float v2 = __shfl_xor(bv, o);
        const int i2 = __shfl_xor(bi, o);
        if (v2 > bv || (v2 == bv && i2 > bi)) {
            bv = v2;
            bi = i2;
        }
    }
    __shared__ float sv[4];
    __shared__ int si[4];
    const int w = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) {
        sv[w] = bv;
        si[w] = bi;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int q = 1; q < 4; q++)
            if (sv[q] > bv || (sv[q] == bv && si[q] > bi)) {
                bv = sv[q];
                bi = si[q];
            }
        pv[(size_t)r * gridDim.x + s] = bv;
        pi[(size_t)r * gridDim.x + s] = bi;
    }
}

// Pass 2: one wave per row.  The winner is the lexicographic maximum of
// (value, index) over the partials and the start (-inf, 0), the order the
// sequential scan of argmax (sampler.rs:1130-1154) keeps: a larger value wins,
// an equal value with a higher index wins, NaN never wins.  A maximum is
// order-free, so the lanes' strided scans and the butterfly give the same
// index as one scan over all partials.
__global__ __launch_bounds__(64) void k_argmax_final(const float* __restrict__ pv, const int* __restrict__ pi,
                                                     int ns, int nrows, int* __restrict__ out) {
    const int r = blockIdx.x, lane = threadIdx.x;
    if (r >= nrows) return;
    float bv = -INFINITY;
    int bi = 0;
    for (int s = lane; s < ns; s += 64) argmax_take(bv, bi, pv[(size_t)r * ns + s], pi[(size_t)r * ns + s]);
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const float v2 = __shfl_xor(bv, o);
        const int i2 = __shfl_xor(bi, o);
        argmax_take(bv, bi, v2, i2);
    }
    if (lane == 0) out[r] = bi;
}

// ---------------------------------------------------------------------------
// host launchers
// ---------------------------------------------------------------------------
void launch_embed(const int* toks, const EmbedSrc& e, int H, float* out, int ldo, int nb,
                  hipStream_t st, const int* tok0) {
    hipLaunchKernelGGL(k_embed, dim3(nb), dim3(256), 0, st, toks, tok0, e, H, out, ldo);
}

void launch_attention(const AttnArgs& a, int max_len, hipStream_t st, bool merge) {
    if (!a.attend) {  // a one-wave-per-row append: the attention grid's chunks would all idle
        hipLaunchKernelGGL(k_kv_append, dim3(a.nb, a.nkv), dim3(64), 0, st, a);
        return;
    }
    const int nch = (max_len + ATT_C - 1) / ATT_C;
    const int nqw = (a.nb * (a.nh / a.nkv) + 3) / 4;  // queries per wave
    void (*k)(AttnArgs) = nullptr;
    switch (nqw) {
        case 0:
        case 1: k = k_attention<1>; break;
        case 2: k = k_attention<2>; break;
        case 3: k = k_attention<3>; break;
        case 4: k = k_attention<4>; break;
        case 5: k = k_attention<5>; break;
        case 6: k = k_attention<6>; break;
        case 7: k = k_attention<7>; break;
        default: k = k_attention<8>; break;
    }
    hipLaunchKernelGGL(k, dim3(a.nkv, nch), dim3(256), 0, st, a);
    if (!a.attend || !merge) return;
    hipLaunchKernelGGL(k_attn_merge, dim3(a.nb * a.nh), dim3(64), 0, st, a);
}

int launch_argmax_part(const float* x, int ld, int n, int nrows, float* pv, int* pi, hipStream_t st) {
    const int slice = 4096, ns = (n + slice - 1) / slice;
    hipLaunchKernelGGL(k_argmax_part, dim3(ns, nrows), dim3(256), 0, st, x, ld, n, slice, pv, pi);
    return ns;
}
void launch_argmax(const float* x, int ld, int n, int nrows, float* pv, int* pi, int* out,
                   hipStream_t st) {
    const int ns = launch_argmax_part(x, ld, n, nrows, pv, pi, st);
    hipLaunchKernelGGL(k_argmax_final, dim3(nrows), dim3(64), 0, st, pv, pi, ns, nrows,
                       out);
}

}  // namespace cmf
