// Causal attention of a prefill chunk (head_dim 128) for gfx950.
//
// The chunk's rows sit at positions p0 .. p0 + cnt - 1 (p0 known to the
// host).  k_prefill_qk applies q-norm + RoPE to the queries (into a scratch
// buffer) and k-norm + RoPE to the new K rows, appending K and V to the
// cache (attention.rs:606-624, 818-890; kv_cache.rs:366-505), exactly as the
// decode kernels do.  k_prefill_attn then runs the attention of 16 query rows
// per workgroup — 16 / HPK positions times the HPK query heads of one kv
// head, which share its K / V — over 64-position key tiles with a running
// (online) softmax:
//   - the tile's K as f16 hi / lo halves and V (f32) in LDS, the next tile's
//     K / V requested into registers while the current one is used;
//   - scores on the f16 MFMA (q.k = qh.kh + qh.kl + ql.kh, 22-bit operands,
//     f32 sums), wave w the tile's keys 16 w .. 16 w + 15, causal limit the
//     row's position (kv_cache.rs:521-690);
//   - per row the running maximum m, the sum l and the factor exp(m_old -
//     m_new) applied to the row's output before the tile's values are added;
//   - values on the fp32 MFMA (16x16x4), wave w output dims 32 w .. 32 w + 31.
// Rows of a workgroup past the chunk see no keys and write nothing.
#include <math.h>

#include "common.h"
#include "layers.h"
#include "wave.h"

namespace cmf {

namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef float float4v __attribute__((ext_vector_type(4)));

constexpr int HD = 128;
constexpr int KT = 64;        // keys per tile
constexpr int KST = HD + 8;   // f16 row stride of Q / K in LDS
constexpr int VST = HD + 16;  // f32 row stride of V in LDS (conflict-free value operand reads)
constexpr int PST = KT + 4;   // f32 row stride of the scores / weights

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

// grid (ceil(cnt / (16 / HPK)), nkv), 256 threads.  Row q (0..15) of block
// qb: chunk row qb * PPW + q % PPW, query head g * HPK + q / PPW.
template <int HPK>
__global__ __launch_bounds__(256) void k_prefill_attn(const float* __restrict__ qbuf, const float* __restrict__ kc,
                                                      const float* __restrict__ vc, int max_seq, int cnt, int p0,
                                                      int nh, float* __restrict__ out) {
    constexpr int PPW = 16 / HPK;  // positions per workgroup
    const int qb = blockIdx.x, g = blockIdx.y, t = threadIdx.x, lane = t & 63;
    const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
    const int r = lane & 15, s = lane >> 4;
    __shared__ __align__(16) _Float16 QHL[2][16][KST];
    __shared__ __align__(16) _Float16 KHL[2][KT][KST];
    __shared__ __align__(16) float VT[KT][VST];
    __shared__ __align__(16) float P[16][PST];
    __shared__ float s_m[16], s_l[16], s_al[16];
    const int i0 = qb * PPW;
    const int npos = min(PPW, cnt - i0);
    // the queries as f16 hi / lo (rows past the chunk: zeros)
    for (int e = t; e < 16 * HD; e += 256) {
        const int q = e / HD, d = e % HD;
        const float v = q % PPW < npos ? qbuf[((size_t)(i0 + q % PPW) * nh + g * HPK + q / PPW) * HD + d] : 0.f;
        split16(v, QHL[0][q][d], QHL[1][q][d]);
    }
    if (t < 16) {
        s_m[t] = -INFINITY;
        s_l[t] = 0.f;
    }
    const int plast = p0 + i0 + npos - 1;  // the block's last query position
    const int ntiles = plast / KT + 1;
    const float* kb = kc + (size_t)g * max_seq * HD;
    const float* vb = vc + (size_t)g * max_seq * HD;
    // thread t moves float4 f = t + 256 u of a tile: key f / 32, dims 4 (f % 32)
    float4v kr[8], vr[8];
    auto load_tile = [&](int tile) {
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const int f = t + 256 * u;
            const int key = min(tile * KT + (f >> 5), plast);  // (keys past the last query: masked)
            kr[u] = *(const float4v*)(kb + (size_t)key * HD + 4 * (f & 31));
            vr[u] = *(const float4v*)(vb + (size_t)key * HD + 4 * (f & 31));
        }
    };
    load_tile(0);
    const float scale = 1.0f / sqrtf((float)HD);
    float4v o[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
    for (int tile = 0; tile < ntiles; tile++) {
        __syncthreads();  // the previous tile's LDS reads are done (and the queries written)
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const int f = t + 256 * u, kl = f >> 5, c = 4 * (f & 31);
            half4 h4, l4;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                _Float16 hh, ll;
                split16(kr[u][i], hh, ll);
                h4[i] = hh;
                l4[i] = ll;
            }
            *(half4*)&KHL[0][kl][c] = h4;
            *(half4*)&KHL[1][kl][c] = l4;
            *(float4v*)&VT[kl][c] = vr[u];
        }
        __syncthreads();
        if (tile + 1 < ntiles) load_tile(tile + 1);
        // scores of keys 16 wave .. + 15 of the tile
        {
            float4v d = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int ks = 0; ks < HD / 32; ks++) {
                const int oo = 32 * ks + 8 * s;
                const half8 qh = *(const half8*)&QHL[0][r][oo], ql = *(const half8*)&QHL[1][r][oo];
                const half8 kh = *(const half8*)&KHL[0][16 * wave + r][oo];
                const half8 kl = *(const half8*)&KHL[1][16 * wave + r][oo];
                d = __builtin_amdgcn_mfma_f32_16x16x32_f16(qh, kh, d, 0, 0, 0);
                d = __builtin_amdgcn_mfma_f32_16x16x32_f16(qh, kl, d, 0, 0, 0);
                d = __builtin_amdgcn_mfma_f32_16x16x32_f16(ql, kh, d, 0, 0, 0);
            }
            const int key = tile * KT + 16 * wave + r;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const int q = 4 * s + e;
                const bool see = q % PPW < npos && key <= p0 + i0 + q % PPW;
                P[q][16 * wave + r] = see ? d[e] * scale : -INFINITY;
            }
        }
        __syncthreads();
        // running softmax: wave w rows 4 w .. 4 w + 3, lane = key
#pragma unroll
        for (int qq = 0; qq < 4; qq++) {
            const int q = 4 * wave + qq;
            const float sv = P[q][lane];
            const float mo = s_m[q];
            const float mn = fmaxf(mo, wave_max(sv));
            const float p = mn == -INFINITY ? 0.f : expf(sv - mn);
            const float lt = wave_sum(p);
            const float al = mo == -INFINITY ? 0.f : expf(mo - mn);
            P[q][lane] = p;
            if (lane == 0) {
                s_m[q] = mn;
                s_l[q] = s_l[q] * al + lt;
                s_al[q] = al;
            }
        }
        __syncthreads();
        // values: output dims 32 wave + 16 tt + r, rows 4 s + e
        {
            float al[4];
#pragma unroll
            for (int e = 0; e < 4; e++) al[e] = s_al[4 * s + e];
#pragma unroll
            for (int tt = 0; tt < 2; tt++)
#pragma unroll
                for (int e = 0; e < 4; e++) o[tt][e] *= al[e];
            const int d0 = 32 * wave;
#pragma unroll
            for (int k = 0; k < KT / 4; k++) {
                const int p = 4 * k + s;
                const float a = P[r][p];
                o[0] = __builtin_amdgcn_mfma_f32_16x16x4f32(a, VT[p][d0 + r], o[0], 0, 0, 0);
                o[1] = __builtin_amdgcn_mfma_f32_16x16x4f32(a, VT[p][d0 + 16 + r], o[1], 0, 0, 0);
            }
        }
    }
    __syncthreads();
#pragma unroll
    for (int tt = 0; tt < 2; tt++)
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const int q = 4 * s + e;
            if (q % PPW < npos) {
                const int row = i0 + q % PPW, head = g * HPK + q / PPW;
                out[(size_t)row * nh * HD + (size_t)head * HD + 32 * wave + 16 * tt + r] = o[tt][e] / s_l[q];
            }
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
    const dim3 grid((a.cnt + ppw - 1) / ppw, a.nkv);
    switch (hpk) {
        case 1: hipLaunchKernelGGL(k_prefill_attn<1>, grid, dim3(256), 0, st, a.qbuf, a.kc, a.vc, a.max_seq, a.cnt, a.p0, a.nh, a.out); break;
        case 2: hipLaunchKernelGGL(k_prefill_attn<2>, grid, dim3(256), 0, st, a.qbuf, a.kc, a.vc, a.max_seq, a.cnt, a.p0, a.nh, a.out); break;
        case 4: hipLaunchKernelGGL(k_prefill_attn<4>, grid, dim3(256), 0, st, a.qbuf, a.kc, a.vc, a.max_seq, a.cnt, a.p0, a.nh, a.out); break;
        case 8: hipLaunchKernelGGL(k_prefill_attn<8>, grid, dim3(256), 0, st, a.qbuf, a.kc, a.vc, a.max_seq, a.cnt, a.p0, a.nh, a.out); break;
        default: hipLaunchKernelGGL(k_prefill_attn<16>, grid, dim3(256), 0, st, a.qbuf, a.kc, a.vc, a.max_seq, a.cnt, a.p0, a.nh, a.out); break;
    }
    return CMF_OK;
}

}  // namespace cmf
