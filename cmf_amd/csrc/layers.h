// Launchers of the decode-layer kernels (layers.hip).
#pragma once

#include "common.h"
#include "gemv.h"
#include "wave.h"

namespace cmf {

constexpr int ATT_C = 64;  // key positions per attention workgroup

// qk-norm + RoPE of one head row x (lane holds dims lane and lane + 64, the
// rotation pair): x * inv * w with inv = 1/sqrt(mean(x^2) + eps) (f64 sum),
// then (a, b) -> (a cos - b sin, a sin + b cos); w0/w1 = w[lane], w[lane +
// 64], cs = the (cos, sin) of the position at lane.
__device__ __forceinline__ float2 norm_rope(float x0, float x1, float w0, float w1, float2 cs, double eps) {
    const double ss = wave_sum((double)x0 * (double)x0 + (double)x1 * (double)x1);
    const float inv = (float)(1.0 / sqrt(ss / 128.0 + eps));
    const float a = x0 * inv * w0, b = x1 * inv * w1;
    return make_float2(a * cs.x - b * cs.y, a * cs.y + b * cs.x);
}

// tok0: row 0 embeds *tok0, row b > 0 toks[b - 1]
void launch_embed(const int* toks, const EmbedSrc& e, int H, float* out, int ldo, int nb,
                  hipStream_t st, const int* tok0 = nullptr);
// One layer's decode attention (head_dim 128): q/k-norm + RoPE, KV append,
// chunked causal attention over the cache and the merge into out
// [nb][nh * 128].  pm/pl [MAXB * nh][nch], po [MAXB * nh][nch][128] hold the
// chunk partials.
struct AttnArgs {
    const float* qkv;   // [nb][ldq] projected q | k | v heads
    int ldq;
    const float* qn;    // q-norm / k-norm weights [128]
    const float* kn;
    const float2* rope; // (cos, sin) [max_seq][64]
    float* kc;          // [nkv][max_seq][128]
    float* vc;
    int max_seq, nb, nh, nkv;
    double eps;
    const int* pbase;   // rows sit at positions *pbase + padd + b
    int padd;
    float *pm, *pl, *po;
    int nch;            // chunk capacity of the partial buffers
    float* out;
    int attend;         // 0: only append the rows' K/V (no queries, no output)
    // optional: the merge also writes the rows as the chunk-scaled q8 operand
    // of the output projection (planes [3][2 nh][4][wop_M] x 16 B, chunk scales
    // [wop_M][2 nh]); this launch's rows are rows wop_b0.. of that operand
    uint8_t* wop = nullptr;
    float* wop_cs = nullptr;
    int wop_M = 0, wop_b0 = 0;
};
// k_attention (chunk partials) then, with merge, k_attn_merge (rows of a.out).
void launch_attention(const AttnArgs& a, int max_len, hipStream_t st, bool merge = true);

// Causal attention of a prefill chunk (prefill_attn.hip): cnt rows at
// positions p0 + i of qkv [cnt][ldq] (q | k | v heads); q/k-norm + RoPE, the
// rows' K / V appended to the cache, out [cnt][nh * 128] (out == nullptr:
// only the append).  qbuf: [cnt][nh][128] scratch for the rotated queries;
// khl: scratch for the rearranged K / V operands, nkv * npad * 128 * 8 bytes
// (npad = ceil((p0 + cnt) / 128) * 128).
struct PrefillAttnArgs {
    const float* qkv;
    int ldq;
    const float *qn, *kn;
    const float2* rope;
    float *kc, *vc;
    int max_seq, cnt, p0, nh, nkv;
    double eps;
    float* qbuf;
    float* out;
    _Float16* khl;
    // placement check of the XCD variant (kv head from the XCD a workgroup
    // runs on): cells [query block][8] take the launch's tag, a collision
    // sets *perr; cells == nullptr or !allow_xcd: the grid-indexed variant
    unsigned long long* cells;
    int* perr;
    unsigned long long tag;
    bool allow_xcd;
};
constexpr int PREFILL_XCD_CELLS = 8 * 1024;  // query blocks of a chunk x 8 kv heads (2048 rows at 2 per block)
bool prefill_attention_fits(int nh, int nkv, int hd);
int launch_prefill_attention(const PrefillAttnArgs& a, hipStream_t st);
// The lexicographic (value, index) maximum step of argmax (sampler.rs:1130-1154
// keeps the higher index on equal values; NaN never wins).
__device__ __forceinline__ void argmax_take(float& bv, int& bi, float v, int i) {
    if (v > bv || (v == bv && i > bi)) {
        bv = v;
        bi = i;
    }
}
// The first pass of launch_argmax alone: per-slice partials of nrows rows
// into pv/pi [nrows][ns]; returns ns.
int launch_argmax_part(const float* x, int ld, int n, int nrows, float* pv, int* pi, hipStream_t st);
void launch_argmax(const float* x, int ld, int n, int nrows, float* pv, int* pi, int* out,
                   hipStream_t st);

}  // namespace cmf
