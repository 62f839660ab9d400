// Launchers of the decode-layer kernels (layers.hip).
#pragma once

#include "common.h"
#include "gemv.h"

namespace cmf {

constexpr int ATT_C = 64;  // key positions per attention wave

// Where a producer writes its prepared activations (see gemv.h).
struct PrepDst {
    int kind;         // 8 (q8 weights) or 16 (q4t / q4tp weights)
    int nk;           // q8: chunks of 64 columns; q4: tiles of 32 columns
    uint8_t* planes;
    float* xs;
};


void launch_add_rmsnorm_prep(float* h, int ldh, const float* delta, int ldd, const float* w, int H,
                             double eps, const PrepDst& d, float* out, int ldo, int nb,
                             hipStream_t st);
void launch_mtp_cat_prep(const int* toks, const float* hid, int ldh, const EmbedSrc& e,
                         const float* enorm, const float* hnorm, int H, double eps, const PrepDst& d,
                         int nb, hipStream_t st);
void launch_embed(const int* toks, const EmbedSrc& e, int H, float* out, int ldo, int nb,
                  hipStream_t st);
void launch_qk_rope_append(const float* qkv, int ldq, const float* qn, const float* kn,
                           const float2* rope, int nh, int nkv, int hd, double eps, const int* pbase,
                           int padd, float* kc, float* vc, int max_seq, float* qout, int ldqo, int nb,
                           hipStream_t st);
void launch_attention(const float* q, int ldq, const float* kc, const float* vc, int max_seq, int nb,
                      int nh, int nkv, const int* pbase, int padd, int max_len, float* pm, float* pl,
                      float* po, int nch_cap, float* out_f32, hipStream_t st);
void launch_silu_mul_prep(const float* gu, int ldg, int I, const PrepDst& d, float* out, int nb,
                          hipStream_t st);
void launch_argmax(const float* x, int ld, int n, int nrows, float* pv, int* pi, int* out,
                   hipStream_t st);

}  // namespace cmf
