/*
 * Oracle timing arm (test infrastructure; never linked into the product):
 * the reference's x86 AVX-512 VNNI a8w8 kernels, used only to time the
 * reference's CPU path on the host cores.  Every function computes exactly
 * the values of the scalar a8w8 arm in quant.c (or_matmat_a8w8): integer dot
 * products are exact in any order, and the float steps below are the same
 * operations in the same order.  The tests pin this arm to the scalar one
 * bit for bit.
 *
 *   q8   row_dot_avx2 with dot_u8p128_i8_vnni (qtensor.rs:8921-8933,
 *        8939-8990): sum (w + 128) * x by 512-bit vpdpbusd in four
 *        accumulators, minus 128 * sum(x);
 *   q4t  dot_q4t_row_vnni (qtensor.rs:4204-4228): per tile one 256-bit
 *        vpdpbusd of |w| and sign(x, w), horizontal sum, acc += d * s;
 *        dot_q4t_row_1x4_vnni (4312-4361) for blocks of four inputs;
 *   q4tp dot_q4tp_row_vnni (4616-4641).
 */
#include <immintrin.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "oracle.h"

#define GROUP 32
#define Q4_TILE 18
#define Q4TP_NIB 16
#define VNNI __attribute__((target("avx2,fma,avx512f,avx512bw,avx512vl,avx512vnni")))

int or_fast_supported(void) {
    __builtin_cpu_init();
    return __builtin_cpu_supports("avx512f") && __builtin_cpu_supports("avx512bw") &&
           __builtin_cpu_supports("avx512vl") && __builtin_cpu_supports("avx512vnni");
}

static inline float f16_at(const uint8_t* p) { return or_f16_to_f32((uint16_t)(p[0] | (p[1] << 8))); }

/* dpbusd_hsum (qtensor.rs:8592-8603): one 256-bit u8 x i8 dot, then the
 * 8 -> 1 integer reduction. */
VNNI static inline int32_t dp_hsum(__m256i aw, __m256i xs) {
    __m256i d = _mm256_dpbusd_epi32(_mm256_setzero_si256(), aw, xs);
    __m128i s = _mm_add_epi32(_mm256_castsi256_si128(d), _mm256_extracti128_si256(d, 1));
    s = _mm_add_epi32(s, _mm_srli_si128(s, 8));
    s = _mm_add_epi32(s, _mm_srli_si128(s, 4));
    return _mm_cvtsi128_si32(s);
}

/* the 32 codes of a tile as int8 (nibble - 8), element order 0..31 */
VNNI static inline __m256i q4_codes(const uint8_t* nib) {
    const __m128i lomask = _mm_set1_epi8(0x0F);
    __m128i b = _mm_loadu_si128((const __m128i*)nib);
    __m128i lo = _mm_and_si128(b, lomask);
    __m128i hi = _mm_and_si128(_mm_srli_epi16(b, 4), lomask);
    return _mm256_sub_epi8(_mm256_set_m128i(_mm_unpackhi_epi8(lo, hi), _mm_unpacklo_epi8(lo, hi)),
                           _mm256_set1_epi8(8));
}

VNNI static int32_t q8_dot(const int8_t* w, const int8_t* x, int n, int32_t xsum) {
    const __m512i flip = _mm512_set1_epi8((char)0x80);
    __m512i a0 = _mm512_setzero_si512(), a1 = a0, a2 = a0, a3 = a0;
    int j = 0;
    for (; j + 256 <= n; j += 256) {
        a0 = _mm512_dpbusd_epi32(a0, _mm512_xor_si512(_mm512_loadu_si512(w + j), flip), _mm512_loadu_si512(x + j));
        a1 = _mm512_dpbusd_epi32(a1, _mm512_xor_si512(_mm512_loadu_si512(w + j + 64), flip),
                                 _mm512_loadu_si512(x + j + 64));
        a2 = _mm512_dpbusd_epi32(a2, _mm512_xor_si512(_mm512_loadu_si512(w + j + 128), flip),
                                 _mm512_loadu_si512(x + j + 128));
        a3 = _mm512_dpbusd_epi32(a3, _mm512_xor_si512(_mm512_loadu_si512(w + j + 192), flip),
                                 _mm512_loadu_si512(x + j + 192));
    }
    for (; j + 64 <= n; j += 64)
        a0 = _mm512_dpbusd_epi32(a0, _mm512_xor_si512(_mm512_loadu_si512(w + j), flip), _mm512_loadu_si512(x + j));
    int32_t t = _mm512_reduce_add_epi32(_mm512_add_epi32(_mm512_add_epi32(a0, a1), _mm512_add_epi32(a2, a3)));
    for (; j < n; j++) t += ((int32_t)(uint8_t)w[j] ^ 0x80) * x[j];
    return (int32_t)((uint32_t)t - 128u * (uint32_t)xsum);
}

VNNI static float q4t_row(const uint8_t* bytes, size_t r, size_t gpr, const int8_t* xq) {
    float acc = 0.0f;
    for (size_t g = 0; g < gpr; g++) {
        const uint8_t* t = bytes + (r * gpr + g) * Q4_TILE;
        __m256i w = q4_codes(t + 2);
        __m256i x = _mm256_loadu_si256((const __m256i*)(xq + g * GROUP));
        acc += (float)dp_hsum(_mm256_abs_epi8(w), _mm256_sign_epi8(x, w)) * f16_at(t);
    }
    return acc;
}

VNNI static float q4tp_row(const uint8_t* nib, size_t r, size_t gpr, const int8_t* xq, const float* sc) {
    float acc = 0.0f;
    for (size_t g = 0; g < gpr; g++) {
        __m256i w = q4_codes(nib + (r * gpr + g) * Q4TP_NIB);
        __m256i x = _mm256_loadu_si256((const __m256i*)(xq + g * GROUP));
        acc += (float)dp_hsum(_mm256_abs_epi8(w), _mm256_sign_epi8(x, w)) * sc[g];
    }
    return acc;
}

VNNI static inline float hsum8(__m256 v) {
    __m128 s = _mm_add_ps(_mm256_castps256_ps128(v), _mm256_extractf128_ps(v, 1));
    s = _mm_add_ps(s, _mm_movehl_ps(s, s));
    s = _mm_add_ss(s, _mm_shuffle_ps(s, s, 0x55));
    return _mm_cvtss_f32(s);
}

VNNI static void q4t_row_1x4(const uint8_t* bytes, size_t r, size_t gpr, const int8_t* const xs[4], float d[4]) {
    __m256 f0 = _mm256_setzero_ps(), f1 = f0, f2 = f0, f3 = f0;
    for (size_t g = 0; g < gpr; g++) {
        const uint8_t* t = bytes + (r * gpr + g) * Q4_TILE;
        __m256 sv = _mm256_set1_ps(f16_at(t));
        __m256i w = q4_codes(t + 2);
        __m256i aw = _mm256_abs_epi8(w);
        size_t off = g * GROUP;
#define DOT4(X)                                                                                          \
    _mm256_cvtepi32_ps(_mm256_dpbusd_epi32(_mm256_setzero_si256(), aw,                                   \
                                           _mm256_sign_epi8(_mm256_loadu_si256((const __m256i*)((X) + off)), w)))
        f0 = _mm256_fmadd_ps(DOT4(xs[0]), sv, f0);
        f1 = _mm256_fmadd_ps(DOT4(xs[1]), sv, f1);
        f2 = _mm256_fmadd_ps(DOT4(xs[2]), sv, f2);
        f3 = _mm256_fmadd_ps(DOT4(xs[3]), sv, f3);
#undef DOT4
    }
    d[0] = hsum8(f0);
    d[1] = hsum8(f1);
    d[2] = hsum8(f2);
    d[3] = hsum8(f3);
}

/* q4tp_scales / the ladder codes, as quant.c reads them */
static void q4tp_row_scales(const uint8_t* bytes, size_t rows, size_t cols, size_t r, float* sc) {
    size_t gpr = cols / GROUP, po, co, st;
    or_q4tp_sections(rows, cols, &po, &co, &st);
    float tab[32];
    or_q4tp_ladder(bytes + po, r, tab);
    for (size_t g = 0; g < gpr; g++) sc[g] = tab[or_q4tp_code(bytes + co + r * st, st, g)];
}

/* Same contract, arguments and output as or_matmat_a8w8 (quant.c); returns
 * -1 (and computes nothing) on a host without AVX-512 VNNI. */
int or_fast_matmat_a8w8(const or_qt* w, const float* xs, int b, float* out, int threads) {
    if (!or_fast_supported() || w->dtype == OR_F32) return -1;
    const int rows = w->rows, cols = w->cols;
    const size_t gpr = (size_t)cols / GROUP;
    int8_t* xq = (int8_t*)malloc((size_t)b * cols + 64);
    int* oi = (int*)malloc(sizeof(int) * (size_t)b * cols);
    float* ov = (float*)malloc(sizeof(float) * (size_t)b * cols);
    float* sx = (float*)malloc(sizeof(float) * (size_t)b);
    int* no = (int*)malloc(sizeof(int) * (size_t)b);
    int32_t* xsum = (int32_t*)malloc(sizeof(int32_t) * (size_t)b);
    for (int i = 0; i < b; i++)
        no[i] = or_split_act(xs + (size_t)i * cols, cols, xq + (size_t)i * cols, &sx[i], oi + (size_t)i * cols,
                             ov + (size_t)i * cols, &xsum[i]);
    if (threads < 1) threads = 1;
#pragma omp parallel num_threads(threads)
    {
        float* sc = (w->dtype == OR_Q4TP) ? (float*)malloc(sizeof(float) * (gpr ? gpr : 1)) : NULL;
        float d4[4];
#pragma omp for schedule(static)
        for (int r = 0; r < rows; r++) {
            if (sc) q4tp_row_scales(w->bytes, rows, cols, r, sc);
            for (int i = 0; i < b; i++) {
                const int8_t* x = xq + (size_t)i * cols;
                float acc;
                if (w->dtype == OR_Q8ROW) {
                    acc = (float)q8_dot(w->q + (size_t)r * cols, x, cols, xsum[i]) * sx[i];
                } else if (w->dtype == OR_Q4T) {
                    if (i < (b & ~3)) {
                        if ((i & 3) == 0) {
                            const int8_t* x4[4] = {x, x + cols, x + 2 * (size_t)cols, x + 3 * (size_t)cols};
                            q4t_row_1x4(w->bytes, r, gpr, x4, d4);
                        }
                        acc = d4[i & 3];
                    } else {
                        acc = q4t_row(w->bytes, r, gpr, x);
                    }
                    acc *= sx[i];
                } else {
                    acc = q4tp_row(w->bytes, r, gpr, x, sc) * sx[i];
                }
                /* outliers: the scalar arm's exact corrections, same order */
                const int* io = oi + (size_t)i * cols;
                const float* vo = ov + (size_t)i * cols;
                for (int o = 0; o < no[i]; o++) {
                    int j = io[o], k = j % GROUP;
                    if (w->dtype == OR_Q8ROW) {
                        acc += (float)w->q[(size_t)r * cols + j] * vo[o];
                    } else if (w->dtype == OR_Q4T) {
                        const uint8_t* t = w->bytes + ((size_t)r * gpr + j / GROUP) * Q4_TILE;
                        uint8_t byte = t[2 + k / 2];
                        int nib = (k & 1) ? (byte >> 4) : (byte & 0x0F);
                        acc += (float)(nib - 8) * f16_at(t) * vo[o];
                    } else {
                        uint8_t byte = w->bytes[((size_t)r * gpr + j / GROUP) * Q4TP_NIB + k / 2];
                        int nib = (k & 1) ? (byte >> 4) : (byte & 0x0F);
                        acc += (float)(nib - 8) * sc[j / GROUP] * vo[o];
                    }
                }
                if (w->dtype == OR_Q8ROW) acc *= w->row_scale[r];
                out[(size_t)i * rows + r] = acc;
            }
        }
        free(sc);
    }
    free(xq);
    free(oi);
    free(ov);
    free(sx);
    free(no);
    free(xsum);
    return 0;
}
