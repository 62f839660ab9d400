/*
 * Oracle (test infrastructure): codec layouts, dequantizers and the CPU
 * matvec contracts of the reference.  See oracle.h for the pinning table.
 */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "oracle.h"

#define GROUP 32
#define Q4_TILE 18
#define Q4TP_NIB 16

/* quant.rs:19-47 — IEEE half to f32, subnormals normalised (b+103 form). */
float or_f16_to_f32(uint16_t h) {
    uint32_t sign = h >> 15, exp = (h >> 10) & 0x1F, mant = h & 0x3FF, bits;
    if (exp == 0) {
        if (mant == 0) {
            bits = sign << 31;
        } else {
            uint32_t e = 0, m = mant;
            while ((m & 0x400) == 0) {
                m <<= 1;
                e++;
            }
            m &= 0x3FF;
            bits = (sign << 31) | ((113 - e) << 23) | (m << 13);
        }
    } else if (exp == 0x1F) {
        bits = (sign << 31) | (0xFFu << 23) | (mant << 13);
    } else {
        bits = (sign << 31) | ((exp + 127 - 15) << 23) | (mant << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* quant.rs:51-82 — f32 to half, round to nearest even. */
uint16_t or_f32_to_f16(float x) {
    uint32_t bits;
    memcpy(&bits, &x, 4);
    uint16_t sign = (uint16_t)((bits >> 16) & 0x8000);
    int32_t exp = (int32_t)((bits >> 23) & 0xFF);
    uint32_t mant = bits & 0x7FFFFF;
    if (exp == 0xFF) return sign | 0x7C00 | (mant ? 0x200 : 0);
    exp -= 127 - 15;
    if (exp >= 0x1F) return sign | 0x7C00;
    if (exp <= 0) {
        if (exp < -10) return sign;
        uint32_t m = mant | 0x800000;
        uint32_t shift = (uint32_t)(14 - exp);
        uint32_t half = m >> shift;
        uint32_t round = (m >> (shift - 1)) & 1;
        return sign | (uint16_t)(half + round);
    }
    uint32_t half = ((uint32_t)exp << 10) | (mant >> 13);
    uint32_t round = (mant >> 12) & 1;
    uint32_t sticky = (mant & 0xFFF) != 0;
    uint32_t bump = round & (sticky | (half & 1));
    return sign | (uint16_t)(half + bump);
}

static inline float rd_f16(const uint8_t* p) { return or_f16_to_f32((uint16_t)(p[0] | (p[1] << 8))); }

/* quant.rs:90-103 — disk q8_row: [i8 rows*cols][f16 rows]. */
void or_dequant_q8_row(const uint8_t* bytes, int rows, int cols, float* dst) {
    const uint8_t* sc = bytes + (size_t)rows * cols;
    for (int o = 0; o < rows; o++) {
        float s = rd_f16(sc + 2 * (size_t)o);
        for (int i = 0; i < cols; i++) dst[(size_t)o * cols + i] = (float)(int8_t)bytes[(size_t)o * cols + i] * s;
    }
}

/* quant.rs:322-344 — 18-byte tiles [f16 scale][16 B nibbles], low first. */
void or_dequant_q4t(const uint8_t* bytes, size_t n, float* dst) {
    size_t ng = (n + GROUP - 1) / GROUP;
    for (size_t g = 0; g < ng; g++) {
        const uint8_t* t = bytes + g * Q4_TILE;
        float s = rd_f16(t);
        for (int k = 0; k < 16; k++) {
            size_t i0 = g * GROUP + 2 * k, i1 = i0 + 1;
            uint8_t b = t[2 + k];
            if (i0 < n) dst[i0] = ((float)(b & 0x0F) - 8.0f) * s;
            if (i1 < n) dst[i1] = ((float)((b >> 4) & 0x0F) - 8.0f) * s;
        }
    }
}

/* quant.rs:355-365 */
size_t or_q4tp_code_stride(size_t gpr) { return (gpr * 5 + 7) / 8; }

void or_q4tp_sections(size_t rows, size_t cols, size_t* params_off, size_t* codes_off,
                      size_t* stride) {
    size_t gpr = cols / GROUP;
    size_t nib = rows * gpr * Q4TP_NIB;
    *params_off = nib;
    *codes_off = nib + rows * 4;
    *stride = or_q4tp_code_stride(gpr);
}

/* quant.rs:367-380 — 5-bit LSB-first field that may span two bytes. */
int or_q4tp_code(const uint8_t* codes, size_t stride, size_t g) {
    size_t bit = g * 5, b = bit / 8, sh = bit % 8;
    uint16_t lo = codes[b];
    uint16_t hi = (sh > 3 && b + 1 < stride) ? codes[b + 1] : 0;
    return (int)(((lo | (hi << 8)) >> sh) & 0x1F);
}

/* quant.rs:383-393 */
void or_q4tp_put_code(uint8_t* codes, size_t g, int code) {
    size_t bit = g * 5, b = bit / 8, sh = bit % 8;
    uint16_t v = (uint16_t)(code & 0x1F);
    codes[b] |= (uint8_t)(v << sh);
    if (sh > 3) codes[b + 1] |= (uint8_t)(v >> (8 - sh));
}

/* quant.rs:399-410 — t[0] = 2^lo, t[c] = t[c-1] * 2^step (f16 lo, step). */
void or_q4tp_ladder(const uint8_t* params, size_t r, float* t) {
    float lo = rd_f16(params + r * 4), st = rd_f16(params + r * 4 + 2);
    float ratio = exp2f(st);
    t[0] = exp2f(lo);
    for (int c = 1; c < 32; c++) t[c] = t[c - 1] * ratio;
}

/* quant.rs:414-431 */
void or_dequant_q4tp(const uint8_t* bytes, int rows, int cols, float* dst) {
    size_t gpr = (size_t)cols / GROUP, po, co, st;
    or_q4tp_sections(rows, cols, &po, &co, &st);
    for (int r = 0; r < rows; r++) {
        float tab[32];
        or_q4tp_ladder(bytes + po, r, tab);
        const uint8_t* codes = bytes + co + (size_t)r * st;
        for (size_t g = 0; g < gpr; g++) {
            float s = tab[or_q4tp_code(codes, st, g)];
            const uint8_t* t = bytes + ((size_t)r * gpr + g) * Q4TP_NIB;
            size_t base = (size_t)r * cols + g * GROUP;
            for (int k = 0; k < 16; k++) {
                dst[base + 2 * k] = ((float)(t[k] & 0x0F) - 8.0f) * s;
                dst[base + 2 * k + 1] = ((float)((t[k] >> 4) & 0x0F) - 8.0f) * s;
            }
        }
    }
}

/* ---------------------------------------------------------------------------
 * Exact contract kernels.
 * ------------------------------------------------------------------------- */

/* qtensor.rs:8687-8718 (dot_i8_f32_avx2): two 8-lane FMA accumulators over
 * 16-element steps, then the 8->4->2->1 horizontal reduction, then the
 * scalar tail.  This is the exact-contract q8 row dot on this x86 host. */
CLONES static float dot_i8_f32(const int8_t* w, const float* x, int n) {
    float a0[8] = {0}, a1[8] = {0};
    int j = 0;
    for (; j + 16 <= n; j += 16)
        for (int l = 0; l < 8; l++) {
            a0[l] = fmaf((float)w[j + l], x[j + l], a0[l]);
            a1[l] = fmaf((float)w[j + 8 + l], x[j + 8 + l], a1[l]);
        }
    float acc[8], s128[4];
    for (int l = 0; l < 8; l++) acc[l] = a0[l] + a1[l];
    for (int l = 0; l < 4; l++) s128[l] = acc[l] + acc[4 + l];
    float s64_0 = s128[0] + s128[2], s64_1 = s128[1] + s128[3];
    float sum = s64_0 + s64_1;
    for (; j < n; j++) sum += (float)w[j] * x[j];
    return sum;
}

/* qtensor.rs:4418-4432 — q4t_row_exact: per tile pairwise (lo, hi) terms,
 * then acc += ga * s, tiles in order. */
CLONES static float q4t_row_exact(const uint8_t* bytes, size_t r, size_t gpr, const float* x) {
    float acc = 0.0f;
    for (size_t g = 0; g < gpr; g++) {
        const uint8_t* t = bytes + (r * gpr + g) * Q4_TILE;
        float s = rd_f16(t);
        const float* xg = x + g * GROUP;
        float ga = 0.0f;
        for (int k = 0; k < 16; k++) {
            uint8_t b = t[2 + k];
            float p0 = ((float)(b & 0x0F) - 8.0f) * xg[2 * k];
            float p1 = ((float)((b >> 4) & 0x0F) - 8.0f) * xg[2 * k + 1];
            ga += p0 + p1;
        }
        acc += ga * s;
    }
    return acc;
}

/* qtensor.rs:4473-4513 — Q4tpView::scales_into (same codes as q4tp_code). */
static void q4tp_scales(const uint8_t* bytes, size_t rows, size_t cols, size_t r, float* sc) {
    size_t gpr = cols / GROUP, po, co, st;
    or_q4tp_sections(rows, cols, &po, &co, &st);
    float tab[32];
    or_q4tp_ladder(bytes + po, r, tab);
    const uint8_t* codes = bytes + co + r * st;
    for (size_t g = 0; g < gpr; g++) sc[g] = tab[or_q4tp_code(codes, st, g)];
}

/* qtensor.rs:4647-4661 — q4tp_row_exact. */
CLONES static float q4tp_row_exact(const uint8_t* nib, size_t r, size_t gpr, const float* x,
                            const float* sc) {
    float acc = 0.0f;
    for (size_t g = 0; g < gpr; g++) {
        const uint8_t* t = nib + (r * gpr + g) * Q4TP_NIB;
        const float* xg = x + g * GROUP;
        float ga = 0.0f;
        for (int k = 0; k < 16; k++) {
            float p0 = ((float)(t[k] & 0x0F) - 8.0f) * xg[2 * k];
            float p1 = ((float)((t[k] >> 4) & 0x0F) - 8.0f) * xg[2 * k + 1];
            ga += p0 + p1;
        }
        acc += ga * sc[g];
    }
    return acc;
}

/* Row-parallel dispatch (pool.rs:320 run_rows): every row is computed by
 * one thread in its own order, so the result does not depend on threads. */
void or_matmat(const or_qt* w, const float* xs, int b, float* out, int threads) {
    const int rows = w->rows, cols = w->cols;
    const size_t gpr = (size_t)cols / GROUP;
    if (threads < 1) threads = 1;
#pragma omp parallel num_threads(threads)
    {
        float* sc = (w->dtype == OR_Q4TP) ? (float*)malloc(sizeof(float) * (gpr ? gpr : 1)) : NULL;
#pragma omp for schedule(static)
        for (int r = 0; r < rows; r++) {
            if (w->dtype == OR_F32) {
                /* QTensor::F32 -> matvec_rows (pool.rs:535-548): sequential sum */
                const float* row = (const float*)w->bytes + (size_t)r * cols;
                for (int bi = 0; bi < b; bi++) {
                    const float* x = xs + (size_t)bi * cols;
                    float sum = 0.0f;
                    for (int j = 0; j < cols; j++) sum += row[j] * x[j];
                    out[(size_t)bi * rows + r] = sum;
                }
            } else if (w->dtype == OR_Q8ROW) {
                /* qtensor.rs:10033-10046: dot_i8_f32(row, xs) * row_scale */
                const int8_t* row = w->q + (size_t)r * cols;
                for (int bi = 0; bi < b; bi++)
                    out[(size_t)bi * rows + r] = dot_i8_f32(row, xs + (size_t)bi * cols, cols) * w->row_scale[r];
            } else if (w->dtype == OR_Q4T) {
                for (int bi = 0; bi < b; bi++)
                    out[(size_t)bi * rows + r] = q4t_row_exact(w->bytes, r, gpr, xs + (size_t)bi * cols);
            } else {
                q4tp_scales(w->bytes, rows, cols, r, sc);
                for (int bi = 0; bi < b; bi++)
                    out[(size_t)bi * rows + r] = q4tp_row_exact(w->bytes, r, gpr, xs + (size_t)bi * cols, sc);
            }
        }
        free(sc);
    }
}

void or_matvec(const or_qt* w, const float* x, float* out, int threads) {
    or_matmat(w, x, 1, out, threads);
}

/* ---------------------------------------------------------------------------
 * a8w8 contract.
 * ------------------------------------------------------------------------- */

/* Rust f32::round: half away from zero. */
static inline float round_away(float v) { return roundf(v); }

/* qtensor.rs:9237-9281 */
int or_split_act(const float* x, int n, int8_t* xq, float* sx_out, int* oi, float* ov,
                 int32_t* xsum) {
    double ss = 0.0;
    for (int j = 0; j < n; j++) ss += (double)(x[j] * x[j]);
    float rms = (float)sqrt(ss / (double)(n > 1 ? n : 1));
    float thr = 8.0f * rms;
    int no = 0;
    float amax = 0.0f;
    for (int j = 0; j < n; j++) {
        float a = fabsf(x[j]);
        if (a > thr) {
            oi[no] = j;
            ov[no] = x[j];
            no++;
        } else if (a > amax) {
            amax = a;
        }
    }
    float sx = amax > 0.0f ? amax / 127.0f : 1.0f;
    float inv = 1.0f / sx;
    int32_t s = 0;
    for (int j = 0; j < n; j++) {
        int8_t q;
        if (no && fabsf(x[j]) > thr) {
            q = 0;
        } else {
            float v = round_away(x[j] * inv);
            if (v < -127.0f) v = -127.0f;
            if (v > 127.0f) v = 127.0f;
            q = (int8_t)v;
        }
        xq[j] = q;
        s += q;
    }
    *sx_out = sx;
    *xsum = s;
    return no;
}

/* The integer tile dot of one q4 tile (32 codes, element 2k = low nibble of
 * byte k) against 32 int8 activations. */
static int32_t q4_tile_dot(const uint8_t* nib, const int8_t* xq) {
    int32_t d = 0;
    for (int k = 0; k < 16; k++)
        d += ((int)(nib[k] & 0x0F) - 8) * xq[2 * k] + ((int)((nib[k] >> 4) & 0x0F) - 8) * xq[2 * k + 1];
    return d;
}

/* The exact outlier corrections of one output (q8: qtensor.rs:8921-8933;
 * q4t_outlier qtensor.rs:4405-4413: (w * s) * xv; q4tp 4690-4700). */
static float a8w8_outliers(const or_qt* w, size_t r, size_t gpr, const float* sc, const int* oi,
                           const float* ov, int no, float acc) {
    for (int o = 0; o < no; o++) {
        int j = oi[o], k = j % GROUP;
        if (w->dtype == OR_Q8ROW) {
            acc += (float)w->q[r * (size_t)w->cols + j] * ov[o];
        } else if (w->dtype == OR_Q4T) {
            const uint8_t* t = w->bytes + (r * gpr + j / GROUP) * Q4_TILE;
            uint8_t byte = t[2 + k / 2];
            int nib = (k & 1) ? (byte >> 4) : (byte & 0x0F);
            acc += (float)(nib - 8) * rd_f16(t) * ov[o];
        } else {
            uint8_t byte = w->bytes[(r * gpr + j / GROUP) * Q4TP_NIB + k / 2];
            int nib = (k & 1) ? (byte >> 4) : (byte & 0x0F);
            acc += (float)(nib - 8) * sc[j / GROUP] * ov[o];
        }
    }
    return acc;
}

/* dot_q4t_row_1x4 (qtensor.rs:4315-4361, the x86 VNNI arm of q4t_matmat's
 * blocked path, 5908-5928): per tile, lane l of 8 holds the integer dot of
 * elements 4l..4l+3, converted to f32 and fused-multiply-added with the tile
 * scale into that lane's accumulator; the row result is the 8->4->2->1
 * horizontal sum (hsum256_ps, qtensor.rs:4300-4310). */
static float q4t_row_1x4_order(const uint8_t* bytes, size_t r, size_t gpr, const int8_t* xq) {
    float f[8] = {0};
    for (size_t g = 0; g < gpr; g++) {
        const uint8_t* t = bytes + (r * gpr + g) * Q4_TILE;
        float s = rd_f16(t);
        for (int l = 0; l < 8; l++) {
            int32_t p = 0;
            for (int e = 4 * l; e < 4 * l + 4; e++) {
                uint8_t byte = t[2 + e / 2];
                int nib = (e & 1) ? (byte >> 4) : (byte & 0x0F);
                p += (nib - 8) * xq[g * GROUP + e];
            }
            f[l] = fmaf((float)p, s, f[l]);
        }
    }
    float h[4];
    for (int l = 0; l < 4; l++) h[l] = f[l] + f[4 + l];
    float a = h[0] + h[2], b = h[1] + h[3];
    return a + b;
}

/* One batch under the a8w8 contract on an x86 host with AVX-512 VNNI (the
 * reference's default there): split_act per input row, then per weight row
 *   q8   (qmatmat x86 arm, qtensor.rs:3456-3470 with row_dot_avx2 8921-8933):
 *        integer dot * sx + outliers, * row_scale, every input alone;
 *   q4t  (q4t_matmat, qtensor.rs:5866-5948): inputs in blocks of four by the
 *        1x4 order above, the rest by dot_q4t_row_i8 (4106-4130: per tile
 *        acc += d * s), * sx, + outliers;
 *   q4tp (dot_q4tp_row_i8 order, 4517-4544), every input alone.
 * Rows are split into contiguous ranges (pool.rs:320 run_rows); each output
 * is computed by one thread in a fixed order, so threads do not change it. */
void or_matmat_a8w8(const or_qt* w, const float* xs, int b, float* out, int threads) {
    const int rows = w->rows, cols = w->cols;
    const size_t gpr = (size_t)cols / GROUP;
    int8_t* xq = (int8_t*)malloc((size_t)b * cols);
    int* oi = (int*)malloc(sizeof(int) * (size_t)b * cols);
    float* ov = (float*)malloc(sizeof(float) * (size_t)b * cols);
    float* sx = (float*)malloc(sizeof(float) * (size_t)b);
    int* no = (int*)malloc(sizeof(int) * (size_t)b);
    for (int i = 0; i < b; i++) {
        int32_t xsum;
        no[i] = or_split_act(xs + (size_t)i * cols, cols, xq + (size_t)i * cols, &sx[i], oi + (size_t)i * cols,
                             ov + (size_t)i * cols, &xsum);
    }
    if (threads < 1) threads = 1;
#pragma omp parallel num_threads(threads)
    {
        float* sc = (w->dtype == OR_Q4TP) ? (float*)malloc(sizeof(float) * (gpr ? gpr : 1)) : NULL;
#pragma omp for schedule(static)
        for (int r = 0; r < rows; r++) {
            if (sc) q4tp_scales(w->bytes, rows, cols, r, sc);
            for (int i = 0; i < b; i++) {
                const int8_t* x = xq + (size_t)i * cols;
                float acc;
                if (w->dtype == OR_Q8ROW) {
                    const int8_t* row = w->q + (size_t)r * cols;
                    int64_t d = 0;
                    for (int j = 0; j < cols; j++) d += (int64_t)row[j] * x[j];
                    acc = (float)(int32_t)d * sx[i];
                } else if (w->dtype == OR_Q4T) {
                    if (i < (b & ~3)) {
                        acc = q4t_row_1x4_order(w->bytes, r, gpr, x);
                    } else {
                        acc = 0.0f;
                        for (size_t g = 0; g < gpr; g++) {
                            const uint8_t* t = w->bytes + ((size_t)r * gpr + g) * Q4_TILE;
                            acc += (float)q4_tile_dot(t + 2, x + g * GROUP) * rd_f16(t);
                        }
                    }
                    acc *= sx[i];
                } else {
                    acc = 0.0f;
                    for (size_t g = 0; g < gpr; g++)
                        acc += (float)q4_tile_dot(w->bytes + ((size_t)r * gpr + g) * Q4TP_NIB, x + g * GROUP) * sc[g];
                    acc *= sx[i];
                }
                acc = a8w8_outliers(w, r, gpr, sc, oi + (size_t)i * cols, ov + (size_t)i * cols, no[i], acc);
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
}

void or_matvec_a8w8(const or_qt* w, const float* x, float* out, int threads) {
    or_matmat_a8w8(w, x, 1, out, threads);
}
