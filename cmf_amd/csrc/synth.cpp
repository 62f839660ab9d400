// Seeded synthetic inputs for the decode hot path (host code, no GPU).
//
// Generator: SplitMix64 (the engine's own RNG, sampler.rs:54-84) feeding
// Box-Muller for N(0,1).  Every row of every tensor draws from its own
// stream, seeded from (tensor seed, row), so tensors are identical however
// many threads build them.  The byte layouts produced are exactly the
// reference's (cortiq-core/src/quant.rs): q8 in the engine's in-memory form
// (int8 rows + f32 row_scale, qtensor.rs:196-231), q4_tiled 18-byte tiles,
// q4tp [nibbles][row params][codes].
#include <math.h>
#include <stdint.h>
#include <string.h>

#include <algorithm>
#include <thread>
#include <vector>

#include "../../include/cmf_hip.h"

namespace {

struct Rng {
    uint64_t s;
    uint64_t next() {
        s += 0x9E3779B97F4A7C15ull;
        uint64_t z = s;
        z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
        z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
        return z ^ (z >> 31);
    }
    // Box-Muller on two 53-bit uniforms; u1 in (0, 1].
    double normal() {
        double u1 = ((next() >> 11) + 1) * (1.0 / 9007199254740992.0);
        double u2 = (next() >> 11) * (1.0 / 9007199254740992.0);
        return sqrt(-2.0 * log(u1)) * cos(6.283185307179586 * u2);
    }
};

inline uint64_t row_seed(uint64_t seed, uint64_t row) {
    Rng r{seed ^ (row * 0xD1B54A32D192ED03ull)};
    return r.next();
}

template <class F>
void par_rows(int64_t rows, F f) {
    unsigned nt = std::max(1u, std::min(16u, std::thread::hardware_concurrency()));
    if (rows < 64) nt = 1;
    std::vector<std::thread> ts;
    int64_t per = (rows + nt - 1) / nt;
    for (unsigned t = 0; t < nt; t++) {
        int64_t a = t * per, b = std::min<int64_t>(rows, a + per);
        if (a >= b) break;
        ts.emplace_back([=] {
            for (int64_t r = a; r < b; r++) f(r);
        });
    }
    for (auto& t : ts) t.join();
}

// quant.rs:51-82 (RNE f32 -> f16), restated for the encoder side.
uint16_t f32_to_f16(float x) {
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
        uint32_t m = mant | 0x800000, shift = (uint32_t)(14 - exp);
        return sign | (uint16_t)((m >> shift) + ((m >> (shift - 1)) & 1));
    }
    uint32_t half = ((uint32_t)exp << 10) | (mant >> 13);
    uint32_t round = (mant >> 12) & 1, sticky = (mant & 0xFFF) != 0;
    return sign | (uint16_t)(half + (round & (sticky | (half & 1))));
}

float f16_to_f32(uint16_t h) {
    uint32_t sign = h >> 15, exp = (h >> 10) & 0x1F, mant = h & 0x3FF, bits;
    if (exp == 0) {
        if (mant == 0) {
            bits = sign << 31;
        } else {
            uint32_t e = 0, m = mant;
            while (!(m & 0x400)) {
                m <<= 1;
                e++;
            }
            bits = (sign << 31) | ((113 - e) << 23) | ((m & 0x3FF) << 13);
        }
    } else if (exp == 0x1F) {
        bits = (sign << 31) | (0xFFu << 23) | (mant << 13);
    } else {
        bits = (sign << 31) | ((exp + 112) << 23) | (mant << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

inline void put_code(uint8_t* codes, size_t g, int code) {
    size_t bit = g * 5, b = bit / 8, sh = bit % 8;
    uint16_t v = (uint16_t)(code & 0x1F);
    codes[b] |= (uint8_t)(v << sh);
    if (sh > 3) codes[b + 1] |= (uint8_t)(v >> (8 - sh));
}

}  // namespace

extern "C" {

void cmf_synth_normal(uint64_t seed, int64_t n, float sigma, float* out) {
    const int64_t blk = 4096;
    par_rows((n + blk - 1) / blk, [&](int64_t r) {
        Rng g{row_seed(seed, (uint64_t)r)};
        for (int64_t i = r * blk; i < std::min(n, (r + 1) * blk); i++) out[i] = (float)(g.normal() * sigma);
    });
}

// Config 1: W int8 uniform in [-127,127], f32 row scale |N(0,1)|*0.01.
void cmf_synth_q8_uniform(uint64_t seed, int rows, int cols, int8_t* q, float* row_scale) {
    par_rows(rows, [&](int64_t r) {
        Rng g{row_seed(seed, (uint64_t)r)};
        row_scale[r] = (float)(fabs(g.normal()) * 0.01);
        for (int c = 0; c < cols; c++) q[(size_t)r * cols + c] = (int8_t)((int)(g.next() % 255) - 127);
    });
}

// Config 2: q4_tiled, nibbles uniform 0..15, f16 scale |N(0,1)|*sigma.
void cmf_synth_q4t_uniform(uint64_t seed, int rows, int cols, float sigma, uint8_t* bytes) {
    const int gpr = cols / 32;
    par_rows(rows, [&](int64_t r) {
        Rng g{row_seed(seed, (uint64_t)r)};
        for (int t = 0; t < gpr; t++) {
            uint8_t* tile = bytes + ((size_t)r * gpr + t) * 18;
            uint16_t s = f32_to_f16((float)(fabs(g.normal()) * sigma));
            tile[0] = (uint8_t)(s & 0xFF);
            tile[1] = (uint8_t)(s >> 8);
            uint64_t u = g.next(), v = g.next();
            for (int k = 0; k < 8; k++) tile[2 + k] = (uint8_t)(u >> (8 * k));
            for (int k = 0; k < 8; k++) tile[10 + k] = (uint8_t)(v >> (8 * k));
        }
    });
}

// Config 3: q4tp, per row lo = log2(|N|*sigma), step = log2(ratio) (both
// f16), 5-bit codes uniform 0..31, nibbles uniform.
void cmf_synth_q4tp_uniform(uint64_t seed, int rows, int cols, float sigma, float ratio,
                            uint8_t* bytes) {
    const size_t gpr = cols / 32, nib = (size_t)rows * gpr * 16, stride = (gpr * 5 + 7) / 8;
    uint8_t* params = bytes + nib;
    uint8_t* codes = params + (size_t)rows * 4;
    memset(codes, 0, (size_t)rows * stride);
    par_rows(rows, [&](int64_t r) {
        Rng g{row_seed(seed, (uint64_t)r)};
        double base = fabs(g.normal()) * sigma;
        if (base < 1e-30) base = 1e-30;
        uint16_t lo = f32_to_f16((float)log2(base)), st = f32_to_f16((float)log2((double)ratio));
        params[r * 4 + 0] = (uint8_t)(lo & 0xFF);
        params[r * 4 + 1] = (uint8_t)(lo >> 8);
        params[r * 4 + 2] = (uint8_t)(st & 0xFF);
        params[r * 4 + 3] = (uint8_t)(st >> 8);
        for (size_t t = 0; t < gpr; t++) {
            put_code(codes + (size_t)r * stride, t, (int)(g.next() & 31));
            uint8_t* tile = bytes + ((size_t)r * gpr + t) * 16;
            uint64_t u = g.next(), v = g.next();
            for (int k = 0; k < 8; k++) tile[k] = (uint8_t)(u >> (8 * k));
            for (int k = 0; k < 8; k++) tile[8 + k] = (uint8_t)(v >> (8 * k));
        }
    });
}

// Weights ~N(0, sigma^2) quantized to q8_row: scale = absmax/127 stored as
// f16 (quant.rs:4-5) and expanded to the engine's f32 row_scale; q =
// round(w / scale) clamped to [-127, 127].
void cmf_synth_q8_normal(uint64_t seed, int rows, int cols, float sigma, int8_t* q,
                         float* row_scale) {
    par_rows(rows, [&](int64_t r) {
        Rng g{row_seed(seed, (uint64_t)r)};
        std::vector<float> w(cols);
        float amax = 0.f;
        for (int c = 0; c < cols; c++) {
            w[c] = (float)(g.normal() * sigma);
            amax = std::max(amax, fabsf(w[c]));
        }
        float s = f16_to_f32(f32_to_f16(amax / 127.0f));
        row_scale[r] = s;
        float inv = s > 0.f ? 1.0f / s : 0.f;
        for (int c = 0; c < cols; c++) {
            float v = roundf(w[c] * inv);
            q[(size_t)r * cols + c] = (int8_t)std::max(-127.f, std::min(127.f, v));
        }
    });
}

// Weights ~N(0, sigma^2) quantized to q4_tiled: per 32-group scale =
// absmax/7 (f16), nibble = clamp(round(w/scale) + 8, 0, 15).
void cmf_synth_q4t_normal(uint64_t seed, int rows, int cols, float sigma, uint8_t* bytes) {
    const int gpr = cols / 32;
    par_rows(rows, [&](int64_t r) {
        Rng g{row_seed(seed, (uint64_t)r)};
        for (int t = 0; t < gpr; t++) {
            float w[32], amax = 0.f;
            for (int k = 0; k < 32; k++) {
                w[k] = (float)(g.normal() * sigma);
                amax = std::max(amax, fabsf(w[k]));
            }
            uint16_t sh = f32_to_f16(amax / 7.0f);
            float s = f16_to_f32(sh), inv = s > 0.f ? 1.0f / s : 0.f;
            uint8_t* tile = bytes + ((size_t)r * gpr + t) * 18;
            tile[0] = (uint8_t)(sh & 0xFF);
            tile[1] = (uint8_t)(sh >> 8);
            for (int k = 0; k < 16; k++) {
                int a = (int)roundf(w[2 * k] * inv) + 8, b = (int)roundf(w[2 * k + 1] * inv) + 8;
                a = std::max(0, std::min(15, a));
                b = std::max(0, std::min(15, b));
                tile[2 + k] = (uint8_t)(a | (b << 4));
            }
        }
    });
}

// Uniform token ids in [0, vocab).
void cmf_synth_ids(uint64_t seed, int n, int vocab, int32_t* out) {
    Rng g{seed};
    for (int i = 0; i < n; i++) out[i] = (int32_t)(g.next() % (uint64_t)vocab);
}

}  // extern "C"
