// Wave-wide (64-lane) reductions by DPP row operations, no LDS permutes:
// pair and quad swaps, row_shr 4 and 8 (a row's total in its lanes 12..15),
// row_bcast 15 and 31 (rows 0+1 in lane 31, the wave's total in lane 63),
// then lane 63 is read into a wave-uniform value.  Lanes a DPP step cannot
// source keep the operation's identity.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace cmf {

template <int CTRL, int ROWS>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v, uint32_t ident) {
    return (uint32_t)__builtin_amdgcn_update_dpp((int)ident, (int)v, CTRL, ROWS, 0xf, false);
}

template <typename Op>
__device__ __forceinline__ double wave_reduce_f64(double v, double ident, Op op) {
    const uint64_t iu = __builtin_bit_cast(uint64_t, ident);
    auto step = [&](auto ctrl, auto rows) {
        constexpr int C = decltype(ctrl)::value, R = decltype(rows)::value;
        const uint64_t u = __builtin_bit_cast(uint64_t, v);
        const uint32_t lo = dpp_u32<C, R>((uint32_t)u, (uint32_t)iu);
        const uint32_t hi = dpp_u32<C, R>((uint32_t)(u >> 32), (uint32_t)(iu >> 32));
        v = op(v, __builtin_bit_cast(double, ((uint64_t)hi << 32) | lo));
    };
    step(std::integral_constant<int, 0xb1>{}, std::integral_constant<int, 0xf>{});   // quad_perm [1,0,3,2]
    step(std::integral_constant<int, 0x4e>{}, std::integral_constant<int, 0xf>{});   // quad_perm [2,3,0,1]
    step(std::integral_constant<int, 0x114>{}, std::integral_constant<int, 0xf>{});  // row_shr 4
    step(std::integral_constant<int, 0x118>{}, std::integral_constant<int, 0xf>{});  // row_shr 8
    step(std::integral_constant<int, 0x142>{}, std::integral_constant<int, 0xa>{});  // row_bcast 15 -> rows 1, 3
    step(std::integral_constant<int, 0x143>{}, std::integral_constant<int, 0xc>{});  // row_bcast 31 -> rows 2, 3
    const uint64_t u = __builtin_bit_cast(uint64_t, v);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)u, 63);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(u >> 32), 63);
    return __builtin_bit_cast(double, ((uint64_t)hi << 32) | lo);
}

template <typename Op>
__device__ __forceinline__ float wave_reduce_f32(float v, float ident, Op op) {
    const uint32_t iu = __builtin_bit_cast(uint32_t, ident);
    auto step = [&](auto ctrl, auto rows) {
        constexpr int C = decltype(ctrl)::value, R = decltype(rows)::value;
        v = op(v, __builtin_bit_cast(float, dpp_u32<C, R>(__builtin_bit_cast(uint32_t, v), iu)));
    };
    step(std::integral_constant<int, 0xb1>{}, std::integral_constant<int, 0xf>{});
    step(std::integral_constant<int, 0x4e>{}, std::integral_constant<int, 0xf>{});
    step(std::integral_constant<int, 0x114>{}, std::integral_constant<int, 0xf>{});
    step(std::integral_constant<int, 0x118>{}, std::integral_constant<int, 0xf>{});
    step(std::integral_constant<int, 0x142>{}, std::integral_constant<int, 0xa>{});
    step(std::integral_constant<int, 0x143>{}, std::integral_constant<int, 0xc>{});
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}

// N f64 sums over the wave at once: every DPP step is applied to all N
// values before the next, so the N chains overlap instead of running one
// after another; the totals are wave-uniform.
template <int N>
__device__ __forceinline__ void wave_sum_n(double (&v)[N]) {
    auto step = [&](auto ctrl, auto rows) {
        constexpr int C = decltype(ctrl)::value, R = decltype(rows)::value;
        uint32_t lo[N], hi[N];
#pragma unroll
        for (int i = 0; i < N; i++) {
            const uint64_t u = __builtin_bit_cast(uint64_t, v[i]);
            lo[i] = dpp_u32<C, R>((uint32_t)u, 0u);
            hi[i] = dpp_u32<C, R>((uint32_t)(u >> 32), 0u);
        }
#pragma unroll
        for (int i = 0; i < N; i++) v[i] += __builtin_bit_cast(double, ((uint64_t)hi[i] << 32) | lo[i]);
    };
    step(std::integral_constant<int, 0xb1>{}, std::integral_constant<int, 0xf>{});
    step(std::integral_constant<int, 0x4e>{}, std::integral_constant<int, 0xf>{});
    step(std::integral_constant<int, 0x114>{}, std::integral_constant<int, 0xf>{});
    step(std::integral_constant<int, 0x118>{}, std::integral_constant<int, 0xf>{});
    step(std::integral_constant<int, 0x142>{}, std::integral_constant<int, 0xa>{});
    step(std::integral_constant<int, 0x143>{}, std::integral_constant<int, 0xc>{});
#pragma unroll
    for (int i = 0; i < N; i++) {
        const uint64_t u = __builtin_bit_cast(uint64_t, v[i]);
        const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)u, 63);
        const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(u >> 32), 63);
        v[i] = __builtin_bit_cast(double, ((uint64_t)hi << 32) | lo);
    }
}

// sum over the wave (f64), the same value in every lane
__device__ __forceinline__ double wave_sum(double v) {
    return wave_reduce_f64(v, 0.0, [](double x, double y) { return x + y; });
}
__device__ __forceinline__ float wave_sum(float v) {
    return wave_reduce_f32(v, 0.f, [](float x, float y) { return x + y; });
}
// max over the wave (NaN-free inputs; -inf is the identity)
__device__ __forceinline__ float wave_max(float v) {
    return wave_reduce_f32(v, -INFINITY, [](float x, float y) { return fmaxf(x, y); });
}

}  // namespace cmf
