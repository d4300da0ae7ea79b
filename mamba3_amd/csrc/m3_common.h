// Device-side helpers shared by the Mamba-3 kernels (gfx950, wave64).
#pragma once
#include <type_traits>

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace m3 {

typedef __bf16 bf16;
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kWave = 64;

__device__ __forceinline__ float ld_f32(const float* p) { return *p; }
__device__ __forceinline__ float ld_f32(const bf16* p) { return (float)(*p); }

template <typename T> __device__ __forceinline__ T cvt_out(float x);
template <> __device__ __forceinline__ float cvt_out<float>(float x) { return x; }
template <> __device__ __forceinline__ bf16 cvt_out<bf16>(float x) { return (bf16)x; }

// torch.nn.functional.softplus with beta=1, threshold=20.
__device__ __forceinline__ float softplus_f(float x) {
    return x > 20.f ? x : log1pf(expf(x));
}
__device__ __forceinline__ float sigmoid_f(float x) { return 1.f / (1.f + expf(-x)); }
__device__ __forceinline__ float silu_f(float x) { return x / (1.f + expf(-x)); }

// Butterfly sum over aligned groups of `width` lanes (width a power of two <= 64).
template <int width>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
    for (int off = width / 2; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
    return v;
}

// The same sum with DPP lane moves inside a row of 16 lanes (swap neighbours, swap pairs,
// mirror within the half-row, mirror within the row; every source lane is valid) and lane
// shuffles across rows: after each step every lane holds the sum of its aligned group.
template <int width>
__device__ __forceinline__ float lane_sum(float v) {
    auto dpp = [](float x, auto ctrl) {
        return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), decltype(ctrl)::value, 0xF, 0xF, false));
    };
    if constexpr (width >= 2) v += dpp(v, std::integral_constant<int, 0xB1>{});
    if constexpr (width >= 4) v += dpp(v, std::integral_constant<int, 0x4E>{});
    if constexpr (width >= 8) v += dpp(v, std::integral_constant<int, 0x141>{});
    if constexpr (width >= 16) v += dpp(v, std::integral_constant<int, 0x140>{});
    if constexpr (width >= 32) v += __shfl_xor(v, 16, kWave);
    if constexpr (width >= 64) v += __shfl_xor(v, 32, kWave);
    return v;
}

__device__ __forceinline__ float group_sum_rt(float v, int width) {
    for (int off = width / 2; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
    return v;
}

// Per-head scalars of one token (mamba3/mamba3.py:200-204, 212-216, 290-296).
struct TokenGate {
    float dt;      // softplus(dt_raw + dt_bias) [* dt_scale]
    float logdA;   // A * dt  (A = -exp(A_log))
    float lam;     // sigmoid(lambda_raw) or 1 when the trapezoid is off
};

__device__ __forceinline__ TokenGate token_gate(float dt_raw, float dt_bias, float scale,
                                                float A, float lam_raw, bool trap) {
    TokenGate g;
    g.dt = softplus_f(dt_raw + dt_bias) * scale;
    g.logdA = A * g.dt;
    g.lam = trap ? sigmoid_f(lam_raw) : 1.f;
    return g;
}

}  // namespace m3
