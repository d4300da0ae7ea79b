// Device helpers shared by the MFMA prefill kernels (gfx950, wave64): operand types,
// the f16 MFMA, the LDS transpose read, lane exchanges and fast transcendental forms.
#pragma once

#include "m3_common.h"
#include "mamba3_amd.h"

namespace m3 {

constexpr float kLog2e = 1.4426950408889634f;

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
// MFMA operand tiles are f16: same dense rate as bf16 on gfx950, three more mantissa
// bits, and packed f16 arithmetic for the RoPE rotation.
typedef _Float16 f16;
typedef f16 f16x8 __attribute__((ext_vector_type(8)));
typedef f16 f16x4 __attribute__((ext_vector_type(4)));
typedef f16 f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

// Returns v through an empty asm statement the compiler cannot see through or move:
// values derived from it are recomputed where used instead of being hoisted out of the
// chunk loop and held in registers across it.
__device__ __forceinline__ int opaque(int v) {
    asm volatile("" : "+v"(v));
    return v;
}

__device__ __forceinline__ f32x4 mfma16(const f16x8& a, const f16x8& b, const f32x4& c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// sin and cos of an angle in radians, reduced to [-0.5, 0.5) turns for the hardware.
__device__ __forceinline__ void fast_sincos(float x, float& s, float& c) {
    float rev = x * 0.15915494309189535f;
    rev = rev - rintf(rev);
    s = __builtin_amdgcn_sinf(rev);
    c = __builtin_amdgcn_cosf(rev);
}

__device__ __forceinline__ float fast_exp(float x) { return __builtin_amdgcn_exp2f(x * kLog2e); }

__device__ __forceinline__ float fast_silu(float x) {
    return x * __builtin_amdgcn_rcpf(1.f + fast_exp(-x));
}

__device__ __forceinline__ float fast_softplus(float x) {
    return x > 20.f ? x : __logf(1.f + fast_exp(x));
}
// The same through the hardware log2 alone: 1 + e^x >= 1 needs no denormal range handling
// (about 20 instructions fewer than __logf; results differ in the last bits).
__device__ __forceinline__ float fast_softplus_hw(float x) {
    return x > 20.f ? x : __builtin_amdgcn_logf(1.f + fast_exp(x)) * 0.69314718055994531f;
}

// Lane exchange through ds_bpermute: value of lane src. The index is computed by the
// caller from its own lane number, so no address register lives across loops.
__device__ __forceinline__ float bperm(float v, int src) {
    return __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute(src << 2, __builtin_bit_cast(int, v)));
}
// DPP move: lanes whose source is outside the row (or outside row_mask) read 0.
template <int kCtrl, int kRowMask = 0xf>
__device__ __forceinline__ float dpp0(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), kCtrl, kRowMask,
                                                                 0xf, true));
}
constexpr int kRowShr = 0x110;      // row_shr:n = kRowShr + n
constexpr int kRowBcast15 = 0x142;  // lane 15 of each row to the next row
constexpr int kRowBcast31 = 0x143;  // lane 31 to rows 2 and 3
// Inclusive prefix sum over the 64 lanes: within 16-lane rows by row shifts, then across
// rows by the row broadcasts.
__device__ __forceinline__ float wave_incl_scan(float v) {
    v += dpp0<kRowShr + 1>(v);
    v += dpp0<kRowShr + 2>(v);
    v += dpp0<kRowShr + 4>(v);
    v += dpp0<kRowShr + 8>(v);
    v += dpp0<kRowBcast15, 0xa>(v);
    v += dpp0<kRowBcast31, 0xc>(v);
    return v;
}

typedef short s16x4 __attribute__((vector_size(8)));
// ds_read_b64_tr_b16: within each 16-lane group, lane j addresses 4 consecutive 16-bit
// elements (row j/4, column group j%4 of a 4 x 16 block); lane i receives element m of
// row m, column i. Two of these give the 8 k-values of an MFMA operand column from a
// row-major [k][col] tile.
__device__ __forceinline__ f16x4 ld_tr(const f16* p) {
    const s16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (__attribute__((address_space(3))) s16x4*)(p));
    return __builtin_bit_cast(f16x4, v);
}
__device__ __forceinline__ f16x2 as_f16x2(unsigned u) { return __builtin_bit_cast(f16x2, u); }
__device__ __forceinline__ unsigned bits(f16x2 v) { return __builtin_bit_cast(unsigned, v); }

// ---- buffer-descriptor global access (gfx950 raw buffer instructions)
// Descriptor flags of every buffer resource built here.
constexpr int kRsrcFlags = 0x00020000;
// Cache policy of the reads and writes that touch their data once (x, z, y): non-temporal,
// so they do not evict the normalised B^ / C^ rows that all heads of a batch row share
// from L2.
constexpr int kStream = 2;

// A buffer resource over [base, base + bytes): reads past the end return zero, stores past
// the end are dropped.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, int64_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0,
                                             (int)(bytes < 0x7fffffff ? bytes : 0x7fffffff),
                                             kRsrcFlags);
}

// 16-bit load kept zero-extended in its own 32-bit register. Holding loaded bf16 values
// as bf16 lets the compiler pack two per register, which forces a wait on the load right
// after it is issued; the value is widened only where it is used (bf16_f32).
__device__ __forceinline__ unsigned ld_u16(__amdgpu_buffer_rsrc_t r, int off_bytes) {
    return __builtin_amdgcn_raw_buffer_load_b16(r, off_bytes, 0, 0);
}
__device__ __forceinline__ float bf16_f32(unsigned u) { return __builtin_bit_cast(float, u << 16); }

__device__ __forceinline__ u32x2 ld_b64(__amdgpu_buffer_rsrc_t r, int off_elems) {
    return __builtin_amdgcn_raw_buffer_load_b64(r, off_elems * 2, 0, 0);
}

// Scheduling fence: keeps LDS operand reads issued ahead of the MFMAs that consume them
// (the compiler otherwise sinks each read next to its use and waits on it).
#define M3_FENCE() __builtin_amdgcn_sched_barrier(0)
// Compiler memory fence between LDS stores (no instruction): stops the pairing of
// neighbouring stores into ds_write2_b64, which is about twice as slow as two single
// 64-bit stores on gfx950.
#define M3_LDS_FENCE() asm volatile("" ::: "memory")

__device__ __forceinline__ f16x8 cat8(const f16x4& lo, const f16x4& hi) {
    return f16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
}

// ---- power-of-two scales of the f16 MFMA operands
// The bf16 prefill kernels hold the normalised B^ / C^ values, x * mimo_x, the decay-masked
// scores and a copy of the state as f16 operands. A layer whose parameters would take them
// past the f16 range holds B^ / sB, C^ / sC and x * mimo_x / sX instead, each s the least
// power of two >= 1 that brings the parameter bound below its limit; scaling by a power of
// two changes no mantissa bit, and with every s = 1 the arithmetic is the unscaled one.
// The fp32 epilogues undo the scales: y by sB sC sX (folded into mimo_down), the skip term
// D enters the scores divided by sB sC, and the state (carried as h / (sB sX)) is
// multiplied back by sB sX where it leaves the kernel (final state, prev_BX).
//
// Bound of one rank's B^ row (N values): the RMS-normalised row over N R values has norm
// sqrt(N R), so the row of w * v + bias has norm at most sqrt(N R) max|w| + sqrt(N) max|bias|.
// Limit 128 keeps every score |C~ . B~| <= 16384 before the decay mask; mimo_x is brought to
// |mimo_x| / sX <= 256 (x * mimo_x / sX below 65504 for |x| < 256). bc_norm and the chunk
// kernels evaluate the same expressions on the same parameters, so they agree bit for bit.
constexpr float kBcRowLimit = 128.f;
constexpr float kMimoXLimit = 256.f;

// Least power of two s >= 1 with bound <= limit * s (limit a power of two; a non-finite
// bound gets 2^100).
__device__ __forceinline__ float f16_down_scale(float bound, float limit) {
    const float q = fminf(bound * (1.f / limit), 0x1p100f);  // fminf(NaN, c) = c
    if (!(q > 1.f)) return 1.f;
    int e;
    const float m = frexpf(q, &e);  // q = m 2^e, m in [0.5, 1)
    return ldexpf(1.f, m == 0.5f ? e - 1 : e);
}

template <int N, int R>
__device__ __forceinline__ float bc_row_scale(float max_w, float max_bias) {
    const float bound = __builtin_fmaf(__builtin_sqrtf((float)(N * R)), max_w,
                                       __builtin_sqrtf((float)N) * max_bias);
    return f16_down_scale(bound, kBcRowLimit);
}

// Max over the 64 lanes of a wave (every lane gets it, the same value): DPP permutations
// inside each 16-lane row (swap neighbours, swap pairs, half-row and row mirrors), then
// the four row maxima through readlane. No LDS traffic.
__device__ __forceinline__ float wave_max(float v) {
    auto dpp = [](float x, auto ctrl) {
        return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x),
                                                                     decltype(ctrl)::value, 0xF, 0xF, false));
    };
    v = fmaxf(v, dpp(v, std::integral_constant<int, 0xB1>{}));
    v = fmaxf(v, dpp(v, std::integral_constant<int, 0x4E>{}));
    v = fmaxf(v, dpp(v, std::integral_constant<int, 0x141>{}));
    v = fmaxf(v, dpp(v, std::integral_constant<int, 0x140>{}));
    auto rl = [&](int l) { return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), l)); };
    return fmaxf(fmaxf(rl(0), rl(16)), fmaxf(rl(32), rl(48)));
}

// max |p[i]| over i < n, by one wave (every lane gets it).
__device__ __forceinline__ float wave_absmax(const float* p, int n, int lane) {
    float m = 0.f;
    for (int i = lane; i < n; i += kWave) m = fmaxf(m, fabsf(p[i]));
    return wave_max(m);
}

__device__ __forceinline__ float uniform(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, v)));
}

// The scales of one (group, head) of a layer, by one wave.
struct F16Scales {
    float inv_x;   // 1 / sX: multiplies mimo_x in the X operands
    float inv_bc;  // 1 / (sB sC): multiplies D in the scores
    float out;     // sB sC sX: multiplies y
    float state;   // sB sX: multiplies the state where it leaves the kernel
    // the same values held in scalar registers (read from LDS by every lane)
    __device__ __forceinline__ F16Scales in_sgprs() const {
        return F16Scales{uniform(inv_x), uniform(inv_bc), uniform(out), uniform(state)};
    }
};

// sX of head h alone (its x * mimo_x operands): the state-only pass needs nothing else.
template <int R>
__device__ __forceinline__ float mimo_x_scale(const m3_layer_params& prm, int h, int P, int lane) {
    return f16_down_scale(wave_absmax(prm.mimo_x + (int64_t)h * P * R, P * R, lane), kMimoXLimit);
}

template <int N, int R>
__device__ __forceinline__ F16Scales layer_f16_scales(const m3_layer_params& prm, int grp, int h,
                                                      int P, int lane) {
    const float mwb = wave_absmax(prm.B_norm_w, N * R, lane);
    const float mwc = wave_absmax(prm.C_norm_w, N * R, lane);
    const float mbb = wave_absmax(prm.B_bias + (int64_t)grp * N * R, N * R, lane);
    const float mbc = wave_absmax(prm.C_bias + (int64_t)grp * N * R, N * R, lane);
    const float mx = wave_absmax(prm.mimo_x + (int64_t)h * P * R, P * R, lane);
    const float sb = bc_row_scale<N, R>(mwb, mbb), sc = bc_row_scale<N, R>(mwc, mbc);
    const float sx = f16_down_scale(mx, kMimoXLimit);
    return F16Scales{1.f / sx, 1.f / (sb * sc), sb * sc * sx, sb * sx};
}

}  // namespace m3
