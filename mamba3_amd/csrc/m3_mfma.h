// Device helpers shared by the MFMA prefill kernels (gfx950, wave64): operand types,
// the f16 MFMA, the LDS transpose read, lane exchanges and fast transcendental forms.
#pragma once

#include "m3_common.h"

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

}  // namespace m3
