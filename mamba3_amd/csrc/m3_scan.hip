// Inter-chunk state scan (replaces mamba3/csrc/scan.cu:10-50 and mamba3/scan.py:34-44).
//
//   h_states[b,0,h,:]   = h_init[b,h,:] or 0
//   h_states[b,k+1,h,:] = decay[b,k,h] * h_states[b,k,h,:] + h_chunk[b,k,h,:]
//
// Design: the recurrence is independent per (b,h,j) column, so lanes own float4 column
// slices and walk k. HBM-bound: B*K*H*PN*8 bytes + decay. Every h_chunk element is read
// once and every state written once, so both go through non-temporal (streaming) loads and
// stores, which keep them out of the caches' way. Memory-level parallelism comes from
// several columns per lane, not from several k per column: a lane owns kScanCols float4
// columns 64 apart, so a wave's loads of one k cover kScanCols KiB contiguous. Loads of
// consecutive k of one column lie H*PN*4 bytes apart, a power of two for the usual
// shapes (4 MiB at 32 heads x 256 x 128), and a burst of them measured 20% slower at that
// stride. The older one-column-per-lane kernels (kScanUnroll k ahead) serve rows that are
// not a multiple of 64 * kScanCols float4 columns, and problems too small to give the
// column-blocked kernels two waves per CU.
#include "m3_common.h"
#include "m3_kernels.h"
#include "m3_mfma.h"

namespace m3 {

constexpr int kScanUnroll = 8;
constexpr int kScanBlock = 256;
constexpr int kScanCols = 8;  // float4 columns per lane of the column-blocked kernels
// The column-blocked kernels run when they still give every CU two waves (512 waves of
// 64 x kScanCols columns); below that the one-column-per-lane kernels keep more loads in
// flight (backward at (4, 33, 24, 8192), 384 waves: 56 against 82 us; at (8, 128, 24,
// 8192), 768 waves: 0.461 against 0.415 ms the other way).
constexpr int64_t kScanColsMin = 512 * 64 * kScanCols;

// A wave's columns: 64 * kScanCols consecutive float4 columns of one (b, h) row; lane l
// owns j4 = j40 + 64 c, c < kScanCols.
struct ScanCols {
    int64_t bh, base;  // (b, h); float4 offset of (b, 0, h, j40)
    int64_t kstride;   // float4 units between k
    int j40, h, w;     // first column of the lane, head, wave index within the row
    const float* dptr; // decay[b, k, h] at k * H
    __device__ ScanCols(const float* decay, int64_t wcol0, int K, int H, int pn4, int lane) {
        bh = wcol0 / pn4;
        j40 = (int)(wcol0 % pn4) + lane;
        w = (int)(wcol0 % pn4) / (64 * kScanCols);
        h = (int)(bh % H);
        const int64_t b = bh / H;
        kstride = (int64_t)H * pn4;
        base = (b * K * H + h) * (int64_t)pn4 + j40;
        dptr = decay + b * K * H + h;
    }
};

// Forward, column-blocked: per k the wave issues kScanCols 1 KiB loads before the FMAs.
__global__ __launch_bounds__(kScanBlock) void scan_fwd_cols(
    const float* __restrict__ decay, const f32x4* __restrict__ h_chunk,
    const f32x4* __restrict__ h_init, f32x4* __restrict__ h_states, int K, int H,
    int pn4, int64_t total_cols) {
    const int lane = threadIdx.x & 63;
    const int64_t wcol0 = ((int64_t)blockIdx.x * (kScanBlock / 64) + (threadIdx.x >> 6)) * (64 * kScanCols);
    if (wcol0 >= total_cols) return;  // whole waves
    const ScanCols c(decay, wcol0, K, H, pn4, lane);
    f32x4 s[kScanCols];
#pragma unroll
    for (int i = 0; i < kScanCols; ++i) {
        s[i] = h_init ? h_init[c.bh * pn4 + c.j40 + 64 * i] : f32x4{0.f, 0.f, 0.f, 0.f};
        __builtin_nontemporal_store(s[i], &h_states[c.base + 64 * i]);
    }
    for (int k = 0; k < K - 1; ++k) {
        const int64_t o = c.base + (int64_t)k * c.kstride;
        f32x4 v[kScanCols];
#pragma unroll
        for (int i = 0; i < kScanCols; ++i) v[i] = __builtin_nontemporal_load(&h_chunk[o + 64 * i]);
        const float d = c.dptr[(int64_t)k * H];
#pragma unroll
        for (int i = 0; i < kScanCols; ++i) {
            s[i] = d * s[i] + v[i];
            __builtin_nontemporal_store(s[i], &h_states[o + c.kstride + 64 * i]);
        }
    }
}

__global__ __launch_bounds__(kScanBlock) void scan_fwd_vec4(
    const float* __restrict__ decay, const f32x4* __restrict__ h_chunk,
    const f32x4* __restrict__ h_init, f32x4* __restrict__ h_states, int K, int H,
    int pn4, int64_t total_cols) {
    const int64_t col = (int64_t)blockIdx.x * kScanBlock + threadIdx.x;
    if (col >= total_cols) return;
    // col enumerates (b, h, j4) with j4 fastest.
    const int j4 = (int)(col % pn4);
    const int64_t bh = col / pn4;
    const int h = (int)(bh % H);
    const int64_t b = bh / H;
    const int64_t kstride = (int64_t)H * pn4;                  // float4 units between k
    const int64_t base = (b * K * H + h) * (int64_t)pn4 + j4;  // (b,0,h,j4)
    const float* dptr = decay + b * K * H + h;                 // decay[b,k,h] at k*H

    f32x4 s = h_init ? h_init[bh * pn4 + j4] : f32x4{0.f, 0.f, 0.f, 0.f};
    h_states[base] = s;

    for (int k0 = 0; k0 < K - 1; k0 += kScanUnroll) {
        f32x4 v[kScanUnroll];
        float d[kScanUnroll];
#pragma unroll
        for (int u = 0; u < kScanUnroll; ++u) {
            if (k0 + u < K - 1) {
                v[u] = __builtin_nontemporal_load(&h_chunk[base + (int64_t)(k0 + u) * kstride]);
                d[u] = dptr[(int64_t)(k0 + u) * H];
            }
        }
#pragma unroll
        for (int u = 0; u < kScanUnroll; ++u) {
            if (k0 + u < K - 1) {
                s = d[u] * s + v[u];
                __builtin_nontemporal_store(s, &h_states[base + (int64_t)(k0 + u + 1) * kstride]);
            }
        }
    }
}

// Scalar fallback for PN not divisible by 4.
__global__ __launch_bounds__(kScanBlock) void scan_fwd_scalar(
    const float* __restrict__ decay, const float* __restrict__ h_chunk,
    const float* __restrict__ h_init, float* __restrict__ h_states, int K, int H, int pn,
    int64_t total_cols) {
    const int64_t col = (int64_t)blockIdx.x * kScanBlock + threadIdx.x;
    if (col >= total_cols) return;
    const int j = (int)(col % pn);
    const int64_t bh = col / pn;
    const int h = (int)(bh % H);
    const int64_t b = bh / H;
    const int64_t kstride = (int64_t)H * pn;
    const int64_t base = (b * K * H + h) * (int64_t)pn + j;
    const float* dptr = decay + b * K * H + h;
    float s = h_init ? h_init[bh * pn + j] : 0.f;
    h_states[base] = s;
    for (int k = 0; k < K - 1; ++k) {
        s = dptr[(int64_t)k * H] * s + __builtin_nontemporal_load(&h_chunk[base + (int64_t)k * kstride]);
        __builtin_nontemporal_store(s, &h_states[base + (int64_t)(k + 1) * kstride]);
    }
}

// ---------------------------------------------------------------------------------
// Backward of the scan (replaces mamba3/csrc/scan.cu:52-126 and mamba3/scan.py:47-62).
// With G[K-1] = dL/dh[K-1] and G[k] = dL/dh[k] + decay[k] G[k+1]:
//   d_chunk[k] = G[k+1] (k < K-1),  d_chunk[K-1] = 0
//   d_decay[k] = sum_j G[k+1][j] h[k][j] (k < K-1),  d_decay[K-1] = 0
//   d_h_init   = G[0]
// Pass 1: lanes own float4 columns (kScanCols each, or one in the fallback kernel) and
// walk k down; each wave reduces its share of the d_decay sum (DPP scan, fixed order) and
// writes one partial per (b,k,h,wave).
// Pass 2 adds the partials of every (b,k,h) in wave order: deterministic, no atomics.
// grad and d_chunk may be one array (the backward then runs in place): every thread reads an
// element of grad before it writes the same element of d_chunk, and touches no other
// thread's elements, so neither pointer is declared __restrict__.
// ---------------------------------------------------------------------------------
constexpr int kScanBwdBlock = 256;

// Sum over the wave in a fixed order (DPP inclusive scan; lane 63 holds the total).
__device__ __forceinline__ float wave_sum_dpp(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, wave_incl_scan(v)), 63));
}

// Backward, column-blocked (columns as in scan_fwd_cols): per k the wave issues its
// 2 kScanCols loads together; its d_decay partial sums the lane's columns in order, then
// the wave (one partial per (b,k,h,wave)).
__global__ __launch_bounds__(kScanBwdBlock) void scan_bwd_cols(
    const float* __restrict__ decay, const f32x4* __restrict__ h_states,
    const f32x4* grad, f32x4* d_chunk, f32x4* __restrict__ d_h_init,
    float* __restrict__ part, int K, int H, int pn4, int64_t total_cols) {
    const int lane = threadIdx.x & 63;
    const int64_t wcol0 = ((int64_t)blockIdx.x * (kScanBwdBlock / 64) + (threadIdx.x >> 6)) * (64 * kScanCols);
    if (wcol0 >= total_cols) return;  // whole waves
    const ScanCols c(decay, wcol0, K, H, pn4, lane);
    const int nw = pn4 / (64 * kScanCols);
    float* pptr = part + (c.base - c.j40) / pn4 * nw + c.w;  // (b,k,h,w) at k * H * nw
    f32x4 g[kScanCols];
    const int64_t last = c.base + (int64_t)(K - 1) * c.kstride;
#pragma unroll
    for (int i = 0; i < kScanCols; ++i) {
        g[i] = __builtin_nontemporal_load(&grad[last + 64 * i]);
        __builtin_nontemporal_store(f32x4{0.f, 0.f, 0.f, 0.f}, &d_chunk[last + 64 * i]);
    }
    for (int k = K - 2; k >= 0; --k) {
        const int64_t o = c.base + (int64_t)k * c.kstride;
        f32x4 hs[kScanCols], gk[kScanCols];
#pragma unroll
        for (int i = 0; i < kScanCols; ++i) {
            hs[i] = __builtin_nontemporal_load(&h_states[o + 64 * i]);
            gk[i] = __builtin_nontemporal_load(&grad[o + 64 * i]);
        }
        float dot = 0.f;
#pragma unroll
        for (int i = 0; i < kScanCols; ++i) {
            __builtin_nontemporal_store(g[i], &d_chunk[o + 64 * i]);
            dot += g[i][0] * hs[i][0] + g[i][1] * hs[i][1] + g[i][2] * hs[i][2] + g[i][3] * hs[i][3];
        }
        const float acc = wave_sum_dpp(dot);
        if (lane == 0) pptr[(int64_t)k * H * nw] = acc;
        const float d = c.dptr[(int64_t)k * H];
#pragma unroll
        for (int i = 0; i < kScanCols; ++i) g[i] = gk[i] + d * g[i];
    }
    if (d_h_init) {
#pragma unroll
        for (int i = 0; i < kScanCols; ++i) d_h_init[c.bh * pn4 + c.j40 + 64 * i] = g[i];
    }
}

// PN % 256 == 0: a wave's 64 float4 columns belong to one (b,h); nw = PN / 256 waves per (b,h).
__global__ __launch_bounds__(kScanBwdBlock) void scan_bwd_vec4(
    const float* __restrict__ decay, const f32x4* __restrict__ h_states,
    const f32x4* grad, f32x4* d_chunk, f32x4* __restrict__ d_h_init,
    float* __restrict__ part, int K, int H, int pn4, int64_t total_cols) {
    const int64_t col = (int64_t)blockIdx.x * kScanBwdBlock + threadIdx.x;
    if (col >= total_cols) return;  // total_cols is a multiple of 64: whole waves exit
    const int j4 = (int)(col % pn4);
    const int64_t bh = col / pn4;
    const int h = (int)(bh % H);
    const int64_t b = bh / H;
    const int nw = pn4 / 64, w = j4 / 64;
    const int64_t kstride = (int64_t)H * pn4;
    const int64_t base = (b * K * H + h) * (int64_t)pn4 + j4;
    const float* dptr = decay + b * K * H + h;
    float* pptr = part + (b * K * H + h) * (int64_t)nw + w;  // (b,k,h,w) at k * H * nw

    f32x4 g = __builtin_nontemporal_load(&grad[base + (int64_t)(K - 1) * kstride]);
    __builtin_nontemporal_store(f32x4{0.f, 0.f, 0.f, 0.f}, &d_chunk[base + (int64_t)(K - 1) * kstride]);
    for (int k = K - 2; k >= 0; --k) {
        const int64_t o = base + (int64_t)k * kstride;
        const f32x4 hs = __builtin_nontemporal_load(&h_states[o]);
        const f32x4 gk = __builtin_nontemporal_load(&grad[o]);
        __builtin_nontemporal_store(g, &d_chunk[o]);
        const float acc = wave_sum_dpp(g[0] * hs[0] + g[1] * hs[1] + g[2] * hs[2] + g[3] * hs[3]);
        if ((threadIdx.x & 63) == 0) pptr[(int64_t)k * H * nw] = acc;
        g = gk + dptr[(int64_t)k * H] * g;
    }
    if (d_h_init) d_h_init[bh * pn4 + j4] = g;
}

// d_decay[b,k,h] = sum over the nw partials (k < K-1), 0 for k = K-1.
__global__ __launch_bounds__(kScanBwdBlock) void scan_bwd_reduce(const float* __restrict__ part,
                                                                 float* __restrict__ d_decay,
                                                                 int K, int H, int nw,
                                                                 int64_t total) {
    const int64_t i = (int64_t)blockIdx.x * kScanBwdBlock + threadIdx.x;  // (b,k,h)
    if (i >= total) return;
    const int k = (int)((i / H) % K);
    float acc = 0.f;
    if (k < K - 1)
        for (int w = 0; w < nw; ++w) acc += part[i * nw + w];
    d_decay[i] = acc;
}

// Any PN and any alignment: one workgroup per (b,h). The columns are walked in tiles of
// 256 * 64 (64 per thread in registers); within a tile the chunks are walked down with the
// d_decay sum of every k reduced through LDS, and the tiles' sums are added in tile order,
// so the result does not depend on timing.
__global__ __launch_bounds__(kScanBwdBlock) void scan_bwd_block(
    const float* __restrict__ decay, const float* __restrict__ h_states,
    const float* grad, float* d_chunk, float* __restrict__ d_decay,
    float* __restrict__ d_h_init, int K, int H, int PN) {
    constexpr int kMaxPer = 64;                      // columns per thread and tile
    constexpr int kTile = kScanBwdBlock * kMaxPer;  // columns per tile
    __shared__ float red[kScanBwdBlock / 64];
    const int64_t bh = blockIdx.x;
    const int h = (int)(bh % H);
    const int64_t b = bh / H;
    const int64_t kstride = (int64_t)H * PN;
    const int64_t db = b * K * H + h;
    const int tid = threadIdx.x;
    if (tid == 0) d_decay[db + (int64_t)(K - 1) * H] = 0.f;
    for (int c0 = 0; c0 < PN; c0 += kTile) {
        const int64_t base = (b * K * H + h) * (int64_t)PN + c0;
        const int cols = PN - c0 < kTile ? PN - c0 : kTile;
        float g[kMaxPer];
        for (int i = 0; i < kMaxPer; ++i) {
            const int j = tid + i * kScanBwdBlock;
            if (j < cols) {
                g[i] = grad[base + (int64_t)(K - 1) * kstride + j];
                d_chunk[base + (int64_t)(K - 1) * kstride + j] = 0.f;
            }
        }
        for (int k = K - 2; k >= 0; --k) {
            const int64_t o = base + (int64_t)k * kstride;
            const float d = decay[db + (int64_t)k * H];
            float acc = 0.f;
            for (int i = 0; i < kMaxPer; ++i) {
                const int j = tid + i * kScanBwdBlock;
                if (j < cols) {
                    acc += g[i] * h_states[o + j];
                    const float gk = grad[o + j];
                    d_chunk[o + j] = g[i];
                    g[i] = gk + d * g[i];
                }
            }
            acc = wave_sum_dpp(acc);
            if ((tid & 63) == 0) red[tid >> 6] = acc;
            __syncthreads();
            if (tid == 0) {
                float s = 0.f;
                for (int w = 0; w < kScanBwdBlock / 64; ++w) s += red[w];
                float* dd = &d_decay[db + (int64_t)k * H];
                *dd = c0 == 0 ? s : *dd + s;
            }
            __syncthreads();
        }
        if (d_h_init)
            for (int i = 0; i < kMaxPer; ++i) {
                const int j = tid + i * kScanBwdBlock;
                if (j < cols) d_h_init[bh * PN + c0 + j] = g[i];
            }
    }
}

size_t scan_bwd_workspace(int64_t B, int64_t K, int64_t H, int64_t PN) {
    if (PN % 256 != 0) return 0;
    return (size_t)(B * K * H * (PN / 256)) * sizeof(float);
}

int launch_scan_bwd(const float* decay, const float* h_states, const float* grad,
                    float* d_decay, float* d_chunk, float* d_h_init, float* workspace,
                    int64_t B, int64_t K, int64_t H, int64_t PN, hipStream_t stream) {
    const bool vec = (PN % 256 == 0) &&
                     ((reinterpret_cast<uintptr_t>(h_states) | reinterpret_cast<uintptr_t>(grad) |
                       reinterpret_cast<uintptr_t>(d_chunk) | reinterpret_cast<uintptr_t>(d_h_init)) % 16 == 0);
    if (vec && (PN / 4) % (64 * kScanCols) == 0 && B * H * (PN / 4) >= kScanColsMin) {
        const int64_t cols = B * H * (PN / 4);
        const int64_t waves = cols / (64 * kScanCols);
        hipLaunchKernelGGL(scan_bwd_cols, dim3((unsigned)((waves + kScanBwdBlock / 64 - 1) / (kScanBwdBlock / 64))),
                           dim3(kScanBwdBlock), 0, stream, decay,
                           reinterpret_cast<const f32x4*>(h_states), reinterpret_cast<const f32x4*>(grad),
                           reinterpret_cast<f32x4*>(d_chunk), reinterpret_cast<f32x4*>(d_h_init), workspace,
                           (int)K, (int)H, (int)(PN / 4), cols);
        const int64_t n = B * K * H;
        hipLaunchKernelGGL(scan_bwd_reduce, dim3((unsigned)((n + kScanBwdBlock - 1) / kScanBwdBlock)),
                           dim3(kScanBwdBlock), 0, stream, workspace, d_decay, (int)K, (int)H,
                           (int)(PN / (256 * kScanCols)), n);
    } else if (vec) {
        const int64_t cols = B * H * (PN / 4);
        hipLaunchKernelGGL(scan_bwd_vec4, dim3((unsigned)((cols + kScanBwdBlock - 1) / kScanBwdBlock)),
                           dim3(kScanBwdBlock), 0, stream, decay,
                           reinterpret_cast<const f32x4*>(h_states), reinterpret_cast<const f32x4*>(grad),
                           reinterpret_cast<f32x4*>(d_chunk), reinterpret_cast<f32x4*>(d_h_init), workspace,
                           (int)K, (int)H, (int)(PN / 4), cols);
        const int64_t n = B * K * H;
        hipLaunchKernelGGL(scan_bwd_reduce, dim3((unsigned)((n + kScanBwdBlock - 1) / kScanBwdBlock)),
                           dim3(kScanBwdBlock), 0, stream, workspace, d_decay, (int)K, (int)H,
                           (int)(PN / 256), n);
    } else {
        hipLaunchKernelGGL(scan_bwd_block, dim3((unsigned)(B * H)), dim3(kScanBwdBlock), 0, stream,
                           decay, h_states, grad, d_chunk, d_decay, d_h_init, (int)K, (int)H, (int)PN);
    }
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

int launch_scan_fwd(const float* decay, const float* h_chunk, const float* h_init,
                    float* h_states, int64_t B, int64_t K, int64_t H, int64_t PN,
                    hipStream_t stream) {
    const bool vec = (PN % 4 == 0) &&
                     ((reinterpret_cast<uintptr_t>(h_chunk) | reinterpret_cast<uintptr_t>(h_states) |
                       reinterpret_cast<uintptr_t>(h_init)) % 16 == 0);
    if (vec && (PN / 4) % (64 * kScanCols) == 0 && B * H * (PN / 4) >= kScanColsMin) {
        const int64_t cols = B * H * (PN / 4);
        const int64_t waves = cols / (64 * kScanCols);
        hipLaunchKernelGGL(scan_fwd_cols, dim3((unsigned)((waves + kScanBlock / 64 - 1) / (kScanBlock / 64))),
                           dim3(kScanBlock), 0, stream, decay, reinterpret_cast<const f32x4*>(h_chunk),
                           reinterpret_cast<const f32x4*>(h_init), reinterpret_cast<f32x4*>(h_states),
                           (int)K, (int)H, (int)(PN / 4), cols);
    } else if (vec) {
        const int64_t cols = B * H * (PN / 4);
        const int64_t blocks = (cols + kScanBlock - 1) / kScanBlock;
        hipLaunchKernelGGL(scan_fwd_vec4, dim3((unsigned)blocks), dim3(kScanBlock), 0, stream,
                           decay, reinterpret_cast<const f32x4*>(h_chunk),
                           reinterpret_cast<const f32x4*>(h_init),
                           reinterpret_cast<f32x4*>(h_states), (int)K, (int)H, (int)(PN / 4),
                           cols);
    } else {
        const int64_t cols = B * H * PN;
        const int64_t blocks = (cols + kScanBlock - 1) / kScanBlock;
        hipLaunchKernelGGL(scan_fwd_scalar, dim3((unsigned)blocks), dim3(kScanBlock), 0, stream,
                           decay, h_chunk, h_init, h_states, (int)K, (int)H, (int)PN, cols);
    }
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

}  // namespace m3
