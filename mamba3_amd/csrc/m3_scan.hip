// Inter-chunk state scan (replaces mamba3/csrc/scan.cu:10-50 and mamba3/scan.py:34-44).
//
//   h_states[b,0,h,:]   = h_init[b,h,:] or 0
//   h_states[b,k+1,h,:] = decay[b,k,h] * h_states[b,k,h,:] + h_chunk[b,k,h,:]
//
// Design: the recurrence is independent per (b,h,j) column, so every lane owns one
// float4 column slice and walks k. A wave reads/writes 1 KiB contiguous per k, and the
// loads of kUnroll consecutive chunks are issued before the dependent FMA chain, so
// each wave keeps kUnroll x 1 KiB in flight. HBM-bound: B*K*H*PN*8 bytes + decay. Every
// h_chunk element is read once and every state written once, so both go through
// non-temporal (streaming) loads and stores, which keep them out of the caches' way.
#include "m3_common.h"
#include "m3_kernels.h"

namespace m3 {

constexpr int kScanUnroll = 8;
constexpr int kScanBlock = 256;

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

int launch_scan_fwd(const float* decay, const float* h_chunk, const float* h_init,
                    float* h_states, int64_t B, int64_t K, int64_t H, int64_t PN,
                    hipStream_t stream) {
    const bool vec = (PN % 4 == 0) &&
                     ((reinterpret_cast<uintptr_t>(h_chunk) | reinterpret_cast<uintptr_t>(h_states) |
                       reinterpret_cast<uintptr_t>(h_init)) % 16 == 0);
    if (vec) {
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
