// RMSNorm of the residual blocks (mamba3/mamba3.py:19-35, used by mamba3/block.py:45-72) in
// one pass over the activations, and its backward; and SwiGLU's silu * mul over a
// concatenated gate / up projection.
//
// Forward, per row of d elements (the reference's arithmetic and roundings):
//   s = rsqrt(mean(x^2) + eps)   in fp32
//   y = (x * T(s)) * w           each product rounded to the output dtype
// where T is the activation dtype: with bf16 activations the scale is rounded to bf16 and
// x * s to bf16 before the weight multiplies (mamba3/mamba3.py:30-35). s is kept (fp32) for
// the backward.
// Backward (fp32 arithmetic), with g = dL/dy and a = sum_j w_j g_j x_j:
//   dx_j = s w_j g_j - x_j s^3 a / d
//   dw_j = sum over rows of g_j x_j s   (per-block column partials summed in block order,
//          so the result does not depend on timing)
#include <hip/hip_runtime.h>

#include <type_traits>

#include "m3_common.h"
#include "m3_kernels.h"

namespace m3 {

constexpr int kNormThreads = 256;    // four rows (one wave each) per block
constexpr int kNormRowsPerPart = 256;

template <typename T>
__device__ __forceinline__ float ldf(const void* p, int64_t i) {
    return (float)reinterpret_cast<const T*>(p)[i];
}
template <typename T>
__device__ __forceinline__ void stf(void* p, int64_t i, float v) {
    reinterpret_cast<T*>(p)[i] = (T)v;
}

template <typename TX, typename TW, typename TY>
__global__ __launch_bounds__(kNormThreads) void rmsnorm_fwd_kernel(
    const void* __restrict__ x, const void* __restrict__ w, void* __restrict__ y,
    float* __restrict__ rstd, int64_t rows, int d, float eps) {
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * (kNormThreads / 64) + (threadIdx.x >> 6);
    if (row >= rows) return;
    const int64_t base = row * d;
    float ss = 0.f;
    for (int j = lane; j < d; j += 64) {
        const float v = ldf<TX>(x, base + j);
        ss += v * v;
    }
    ss = group_sum<64>(ss);
    const float s = rsqrtf(ss / (float)d + eps);
    if (rstd && lane == 0) rstd[row] = s;
    const float st = (float)(TX)s;  // the scale in the activation dtype
    for (int j = lane; j < d; j += 64) {
        const float xs = (float)(TX)(ldf<TX>(x, base + j) * st);
        stf<TY>(y, base + j, xs * ldf<TW>(w, j));
    }
}

// bf16 rows of d % 8 == 0 elements, 16-byte aligned: the same arithmetic on 16-byte pieces
// (each lane sums the squares of its pieces, then the 64-lane butterfly).
typedef __bf16 nb16x8 __attribute__((ext_vector_type(8)));

template <typename TW, typename TY>
__global__ __launch_bounds__(kNormThreads) void rmsnorm_fwd_vec_kernel(
    const bf16* __restrict__ x, const TW* __restrict__ w, TY* __restrict__ y,
    float* __restrict__ rstd, int64_t rows, int d, float eps) {
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * (kNormThreads / 64) + (threadIdx.x >> 6);
    if (row >= rows) return;
    const int pieces = d / 8;
    const nb16x8* xr = reinterpret_cast<const nb16x8*>(x + row * d);
    float ss = 0.f;
    for (int c = lane; c < pieces; c += 64) {
        const nb16x8 v = xr[c];
#pragma unroll
        for (int e = 0; e < 8; ++e) ss += (float)v[e] * (float)v[e];
    }
    ss = group_sum<64>(ss);
    const float s = rsqrtf(ss / (float)d + eps);
    if (rstd && lane == 0) rstd[row] = s;
    const float st = (float)(bf16)s;  // the scale in the activation dtype
    for (int c = lane; c < pieces; c += 64) {
        const nb16x8 v = xr[c];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const float xs = (float)(bf16)((float)v[e] * st);
            y[row * d + c * 8 + e] = (TY)(xs * (float)w[c * 8 + e]);
        }
    }
}

// SwiGLU's element-wise step (mamba3/block.py:16-26) on the concatenated gate / up
// projection gu (rows x row_stride, gate in columns [0, d_ff), up in [d_ff, 2 d_ff)):
// out = silu(gate) * up in fp32, rounded once to bf16.
__global__ __launch_bounds__(256) void silu_mul_kernel(const bf16* __restrict__ gu,
                                                       bf16* __restrict__ out, int64_t rows,
                                                       int dff, int64_t stride) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int pieces = dff / 8;
    if (i >= rows * pieces) return;
    const int64_t r = i / pieces;
    const int c = (int)(i - r * pieces);
    const nb16x8 g = *reinterpret_cast<const nb16x8*>(gu + r * stride + c * 8);
    const nb16x8 u = *reinterpret_cast<const nb16x8*>(gu + r * stride + dff + c * 8);
    nb16x8 o;
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = (bf16)(silu_f((float)g[e]) * (float)u[e]);
    *reinterpret_cast<nb16x8*>(out + r * dff + c * 8) = o;
}

__global__ __launch_bounds__(256) void silu_mul_scalar_kernel(const bf16* __restrict__ gu,
                                                              bf16* __restrict__ out,
                                                              int64_t rows, int dff,
                                                              int64_t stride) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= rows * dff) return;
    const int64_t r = i / dff;
    const int j = (int)(i - r * dff);
    out[r * dff + j] = (bf16)(silu_f((float)gu[r * stride + j]) * (float)gu[r * stride + dff + j]);
}

int launch_silu_mul(const void* gu, void* out, int64_t rows, int dff, int64_t stride,
                    hipStream_t stream) {
    const bf16* g = reinterpret_cast<const bf16*>(gu);
    bf16* o = reinterpret_cast<bf16*>(out);
    const bool vec = dff % 8 == 0 && stride % 8 == 0 && reinterpret_cast<uintptr_t>(gu) % 16 == 0 &&
                     reinterpret_cast<uintptr_t>(out) % 16 == 0;
    const int64_t n = vec ? rows * (dff / 8) : rows * dff;
    const dim3 grid((unsigned)((n + 255) / 256));
    if (vec) hipLaunchKernelGGL(silu_mul_kernel, grid, dim3(256), 0, stream, g, o, rows, dff, stride);
    else hipLaunchKernelGGL(silu_mul_scalar_kernel, grid, dim3(256), 0, stream, g, o, rows, dff, stride);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

template <typename TX, typename TW, typename TG>
__global__ __launch_bounds__(kNormThreads) void rmsnorm_dx_kernel(
    const void* __restrict__ x, const void* __restrict__ w, const float* __restrict__ rstd,
    const void* __restrict__ g, void* __restrict__ dx, int64_t rows, int d) {
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * (kNormThreads / 64) + (threadIdx.x >> 6);
    if (row >= rows) return;
    const int64_t base = row * d;
    const float s = rstd[row];
    float acc = 0.f;
    for (int j = lane; j < d; j += 64)
        acc += ldf<TW>(w, j) * ldf<TG>(g, base + j) * ldf<TX>(x, base + j);
    acc = group_sum<64>(acc);
    const float c = s * s * s * acc / (float)d;
    for (int j = lane; j < d; j += 64)
        stf<TX>(dx, base + j, s * ldf<TW>(w, j) * ldf<TG>(g, base + j) - ldf<TX>(x, base + j) * c);
}

// Column partials of dw: block (i, c) sums rows i*kNormRowsPerPart .. +kNormRowsPerPart-1 for
// columns c*256 .. c*256+255, one column per thread.
template <typename TX, typename TG>
__global__ __launch_bounds__(kNormThreads) void rmsnorm_dw_part_kernel(
    const void* __restrict__ x, const float* __restrict__ rstd, const void* __restrict__ g,
    float* __restrict__ part, int64_t rows, int d) {
    const int j = blockIdx.y * kNormThreads + threadIdx.x;
    if (j >= d) return;
    const int64_t r0 = (int64_t)blockIdx.x * kNormRowsPerPart;
    const int64_t r1 = r0 + kNormRowsPerPart < rows ? r0 + kNormRowsPerPart : rows;
    float acc = 0.f;
    for (int64_t r = r0; r < r1; ++r) acc += ldf<TG>(g, r * d + j) * ldf<TX>(x, r * d + j) * rstd[r];
    part[(int64_t)blockIdx.x * d + j] = acc;
}

template <typename TW>
__global__ __launch_bounds__(kNormThreads) void rmsnorm_dw_sum_kernel(
    const float* __restrict__ part, void* __restrict__ dw, int nparts, int d) {
    const int j = blockIdx.x * kNormThreads + threadIdx.x;
    if (j >= d) return;
    float acc = 0.f;
    for (int i = 0; i < nparts; ++i) acc += part[(int64_t)i * d + j];
    stf<TW>(dw, j, acc);
}

size_t rmsnorm_bwd_workspace(int64_t rows, int d) {
    const int64_t nparts = (rows + kNormRowsPerPart - 1) / kNormRowsPerPart;
    return (size_t)nparts * d * sizeof(float);
}

template <typename TX, typename TW>
static void launch_fwd_w(int ydtype, const void* x, const void* w, void* y, float* rstd,
                         int64_t rows, int d, float eps, hipStream_t stream) {
    const dim3 grid((unsigned)((rows + 3) / 4));
    if constexpr (std::is_same<TX, bf16>::value) {
        if (d % 8 == 0 && reinterpret_cast<uintptr_t>(x) % 16 == 0) {
            const bf16* xb = reinterpret_cast<const bf16*>(x);
            const TW* wt = reinterpret_cast<const TW*>(w);
            if (ydtype == M3_DTYPE_BF16)
                hipLaunchKernelGGL((rmsnorm_fwd_vec_kernel<TW, bf16>), grid, dim3(kNormThreads), 0,
                                   stream, xb, wt, reinterpret_cast<bf16*>(y), rstd, rows, d, eps);
            else
                hipLaunchKernelGGL((rmsnorm_fwd_vec_kernel<TW, float>), grid, dim3(kNormThreads), 0,
                                   stream, xb, wt, reinterpret_cast<float*>(y), rstd, rows, d, eps);
            return;
        }
    }
    if (ydtype == M3_DTYPE_BF16)
        hipLaunchKernelGGL((rmsnorm_fwd_kernel<TX, TW, bf16>), grid, dim3(kNormThreads), 0, stream,
                           x, w, y, rstd, rows, d, eps);
    else
        hipLaunchKernelGGL((rmsnorm_fwd_kernel<TX, TW, float>), grid, dim3(kNormThreads), 0, stream,
                           x, w, y, rstd, rows, d, eps);
}

int launch_rmsnorm_fwd(const void* x, int xdtype, const void* w, int wdtype, void* y,
                       int ydtype, float* rstd, int64_t rows, int d, float eps,
                       hipStream_t stream) {
    if (xdtype == M3_DTYPE_BF16) {
        if (wdtype == M3_DTYPE_BF16) launch_fwd_w<bf16, bf16>(ydtype, x, w, y, rstd, rows, d, eps, stream);
        else launch_fwd_w<bf16, float>(ydtype, x, w, y, rstd, rows, d, eps, stream);
    } else {
        if (wdtype == M3_DTYPE_BF16) launch_fwd_w<float, bf16>(ydtype, x, w, y, rstd, rows, d, eps, stream);
        else launch_fwd_w<float, float>(ydtype, x, w, y, rstd, rows, d, eps, stream);
    }
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

template <typename TX, typename TW, typename TG>
static void launch_bwd_t(const void* x, const void* w, const float* rstd, const void* g,
                         void* dx, void* dw, float* part, int64_t rows, int d, hipStream_t stream) {
    hipLaunchKernelGGL((rmsnorm_dx_kernel<TX, TW, TG>), dim3((unsigned)((rows + 3) / 4)),
                       dim3(kNormThreads), 0, stream, x, w, rstd, g, dx, rows, d);
    const int64_t nparts = (rows + kNormRowsPerPart - 1) / kNormRowsPerPart;
    const unsigned cb = (unsigned)((d + kNormThreads - 1) / kNormThreads);
    hipLaunchKernelGGL((rmsnorm_dw_part_kernel<TX, TG>), dim3((unsigned)nparts, cb),
                       dim3(kNormThreads), 0, stream, x, rstd, g, part, rows, d);
    hipLaunchKernelGGL((rmsnorm_dw_sum_kernel<TW>), dim3(cb), dim3(kNormThreads), 0, stream, part,
                       dw, (int)nparts, d);
}

template <typename TX, typename TW>
static void launch_bwd_g(int gdtype, const void* x, const void* w, const float* rstd,
                         const void* g, void* dx, void* dw, float* part, int64_t rows, int d,
                         hipStream_t stream) {
    if (gdtype == M3_DTYPE_BF16) launch_bwd_t<TX, TW, bf16>(x, w, rstd, g, dx, dw, part, rows, d, stream);
    else launch_bwd_t<TX, TW, float>(x, w, rstd, g, dx, dw, part, rows, d, stream);
}

int launch_rmsnorm_bwd(const void* x, int xdtype, const void* w, int wdtype, const float* rstd,
                       const void* g, int gdtype, void* dx, void* dw, void* workspace,
                       int64_t rows, int d, hipStream_t stream) {
    float* part = reinterpret_cast<float*>(workspace);
    if (xdtype == M3_DTYPE_BF16) {
        if (wdtype == M3_DTYPE_BF16) launch_bwd_g<bf16, bf16>(gdtype, x, w, rstd, g, dx, dw, part, rows, d, stream);
        else launch_bwd_g<bf16, float>(gdtype, x, w, rstd, g, dx, dw, part, rows, d, stream);
    } else {
        if (wdtype == M3_DTYPE_BF16) launch_bwd_g<float, bf16>(gdtype, x, w, rstd, g, dx, dw, part, rows, d, stream);
        else launch_bwd_g<float, float>(gdtype, x, w, rstd, g, dx, dw, part, rows, d, stream);
    }
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

}  // namespace m3
