// RMSNorm of the residual blocks (mamba3/mamba3.py:19-35, used by mamba3/block.py:45-72) in
// one pass over the activations, and its backward.
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
