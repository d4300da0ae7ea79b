// O(1) decode step of one KulaMamba layer (replaces mamba3/mamba3.py:275-316).
//
// One workgroup per (batch, head). Each lane owns four consecutive state columns
// n0..n0+3 of one headdim row p, so a row of N columns is spread over LPR = N/4 lanes
// and a wave covers 64/LPR rows. The lane recomputes the RMSNorm / bias / RoPE of its
// four B and C columns (a butterfly over the LPR lanes gives the row RMS), then streams
// its rows of h and prev_BX with 16-byte loads:
//
//   curr[p,n] = sum_r B~[n,r] x[p,r]
//   h'[p,n]   = dA h[p,n] + gamma curr[p,n] + beta prev[p,n]      (fp32)
//   y[p,r]    = sum_n C~[n,r] h'[p,n] + D x[p,r]                 (butterfly over LPR lanes)
//   out[p]    = sum_r mimo_down[p,r] y[p,r] silu(z[p] mimo_z[p,r])
//
// All loads of a lane's rows are issued before the dependent arithmetic so each wave
// keeps up to kStepRowsPerLane * 32 bytes per lane in flight. HBM-bound: 16*P*N bytes
// per (batch, head).
#include "m3_common.h"
#include "m3_kernels.h"

namespace m3 {

constexpr int kStepThreads = 256;
constexpr int kStepRowsPerLane = 8;

struct StepArgs {
    int H, P, N, G;
    int trap, cplx;
    float eps;
    int64_t row_stride;
    ProjLayout pl;
    m3_layer_params prm;
    const void* proj;
    const float* dt_scale;
    const float* h_in;
    const float* prev_in;
    const void* angle_in;
    void* y_out;
    float* h_out;
    float* prev_out;
    void* angle_out;
};

template <typename T, typename TA, int R, int LPR>
__global__ __launch_bounds__(kStepThreads) void step_kernel(StepArgs a) {
    constexpr int kRows = kStepThreads / LPR;  // rows handled per pass of the block
    const int tid = threadIdx.x;
    const int b = blockIdx.x / a.H, h = blockIdx.x % a.H;
    const int g = h / (a.H / a.G);
    const int P = a.P, N = a.N, Nh = N / 2, NR = N * R;
    const int q = tid % LPR;   // column group
    const int row0 = tid / LPR;
    const int n0 = q * 4;
    const T* pr = reinterpret_cast<const T*>(a.proj) + (int64_t)b * a.row_stride;

    // Per-head scalars (mamba3/mamba3.py:278-282, 290-296).
    const float Ah = -expf(a.prm.A_log[h]);
    const float sc = a.dt_scale ? a.dt_scale[(int64_t)b * a.H + h] : 1.f;
    const TokenGate tg = token_gate(ld_f32(pr + a.pl.dt + h), a.prm.dt_bias[h], sc, Ah,
                                    a.trap ? ld_f32(pr + a.pl.lam + h) : 0.f, a.trap != 0);
    const float dA = expf(tg.logdA);
    const float gamma = a.trap ? tg.lam * tg.dt : tg.dt;
    const float beta = a.trap ? (1.f - tg.lam) * tg.dt * dA : 0.f;

    // B~, C~ for columns n0..n0+3 (mamba3/mamba3.py:170-190).
    float Bv[4][R], Cv[4][R];
    float ssb = 0.f, ssc = 0.f;
    const T* Braw = pr + a.pl.B + (int64_t)g * NR + n0 * R;
    const T* Craw = pr + a.pl.C + (int64_t)g * NR + n0 * R;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
            Bv[j][r] = ld_f32(Braw + j * R + r);
            Cv[j][r] = ld_f32(Craw + j * R + r);
            ssb += Bv[j][r] * Bv[j][r];
            ssc += Cv[j][r] * Cv[j][r];
        }
    }
    ssb = group_sum<LPR>(ssb);
    ssc = group_sum<LPR>(ssc);
    const float rb = rsqrtf(ssb / NR + a.eps), rc = rsqrtf(ssc / NR + a.eps);
    const float* wB = a.prm.B_norm_w + n0 * R;
    const float* wC = a.prm.C_norm_w + n0 * R;
    const float* bB = a.prm.B_bias + (int64_t)g * NR + n0 * R;
    const float* bC = a.prm.C_bias + (int64_t)g * NR + n0 * R;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
            Bv[j][r] = Bv[j][r] * rb * wB[j * R + r] + bB[j * R + r];
            Cv[j][r] = Cv[j][r] * rc * wC[j * R + r] + bC[j * R + r];
        }
    }
    if (a.cplx) {
        const TA* ain = reinterpret_cast<const TA*>(a.angle_in) + ((int64_t)b * a.H + h) * Nh;
        TA* aout = reinterpret_cast<TA*>(a.angle_out) + ((int64_t)b * a.H + h) * Nh;
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int i = n0 / 2 + j;
            const float phi = ld_f32(ain + i) - tg.dt * ld_f32(pr + a.pl.theta + i);
            if (row0 == 0) aout[i] = cvt_out<TA>(phi);
            float sn, cs;
            sincosf(phi, &sn, &cs);
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const float be = Bv[2 * j][r], bo = Bv[2 * j + 1][r];
                Bv[2 * j][r] = be * cs - bo * sn;
                Bv[2 * j + 1][r] = be * sn + bo * cs;
                const float ce = Cv[2 * j][r], co = Cv[2 * j + 1][r];
                Cv[2 * j][r] = ce * cs - co * sn;
                Cv[2 * j + 1][r] = ce * sn + co * cs;
            }
        }
    } else if (row0 == 0 && a.angle_out) {
        // Angle stays zero without complex RoPE; pass the input through.
        const TA* ain = reinterpret_cast<const TA*>(a.angle_in) + ((int64_t)b * a.H + h) * Nh;
        TA* aout = reinterpret_cast<TA*>(a.angle_out) + ((int64_t)b * a.H + h) * Nh;
        for (int i = n0 / 2; i < n0 / 2 + 2; ++i) aout[i] = ain[i];
    }

    const float Dh = a.prm.D[h];
    const float* mx = a.prm.mimo_x + (int64_t)h * P * R;
    const float* mz = a.prm.mimo_z + (int64_t)h * P * R;
    const float* md = a.prm.mimo_down + (int64_t)h * P * R;
    const int64_t sbase = ((int64_t)b * a.H + h) * P * N;
    const f32x4* hin = reinterpret_cast<const f32x4*>(a.h_in + sbase);
    const f32x4* pin = reinterpret_cast<const f32x4*>(a.prev_in + sbase);
    f32x4* hout = reinterpret_cast<f32x4*>(a.h_out + sbase);
    f32x4* pout = reinterpret_cast<f32x4*>(a.prev_out + sbase);
    T* yo = reinterpret_cast<T*>(a.y_out) + (int64_t)b * a.H * P + (int64_t)h * P;
    const int n4 = N / 4;

    for (int pbase = row0; pbase < P; pbase += kRows * kStepRowsPerLane) {
        f32x4 hv[kStepRowsPerLane], pv[kStepRowsPerLane];
        float xv[kStepRowsPerLane];
#pragma unroll
        for (int it = 0; it < kStepRowsPerLane; ++it) {
            const int p = pbase + it * kRows;
            if (p < P) {
                // streaming reads of the incoming state; the outgoing state is stored
                // normally so the next step finds it in the caches
                hv[it] = __builtin_nontemporal_load(&hin[p * n4 + q]);
                pv[it] = __builtin_nontemporal_load(&pin[p * n4 + q]);
                xv[it] = ld_f32(pr + a.pl.x + (int64_t)h * P + p);
            }
        }
#pragma unroll
        for (int it = 0; it < kStepRowsPerLane; ++it) {
            const int p = pbase + it * kRows;
            if (p < P) {
                float xr[R];
#pragma unroll
                for (int r = 0; r < R; ++r) xr[r] = xv[it] * mx[p * R + r];
                f32x4 cur, hn;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    float c = 0.f;
#pragma unroll
                    for (int r = 0; r < R; ++r) c += Bv[j][r] * xr[r];
                    cur[j] = c;
                    hn[j] = dA * hv[it][j] + gamma * c + beta * pv[it][j];
                }
                hout[p * n4 + q] = hn;
                pout[p * n4 + q] = cur;
                float yr[R];
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    float acc = 0.f;
#pragma unroll
                    for (int j = 0; j < 4; ++j) acc += Cv[j][r] * hn[j];
                    yr[r] = group_sum<LPR>(acc);
                }
                if (q == 0) {
                    const float z = ld_f32(pr + a.pl.z + (int64_t)h * P + p);
                    float out = 0.f;
#pragma unroll
                    for (int r = 0; r < R; ++r) {
                        const float y = yr[r] + Dh * xr[r];
                        out += md[p * R + r] * y * silu_f(z * mz[p * R + r]);
                    }
                    yo[p] = cvt_out<T>(out);
                }
            }
        }
    }
}

int step_supported(int N, int R) {
    const bool n_ok = N == 8 || N == 16 || N == 32 || N == 64 || N == 128 || N == 256;
    const bool r_ok = R >= 1 && R <= 4;
    return n_ok && r_ok;
}

template <typename T, typename TA, int R>
static void launch_step_r(int lpr, dim3 grid, hipStream_t stream, const StepArgs& a) {
    switch (lpr) {
        case 2: hipLaunchKernelGGL((step_kernel<T, TA, R, 2>), grid, dim3(kStepThreads), 0, stream, a); break;
        case 4: hipLaunchKernelGGL((step_kernel<T, TA, R, 4>), grid, dim3(kStepThreads), 0, stream, a); break;
        case 8: hipLaunchKernelGGL((step_kernel<T, TA, R, 8>), grid, dim3(kStepThreads), 0, stream, a); break;
        case 16: hipLaunchKernelGGL((step_kernel<T, TA, R, 16>), grid, dim3(kStepThreads), 0, stream, a); break;
        case 32: hipLaunchKernelGGL((step_kernel<T, TA, R, 32>), grid, dim3(kStepThreads), 0, stream, a); break;
        default: hipLaunchKernelGGL((step_kernel<T, TA, R, 64>), grid, dim3(kStepThreads), 0, stream, a); break;
    }
}

template <typename T, typename TA>
static void launch_step_t(int R, int lpr, dim3 grid, hipStream_t stream, const StepArgs& a) {
    switch (R) {
        case 1: launch_step_r<T, TA, 1>(lpr, grid, stream, a); break;
        case 2: launch_step_r<T, TA, 2>(lpr, grid, stream, a); break;
        case 3: launch_step_r<T, TA, 3>(lpr, grid, stream, a); break;
        default: launch_step_r<T, TA, 4>(lpr, grid, stream, a); break;
    }
}

int launch_step(const m3_layer_desc& d, const m3_layer_params& p, const void* proj,
                const float* dt_scale, const float* h_in, const float* prev_in,
                const void* angle_in, int angle_dtype, void* y_out, float* h_out,
                float* prev_out, void* angle_out, hipStream_t stream) {
    StepArgs a;
    a.H = d.nheads; a.P = d.headdim; a.N = d.d_state; a.G = d.ngroups;
    a.trap = d.use_trapezoidal; a.cplx = d.use_complex; a.eps = d.rms_eps;
    a.row_stride = d.proj_row_stride;
    a.pl = proj_layout(d);
    a.prm = p;
    a.proj = proj; a.dt_scale = dt_scale; a.h_in = h_in; a.prev_in = prev_in;
    a.angle_in = angle_in; a.y_out = y_out; a.h_out = h_out; a.prev_out = prev_out;
    a.angle_out = angle_out;
    const int lpr = d.d_state / 4;
    const dim3 grid((unsigned)(d.batch * d.nheads));
    const bool bf = d.dtype == M3_DTYPE_BF16;
    const bool abf = angle_dtype == M3_DTYPE_BF16;
    if (bf && abf) launch_step_t<bf16, bf16>(d.mimo_rank, lpr, grid, stream, a);
    else if (bf) launch_step_t<bf16, float>(d.mimo_rank, lpr, grid, stream, a);
    else if (abf) launch_step_t<float, bf16>(d.mimo_rank, lpr, grid, stream, a);
    else launch_step_t<float, float>(d.mimo_rank, lpr, grid, stream, a);
    return hipGetLastError() == hipSuccess ? M3_OK : M3_ERR_LAUNCH;
}

}  // namespace m3
