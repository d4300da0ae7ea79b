// O(1) decode step of one KulaMamba layer (replaces mamba3/mamba3.py:275-316).
//
// One workgroup per (batch, head). Each lane owns NV vectors of VW consecutive state
// columns (CPL = NV * VW columns, n0 = q * CPL) of one headdim row p, so a row of N
// columns is spread over ceil(N / CPL) lanes, rounded up to LPR (a power of two; lanes
// past the row end hold no columns), and a wave covers 64 / LPR rows. The lane recomputes
// the RMSNorm / bias / RoPE of its B and C columns (a butterfly over the LPR lanes gives
// the row RMS), then streams its rows of h and prev_BX with VW*4-byte loads:
//
//   curr[p,n] = sum_r B~[n,r] x[p,r]
//   h'[p,n]   = dA h[p,n] + gamma curr[p,n] + beta prev[p,n]      (fp32)
//   y[p,r]    = sum_n C~[n,r] h'[p,n] + D x[p,r]                 (butterfly over LPR lanes)
//   out[p]    = sum_r mimo_down[p,r] y[p,r] silu(z[p] mimo_z[p,r])
//
// Shapes: any even N <= 512 and mimo_rank R <= 8 (R <= RM, a template bound). VW = 4 when
// N % 4 == 0 (16-byte rows), else 2; NV = 2 when N > 64 * VW (or N > 256 with VW = 2),
// else 1. All loads of a lane's rows are issued before the dependent arithmetic so each
// wave keeps up to kStepRowsPerLane rows per lane in flight. HBM-bound: 16*P*N bytes per
// (batch, head).
#include "m3_common.h"
#include "m3_kernels.h"

namespace m3 {

constexpr int kStepThreads = 256;
constexpr int kStepRowsPerLane = 8;

struct StepArgs {
    int H, P, N, G, R;
    int trap, cplx;
    int angle_bf16;
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

template <int VW> struct StepVec;
template <> struct StepVec<4> { typedef f32x4 type; };
template <> struct StepVec<2> { typedef float type __attribute__((ext_vector_type(2))); };

__device__ __forceinline__ float ld_angle(const void* p, int64_t i, bool is_bf16) {
    return is_bf16 ? (float)reinterpret_cast<const bf16*>(p)[i] : reinterpret_cast<const float*>(p)[i];
}
__device__ __forceinline__ void st_angle(void* p, int64_t i, float v, bool is_bf16) {
    if (is_bf16) reinterpret_cast<bf16*>(p)[i] = (bf16)v;
    else reinterpret_cast<float*>(p)[i] = v;
}

template <typename T, int RM, bool kExactR, int LPR, int VW, int NV>
__global__ __launch_bounds__(kStepThreads) void step_kernel(StepArgs a) {
    typedef typename StepVec<VW>::type vec;
    constexpr int CPL = VW * NV;               // state columns per lane
    constexpr int kRows = kStepThreads / LPR;  // rows handled per pass of the block
    const int tid = threadIdx.x;
    const int b = blockIdx.x / a.H, h = blockIdx.x % a.H;
    const int g = h / (a.H / a.G);
    // the rank: RM itself, or a.R <= RM (ranks 3, 5, 6 and 7 run under RM = 4 or 8)
    const int R = kExactR ? RM : a.R;
    const int P = a.P, N = a.N, Nh = N / 2, NR = N * R;
    const int q = tid % LPR;   // column group
    const int row0 = tid / LPR;
    const int n0 = q * CPL;
    // vectors of this lane inside the row (0: the lane is past the row end)
    const int nvq = n0 >= N ? 0 : ((N - n0) / VW < NV ? (N - n0) / VW : NV);
    const T* pr = reinterpret_cast<const T*>(a.proj) + (int64_t)b * a.row_stride;

    // Per-head scalars (mamba3/mamba3.py:278-282, 290-296).
    const float Ah = -expf(a.prm.A_log[h]);
    const float sc = a.dt_scale ? a.dt_scale[(int64_t)b * a.H + h] : 1.f;
    const TokenGate tg = token_gate(ld_f32(pr + a.pl.dt + h), a.prm.dt_bias[h], sc, Ah,
                                    a.trap ? ld_f32(pr + a.pl.lam + h) : 0.f, a.trap != 0);
    const float dA = expf(tg.logdA);
    const float gamma = a.trap ? tg.lam * tg.dt : tg.dt;
    const float beta = a.trap ? (1.f - tg.lam) * tg.dt * dA : 0.f;

    // B~, C~ for columns n0 .. n0 + CPL - 1 (mamba3/mamba3.py:170-190).
    float Bv[CPL][RM], Cv[CPL][RM];
    float ssb = 0.f, ssc = 0.f;
    const T* Braw = pr + a.pl.B + (int64_t)g * NR + (int64_t)n0 * R;
    const T* Craw = pr + a.pl.C + (int64_t)g * NR + (int64_t)n0 * R;
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
        const bool live = j < nvq * VW;
#pragma unroll
        for (int r = 0; r < RM; ++r) {
            const bool ok = live && r < R;
            Bv[j][r] = ok ? ld_f32(Braw + j * R + r) : 0.f;
            Cv[j][r] = ok ? ld_f32(Craw + j * R + r) : 0.f;
            ssb += Bv[j][r] * Bv[j][r];
            ssc += Cv[j][r] * Cv[j][r];
        }
    }
    ssb = group_sum<LPR>(ssb);
    ssc = group_sum<LPR>(ssc);
    const float rb = rsqrtf(ssb / NR + a.eps), rc = rsqrtf(ssc / NR + a.eps);
    const float* wB = a.prm.B_norm_w + (int64_t)n0 * R;
    const float* wC = a.prm.C_norm_w + (int64_t)n0 * R;
    const float* bB = a.prm.B_bias + (int64_t)g * NR + (int64_t)n0 * R;
    const float* bC = a.prm.C_bias + (int64_t)g * NR + (int64_t)n0 * R;
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
        const bool live = j < nvq * VW;
#pragma unroll
        for (int r = 0; r < RM; ++r) {
            if (live && r < R) {
                Bv[j][r] = Bv[j][r] * rb * wB[j * R + r] + bB[j * R + r];
                Cv[j][r] = Cv[j][r] * rc * wC[j * R + r] + bC[j * R + r];
            }
        }
    }
    const int64_t abase = ((int64_t)b * a.H + h) * Nh;
    const bool abf = a.angle_bf16 != 0;
    if (a.cplx) {
#pragma unroll
        for (int j = 0; j < CPL / 2; ++j) {
            if (2 * j < nvq * VW) {
                const int i = n0 / 2 + j;
                const float phi = ld_angle(a.angle_in, abase + i, abf) - tg.dt * ld_f32(pr + a.pl.theta + i);
                if (row0 == 0) st_angle(a.angle_out, abase + i, phi, abf);
                float sn, cs;
                sincosf(phi, &sn, &cs);
#pragma unroll
                for (int r = 0; r < RM; ++r) {
                    const float be = Bv[2 * j][r], bo = Bv[2 * j + 1][r];
                    Bv[2 * j][r] = be * cs - bo * sn;
                    Bv[2 * j + 1][r] = be * sn + bo * cs;
                    const float ce = Cv[2 * j][r], co = Cv[2 * j + 1][r];
                    Cv[2 * j][r] = ce * cs - co * sn;
                    Cv[2 * j + 1][r] = ce * sn + co * cs;
                }
            }
        }
    } else if (row0 == 0 && a.angle_out) {
        // Angle stays zero without complex RoPE; pass the input through.
        for (int j = 0; j < CPL / 2; ++j)
            if (2 * j < nvq * VW) {
                const int i = n0 / 2 + j;
                st_angle(a.angle_out, abase + i, ld_angle(a.angle_in, abase + i, abf), abf);
            }
    }

    const float Dh = a.prm.D[h];
    const float* mx = a.prm.mimo_x + (int64_t)h * P * R;
    const float* mz = a.prm.mimo_z + (int64_t)h * P * R;
    const float* md = a.prm.mimo_down + (int64_t)h * P * R;
    const int64_t sbase = ((int64_t)b * a.H + h) * P * N;
    const vec* hin = reinterpret_cast<const vec*>(a.h_in + sbase);
    const vec* pin = reinterpret_cast<const vec*>(a.prev_in + sbase);
    vec* hout = reinterpret_cast<vec*>(a.h_out + sbase);
    vec* pout = reinterpret_cast<vec*>(a.prev_out + sbase);
    T* yo = reinterpret_cast<T*>(a.y_out) + (int64_t)b * a.H * P + (int64_t)h * P;
    const int nvr = N / VW;       // vectors per row (P * N <= 256 * 512: int offsets)
    const int v0 = q * NV;        // this lane's first vector in the row

    for (int pbase = row0; pbase < P; pbase += kRows * kStepRowsPerLane) {
        vec hv[kStepRowsPerLane][NV], pv[kStepRowsPerLane][NV];
        float xv[kStepRowsPerLane];
#pragma unroll
        for (int it = 0; it < kStepRowsPerLane; ++it) {
            const int p = pbase + it * kRows;
            if (p < P) {
                // streaming reads of the incoming state; the outgoing state is stored
                // normally so the next step finds it in the caches
#pragma unroll
                for (int v = 0; v < NV; ++v)
                    if (v < nvq) {
                        hv[it][v] = __builtin_nontemporal_load(&hin[p * nvr + v0 + v]);
                        pv[it][v] = __builtin_nontemporal_load(&pin[p * nvr + v0 + v]);
                    }
                xv[it] = ld_f32(pr + a.pl.x + (int64_t)h * P + p);
            }
        }
#pragma unroll
        for (int it = 0; it < kStepRowsPerLane; ++it) {
            const int p = pbase + it * kRows;
            if (p < P) {
                float xr[RM];
#pragma unroll
                for (int r = 0; r < RM; ++r) xr[r] = r < R ? xv[it] * mx[p * R + r] : 0.f;
                float yacc[RM];
#pragma unroll
                for (int r = 0; r < RM; ++r) yacc[r] = 0.f;
#pragma unroll
                for (int v = 0; v < NV; ++v) {
                    if (v < nvq) {
                        vec cur, hn;
#pragma unroll
                        for (int e = 0; e < VW; ++e) {
                            const int j = v * VW + e;
                            float c = 0.f;
#pragma unroll
                            for (int r = 0; r < RM; ++r) c += Bv[j][r] * xr[r];
                            cur[e] = c;
                            hn[e] = dA * hv[it][v][e] + gamma * c + beta * pv[it][v][e];
#pragma unroll
                            for (int r = 0; r < RM; ++r) yacc[r] += Cv[j][r] * hn[e];
                        }
                        hout[p * nvr + v0 + v] = hn;
                        pout[p * nvr + v0 + v] = cur;
                    }
                }
                float yr[RM];
#pragma unroll
                for (int r = 0; r < RM; ++r) yr[r] = group_sum<LPR>(yacc[r]);
                if (q == 0) {
                    const float z = ld_f32(pr + a.pl.z + (int64_t)h * P + p);
                    float out = 0.f;
#pragma unroll
                    for (int r = 0; r < RM; ++r) {
                        if (r < R) {
                            const float y = yr[r] + Dh * xr[r];
                            out += md[p * R + r] * y * silu_f(z * mz[p * R + r]);
                        }
                    }
                    yo[p] = cvt_out<T>(out);
                }
            }
        }
    }
}

// Every even d_state up to 512 and every mimo_rank up to 8.
int step_supported(int N, int R) { return N >= 2 && N <= 512 && N % 2 == 0 && R >= 1 && R <= 8; }

// Lane layout of a row of N columns: vector width, vectors per lane, lanes per row.
static void step_layout(int N, int& vw, int& nv, int& lpr) {
    vw = N % 4 == 0 ? 4 : 2;
    nv = (N > 64 * vw) ? 2 : 1;
    if (vw == 2 && N > 256) nv = 4;
    const int lanes = (N + vw * nv - 1) / (vw * nv);
    lpr = 1;
    while (lpr < lanes) lpr *= 2;
}

// Reachable layouts: one vector per lane for any power-of-two lane count (N <= 64 VW);
// several vectors per lane only with all 64 lanes (N > 256, or N > 128 with VW = 2).
template <typename T, int RM, bool kX, int VW>
static void launch_step_l(int lpr, dim3 grid, hipStream_t stream, const StepArgs& a) {
    switch (lpr) {
        case 1: hipLaunchKernelGGL((step_kernel<T, RM, kX, 1, VW, 1>), grid, dim3(kStepThreads), 0, stream, a); break;
        case 2: hipLaunchKernelGGL((step_kernel<T, RM, kX, 2, VW, 1>), grid, dim3(kStepThreads), 0, stream, a); break;
        case 4: hipLaunchKernelGGL((step_kernel<T, RM, kX, 4, VW, 1>), grid, dim3(kStepThreads), 0, stream, a); break;
        case 8: hipLaunchKernelGGL((step_kernel<T, RM, kX, 8, VW, 1>), grid, dim3(kStepThreads), 0, stream, a); break;
        case 16: hipLaunchKernelGGL((step_kernel<T, RM, kX, 16, VW, 1>), grid, dim3(kStepThreads), 0, stream, a); break;
        case 32: hipLaunchKernelGGL((step_kernel<T, RM, kX, 32, VW, 1>), grid, dim3(kStepThreads), 0, stream, a); break;
        default: hipLaunchKernelGGL((step_kernel<T, RM, kX, 64, VW, 1>), grid, dim3(kStepThreads), 0, stream, a); break;
    }
}

// Reachable layouts: one vector per lane for any power-of-two lane count (N <= 64 VW);
// several vectors per lane only with all 64 lanes (N > 256, or N > 128 with VW = 2).
template <typename T, int RM, bool kX>
static void launch_step_v(int vw, int nv, int lpr, dim3 grid, hipStream_t stream, const StepArgs& a) {
    if (nv == 1) {
        if (vw == 4) launch_step_l<T, RM, kX, 4>(lpr, grid, stream, a);
        else launch_step_l<T, RM, kX, 2>(lpr, grid, stream, a);
    } else if (vw == 4) {
        hipLaunchKernelGGL((step_kernel<T, RM, kX, 64, 4, 2>), grid, dim3(kStepThreads), 0, stream, a);
    } else if (nv == 2) {
        hipLaunchKernelGGL((step_kernel<T, RM, kX, 64, 2, 2>), grid, dim3(kStepThreads), 0, stream, a);
    } else {
        hipLaunchKernelGGL((step_kernel<T, RM, kX, 64, 2, 4>), grid, dim3(kStepThreads), 0, stream, a);
    }
}

// Ranks 1, 2 and 4 are compile-time constants; the others run under RM = 8 with the rank
// as a run-time bound.
template <typename T>
static void launch_step_t(int R, int vw, int nv, int lpr, dim3 grid, hipStream_t stream,
                          const StepArgs& a) {
    if (R == 1) launch_step_v<T, 1, true>(vw, nv, lpr, grid, stream, a);
    else if (R == 2) launch_step_v<T, 2, true>(vw, nv, lpr, grid, stream, a);
    else if (R == 4) launch_step_v<T, 4, true>(vw, nv, lpr, grid, stream, a);
    else launch_step_v<T, 8, false>(vw, nv, lpr, grid, stream, a);
}

int launch_step(const m3_layer_desc& d, const m3_layer_params& p, const void* proj,
                const float* dt_scale, const float* h_in, const float* prev_in,
                const void* angle_in, int angle_dtype, void* y_out, float* h_out,
                float* prev_out, void* angle_out, hipStream_t stream) {
    StepArgs a;
    a.H = d.nheads; a.P = d.headdim; a.N = d.d_state; a.G = d.ngroups; a.R = d.mimo_rank;
    a.trap = d.use_trapezoidal; a.cplx = d.use_complex; a.eps = d.rms_eps;
    a.angle_bf16 = angle_dtype == M3_DTYPE_BF16;
    a.row_stride = d.proj_row_stride;
    a.pl = proj_layout(d);
    a.prm = p;
    a.proj = proj; a.dt_scale = dt_scale; a.h_in = h_in; a.prev_in = prev_in;
    a.angle_in = angle_in; a.y_out = y_out; a.h_out = h_out; a.prev_out = prev_out;
    a.angle_out = angle_out;
    int vw, nv, lpr;
    step_layout(d.d_state, vw, nv, lpr);
    const dim3 grid((unsigned)(d.batch * d.nheads));
    if (d.dtype == M3_DTYPE_BF16) launch_step_t<bf16>(d.mimo_rank, vw, nv, lpr, grid, stream, a);
    else launch_step_t<float>(d.mimo_rank, vw, nv, lpr, grid, stream, a);
    return hipGetLastError() == hipSuccess ? M3_OK : M3_ERR_LAUNCH;
}

}  // namespace m3
