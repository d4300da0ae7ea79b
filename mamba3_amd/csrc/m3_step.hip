// O(1) decode step of one KulaMamba layer (replaces mamba3/mamba3.py:275-316).
//
// One workgroup per (batch, head), or at small batch per (batch, head, block of P / psplit
// rows), so that about 1024 workgroups share the step. Each lane owns NV vectors of VW
// consecutive state columns (CPL = NV * VW columns, n0 = q * CPL) of one headdim row p, so a
// row of N columns is spread over ceil(N / CPL) lanes, rounded up to LPR (a power of two;
// lanes past the row end hold no columns), and a wave covers 64 / LPR rows. The lane recomputes
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
// else 1. Full layouts (power-of-two N >= 4 with rank 1, 2 or 4: every lane inside the row)
// read a lane's B / C entries, norm weights and biases as contiguous runs with wide loads;
// the others read entry by entry, clamped into the row and masked. Every prologue load is
// issued before the dependent arithmetic, as are all loads of a lane's rows, so each wave
// keeps up to kStepRowsPerLane rows per lane in flight. HBM-bound: 16*P*N bytes per
// (batch, head).
#include "m3_common.h"
#include "m3_kernels.h"

namespace m3 {

constexpr int kStepThreads = 256;
constexpr int kStepRowsPerLane = 8;

struct StepArgs {
    int H, P, N, G, R;
    int psplit;  // workgroups per (batch, head), each P / psplit rows
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

// Element i of a bf16 or fp32 angle array, read as 16-bit halves so neither dtype needs a
// branch (a bf16 element is the high half of its fp32 value; an fp32 element's halves are
// little-endian).
__device__ __forceinline__ float ld_angle(const void* p, int64_t i, bool is_bf16) {
    const unsigned short* u = reinterpret_cast<const unsigned short*>(p);
    const int64_t e = is_bf16 ? i : 2 * i;
    const unsigned lo = u[e], hi = u[is_bf16 ? e : e + 1];
    const unsigned sh = is_bf16 ? 16u : 0u, hmask = is_bf16 ? 0u : 0xffff0000u;
    return __uint_as_float((lo << sh) | ((hi << 16) & hmask));
}
__device__ __forceinline__ void st_angle(void* p, int64_t i, float v, bool is_bf16) {
    if (is_bf16) reinterpret_cast<bf16*>(p)[i] = (bf16)v;
    else reinterpret_cast<float*>(p)[i] = v;
}

// RPL: rows in flight per lane (kStepRowsPerLane, or 1 when a workgroup's rows are one per
// lane: then those rows' reads are issued with the prologue's, before its arithmetic).
template <typename T, int RM, bool kExactR, int LPR, int VW, int NV, bool kFull, int RPL>
__global__ __launch_bounds__(kStepThreads) void step_kernel(StepArgs a) {
    typedef typename StepVec<VW>::type vec;
    constexpr bool kEarly = RPL == 1;
    constexpr int CPL = VW * NV;               // state columns per lane
    constexpr int kRows = kStepThreads / LPR;  // rows handled per pass of the block
    const int tid = threadIdx.x;
    const int bh = blockIdx.x / a.psplit, ps = blockIdx.x - bh * a.psplit;
    const int b = bh / a.H, h = bh % a.H;
    const int g = h / (a.H / a.G);
    // the rank: RM itself, or a.R <= RM (ranks 3, 5, 6 and 7 run under RM = 4 or 8)
    const int R = kExactR ? RM : a.R;
    const int P = a.P, N = a.N, Nh = N / 2, NR = N * R;
    const int q = tid % LPR;   // column group
    const int row0 = tid / LPR;
    const int n0 = q * CPL;
    // vectors of this lane inside the row (0: the lane is past the row end)
    const int nvq = kFull ? NV : n0 >= N ? 0 : ((N - n0) / VW < NV ? (N - n0) / VW : NV);
    const T* pr = reinterpret_cast<const T*>(a.proj) + (int64_t)b * a.row_stride;

    // Prologue loads, all unconditional and issued as one flight before the arithmetic:
    // absent inputs, and entries past the row end or the rank, read a valid element and are
    // blended out arithmetically (a select on a loaded value lets the compiler move the load
    // under a branch, which serialises the flight).
    constexpr int NPL = CPL / 2;  // column pairs per lane
    const float dt_raw = ld_f32(pr + a.pl.dt + h);
    const float trapf = a.trap ? 1.f : 0.f;
    const float lam_raw = ld_f32(pr + (a.trap ? a.pl.lam + h : 0));
    const float scf = a.dt_scale ? 1.f : 0.f;
    const float sc_raw = *(a.dt_scale ? a.dt_scale + (int64_t)b * a.H + h : a.prm.dt_bias + h);
    const float A_log = a.prm.A_log[h], dt_bias = a.prm.dt_bias[h];
    // running angle and theta of the lane's column pairs (pairs past the row end read pair
    // 0; without complex RoPE theta reads element 0 of the row and is unused)
    const int64_t abase = ((int64_t)b * a.H + h) * Nh;
    const bool abf = a.angle_bf16 != 0;
    float ang[NPL], th[NPL];
#pragma unroll
    for (int j = 0; j < NPL; ++j) {
        const int i = 2 * j < nvq * VW ? n0 / 2 + j : 0;
        ang[j] = ld_angle(a.angle_in, abase + i, abf);
        th[j] = ld_f32(pr + (a.cplx ? a.pl.theta + i : 0));
    }
    // B, C columns n0 .. n0 + CPL - 1, with their norm weights and biases when the lane
    // holds at most 16 entries (more would cost occupancy; those load them below). In the
    // full layouts (every lane's columns inside the row, the rank a compile-time constant:
    // every power-of-two d_state >= 4 with rank 1, 2 or 4) a lane's CPL * RM entries are one
    // contiguous run from n0 * RM, which the compiler reads with wide loads; otherwise each
    // entry is read on its own, clamped into the row.
    constexpr bool kPreW = CPL * RM <= 16;
    constexpr int WD = kPreW ? CPL : 1, WR = kPreW ? RM : 1;
    float Bv[CPL][RM], Cv[CPL][RM], msk[CPL][RM];
    float wb[WD][WR], wc[WD][WR], bb[WD][WR], bc[WD][WR];
    const T* Braw = pr + a.pl.B + (int64_t)g * NR;
    const T* Craw = pr + a.pl.C + (int64_t)g * NR;
    const float* bB = a.prm.B_bias + (int64_t)g * NR;
    const float* bC = a.prm.C_bias + (int64_t)g * NR;
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
#pragma unroll
        for (int r = 0; r < RM; ++r) {
            bool ok;
            int o;
            if constexpr (kFull) {
                ok = true;
                o = n0 * RM + j * RM + r;
            } else {
                ok = j < nvq * VW && r < R;
                o = ok ? (n0 + j) * R + r : 0;
            }
            msk[j][r] = ok ? 1.f : 0.f;
            Bv[j][r] = ld_f32(Braw + o);
            Cv[j][r] = ld_f32(Craw + o);
            if constexpr (kPreW) {
                wb[j][r] = a.prm.B_norm_w[o];
                wc[j][r] = a.prm.C_norm_w[o];
                bb[j][r] = bB[o];
                bc[j][r] = bC[o];
            }
        }
    }

    // Incoming state rows (the outgoing state is stored normally so the next step finds it
    // in the caches). All loads are unconditional and issued before the arithmetic that uses
    // them: rows past the block's end read its last row and lanes past the row end read the
    // row's last vector (their B / C columns are zero); neither stores anything.
    const int64_t sbase = ((int64_t)b * a.H + h) * P * N;
    const vec* hin = reinterpret_cast<const vec*>(a.h_in + sbase);
    const vec* pin = reinterpret_cast<const vec*>(a.prev_in + sbase);
    vec* hout = reinterpret_cast<vec*>(a.h_out + sbase);
    vec* pout = reinterpret_cast<vec*>(a.prev_out + sbase);
    const int nvr = N / VW;       // vectors per row (P * N <= 256 * 512: int offsets)
    const int v0 = q * NV;        // this lane's first vector in the row
    // this workgroup's rows [pb, pe)
    const int pb = ps * (P / a.psplit), pe = pb + P / a.psplit;
    vec hv[RPL][NV], pv[RPL][NV];
    T xv[RPL];
    auto load_rows = [&](int pbase) {
#pragma unroll
        for (int it = 0; it < RPL; ++it) {
            const int p = pbase + it * kRows < pe ? pbase + it * kRows : pe - 1;
#pragma unroll
            for (int v = 0; v < NV; ++v) {
                const int vi = v0 + v < nvr ? v0 + v : nvr - 1;
                hv[it][v] = __builtin_nontemporal_load(&hin[p * nvr + vi]);
                pv[it][v] = __builtin_nontemporal_load(&pin[p * nvr + vi]);
            }
            xv[it] = pr[a.pl.x + (int64_t)h * P + p];
        }
    };
    if constexpr (kEarly) load_rows(pb + row0 < pe ? pb + row0 : pe - 1);

    // Per-head scalars (mamba3/mamba3.py:278-282, 290-296).
    const float sc = sc_raw * scf + (1.f - scf);
    const TokenGate tg = token_gate(dt_raw, dt_bias, sc, -expf(A_log), lam_raw * trapf, a.trap != 0);
    const float dA = expf(tg.logdA);
    const float gamma = a.trap ? tg.lam * tg.dt : tg.dt;
    const float beta = a.trap ? (1.f - tg.lam) * tg.dt * dA : 0.f;

    // B~, C~: RMSNorm over the group's N*R entries, weight and bias (mamba3/mamba3.py:170-184)
    float ssb = 0.f, ssc = 0.f;
#pragma unroll
    for (int j = 0; j < CPL; ++j)
#pragma unroll
        for (int r = 0; r < RM; ++r) {
            Bv[j][r] *= msk[j][r];
            Cv[j][r] *= msk[j][r];
            ssb += Bv[j][r] * Bv[j][r];
            ssc += Cv[j][r] * Cv[j][r];
        }
    ssb = lane_sum<LPR>(ssb);
    ssc = lane_sum<LPR>(ssc);
    const float rb = rsqrtf(ssb / NR + a.eps), rc = rsqrtf(ssc / NR + a.eps);
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
#pragma unroll
        for (int r = 0; r < RM; ++r) {
            if constexpr (kPreW) {
                Bv[j][r] = (Bv[j][r] * rb * wb[j][r] + bb[j][r]) * msk[j][r];
                Cv[j][r] = (Cv[j][r] * rc * wc[j][r] + bc[j][r]) * msk[j][r];
            } else {
                const int o = j < nvq * VW && r < R ? (n0 + j) * R + r : 0;
                Bv[j][r] = (Bv[j][r] * rb * a.prm.B_norm_w[o] + bB[o]) * msk[j][r];
                Cv[j][r] = (Cv[j][r] * rc * a.prm.C_norm_w[o] + bC[o]) * msk[j][r];
            }
        }
    }
    if (a.cplx) {
#pragma unroll
        for (int j = 0; j < NPL; ++j) {
            // pairs past the row end rotate zero columns and store nothing
            const float phi = ang[j] - tg.dt * th[j];
            if (row0 == 0 && ps == 0 && 2 * j < nvq * VW) st_angle(a.angle_out, abase + n0 / 2 + j, phi, abf);
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
    } else if (row0 == 0 && ps == 0) {
        // Angle stays zero without complex RoPE; pass the input through.
#pragma unroll
        for (int j = 0; j < NPL; ++j)
            if (2 * j < nvq * VW) st_angle(a.angle_out, abase + n0 / 2 + j, ang[j], abf);
    }

    const float Dh = a.prm.D[h];
    const float* mx = a.prm.mimo_x + (int64_t)h * P * R;
    const float* mz = a.prm.mimo_z + (int64_t)h * P * R;
    const float* md = a.prm.mimo_down + (int64_t)h * P * R;
    T* yo = reinterpret_cast<T*>(a.y_out) + (int64_t)b * a.H * P + (int64_t)h * P;

    for (int pbase = pb + row0; pbase < pe; pbase += kRows * RPL) {
        if (!kEarly || pbase != pb + row0) load_rows(pbase);
#pragma unroll
        for (int it = 0; it < RPL; ++it) {
            const int p = pbase + it * kRows;
            if (p < pe) {
                float xr[RM];
#pragma unroll
                for (int r = 0; r < RM; ++r) xr[r] = r < R ? (float)xv[it] * mx[p * R + r] : 0.f;
                float yacc[RM];
#pragma unroll
                for (int r = 0; r < RM; ++r) yacc[r] = 0.f;
#pragma unroll
                for (int v = 0; v < NV; ++v) {
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
                    if (v < nvq) {
                        hout[p * nvr + v0 + v] = hn;
                        pout[p * nvr + v0 + v] = cur;
                    }
                }
                float yr[RM];
#pragma unroll
                for (int r = 0; r < RM; ++r) yr[r] = lane_sum<LPR>(yacc[r]);
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
template <typename T, int RM, bool kX, int VW, bool kF, int RPL>
static void launch_step_l(int lpr, dim3 grid, hipStream_t stream, const StepArgs& a) {
    switch (lpr) {
        case 1: hipLaunchKernelGGL((step_kernel<T, RM, kX, 1, VW, 1, kF, RPL>), grid, dim3(kStepThreads), 0, stream, a); break;
        case 2: hipLaunchKernelGGL((step_kernel<T, RM, kX, 2, VW, 1, kF, RPL>), grid, dim3(kStepThreads), 0, stream, a); break;
        case 4: hipLaunchKernelGGL((step_kernel<T, RM, kX, 4, VW, 1, kF, RPL>), grid, dim3(kStepThreads), 0, stream, a); break;
        case 8: hipLaunchKernelGGL((step_kernel<T, RM, kX, 8, VW, 1, kF, RPL>), grid, dim3(kStepThreads), 0, stream, a); break;
        case 16: hipLaunchKernelGGL((step_kernel<T, RM, kX, 16, VW, 1, kF, RPL>), grid, dim3(kStepThreads), 0, stream, a); break;
        case 32: hipLaunchKernelGGL((step_kernel<T, RM, kX, 32, VW, 1, kF, RPL>), grid, dim3(kStepThreads), 0, stream, a); break;
        default: hipLaunchKernelGGL((step_kernel<T, RM, kX, 64, VW, 1, kF, RPL>), grid, dim3(kStepThreads), 0, stream, a); break;
    }
}

template <typename T, int RM, bool kX>
static void launch_step_v(int vw, int nv, int lpr, dim3 grid, hipStream_t stream, const StepArgs& a) {
    constexpr int R8 = kStepRowsPerLane;
    if (nv == 1) {
        if (vw == 4) launch_step_l<T, RM, kX, 4, false, R8>(lpr, grid, stream, a);
        else launch_step_l<T, RM, kX, 2, false, R8>(lpr, grid, stream, a);
    } else if (vw == 4) {
        hipLaunchKernelGGL((step_kernel<T, RM, kX, 64, 4, 2, false, R8>), grid, dim3(kStepThreads), 0, stream, a);
    } else if (nv == 2) {
        hipLaunchKernelGGL((step_kernel<T, RM, kX, 64, 2, 2, false, R8>), grid, dim3(kStepThreads), 0, stream, a);
    } else {
        hipLaunchKernelGGL((step_kernel<T, RM, kX, 64, 2, 4, false, R8>), grid, dim3(kStepThreads), 0, stream, a);
    }
}

// Full layouts (4-column vectors, every lane inside the row, exact rank). one_row: each
// workgroup's P / psplit rows are at most one per lane (small batches).
template <typename T, int RM>
static void launch_step_full(int nv, int lpr, bool one_row, dim3 grid, hipStream_t stream, const StepArgs& a) {
    constexpr int R8 = kStepRowsPerLane;
    if (nv == 2) {
        if (one_row) hipLaunchKernelGGL((step_kernel<T, RM, true, 64, 4, 2, true, 1>), grid, dim3(kStepThreads), 0, stream, a);
        else hipLaunchKernelGGL((step_kernel<T, RM, true, 64, 4, 2, true, R8>), grid, dim3(kStepThreads), 0, stream, a);
    } else if (one_row) {
        launch_step_l<T, RM, true, 4, true, 1>(lpr, grid, stream, a);
    } else {
        launch_step_l<T, RM, true, 4, true, R8>(lpr, grid, stream, a);
    }
}

// Ranks 1, 2 and 4 are compile-time constants; the others run under RM = 8 with the rank
// as a run-time bound.
template <typename T>
static void launch_step_t(int N, int R, int vw, int nv, int lpr, bool one_row, dim3 grid, hipStream_t stream,
                          const StepArgs& a) {
    const bool full = vw == 4 && N == lpr * vw * nv;
    if (R == 1) {
        if (full) launch_step_full<T, 1>(nv, lpr, one_row, grid, stream, a);
        else launch_step_v<T, 1, true>(vw, nv, lpr, grid, stream, a);
    } else if (R == 2) {
        if (full) launch_step_full<T, 2>(nv, lpr, one_row, grid, stream, a);
        else launch_step_v<T, 2, true>(vw, nv, lpr, grid, stream, a);
    } else if (R == 4) {
        if (full) launch_step_full<T, 4>(nv, lpr, one_row, grid, stream, a);
        else launch_step_v<T, 4, true>(vw, nv, lpr, grid, stream, a);
    } else {
        launch_step_v<T, 8, false>(vw, nv, lpr, grid, stream, a);
    }
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
    // Small batches split each (batch, head) over up to 8 workgroups of P / psplit rows
    // (the per-head prologue is repeated), so that about 1024 workgroups share the work.
    a.psplit = 1;
    while (a.psplit < 8 && (int64_t)d.batch * d.nheads * a.psplit < 1024 && d.headdim % (2 * a.psplit) == 0)
        a.psplit *= 2;
    const dim3 grid((unsigned)(d.batch * d.nheads * a.psplit));
    const bool one_row = d.headdim / a.psplit <= kStepThreads / lpr;
    if (d.dtype == M3_DTYPE_BF16) launch_step_t<bf16>(d.d_state, d.mimo_rank, vw, nv, lpr, one_row, grid, stream, a);
    else launch_step_t<float>(d.d_state, d.mimo_rank, vw, nv, lpr, one_row, grid, stream, a);
    return hipGetLastError() == hipSuccess ? M3_OK : M3_ERR_LAUNCH;
}

}  // namespace m3
