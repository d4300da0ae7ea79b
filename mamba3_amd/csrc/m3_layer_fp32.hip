// fp32 layer prefill on the fp32-MFMA chunk kernels: the region between in_proj and out_proj
// (mamba3/mamba3.py:199-256) for fp32 layers, as
//   lp_dt      dt = softplus(dt_raw + dt_bias) [* dt_scale], A = -exp(A_log)
//              (mamba3/mamba3.py:200-204)
//   lp_angle_sums, lp_angles
//              the RoPE angle prefix phi_t = -sum_{s<=t} dt_s theta_s (mamba3/mamba3.py:160-162)
//              in chunks of 64 tokens
//   lp_prep    per token: B/C RMSNorm + weight + bias per group (mamba3/mamba3.py:19-35,
//              147-157), the rotation by phi per head (mamba3/mamba3.py:38-45, 163-166), the
//              MIMO x (mamba3/mamba3.py:219) and the trapezoid terms x_g = lambda x_r,
//              x_b = (1 - lambda) dA x_r[t-1], B_b = B~[t-1] (mamba3/mamba3.py:221-229)
//   chunked SSD forward (m3_ssd_bwd.hip, fp32 MFMA)
//   lp_gate    out = sum_r mimo_down y silu(z mimo_z) (mamba3/mamba3.py:233-239)
//   lp_state   angle = phi_{T-1}, prev_BX = B~_{T-1} x_r,{T-1}^T (mamba3/mamba3.py:241-256)
// The intermediate tensors (chunked_ssd's inputs, in its (B,T,H,X,R) layouts) live in the
// caller's workspace.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "m3_kernels.h"

namespace m3 {
namespace lp {

struct Args {
    int B, T, H, P, N, R, G, trap, cplx;
    int HT;  // heads whose sin / cos lp_prep holds in LDS at a time
    int64_t rs;  // proj row stride
    ProjLayout pl;
    float eps;
    m3_layer_params prm;
    const float* proj;
    const float* dt_scale;
    float *dt, *A, *phi, *phi_sum, *xg, *xb, *xr, *Bt, *Bb, *Ct, *ys;  // workspace
    float *y, *h_final, *angle, *prev_bx;                     // outputs
};

constexpr int NTH = 256;

__device__ __forceinline__ float softplus(float v) { return v > 20.f ? v : log1pf(expf(v)); }

// dt[b,t,h] and A[h].
__global__ __launch_bounds__(NTH) void lp_dt(Args a) {
    const int64_t n = (int64_t)a.B * a.T * a.H;
    const int64_t e = (int64_t)blockIdx.x * NTH + threadIdx.x;
    if (e < a.H) a.A[e] = -expf(a.prm.A_log[e]);
    if (e >= n) return;
    const int h = (int)(e % a.H);
    float d = softplus(a.proj[(e / a.H) * a.rs + a.pl.dt + h] + a.prm.dt_bias[h]);
    if (a.dt_scale) d *= a.dt_scale[e];
    a.dt[e] = d;
}

// RoPE angles phi_t = -sum_{s<=t} dt_s theta_s in chunks of kAC tokens: pass 1 writes each
// chunk's sum, pass 2 walks each chunk from the sum of the chunks before it. One thread per
// (b, chunk, h, pair).
constexpr int kAC = 64;

__device__ __forceinline__ void angle_job(const Args& a, int64_t e, int& b, int& c, int& h, int& i) {
    const int NH = a.N / 2;
    i = (int)(e % NH);
    h = (int)((e / NH) % a.H);
    const int64_t bc = e / ((int64_t)NH * a.H);
    const int nc = (a.T + kAC - 1) / kAC;
    c = (int)(bc % nc);
    b = (int)(bc / nc);
}

__global__ __launch_bounds__(NTH) void lp_angle_sums(Args a) {
    const int nc = (a.T + kAC - 1) / kAC;
    const int64_t n = (int64_t)a.B * nc * a.H * (a.N / 2);
    const int64_t e = (int64_t)blockIdx.x * NTH + threadIdx.x;
    if (e >= n) return;
    int b, c, h, i;
    angle_job(a, e, b, c, h, i);
    float s = 0.f;
    const int t1 = min(a.T, (c + 1) * kAC);
    const float* dtp = a.dt + (int64_t)b * a.T * a.H + h;                  // stride H
    const float* thp = a.proj + (int64_t)b * a.T * a.rs + a.pl.theta + i;  // stride rs
    int t = c * kAC;
    for (; t + 8 <= t1; t += 8) {  // tokens added in order; eight loads ahead of their products
        float dv[8], tv[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            dv[u] = dtp[(int64_t)(t + u) * a.H];
            tv[u] = thp[(int64_t)(t + u) * a.rs];
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) s += dv[u] * tv[u];
    }
    for (; t < t1; ++t) s += dtp[(int64_t)t * a.H] * thp[(int64_t)t * a.rs];
    a.phi_sum[e] = s;
}

__global__ __launch_bounds__(NTH) void lp_angles(Args a) {
    const int nc = (a.T + kAC - 1) / kAC;
    const int NH = a.N / 2;
    const int64_t n = (int64_t)a.B * nc * a.H * NH;
    const int64_t e = (int64_t)blockIdx.x * NTH + threadIdx.x;
    if (e >= n) return;
    int b, c, h, i;
    angle_job(a, e, b, c, h, i);
    float s = 0.f;
    for (int cc = 0; cc < c; ++cc) s += a.phi_sum[(((int64_t)b * nc + cc) * a.H + h) * NH + i];
    const int t1 = min(a.T, (c + 1) * kAC);
    const float* dtp = a.dt + (int64_t)b * a.T * a.H + h;                  // stride H
    const float* thp = a.proj + (int64_t)b * a.T * a.rs + a.pl.theta + i;  // stride rs
    float* php = a.phi + ((int64_t)b * a.T * a.H + h) * NH + i;            // stride H*NH
    const int64_t ps = (int64_t)a.H * NH;
    // tokens in order; phi is a buffer of its own, so eight tokens' loads go out ahead of the
    // running sums and their stores
    int t = c * kAC;
    for (; t + 8 <= t1; t += 8) {
        float dv[8], tv[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            dv[u] = dtp[(int64_t)(t + u) * a.H];
            tv[u] = thp[(int64_t)(t + u) * a.rs];
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            s += dv[u] * tv[u];
            php[(t + u) * ps] = -s;
        }
    }
    for (; t < t1; ++t) {
        s += dtp[(int64_t)t * a.H] * thp[(int64_t)t * a.rs];
        php[t * ps] = -s;
    }
}

// One block per (b, t), one group at a time: the group's normalised B^ / C^ in LDS, the sin /
// cos of a tile of its heads' RoPE pairs in LDS, then the rotated rows of those heads, as flat
// loops over (head, element); then the x terms of every head.
__global__ __launch_bounds__(NTH) void lp_prep(Args a) {
    // B^ [N*R], C^ [N*R], reduction scratch [2*NTH], sin / cos [HT*N/2] each
    extern __shared__ float sm[];
    const int bt = blockIdx.x, b = bt / a.T, t = bt % a.T;
    const int NR = a.N * a.R, NH = a.N / 2;
    float* Bh = sm;
    float* Ch = sm + NR;
    float* red = sm + 2 * NR;
    float* sn = red + 2 * NTH;
    float* cn = sn + (int64_t)a.HT * NH;
    const float* row = a.proj + ((int64_t)b * a.T + t) * a.rs;
    const int64_t tok0 = ((int64_t)b * a.T + t) * a.H;  // token row of head 0
    const int tid = threadIdx.x;
    const int hpg = a.H / a.G;
    for (int g = 0; g < a.G; ++g) {
        if (g > 0) __syncthreads();  // the previous group's rows and sin / cos are read
        float sb = 0.f, sc = 0.f;
        for (int e = tid; e < NR; e += NTH) {
            const float vb = row[a.pl.B + (int64_t)g * NR + e], vc = row[a.pl.C + (int64_t)g * NR + e];
            sb += vb * vb;
            sc += vc * vc;
        }
        red[tid] = sb;
        red[NTH + tid] = sc;
        __syncthreads();
        for (int w = NTH / 2; w > 0; w >>= 1) {
            if (tid < w) {
                red[tid] += red[tid + w];
                red[NTH + tid] += red[NTH + tid + w];
            }
            __syncthreads();
        }
        const float rb = rsqrtf(red[0] / NR + a.eps), rc = rsqrtf(red[NTH] / NR + a.eps);
        for (int e = tid; e < NR; e += NTH) {
            const int64_t o = (int64_t)g * NR + e;
            Bh[e] = row[a.pl.B + o] * rb * a.prm.B_norm_w[e] + a.prm.B_bias[o];
            Ch[e] = row[a.pl.C + o] * rc * a.prm.C_norm_w[e] + a.prm.C_bias[o];
        }
        __syncthreads();
        // the group's heads in tiles of HT, so the sin / cos of a tile fit in LDS whatever
        // H * N is
        for (int h0 = g * hpg; h0 < (g + 1) * hpg; h0 += a.HT) {
            const int nh = min(a.HT, (g + 1) * hpg - h0);
            if (a.cplx) {
                if (h0 > g * hpg) __syncthreads();  // the previous tile's sin / cos are read
                for (int j = tid; j < nh * NH; j += NTH)
                    sincosf(a.phi[(tok0 + h0) * NH + j], &sn[j], &cn[j]);
                __syncthreads();
            }
            for (int j = tid; j < nh * NR; j += NTH) {
                const int hl = j / NR, h = h0 + hl, e = j % NR;
                const int n = e / a.R, r = e % a.R, i = n >> 1;
                const int ev = (2 * i) * a.R + r, od = ev + a.R;
                float vb = Bh[e], vc = Ch[e];
                if (a.cplx) {
                    const float s = sn[hl * NH + i], c = cn[hl * NH + i];
                    vb = (n & 1) ? Bh[ev] * s + Bh[od] * c : Bh[ev] * c - Bh[od] * s;
                    vc = (n & 1) ? Ch[ev] * s + Ch[od] * c : Ch[ev] * c - Ch[od] * s;
                }
                const int64_t tok = tok0 + h;
                a.Bt[tok * NR + e] = vb;
                a.Ct[tok * NR + e] = vc;
                if (a.trap) {
                    if (t + 1 < a.T) a.Bb[(tok + a.H) * NR + e] = vb;  // B_b[t+1] = B~[t]
                    if (t == 0) a.Bb[tok * NR + e] = 0.f;
                }
            }
        }
    }
    const int PR = a.P * a.R;
    for (int j = tid; j < a.H * PR; j += NTH) {
        const int h = j / PR, e = j % PR, p = e / a.R;
        const int64_t tok = tok0 + h;
        const float mx = a.prm.mimo_x[(int64_t)h * PR + e];
        const float xr = row[a.pl.x + (int64_t)h * a.P + p] * mx;
        float lam = 1.f;
        if (a.trap) lam = 1.f / (1.f + expf(-row[a.pl.lam + h]));
        a.xr[tok * PR + e] = xr;
        a.xg[tok * PR + e] = xr * lam;
        if (a.trap) {
            const float sb = (1.f - lam) * expf(a.A[h] * a.dt[tok]);
            const float xp = t > 0 ? row[a.pl.x + (int64_t)h * a.P + p - a.rs] * mx : 0.f;
            a.xb[tok * PR + e] = xp * sb;
        }
    }
}

// out[b,t,h*P+p] = sum_r mimo_down[h,p,r] y[b,t,h,p,r] silu(z[b,t,h*P+p] mimo_z[h,p,r]).
__global__ __launch_bounds__(NTH) void lp_gate(Args a) {
    const int64_t n = (int64_t)a.B * a.T * a.H * a.P;
    const int64_t HP = (int64_t)a.H * a.P;
    for (int64_t e = (int64_t)blockIdx.x * NTH + threadIdx.x; e < n; e += (int64_t)gridDim.x * NTH) {
        const int64_t tok = e / HP;
        const int hp = (int)(e % HP);
        const float z = a.proj[tok * a.rs + a.pl.z + hp];
        float acc = 0.f;
        for (int r = 0; r < a.R; ++r) {
            const int64_t pr = (int64_t)hp * a.R + r;
            const float zz = z * a.prm.mimo_z[pr];
            acc += a.prm.mimo_down[pr] * a.ys[e * a.R + r] * (zz / (1.f + expf(-zz)));
        }
        a.y[e] = acc;
    }
}

// angle = phi at t = T-1 (0 without RoPE); prev_BX[b,h,p,n] = sum_r B~[T-1,n,r] x_r[T-1,p,r].
__global__ __launch_bounds__(NTH) void lp_state(Args a) {
    const int bh = blockIdx.x, b = bh / a.H, h = bh % a.H;
    const int NH = a.N / 2;
    const int64_t tok = ((int64_t)b * a.T + a.T - 1) * a.H + h;
    if (a.angle)
        for (int i = threadIdx.x; i < NH; i += NTH)
            a.angle[(int64_t)bh * NH + i] = a.cplx ? a.phi[tok * NH + i] : 0.f;
    if (a.prev_bx) {
        const int PN = a.P * a.N;
        for (int e = threadIdx.x; e < PN; e += NTH) {
            const int p = e / a.N, nn = e % a.N;
            float acc = 0.f;
            for (int r = 0; r < a.R; ++r)
                acc += a.Bt[tok * a.N * a.R + (int64_t)nn * a.R + r] * a.xr[tok * a.P * a.R + (int64_t)p * a.R + r];
            a.prev_bx[(int64_t)bh * PN + e] = acc;
        }
    }
}

struct Plan {
    size_t off[11], chunk_off, total;
};

inline size_t al(size_t x) { return (x + 255) & ~(size_t)255; }

Plan plan(const m3_layer_desc& d) {
    const size_t BTH = (size_t)d.batch * d.seqlen * d.nheads;
    const size_t X = BTH * d.headdim * d.mimo_rank, BN = BTH * d.d_state * d.mimo_rank;
    const bool trap = d.use_trapezoidal != 0;
    const size_t nc = (d.seqlen + kAC - 1) / kAC;
    const size_t sizes[11] = {BTH, (size_t)d.nheads, BTH * (d.d_state / 2), X, trap ? X : 0, X,
                              BN, trap ? BN : 0, BN, X,
                              (size_t)d.batch * nc * d.nheads * (d.d_state / 2)};
    Plan p;
    size_t o = 0;
    for (int i = 0; i < 11; ++i) {
        p.off[i] = o;
        o += al(sizes[i] * sizeof(float));
    }
    p.chunk_off = o;
    o += al(chunked_fwd_mfma_workspace(d.batch, d.seqlen, d.nheads, d.headdim, d.d_state,
                                       d.mimo_rank, trap));
    p.total = o;
    return p;
}

}  // namespace lp

namespace {
constexpr size_t kPrepLds = 64 * 1024;

// LDS of lp_prep without the sin / cos tiles: B^ and C^ of one group, the reduction scratch
// (at most 34 KB: d_state <= 512, rank <= 8).
size_t prep_lds_fixed(const m3_layer_desc& d) {
    return (2 * (size_t)d.d_state * d.mimo_rank + 2 * lp::NTH) * sizeof(float);
}
// Heads per sin / cos tile: as many of a group's heads as fit next to the fixed part (0:
// nothing fits).
int prep_heads_per_tile(const m3_layer_desc& d) {
    const size_t fixed = prep_lds_fixed(d);
    if (fixed >= kPrepLds || d.ngroups <= 0 || d.nheads % d.ngroups != 0) return 0;
    const size_t per_head = (size_t)d.d_state * sizeof(float);  // sin and cos of N/2 pairs
    return (int)std::min<size_t>(d.nheads / d.ngroups, (kPrepLds - fixed) / per_head);
}
size_t prep_lds(const m3_layer_desc& d) {
    return prep_lds_fixed(d) + (size_t)prep_heads_per_tile(d) * d.d_state * sizeof(float);
}
}  // namespace

Fp32LayerParts fp32_layer_parts(const m3_layer_desc& d, void* workspace) {
    const lp::Plan pl = lp::plan(d);
    char* ws = reinterpret_cast<char*>(workspace);
    auto part = [&](int i) { return reinterpret_cast<float*>(ws + pl.off[i]); };
    const bool trap = d.use_trapezoidal != 0;
    float* hs = reinterpret_cast<float*>(
        ws + pl.chunk_off + chunked_fwd_hs_offset(d.batch, d.seqlen, d.nheads, d.headdim, d.d_state,
                                                  d.mimo_rank, trap));
    return Fp32LayerParts{part(0), part(1), part(2), part(3), trap ? part(4) : nullptr, part(5),
                          part(6), trap ? part(7) : nullptr, part(8), part(9), hs};
}

// The chunk-start states of the training forward (Fp32LayerParts::Hs) are valid for the
// backward when the fused fp32 forward can keep its B^ rows below them and its C^ rows above
// them in the chunk-kernel region (the staged forward's chunk kernels always write them).
// Decided from the descriptor alone, so the forward that writes them and the backward that
// reads them agree.
size_t fp32_layer_hs_bytes(const m3_layer_desc& d) {
    const int qb = chunked_chunk_tokens(d.mimo_rank, d.use_trapezoidal != 0);
    if (qb <= 0) return 0;
    const size_t K = (d.seqlen + qb - 1) / qb;
    return (size_t)d.batch * (K + 1) * d.nheads * d.headdim * d.d_state * sizeof(float);
}
bool fp32_layer_hs_ok(const m3_layer_desc& d) {
    const bool trap = d.use_trapezoidal != 0;
    const size_t hs = chunked_fwd_hs_offset(d.batch, d.seqlen, d.nheads, d.headdim, d.d_state,
                                            d.mimo_rank, trap);
    const size_t region = chunked_fwd_mfma_workspace(d.batch, d.seqlen, d.nheads, d.headdim,
                                                     d.d_state, d.mimo_rank, trap);
    const size_t rows = (size_t)d.batch * d.seqlen * d.ngroups * d.d_state * d.mimo_rank * sizeof(float);
    const size_t hsb = fp32_layer_hs_bytes(d);
    return hs > 0 && hsb > 0 && rows <= hs && hs + lp::al(hsb) + rows <= region;
}

void* fp32_layer_scratch(const m3_layer_desc& d, void* ws, size_t* bytes) {
    const lp::Plan pl = lp::plan(d);
    *bytes = pl.total - pl.chunk_off;
    return ws ? reinterpret_cast<char*>(ws) + pl.chunk_off : nullptr;
}

bool fp32_layer_supported(const m3_layer_desc& d) {
    return d.dtype == M3_DTYPE_F32 && prep_heads_per_tile(d) > 0 &&
           chunked_fwd_mfma_workspace(d.batch, d.seqlen, d.nheads, d.headdim, d.d_state,
                                      d.mimo_rank, d.use_trapezoidal != 0) > 0;
}

size_t fp32_layer_workspace(const m3_layer_desc& d) {
    return fp32_layer_supported(d) ? lp::plan(d).total : 0;
}

int launch_fp32_layer(const m3_layer_desc& d, const m3_layer_params& p, const void* proj,
                      const float* dt_scale, void* y_out, float* h_final, float* angle,
                      float* prev_bx, void* workspace, hipStream_t stream) {
    using namespace lp;
    const Plan pl = plan(d);
    char* ws = reinterpret_cast<char*>(workspace);
    auto part = [&](int i) { return reinterpret_cast<float*>(ws + pl.off[i]); };
    Args a;
    a.B = d.batch, a.T = d.seqlen, a.H = d.nheads, a.P = d.headdim, a.N = d.d_state;
    a.R = d.mimo_rank, a.G = d.ngroups, a.trap = d.use_trapezoidal, a.cplx = d.use_complex;
    a.rs = d.proj_row_stride, a.pl = proj_layout(d), a.eps = d.rms_eps, a.prm = p;
    a.HT = prep_heads_per_tile(d);
    a.proj = reinterpret_cast<const float*>(proj);
    a.dt_scale = dt_scale;
    a.dt = part(0), a.A = part(1), a.phi = part(2), a.xg = part(3);
    a.xb = a.trap ? part(4) : nullptr;
    a.xr = part(5), a.Bt = part(6), a.Bb = a.trap ? part(7) : nullptr, a.Ct = part(8);
    a.ys = part(9), a.phi_sum = part(10);
    a.y = reinterpret_cast<float*>(y_out), a.h_final = h_final, a.angle = angle;
    a.prev_bx = prev_bx;
    const size_t lds = prep_lds(d);
    if (a.HT <= 0 || lds > kPrepLds) return 1;
    const int64_t nbth = (int64_t)d.batch * d.seqlen * d.nheads;
    hipLaunchKernelGGL(lp_dt, dim3((unsigned)((std::max<int64_t>(nbth, d.nheads) + NTH - 1) / NTH)),
                       dim3(NTH), 0, stream, a);
    if (a.cplx) {
        const int64_t na = (int64_t)d.batch * ((d.seqlen + kAC - 1) / kAC) * d.nheads * (d.d_state / 2);
        const unsigned ga = (unsigned)((na + NTH - 1) / NTH);
        hipLaunchKernelGGL(lp_angle_sums, dim3(ga), dim3(NTH), 0, stream, a);
        hipLaunchKernelGGL(lp_angles, dim3(ga), dim3(NTH), 0, stream, a);
    }
    hipLaunchKernelGGL(lp_prep, dim3(d.batch * d.seqlen), dim3(NTH), lds, stream, a);
    if (launch_chunked_fwd_mfma(a.B, a.T, a.H, a.P, a.N, a.R, a.xg, a.xb, a.Bt, a.Bb, a.Ct, a.dt,
                                a.A, p.D, a.xr, nullptr, a.ys, h_final, ws + pl.chunk_off,
                                stream) != 0)
        return 1;
    const int64_t n = (int64_t)d.batch * d.seqlen * d.nheads * d.headdim;
    const unsigned grid = (unsigned)std::min<int64_t>((n + NTH - 1) / NTH, 65536);
    hipLaunchKernelGGL(lp_gate, dim3(grid), dim3(NTH), 0, stream, a);
    if (angle || prev_bx) hipLaunchKernelGGL(lp_state, dim3(d.batch * d.nheads), dim3(NTH), 0, stream, a);
    return hipGetLastError() == hipSuccess ? 0 : 1;
}

}  // namespace m3
