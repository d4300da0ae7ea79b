// Backward of the O(1) decode step (gfx950): the gradients of KulaMamba.step between in_proj
// and out_proj (mamba3/mamba3.py:267-322 with _process_BC_step :170-190) with respect to the
// in_proj row, the incoming state (h, prev_BX, angle), the layer's small parameters and
// dt_scale, given the gradients of the gated output y and of the new state. The reference
// differentiates this region with ATen's autograd; fp32 arithmetic here.
//
// Forward, per batch row b and head h (group g), recomputed from the inputs:
//   dt = softplus(u) s, u = dt_raw + dt_bias (threshold 20), A = -exp(A_log), dA = exp(A dt)
//   B^ = B r_B w_B + bias_B[g] (r_B = rsqrt(mean(B^2) + eps)), C^ likewise
//   ang' = ang - dt theta; B~, C~ = B^, C^ rotated pairwise by ang' (when RoPE is on)
//   x_r[p,r] = x[p] mimo_x[p,r];  lam = sigmoid(lam_raw), gam = lam dt, bet = (1-lam) dt dA
//   (trapezoid off: gam = dt, bet = 0)
//   cur[p,n] = sum_r B~[n,r] x_r[p,r];  h'[p,n] = dA h + gam cur + bet prev
//   y_r[p,r] = sum_n C~[n,r] h'[p,n] + D x_r[p,r];  y[p] = sum_r md[p,r] y_r silu(z mz[p,r])
//   new state (h', ang', cur).
// Backward (gy = dL/dy, gH = dL/dh', gA' = dL/dang', gP = dL/dprev_BX' = dL/dcur):
//   gyr = gy md silu(z mz);  G[p,n] = gH + sum_r gyr C~[n,r];  dL/dh = dA G;  dL/dprev = bet G
//   gcur = gam G + gP;  gB~[n,r] = sum_p gcur x_r;  gC~[n,r] = sum_p gyr h';
//   gx_r = D gyr + sum_n gcur B~;  the scalars dL/d(dA, gam, bet) = sum G (h, cur, prev);
//   the rotation's adjoint gives dL/dB^, dL/dC^ and dL/dang'; the RMSNorm backward per
//   (b, g) over the heads of the group; every parameter gradient is a per-row partial summed
//   over the batch in row order (deterministic).
//
// Launches: sb_head (one 256-thread block per (b, h)), sb_group (one per (b, g)), sb_colsum
// (the batch sums of the parameter partials).
#include "m3_common.h"
#include "m3_kernels.h"

namespace m3 {
namespace sb {

constexpr int NTH = 256;
constexpr int RMAX = 8;

struct Args {
    int B, H, P, N, R, G, trap, cplx;
    int64_t rs;
    ProjLayout pl;
    float eps;
    m3_layer_params prm;
    const float* proj;      // [B][rs]
    const float* dt_scale;  // [B][H] or null
    const float* h;         // [B][H][P][N]
    const float* prev;
    const float* ang;       // [B][H][N/2]
    const float* gy;        // [B][H*P]
    const float* gH;        // [B][H][P][N] or null
    const float* gP;        // or null
    const float* gA;        // [B][H][N/2] or null
    float* g_proj;          // [B][rs] (the d_in_proj columns)
    float* g_h;             // [B][H][P][N]
    float* g_prev;
    float* g_ang;           // [B][H][N/2]
    float* g_dt_scale;      // [B][H] or null
    // partials (workspace)
    float *pBhat, *pChat;   // [B][H][N*R]
    float* pth;             // [B][H][N/2]
    float *pAlog, *pD, *pdtb;     // [B][H]
    float *pmx, *pmz, *pmd;       // [B][H][P][R]
    float *pBb, *pCb, *pBw, *pCw;  // [B][G][N*R]
};

__device__ __forceinline__ float block_sum(float v, float* red) {
    v = lane_sum<64>(v);
    const int w = threadIdx.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[w] = v;
    __syncthreads();
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < NTH / 64; ++i) s += red[i];
    return s;
}

// LDS of sb_head: B, C raw rows and rotated rows [N*R] each, cos / sin [N/2] each, x_r, gyr,
// gx_r, y_r [P*R] each, x, z [P] each, and a reduction scratch.
inline size_t head_lds(const m3_layer_desc& d) {
    const size_t NR = (size_t)d.d_state * d.mimo_rank, PR = (size_t)d.headdim * d.mimo_rank;
    return (4 * NR + (size_t)d.d_state + 4 * PR + 2 * (size_t)d.headdim + 8) * sizeof(float);
}
inline size_t group_lds(const m3_layer_desc& d) {
    return (3 * (size_t)d.d_state * d.mimo_rank + 8) * sizeof(float);
}

__global__ __launch_bounds__(NTH) void sb_head(Args a) {
    extern __shared__ float sm[];
    const int bh = blockIdx.x, b = bh / a.H, h = bh % a.H;
    const int g = h / (a.H / a.G);
    const int N = a.N, P = a.P, R = a.R, NR = N * R, NH = N / 2, PR = P * R;
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    float* sBr = sm;            // raw B of the group (n, r)
    float* sCr = sBr + NR;
    float* sBt = sCr + NR;      // rotated B~
    float* sCt = sBt + NR;
    float* scs = sCt + NR;      // cos / sin of the new angle per pair
    float* ssn = scs + NH;
    float* sxr = ssn + NH;      // x_r [p][r]
    float* sgy = sxr + PR;      // gyr
    float* sgx = sgy + PR;      // gx_r
    float* syr = sgx + PR;      // y_r
    float* sx = syr + PR;       // x [p]
    float* sz = sx + P;         // z [p]
    float* red = sz + P;        // 8 floats

    const float* row = a.proj + (int64_t)b * a.rs;
    const int64_t hp = (int64_t)h * P;
    // ---- per-head scalars (mamba3/mamba3.py:283-296)
    const float u = row[a.pl.dt + h] + a.prm.dt_bias[h];
    const float sp = u > 20.f ? u : log1pf(expf(u));
    const float sc = a.dt_scale ? a.dt_scale[(int64_t)b * a.H + h] : 1.f;
    const float dt = sp * sc;
    const float A = -expf(a.prm.A_log[h]);
    const float dA = expf(A * dt);
    const float lam = a.trap ? sigmoid_f(row[a.pl.lam + h]) : 1.f;
    const float gam = a.trap ? lam * dt : dt;
    const float bet = a.trap ? (1.f - lam) * dt * dA : 0.f;
    const float Dh = a.prm.D[h];

    // ---- B^ / C^ of the group, RMSNorm in fp32 (mamba3/mamba3.py:19-35, 174-178)
    float sb = 0.f, scc = 0.f;
    for (int e = tid; e < NR; e += NTH) {
        const float vb = row[a.pl.B + (int64_t)g * NR + e], vc = row[a.pl.C + (int64_t)g * NR + e];
        sBr[e] = vb;
        sCr[e] = vc;
        sb += vb * vb;
        scc += vc * vc;
    }
    sb = block_sum(sb, red);
    scc = block_sum(scc, red);
    const float rB = rsqrtf(sb / NR + a.eps), rC = rsqrtf(scc / NR + a.eps);
    // ---- new angle and the rotation (mamba3/mamba3.py:181-189, 38-45)
    for (int i = tid; i < NH; i += NTH) {
        float c = 1.f, s = 0.f;
        if (a.cplx) {
            const float an = a.ang[(int64_t)bh * NH + i] - dt * row[a.pl.theta + i];
            sincosf(an, &s, &c);
        }
        scs[i] = c;
        ssn[i] = s;
    }
    __syncthreads();
    for (int e = tid; e < NR; e += NTH) {
        const int n = e / R, r = e % R, i = n >> 1;
        const int ev = (2 * i) * R + r, od = ev + R;
        const float be = sBr[ev] * rB * a.prm.B_norm_w[ev] + a.prm.B_bias[(int64_t)g * NR + ev];
        const float bo = sBr[od] * rB * a.prm.B_norm_w[od] + a.prm.B_bias[(int64_t)g * NR + od];
        const float ce = sCr[ev] * rC * a.prm.C_norm_w[ev] + a.prm.C_bias[(int64_t)g * NR + ev];
        const float co = sCr[od] * rC * a.prm.C_norm_w[od] + a.prm.C_bias[(int64_t)g * NR + od];
        const float c = scs[i], s = ssn[i];
        sBt[e] = (n & 1) ? be * s + bo * c : be * c - bo * s;
        sCt[e] = (n & 1) ? ce * s + co * c : ce * c - co * s;
    }
    // ---- x_r, z and gyr = gy md silu(z mz)
    float gD = 0.f;
    for (int e = tid; e < PR; e += NTH) {
        const int p = e / R;
        const float xv = row[a.pl.x + hp + p], zv = row[a.pl.z + hp + p];
        const int64_t pe = (hp * R) + e;
        const float xr = xv * a.prm.mimo_x[pe];
        sxr[e] = xr;
        const float az = zv * a.prm.mimo_z[pe];
        const float gyr = a.gy[(int64_t)b * a.H * P + hp + p] * a.prm.mimo_down[pe] * silu_f(az);
        sgy[e] = gyr;
        gD += gyr * xr;
        if (e % R == 0) {
            sx[p] = xv;
            sz[p] = zv;
        }
    }
    gD = block_sum(gD, red);  // (its barriers also publish the tiles above)

    const int64_t st0 = (int64_t)bh * P * N;
    // ---- pass A: a wave per row p, lanes over n: y_r and gx_r (row sums over n), dL/dh and
    // dL/dprev
    for (int p = wv; p < P; p += NTH / 64) {
        float yp[RMAX], gxp[RMAX];
#pragma unroll
        for (int r = 0; r < RMAX; ++r) yp[r] = gxp[r] = 0.f;
        for (int n = lane; n < N; n += 64) {
            const int64_t o = st0 + (int64_t)p * N + n;
            const float h0 = a.h[o], pv = a.prev[o];
            const float gh = a.gH ? a.gH[o] : 0.f, gp = a.gP ? a.gP[o] : 0.f;
            float cur = 0.f, G = gh;
            for (int r = 0; r < R; ++r) {
                cur += sBt[n * R + r] * sxr[p * R + r];
                G += sgy[p * R + r] * sCt[n * R + r];
            }
            const float h1 = dA * h0 + gam * cur + bet * pv;
            a.g_h[o] = dA * G;
            a.g_prev[o] = bet * G;
            const float gc = gam * G + gp;
#pragma unroll
            for (int r = 0; r < RMAX; ++r)
                if (r < R) {
                    yp[r] += sCt[n * R + r] * h1;
                    gxp[r] += gc * sBt[n * R + r];
                }
        }
#pragma unroll
        for (int r = 0; r < RMAX; ++r)
            if (r < R) {
                const float ys = lane_sum<64>(yp[r]), gs = lane_sum<64>(gxp[r]);
                if (lane == 0) {
                    syr[p * R + r] = ys + Dh * sxr[p * R + r];
                    sgx[p * R + r] = gs + Dh * sgy[p * R + r];
                }
            }
    }
    __syncthreads();
    // ---- gate and x backward per p: dL/dz, dL/dx, partials of mimo_down / mimo_z / mimo_x
    for (int p = tid; p < P; p += NTH) {
        const float zv = sz[p], xv = sx[p], gyv = a.gy[(int64_t)b * a.H * P + hp + p];
        float gz = 0.f, gx = 0.f;
        for (int r = 0; r < R; ++r) {
            const int64_t pe = (hp + p) * R + r;
            const float mz = a.prm.mimo_z[pe], md = a.prm.mimo_down[pe];
            const float az = zv * mz, sg = sigmoid_f(az);
            const float yr = syr[p * R + r];
            const float ga = gyv * md * yr * sg * (1.f + az * (1.f - sg));  // dL/d(z mz)
            gz += ga * mz;
            const int64_t pp = (int64_t)b * a.H * P * R + pe;
            a.pmd[pp] = gyv * yr * az * sg;
            a.pmz[pp] = ga * zv;
            a.pmx[pp] = sgx[p * R + r] * xv;
            gx += sgx[p * R + r] * a.prm.mimo_x[pe];
        }
        a.g_proj[(int64_t)b * a.rs + a.pl.z + hp + p] = gz;
        a.g_proj[(int64_t)b * a.rs + a.pl.x + hp + p] = gx;
    }
    // ---- pass B: a thread per column n, rows p in order: dL/dB~, dL/dC~ and the scalar sums
    float gdA = 0.f, ggam = 0.f, gbet = 0.f;
    float gbt[2][RMAX], gct[2][RMAX];
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int r = 0; r < RMAX; ++r) gbt[j][r] = gct[j][r] = 0.f;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int n = tid + NTH * j;
        if (n < N) {
            for (int p = 0; p < P; ++p) {
                const int64_t o = st0 + (int64_t)p * N + n;
                const float h0 = a.h[o], pv = a.prev[o];
                const float gh = a.gH ? a.gH[o] : 0.f, gp = a.gP ? a.gP[o] : 0.f;
                float cur = 0.f, G = gh;
                for (int r = 0; r < R; ++r) {
                    cur += sBt[n * R + r] * sxr[p * R + r];
                    G += sgy[p * R + r] * sCt[n * R + r];
                }
                const float h1 = dA * h0 + gam * cur + bet * pv;
                const float gc = gam * G + gp;
                gdA += G * h0;
                ggam += G * cur;
                gbet += G * pv;
#pragma unroll
                for (int r = 0; r < RMAX; ++r)
                    if (r < R) {
                        gbt[j][r] += gc * sxr[p * R + r];
                        gct[j][r] += sgy[p * R + r] * h1;
                    }
            }
        }
    }
    __syncthreads();
    // rotated-row gradients over the raw rows' LDS (no longer read)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int n = tid + NTH * j;
        if (n < N)
#pragma unroll
            for (int r = 0; r < RMAX; ++r)
                if (r < R) {
                    sBr[n * R + r] = gbt[j][r];
                    sCr[n * R + r] = gct[j][r];
                }
    }
    gdA = block_sum(gdA, red);
    ggam = block_sum(ggam, red);
    gbet = block_sum(gbet, red);
    // ---- the rotation's adjoint, a thread per pair: dL/dB^, dL/dC^, dL/dang
    float gdt_ang = 0.f;
    const int64_t hb = (int64_t)bh * NR;
    for (int i = tid; i < NH; i += NTH) {
        const float c = scs[i], s = ssn[i];
        // without RoPE the angle passes through unchanged (c = 1, s = 0 above)
        float gang = a.gA ? a.gA[(int64_t)bh * NH + i] : 0.f;
        for (int r = 0; r < R; ++r) {
            const int ev = (2 * i) * R + r, od = ev + R;
            const float gbe = sBr[ev], gbo = sBr[od], gce = sCr[ev], gco = sCr[od];
            if (a.cplx) gang += gbo * sBt[ev] - gbe * sBt[od] + gco * sCt[ev] - gce * sCt[od];
            a.pBhat[hb + ev] = gbe * c + gbo * s;
            a.pBhat[hb + od] = gbo * c - gbe * s;
            a.pChat[hb + ev] = gce * c + gco * s;
            a.pChat[hb + od] = gco * c - gce * s;
        }
        a.g_ang[(int64_t)bh * NH + i] = gang;
        if (a.cplx) {
            const float th = row[a.pl.theta + i];
            a.pth[(int64_t)bh * NH + i] = -dt * gang;
            gdt_ang -= gang * th;
        }
    }
    gdt_ang = block_sum(gdt_ang, red);
    // ---- per-head scalars (mamba3/mamba3.py:283-296)
    if (tid == 0) {
        float gdA_t = gdA, gdt = gdt_ang;
        if (a.trap) {
            const float glam = ggam * dt - gbet * dt * dA;
            gdA_t += gbet * (1.f - lam) * dt;
            gdt += ggam * lam + gbet * (1.f - lam) * dA;
            a.g_proj[(int64_t)b * a.rs + a.pl.lam + h] = glam * lam * (1.f - lam);
        } else {
            gdt += ggam;
        }
        gdt += gdA_t * A * dA;
        const float gsp = gdt * sc;
        if (a.g_dt_scale) a.g_dt_scale[(int64_t)b * a.H + h] = gdt * sp;
        const float gu = u > 20.f ? gsp : gsp * sigmoid_f(u);
        a.g_proj[(int64_t)b * a.rs + a.pl.dt + h] = gu;
        a.pdtb[bh] = gu;
        a.pAlog[bh] = gdA_t * dt * dA * A;  // dA/dA_log = dt dA A
        a.pD[bh] = gD;
    }
}

// One block per (b, g): dL/dB^ and dL/dC^ summed over the group's heads, the RMSNorm
// backward into dL/dB, dL/dC (in_proj columns), partials of the norm weights and biases; the
// g = 0 block also sums dL/dtheta over the heads.
__global__ __launch_bounds__(NTH) void sb_group(Args a) {
    extern __shared__ float sm[];
    const int bg = blockIdx.x, b = bg / a.G, g = bg % a.G;
    const int NR = a.N * a.R, hpg = a.H / a.G, NH = a.N / 2;
    const int tid = threadIdx.x;
    float* sx = sm;          // raw row
    float* sgv = sx + NR;    // summed dL/dB^
    float* red = sgv + 2 * NR;
    const float* row = a.proj + (int64_t)b * a.rs;
    for (int which = 0; which < 2; ++which) {
        const int64_t off = (which == 0 ? a.pl.B : a.pl.C) + (int64_t)g * NR;
        const float* w = which == 0 ? a.prm.B_norm_w : a.prm.C_norm_w;
        const float* part = which == 0 ? a.pBhat : a.pChat;
        float* pbias = which == 0 ? a.pBb : a.pCb;
        float* pw = which == 0 ? a.pBw : a.pCw;
        float ss = 0.f, q = 0.f;
        for (int e = tid; e < NR; e += NTH) {
            const float xv = row[off + e];
            float gs = 0.f;
            for (int k = 0; k < hpg; ++k) gs += part[((int64_t)b * a.H + g * hpg + k) * NR + e];
            sx[e] = xv;
            sgv[e] = gs;
            ss += xv * xv;
            q += gs * w[e] * xv;
        }
        ss = block_sum(ss, red);
        q = block_sum(q, red);
        const float r = rsqrtf(ss / NR + a.eps);
        const int64_t pb = (int64_t)bg * NR;
        for (int e = tid; e < NR; e += NTH) {
            const float xv = sx[e], gs = sgv[e];
            pbias[pb + e] = gs;
            pw[pb + e] = gs * xv * r;
            a.g_proj[(int64_t)b * a.rs + off + e] = r * gs * w[e] - xv * r * r * r * q / NR;
        }
        __syncthreads();
    }
    if (g == 0 && a.cplx)
        for (int i = tid; i < NH; i += NTH) {
            float s = 0.f;
            for (int k = 0; k < a.H; ++k) s += a.pth[((int64_t)b * a.H + k) * NH + i];
            a.g_proj[(int64_t)b * a.rs + a.pl.theta + i] = s;
        }
}

// out[m] = sum over rows k < K of in[k M + m], rows in order.
__global__ __launch_bounds__(NTH) void sb_colsum(const float* in, float* out, int64_t M, int64_t K) {
    const int64_t m = (int64_t)blockIdx.x * NTH + threadIdx.x;
    if (m >= M) return;
    float s = 0.f;
    for (int64_t k = 0; k < K; ++k) s += in[k * M + m];
    out[m] = s;
}

struct Plan {
    size_t off[13], total;
};

inline size_t al(size_t x) { return (x + 255) & ~(size_t)255; }

Plan plan(const m3_layer_desc& d) {
    const size_t B = d.batch, H = d.nheads, G = d.ngroups;
    const size_t NR = (size_t)d.d_state * d.mimo_rank, PR = (size_t)d.headdim * d.mimo_rank;
    const size_t sizes[13] = {B * H * NR, B * H * NR, B * H * (d.d_state / 2), B * H, B * H, B * H,
                              B * H * PR, B * H * PR, B * H * PR, B * G * NR, B * G * NR,
                              B * G * NR, B * G * NR};
    Plan p;
    size_t o = 0;
    for (int i = 0; i < 13; ++i) {
        p.off[i] = o;
        o += al(sizes[i] * sizeof(float));
    }
    p.total = o;
    return p;
}

}  // namespace sb

// Both kernels' LDS stays within gfx950's 160 KB per workgroup for every shape the API takes
// (sb_head at most 100 KB: d_state 512, headdim 256, rank 8); above 64 KB a kernel's dynamic
// LDS limit is raised before its launch.
constexpr size_t kStepBwdMaxLds = 160 * 1024;

bool step_bwd_supported(const m3_layer_desc& d) {
    return d.d_state % 2 == 0 && d.d_state <= 2 * sb::NTH && d.mimo_rank >= 1 &&
           d.mimo_rank <= sb::RMAX && sb::head_lds(d) <= kStepBwdMaxLds &&
           sb::group_lds(d) <= kStepBwdMaxLds;
}

size_t step_bwd_workspace(const m3_layer_desc& d) {
    return step_bwd_supported(d) ? sb::plan(d).total : 0;
}

int launch_step_bwd(const m3_layer_desc& d, const m3_layer_params& p, const float* proj,
                    const float* dt_scale, const float* h, const float* prev, const float* ang,
                    const float* gy, const float* gH, const float* gP, const float* gA,
                    float* g_proj, float* g_h, float* g_prev, float* g_ang,
                    const m3_layer_param_grads& out, void* workspace, hipStream_t stream) {
    using namespace sb;
    const Plan pl = plan(d);
    char* ws = reinterpret_cast<char*>(workspace);
    auto part = [&](int i) { return reinterpret_cast<float*>(ws + pl.off[i]); };
    Args a;
    a.B = d.batch, a.H = d.nheads, a.P = d.headdim, a.N = d.d_state, a.R = d.mimo_rank;
    a.G = d.ngroups, a.trap = d.use_trapezoidal, a.cplx = d.use_complex;
    a.rs = d.proj_row_stride, a.pl = proj_layout(d), a.eps = d.rms_eps, a.prm = p;
    a.proj = proj, a.dt_scale = dt_scale, a.h = h, a.prev = prev, a.ang = ang;
    a.gy = gy, a.gH = gH, a.gP = gP, a.gA = gA;
    a.g_proj = g_proj, a.g_h = g_h, a.g_prev = g_prev, a.g_ang = g_ang;
    a.g_dt_scale = out.dt_scale;
    a.pBhat = part(0), a.pChat = part(1), a.pth = part(2), a.pAlog = part(3), a.pD = part(4);
    a.pdtb = part(5), a.pmx = part(6), a.pmz = part(7), a.pmd = part(8);
    a.pBb = part(9), a.pCb = part(10), a.pBw = part(11), a.pCw = part(12);
    auto raise_lds = [](const void* f, size_t lds) {
        return lds <= 64 * 1024 ||
               hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) == hipSuccess;
    };
    if (!raise_lds(reinterpret_cast<const void*>(&sb_head), head_lds(d)) ||
        !raise_lds(reinterpret_cast<const void*>(&sb_group), group_lds(d)))
        return 1;
    hipLaunchKernelGGL(sb_head, dim3((unsigned)(d.batch * d.nheads)), dim3(NTH), head_lds(d), stream, a);
    hipLaunchKernelGGL(sb_group, dim3((unsigned)(d.batch * d.ngroups)), dim3(NTH), group_lds(d), stream, a);
    const int64_t B = d.batch, H = d.nheads, G = d.ngroups;
    const int64_t NR = (int64_t)d.d_state * d.mimo_rank, PR = (int64_t)d.headdim * d.mimo_rank;
    auto colsum = [&](const float* in, float* o, int64_t M, int64_t K) {
        hipLaunchKernelGGL(sb_colsum, dim3((unsigned)((M + NTH - 1) / NTH)), dim3(NTH), 0, stream, in, o, M, K);
    };
    colsum(a.pAlog, out.A_log, H, B);
    colsum(a.pD, out.D, H, B);
    colsum(a.pdtb, out.dt_bias, H, B);
    colsum(a.pmx, out.mimo_x, H * PR, B);
    colsum(a.pmz, out.mimo_z, H * PR, B);
    colsum(a.pmd, out.mimo_down, H * PR, B);
    colsum(a.pBb, out.B_bias, G * NR, B);
    colsum(a.pCb, out.C_bias, G * NR, B);
    colsum(a.pBw, out.B_norm_w, NR, B * G);
    colsum(a.pCw, out.C_norm_w, NR, B * G);
    return hipGetLastError() == hipSuccess ? 0 : 1;
}

}  // namespace m3
