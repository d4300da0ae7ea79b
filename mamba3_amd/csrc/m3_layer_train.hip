// Backward of the fp32 layer prefill (m3_layer_fp32.hip): from dL/d(gated output) (and
// optionally dL/dh, dL/dangle, dL/dprev_BX of the prefill state) to dL/d(in_proj output) and
// the gradients of the small parameters. Replaces, under autograd, the reference's backward
// of mamba3/mamba3.py:197-256 (ATen's backward of softplus, RMSNorm, the RoPE rotation and
// its cumsum, the trapezoid terms, SiLU and the MIMO sums) around chunked_ssd, whose backward
// is m3_ssd_bwd.hip.
//
// Forward (per batch b, token t, head h, group g of h), restated from m3_layer_fp32.hip:
//   dt = softplus(u) s, u = dt_raw + dt_bias, s = dt_scale or 1;  A = -exp(A_log)
//   phi_t[i] = -sum_{t'<=t} dt_t' theta_t'[i]
//   B^[g] = v rho w + bias (v the raw B row of g, rho = rsqrt(mean(v^2) + eps))
//   B~[h] = rot(B^[g], phi[h]): e' = e cos - o sin, o' = e sin + o cos per pair (2i, 2i+1)
//   B_b[t] = B~[t-1];  x_r = x mimo_x;  lambda = sigmoid(lam_raw);  dA = exp(A dt)
//   x_g = lambda x_r;  x_b[t] = (1 - lambda_t) dA_t x_r[t-1]
//   y = chunked_ssd(x_g, x_b, B~, B_b, C~, dt, A, D, x_r)
//   out = sum_r mimo_down y silu(z mimo_z);  angle = phi_{T-1};  prev_BX = B~_{T-1} x_r,{T-1}^T
// Backward, in kernel order:
//   tb_gate   dL/dy, dL/dz and the per-block partials of dL/dmimo_down, dL/dmimo_z
//   (chunked SSD backward: dL/d of x_g, x_b, B~, B_b, C~, dt, A, D, x_r)
//   tb_x      dL/dx_r = g_xr + lambda g_xg + (1 - lambda_{t+1}) dA_{t+1} g_xb[t+1] (+ prev_BX),
//             dL/dx, dL/dlam_raw, the dt and A terms of dA, partials of dL/dmimo_x
//   tb_bc     dL/dB~ (+ g_Bb[t+1], + prev_BX), rotated back (by -phi) and summed over the heads
//             of the group, dL/dphi = sum_r (g_o' e' - g_e' o') over B and C, the RMSNorm
//             backward g_v = rho w g - v rho^3 sum(w g v) / (N R), partials of dL/dw, dL/dbias
//   tb_asum, tb_angle   Phi_t = sum_{t'>=t} dL/dphi_t' (+ dL/dangle), in chunks of 64 tokens
//   tb_tok    dL/dtheta_t = -sum_h dt Phi_t, dL/du = s sigmoid(u) (g_dt + -sum_i theta Phi),
//             dL/ds = softplus(u) (g_dt + -sum_i theta Phi) when dt_scale is differentiated
//   tb_colsum, tb_finish   the parameter gradients from the partials, in a fixed order
// Every reduction runs in a fixed order: results are deterministic.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <initializer_list>

#include "m3_common.h"
#include "m3_kernels.h"

namespace m3 {
namespace tb {

typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int NTH = 256;
constexpr int kW = 64;   // wavefront size

// Sum over the 64 lanes of a wave (butterfly: every lane gets the same result).
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int off = kW / 2; off > 0; off >>= 1) v += __shfl_xor(v, off, kW);
    return v;
}
constexpr int TBK = 64;  // tokens per block of tb_gate / tb_x
constexpr int TBC = 4;   // tokens per block of tb_bc
constexpr int kAC = 64;  // tokens per chunk of the angle suffix scan

struct Args {
    int B, T, H, P, N, R, G, trap, cplx;
    // With the trapezoid: tokens per chunk of the chunked backward and chunks per sequence.
    // gBt then holds dL/dB~ from both B factors except the b part of each chunk's first token,
    // which gBb holds as (B, K, H, N, R) rows (it belongs to the previous chunk's last token).
    int qb, nk;
    int64_t rs;
    ProjLayout pl;
    float eps;
    m3_layer_params prm;
    const float* proj;
    const float* dt_scale;
    Fp32LayerParts f;
    const float *gout, *gh, *gang, *gprev;
    float* gproj;
    m3_layer_param_grads out;
    // workspace
    float *gys, *gxg, *gxb, *gxr, *gBt, *gBb, *gCt, *gdtc, *gAc, *gD, *gdtx, *gphi, *Phi,
        *Phi_sum, *gA_part, *p_md, *p_mz, *p_mx, *p_Bw, *p_Cw, *p_Bb, *p_Cb, *p_dtb;
};

__device__ __forceinline__ float sigm(float v) { return 1.f / (1.f + expf(-v)); }

// The R values of one (token, head, column) of a (B,T,H,X,R) workspace array are contiguous and
// 4R-byte aligned: 16-byte accesses when R % 4 == 0, 8-byte ones when R is
// even, else one per value.
template <int R>
__device__ __forceinline__ void ldr(const float* p, float (&v)[R]) {
    if constexpr (R % 4 == 0) {
#pragma unroll
        for (int j = 0; j < R / 4; ++j) {
            const f32x4 q = *reinterpret_cast<const f32x4*>(p + 4 * j);
#pragma unroll
            for (int k = 0; k < 4; ++k) v[4 * j + k] = q[k];
        }
    } else if constexpr (R % 2 == 0) {
#pragma unroll
        for (int j = 0; j < R / 2; ++j) {
            const f32x2 q = *reinterpret_cast<const f32x2*>(p + 2 * j);
            v[2 * j] = q[0];
            v[2 * j + 1] = q[1];
        }
    } else {
#pragma unroll
        for (int j = 0; j < R; ++j) v[j] = p[j];
    }
}
template <int R>
__device__ __forceinline__ void str(float* p, const float (&v)[R]) {
    if constexpr (R % 4 == 0) {
#pragma unroll
        for (int j = 0; j < R / 4; ++j)
            *reinterpret_cast<f32x4*>(p + 4 * j) = f32x4{v[4 * j], v[4 * j + 1], v[4 * j + 2], v[4 * j + 3]};
    } else if constexpr (R % 2 == 0) {
#pragma unroll
        for (int j = 0; j < R / 2; ++j) *reinterpret_cast<f32x2*>(p + 2 * j) = f32x2{v[2 * j], v[2 * j + 1]};
    } else {
#pragma unroll
        for (int j = 0; j < R; ++j) p[j] = v[j];
    }
}

// Sum over the block (blockDim.x a power of two, at most NTH), in a fixed order.
__device__ float block_sum(float v, float* red) {
    const int tid = threadIdx.x;
    red[tid] = v;
    __syncthreads();
    for (int w = blockDim.x / 2; w > 0; w >>= 1) {
        if (tid < w) red[tid] += red[tid + w];
        __syncthreads();
    }
    const float s = red[0];
    __syncthreads();
    return s;
}

// ---- gate: one block per (b, token block, h) of NTH threads = slots of PT threads (PT = P
// rounded up to a power of two), slot s handling tokens t0 + s, t0 + s + slots, ...; the
// slots' parameter partials are added in order.
template <int R>
__global__ __launch_bounds__(NTH) void tb_gate(Args a) {
    __shared__ float red[2][NTH];
    const int nTB = (a.T + TBK - 1) / TBK;
    const int h = blockIdx.x % a.H, tb = (blockIdx.x / a.H) % nTB, b = blockIdx.x / (a.H * nTB);
    int PT = 64;
    while (PT < a.P) PT *= 2;
    const int slots = NTH / PT;
    const int tid = threadIdx.x, slot = tid / PT, p = tid % PT;
    const bool col = p < a.P;
    const int64_t HP = (int64_t)a.H * a.P;
    float pmd[R], pmz[R], mz[R], md[R];
#pragma unroll
    for (int r = 0; r < R; ++r) pmd[r] = pmz[r] = 0.f;
    const int t1 = min(a.T, (tb + 1) * TBK);
    if (col) {
        // parameters (caller pointers of any alignment): read once per thread
#pragma unroll
        for (int r = 0; r < R; ++r) {
            mz[r] = a.prm.mimo_z[((int64_t)h * a.P + p) * R + r];
            md[r] = a.prm.mimo_down[((int64_t)h * a.P + p) * R + r];
        }
        for (int t = tb * TBK + slot; t < t1; t += slots) {
            const int64_t tok = (int64_t)b * a.T + t;
            const float z = a.proj[tok * a.rs + a.pl.z + (int64_t)h * a.P + p];
            const float g = a.gout[tok * HP + (int64_t)h * a.P + p];
            const int64_t yb = (tok * a.H + h) * a.P * R + (int64_t)p * R;
            float y[R], gy[R];
            ldr<R>(a.f.ys + yb, y);
            float gz = 0.f;
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const float zz = z * mz[r], sg = sigm(zz), silu = zz * sg, ds = sg * (1.f + zz * (1.f - sg));
                gy[r] = g * md[r] * silu;
                gz += g * md[r] * y[r] * ds * mz[r];
                pmd[r] += g * y[r] * silu;
                pmz[r] += g * md[r] * y[r] * ds * z;
            }
            str<R>(a.gys + yb, gy);
            a.gproj[tok * a.rs + a.pl.z + (int64_t)h * a.P + p] = gz;
        }
    }
    const int64_t o = (((int64_t)b * nTB + tb) * HP + (int64_t)h * a.P + p) * R;
#pragma unroll
    for (int r = 0; r < R; ++r) {
        __syncthreads();
        red[0][tid] = pmd[r];
        red[1][tid] = pmz[r];
        __syncthreads();
        if (slot == 0 && col) {
            float sd = 0.f, sz = 0.f;
            for (int k = 0; k < slots; ++k) {
                sd += red[0][k * PT + p];
                sz += red[1][k * PT + p];
            }
            a.p_md[o + r] = sd;
            a.p_mz[o + r] = sz;
        }
    }
}

// ---- x terms: one block per (b, token block, h) of NTH threads = slots of PT threads (PT = P
// rounded up to a power of two): slot s handles tokens t0 + s, t0 + s + slots, ...; the
// per-token sums over p are segmented block sums; the slots' partials are added in order.
template <int R>
__global__ __launch_bounds__(NTH) void tb_x(Args a) {
    __shared__ float red[2][NTH];
    __shared__ float part[NTH / 64];  // per slot: dL/dA
    const int nTB = (a.T + TBK - 1) / TBK;
    const int h = blockIdx.x % a.H, tb = (blockIdx.x / a.H) % nTB, b = blockIdx.x / (a.H * nTB);
    int PT = 64;
    while (PT < a.P) PT *= 2;
    const int slots = NTH / PT;
    const int tid = threadIdx.x, slot = tid / PT, p = tid % PT;
    const bool col = p < a.P;
    const int PR = a.P * R;
    const float Ah = a.f.A[h];
    float pmx[R], mx[R];
#pragma unroll
    for (int r = 0; r < R; ++r) pmx[r] = 0.f;
#pragma unroll
    for (int r = 0; r < R; ++r) mx[r] = col ? a.prm.mimo_x[((int64_t)h * a.P + p) * R + r] : 0.f;
    float gA = 0.f;
    const int t0 = tb * TBK, t1 = min(a.T, (tb + 1) * TBK);
    const int rounds = (t1 - t0 + slots - 1) / slots;
    // One round's inputs, loaded a round ahead of their use (a one-deep software pipeline):
    // lambda and dt of the token and the next one (raw), x, and the gradient / x rows.
    struct In {
        float lr, dtv, lrn, dtn, x;
        float gxr[R], gxg[R], gxb[R], xrv[R], gxbn[R], xrp[R];
    };
    auto fetch = [&](int k, In& v) {
        const int t = t0 + k * slots + slot;
        const bool act = t < t1;
        const int64_t tok = (int64_t)b * a.T + (act ? t : t0);
        const int64_t th = tok * a.H + h;
        const float* row = a.proj + tok * a.rs;
        v.lr = v.dtv = v.lrn = v.dtn = v.x = 0.f;
        if (a.trap && act) {
            v.lr = row[a.pl.lam + h];
            v.dtv = a.f.dt[th];
            if (t + 1 < a.T) {
                v.lrn = row[a.rs + a.pl.lam + h];
                v.dtn = a.f.dt[th + a.H];
            }
        }
        if (col && act) {
            v.x = row[a.pl.x + (int64_t)h * a.P + p];
            const int64_t e0 = th * PR + (int64_t)p * R;
            ldr<R>(a.gxr + e0, v.gxr);
            ldr<R>(a.gxg + e0, v.gxg);
            if (a.trap) {
                ldr<R>(a.gxb + e0, v.gxb);
                ldr<R>(a.f.xr + e0, v.xrv);
                if (t + 1 < a.T) ldr<R>(a.gxb + e0 + (int64_t)a.H * PR, v.gxbn);  // next token's
                if (t > 0) ldr<R>(a.f.xr + e0 - (int64_t)a.H * PR, v.xrp);        // previous token's
            }
        }
    };
    In nxt;
    if (rounds > 0) fetch(0, nxt);
    for (int k = 0; k < rounds; ++k) {
        const In in = nxt;
        if (k + 1 < rounds) fetch(k + 1, nxt);
        const int t = t0 + k * slots + slot;
        const bool act = t < t1;
        const int64_t tok = (int64_t)b * a.T + (act ? t : t0);
        const int64_t th = tok * a.H + h;
        float lam = 1.f, dA = 1.f, lamn = 1.f, dAn = 1.f;
        if (a.trap && act) {
            lam = sigm(in.lr);
            dA = expf(Ah * in.dtv);
            if (t + 1 < a.T) {
                lamn = sigm(in.lrn);
                dAn = expf(Ah * in.dtn);
            }
        }
        float sl = 0.f, sa = 0.f;
        if (col && act) {
            const float x = in.x;
            const float(&gxr)[R] = in.gxr;
            const float(&gxg)[R] = in.gxg;
            const float(&gxb)[R] = in.gxb;
            const float(&xrv)[R] = in.xrv;
            const float(&gxbn)[R] = in.gxbn;
            const float(&xrp)[R] = in.xrp;
            float gx = 0.f;
#pragma unroll
            for (int r = 0; r < R; ++r) {
                float g = gxr[r] + (a.trap ? lam : 1.f) * gxg[r];
                if (a.trap && t + 1 < a.T) g += (1.f - lamn) * dAn * gxbn[r];
                if (t == a.T - 1 && a.gprev) {
                    const float* gp = a.gprev + (((int64_t)b * a.H + h) * a.P + p) * a.N;
                    const float* bt = a.f.Bt + th * a.N * R + r;
                    for (int n = 0; n < a.N; ++n) g += gp[n] * bt[(int64_t)n * R];
                }
                gx += g * mx[r];
                pmx[r] += g * x;
                if (a.trap) sl += gxg[r] * xrv[r];
            }
            if (a.trap && t > 0) {
#pragma unroll
                for (int r = 0; r < R; ++r) sa += gxb[r] * xrp[r];
            }
            a.gproj[tok * a.rs + a.pl.x + (int64_t)h * a.P + p] = gx;
        }
        if (a.trap) {
            // segmented sums over the PT threads of each slot: a butterfly within each wave
            // (a slot of 64 threads is one wave), then, for wider slots, the slot's waves
            // added in order through LDS
            float slt = wave_sum(sl), sat = wave_sum(sa);
            if (PT > kW) {
                const int nw = PT / kW;
                if ((tid & (kW - 1)) == 0) {
                    red[0][tid / kW] = slt;
                    red[1][tid / kW] = sat;
                }
                __syncthreads();
                slt = 0.f;
                sat = 0.f;
                for (int w = 0; w < nw; ++w) {
                    slt += red[0][slot * nw + w];
                    sat += red[1][slot * nw + w];
                }
                __syncthreads();
            }
            if (act) {
                const float glam = slt - sat * dA;   // dL/dlambda
                const float gdA = sat * (1.f - lam);  // dL/d(dA)
                if (p == 0) {
                    a.gproj[tok * a.rs + a.pl.lam + h] = glam * lam * (1.f - lam);
                    a.gdtx[th] = gdA * dA * Ah;
                }
                gA += gdA * dA * in.dtv;
            }
        } else if (act && p == 0) {
            a.gdtx[th] = 0.f;
        }
    }
    // the slots' mimo_x partials and dL/dA, added in slot order
    float* pm = &red[0][0];  // one rank at a time
#pragma unroll
    for (int r = 0; r < R; ++r) {
        __syncthreads();
        pm[tid] = pmx[r];
        __syncthreads();
        if (slot == 0 && col) {
            float s = 0.f;
            for (int k = 0; k < slots; ++k) s += pm[k * PT + p];
            const int64_t o = (((int64_t)b * nTB + tb) * a.H * a.P + (int64_t)h * a.P + p) * R;
            a.p_mx[o + r] = s;
        }
    }
    if (p == 0) part[slot] = gA;
    __syncthreads();
    if (tid == 0) {
        float s = 0.f;
        for (int k = 0; k < slots; ++k) s += part[k];
        a.gA_part[((int64_t)b * nTB + tb) * a.H + h] = s;
    }
}

// ---- B / C: one block per (b, TBC tokens), one group g at a time, token by token. Thread
// (pair i, head slot hg) handles the heads g hpg + hl, hl = hg (mod HS), of pair i and
// accumulates into its own LDS partial of the group's dL/dB^, dL/dC^; the HS partials are
// then summed in order. The rotated rows dL/dphi needs are formed again from the group's
// normalised B^ / C^ (kept in LDS) and the cos / sin, not read back. LDS: the partials,
// dL/dB^, dL/dC^, the parameter partials of the group, B^ / C^, the reduction scratch.
__device__ __forceinline__ int bc_hs(int N) { return max(1, NTH / (N / 2)); }

// The K = 2R values of pair i (even column, ranks 0..R-1, then odd column) are contiguous
// and 8R-byte aligned: 16-byte loads when R is even, else 8-byte ones.
template <int K>
__device__ __forceinline__ void ldv(const float* p, float (&v)[K]) {
    static_assert(K % 2 == 0, "pairs hold an even number of values");
    if constexpr (K % 4 == 0) {
#pragma unroll
        for (int j = 0; j < K / 4; ++j) {
            const f32x4 q = *reinterpret_cast<const f32x4*>(p + 4 * j);
#pragma unroll
            for (int k = 0; k < 4; ++k) v[4 * j + k] = q[k];
        }
    } else {
#pragma unroll
        for (int j = 0; j < K / 2; ++j) {
            const f32x2 q = *reinterpret_cast<const f32x2*>(p + 2 * j);
            v[2 * j] = q[0];
            v[2 * j + 1] = q[1];
        }
    }
}

template <int R>
__global__ __launch_bounds__(NTH) void tb_bc(Args a) {
    extern __shared__ float sm[];
    const int NR = a.N * R, GNR = a.G * NR, NH = a.N / 2, hpg = a.H / a.G;
    const int HS = bc_hs(a.N);
    float* qB = sm;                 // [HS][NR]
    float* qC = qB + HS * NR;       // [HS][NR]
    float* nx = qC + HS * NR;
    float* gBh = HS > 1 ? nx : qB;  // with one head slot its partial is the sum
    float* gCh = HS > 1 ? nx + NR : qC;
    float* pBw = nx + (HS > 1 ? 2 * NR : 0);
    float* pCw = pBw + NR;
    float* pBb = pCw + NR;
    float* pCb = pBb + NR;
    float* Bh = pCb + NR;           // the token's normalised B^ / C^ of group g
    float* Ch = Bh + NR;
    float* red = Ch + NR;
    const int nTB = (a.T + TBC - 1) / TBC;
    const int tb = blockIdx.x % nTB, b = blockIdx.x / nTB;
    const int64_t ob = (int64_t)blockIdx.x;
    const int tid = threadIdx.x;
    const int hg = tid / NH < HS ? tid / NH : hpg;  // hpg: no heads for this thread
    const int i0 = tid % NH;
    for (int e = tid; e < NR; e += NTH) pBw[e] = pCw[e] = 0.f;
    const int t1 = min(a.T, (tb + 1) * TBC);
    for (int g = 0; g < a.G; ++g) {
        for (int e = tid; e < NR; e += NTH) pBb[e] = pCb[e] = 0.f;
        for (int t = tb * TBC; t < t1; ++t) {
            const int64_t tok = (int64_t)b * a.T + t;
            const float* row = a.proj + tok * a.rs;
            const float* vb = row + a.pl.B + (int64_t)g * NR;
            const float* vc = row + a.pl.C + (int64_t)g * NR;
            // RMS of the raw rows, then (with RoPE) B^ / C^ in LDS: the rotated rows of every
            // head are formed from them again below instead of being read back
            float sb = 0.f, sc = 0.f;
            for (int e = tid; e < NR; e += NTH) {
                sb += vb[e] * vb[e];
                sc += vc[e] * vc[e];
            }
            sb = block_sum(sb, red);
            sc = block_sum(sc, red);
            const float rb = rsqrtf(sb / NR + a.eps), rc = rsqrtf(sc / NR + a.eps);
            if (a.cplx) {
                for (int e = tid; e < NR; e += NTH) {
                    Bh[e] = vb[e] * rb * a.prm.B_norm_w[e] + a.prm.B_bias[(int64_t)g * NR + e];
                    Ch[e] = vc[e] * rc * a.prm.C_norm_w[e] + a.prm.C_bias[(int64_t)g * NR + e];
                }
            }
            for (int e = tid; e < HS * NR; e += NTH) qB[e] = qC[e] = 0.f;
            __syncthreads();
            // This thread's heads of the group (one RoPE pair each: N / 2 <= NTH), software-
            // pipelined: the next head's angle and gradient rows are loaded before this head's
            // math. nb: the b part of the next chunk's first token, at chunk ends.
            const bool bnd = a.trap && t + 1 < a.T && (t + 1) % a.qb == 0;
            const int64_t ckb = bnd ? ((int64_t)b * a.nk + (t + 1) / a.qb) * a.H : 0;
            const int i = i0;
            float ph = 0.f, gb[2 * R], gc[2 * R], nb[2 * R];
            auto fetch = [&](int hl) {
                const int64_t th = tok * a.H + g * hpg + hl;
                const int64_t e0 = th * NR + (int64_t)(2 * i) * R;
                if (a.cplx) ph = a.f.phi[th * NH + i];
                ldv<2 * R>(a.gBt + e0, gb);
                ldv<2 * R>(a.gCt + e0, gc);
                if (bnd) ldv<2 * R>(a.gBb + (ckb + g * hpg + hl) * NR + (int64_t)(2 * i) * R, nb);
            };
            if (hg < hpg) fetch(hg);
            for (int hl = hg; hl < hpg; hl += HS) {
                const int h = g * hpg + hl;
                const int64_t th = tok * a.H + h;
                float* qb = qB + (int64_t)hg * NR;
                float* qc = qC + (int64_t)hg * NR;
                float cgb[2 * R], cgc[2 * R];
#pragma unroll
                for (int k = 0; k < 2 * R; ++k) {
                    cgb[k] = bnd ? gb[k] + nb[k] : gb[k];
                    cgc[k] = gc[k];
                }
                const float cph = ph;
                if (hl + HS < hpg) fetch(hl + HS);
                {
                    float s = 0.f, c = 1.f;
                    if (a.cplx) sincosf(cph, &s, &c);
                    float gphi = 0.f;
#pragma unroll
                    for (int r = 0; r < R; ++r) {
                        float gbe = cgb[r], gbo = cgb[R + r];
                        if (t == a.T - 1 && a.gprev) {
                            const float* gp = a.gprev + ((int64_t)b * a.H + h) * a.P * a.N;
                            const float* xr = a.f.xr + th * a.P * R + r;
                            for (int pp = 0; pp < a.P; ++pp) {
                                gbe += gp[(int64_t)pp * a.N + 2 * i] * xr[(int64_t)pp * R];
                                gbo += gp[(int64_t)pp * a.N + 2 * i + 1] * xr[(int64_t)pp * R];
                            }
                        }
                        const float gce = cgc[r], gco = cgc[R + r];
                        const int je = (2 * i) * R + r, jo = je + R;
                        if (a.cplx) {
                            // the rotated rows: e' = e cos - o sin, o' = e sin + o cos
                            const float be = Bh[je] * c - Bh[jo] * s, bo = Bh[je] * s + Bh[jo] * c;
                            const float ce = Ch[je] * c - Ch[jo] * s, co = Ch[je] * s + Ch[jo] * c;
                            gphi += gbo * be - gbe * bo + gco * ce - gce * co;
                        }
                        qb[je] += gbe * c + gbo * s;
                        qb[jo] += gbo * c - gbe * s;
                        qc[je] += gce * c + gco * s;
                        qc[jo] += gco * c - gce * s;
                    }
                    if (a.cplx) a.gphi[th * NH + i] = gphi;
                }
            }
            __syncthreads();
            if (HS > 1) {
                for (int e = tid; e < NR; e += NTH) {
                    float sbh = 0.f, sch = 0.f;
                    for (int k = 0; k < HS; ++k) {
                        sbh += qB[(int64_t)k * NR + e];
                        sch += qC[(int64_t)k * NR + e];
                    }
                    gBh[e] = sbh;
                    gCh[e] = sch;
                }
                __syncthreads();
            }
            // RMSNorm backward of group g; parameter partials
            float wb = 0.f, wc = 0.f;
            for (int e = tid; e < NR; e += NTH) {
                wb += gBh[e] * a.prm.B_norm_w[e] * vb[e];
                wc += gCh[e] * a.prm.C_norm_w[e] * vc[e];
            }
            wb = block_sum(wb, red);
            wc = block_sum(wc, red);
            const float kb = rb * rb * rb * wb / NR, kc = rc * rc * rc * wc / NR;
            for (int e = tid; e < NR; e += NTH) {
                const float gb = gBh[e], gc = gCh[e];
                a.gproj[tok * a.rs + a.pl.B + (int64_t)g * NR + e] = rb * a.prm.B_norm_w[e] * gb - vb[e] * kb;
                a.gproj[tok * a.rs + a.pl.C + (int64_t)g * NR + e] = rc * a.prm.C_norm_w[e] * gc - vc[e] * kc;
                pBw[e] += gb * vb[e] * rb;
                pCw[e] += gc * vc[e] * rc;
                pBb[e] += gb;
                pCb[e] += gc;
            }
            __syncthreads();
        }
        for (int e = tid; e < NR; e += NTH) {
            a.p_Bb[ob * GNR + (int64_t)g * NR + e] = pBb[e];
            a.p_Cb[ob * GNR + (int64_t)g * NR + e] = pCb[e];
        }
    }
    for (int e = tid; e < NR; e += NTH) {
        a.p_Bw[ob * NR + e] = pBw[e];
        a.p_Cw[ob * NR + e] = pCw[e];
    }
}

// ---- Phi_t = sum_{t'>=t} dL/dphi_t' + dL/dangle: chunk sums, then each chunk walked down
// from the sum of the chunks after it. One thread per (b, chunk, h, pair).
__device__ __forceinline__ void ajob(const Args& a, int64_t e, int& b, int& c, int& h, int& i) {
    const int NH = a.N / 2;
    const int nc = (a.T + kAC - 1) / kAC;
    i = (int)(e % NH);
    h = (int)((e / NH) % a.H);
    const int64_t bc = e / ((int64_t)NH * a.H);
    c = (int)(bc % nc);
    b = (int)(bc / nc);
}

__global__ __launch_bounds__(NTH) void tb_asum(Args a) {
    const int NH = a.N / 2, nc = (a.T + kAC - 1) / kAC;
    const int64_t e = (int64_t)blockIdx.x * NTH + threadIdx.x;
    if (e >= (int64_t)a.B * nc * a.H * NH) return;
    int b, c, h, i;
    ajob(a, e, b, c, h, i);
    float s = 0.f;
    const int t1 = min(a.T, (c + 1) * kAC);
    const int64_t ts = (int64_t)a.H * NH;  // token stride
    const float* gp = a.gphi + (((int64_t)b * a.T) * a.H + h) * NH + i;
    int t = c * kAC;
    for (; t + 8 <= t1; t += 8) {  // tokens added in order; eight loads ahead of their adds
        float v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) v[u] = gp[(t + u) * ts];
#pragma unroll
        for (int u = 0; u < 8; ++u) s += v[u];
    }
    for (; t < t1; ++t) s += gp[t * ts];
    a.Phi_sum[e] = s;
}

__global__ __launch_bounds__(NTH) void tb_angle(Args a) {
    const int NH = a.N / 2, nc = (a.T + kAC - 1) / kAC;
    const int64_t e = (int64_t)blockIdx.x * NTH + threadIdx.x;
    if (e >= (int64_t)a.B * nc * a.H * NH) return;
    int b, c, h, i;
    ajob(a, e, b, c, h, i);
    float s = a.gang ? a.gang[((int64_t)b * a.H + h) * NH + i] : 0.f;
    for (int cc = nc - 1; cc > c; --cc) s += a.Phi_sum[(((int64_t)b * nc + cc) * a.H + h) * NH + i];
    const int t1 = min(a.T, (c + 1) * kAC);
    const int64_t ts = (int64_t)a.H * NH;  // token stride
    const int64_t o0 = (((int64_t)b * a.T) * a.H + h) * NH + i;
    // tokens walked down in order; gphi and Phi are separate buffers, so eight loads of gphi
    // go out ahead of the running sums
    int t = t1 - 1;
    for (; t - 7 >= c * kAC; t -= 8) {
        float v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) v[u] = a.gphi[o0 + (t - u) * ts];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            s += v[u];
            a.Phi[o0 + (t - u) * ts] = s;
        }
    }
    for (; t >= c * kAC; --t) {
        s += a.gphi[o0 + t * ts];
        a.Phi[o0 + t * ts] = s;
    }
}

// ---- per token: dL/dtheta, dL/ddt_raw and the dt_bias partials. One block per (b, t).
__global__ __launch_bounds__(NTH) void tb_tok(Args a) {
    const int64_t tok = blockIdx.x;
    const int NH = a.N / 2;
    const float* row = a.proj + tok * a.rs;
    if (a.cplx) {
        for (int i = threadIdx.x; i < NH; i += NTH) {
            // heads added in order; eight heads' loads go out before their products
            float s = 0.f;
            int h = 0;
            for (; h + 8 <= a.H; h += 8) {
                float dv[8], pv[8];
#pragma unroll
                for (int u = 0; u < 8; ++u) {
                    dv[u] = a.f.dt[tok * a.H + h + u];
                    pv[u] = a.Phi[(tok * a.H + h + u) * NH + i];
                }
#pragma unroll
                for (int u = 0; u < 8; ++u) s += dv[u] * pv[u];
            }
            for (; h < a.H; ++h) s += a.f.dt[tok * a.H + h] * a.Phi[(tok * a.H + h) * NH + i];
            a.gproj[tok * a.rs + a.pl.theta + i] = -s;
        }
    }
    for (int h = threadIdx.x; h < a.H; h += NTH) {
        const int64_t th = tok * a.H + h;
        float g = a.gdtc[th] + a.gdtx[th];
        if (a.cplx) {
            float s = 0.f;
            int i = 0;
            for (; i + 8 <= NH; i += 8) {
                float tv[8], pv[8];
#pragma unroll
                for (int u = 0; u < 8; ++u) {
                    tv[u] = row[a.pl.theta + i + u];
                    pv[u] = a.Phi[th * NH + i + u];
                }
#pragma unroll
                for (int u = 0; u < 8; ++u) s += tv[u] * pv[u];
            }
            for (; i < NH; ++i) s += row[a.pl.theta + i] * a.Phi[th * NH + i];
            g -= s;
        }
        const float u = row[a.pl.dt + h] + a.prm.dt_bias[h];
        const float gu = g * (a.dt_scale ? a.dt_scale[th] : 1.f) * sigm(u);
        a.gproj[tok * a.rs + a.pl.dt + h] = gu;
        a.p_dtb[th] = gu;
        // dt = softplus(u) s: dL/ds = dL/ddt softplus(u)
        if (a.out.dt_scale) a.out.dt_scale[th] = g * softplus_f(u);
    }
}

// ---- parameter gradients: column sums of the (K x M) partial matrices in a fixed order.
// A block sums a slab of 256 rows for 64 columns (4 row groups of 64 rows each, then the
// groups in order); slabs are summed by the next pass.
constexpr int kSlab = 256;

// Up to four column-sum jobs of the same row count K in one launch (blockIdx.z picks one);
// each has its own input, output and column count.
struct ColJobs {
    const float* in[4];
    float* out[4];
    int M[4];
};

__global__ __launch_bounds__(NTH) void tb_colsum(ColJobs jobs, int64_t K) {
    __shared__ float red[4][64];
    const float* in = jobs.in[blockIdx.z];
    float* out = jobs.out[blockIdx.z];
    const int M = jobs.M[blockIdx.z];
    const int c = threadIdx.x & 63, grp = threadIdx.x >> 6;
    const int col = blockIdx.x * 64 + c;
    const int64_t r0 = (int64_t)blockIdx.y * kSlab, r1 = min(K, r0 + kSlab);
    float s = 0.f;
    if (col < M) {
        // rows r0+grp, +4, +8, ... added in that order; eight loads go out before their adds
        int64_t r = r0 + grp;
        for (; r + 28 < r1; r += 32) {
            float v[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) v[u] = in[(r + 4 * u) * M + col];
#pragma unroll
            for (int u = 0; u < 8; ++u) s += v[u];
        }
        for (; r < r1; r += 4) s += in[r * M + col];
    }
    red[grp][c] = s;
    __syncthreads();
    if (grp == 0 && col < M) out[(int64_t)blockIdx.y * M + col] = red[0][c] + red[1][c] + red[2][c] + red[3][c];
}

// dL/dA_log = (dL/dA of the chunked SSD + of the trapezoid decays) A;  dL/dD.
__global__ __launch_bounds__(NTH) void tb_finish(Args a, const float* gA_x) {
    const int h = blockIdx.x * NTH + threadIdx.x;
    if (h >= a.H) return;
    a.out.A_log[h] = (a.gAc[h] + gA_x[h]) * a.f.A[h];
    a.out.D[h] = a.gD[h];
}

struct Plan {
    size_t off[26], chunk_off, total;
};

// Largest slab-sum matrix of the parameter reductions (rows ceil(K / kSlab) x M).
size_t colsum_scratch(const m3_layer_desc& d) {
    const size_t B = d.batch, T = d.seqlen, H = d.nheads;
    const size_t NR = (size_t)d.d_state * d.mimo_rank, HPR = H * d.headdim * d.mimo_rank;
    const size_t nTB = (T + TBK - 1) / TBK, nTC = (T + TBC - 1) / TBC;
    const size_t KM[4][2] = {{B * T, H}, {B * nTC, d.ngroups * NR}, {B * nTB, HPR}, {B * nTB, H}};
    size_t m = 0;
    for (const auto& km : KM) m = std::max(m, (km[0] + kSlab - 1) / kSlab * km[1]);
    return m;
}

inline size_t al(size_t x) { return (x + 255) & ~(size_t)255; }

Plan plan(const m3_layer_desc& d) {
    const size_t B = d.batch, T = d.seqlen, H = d.nheads, P = d.headdim, N = d.d_state,
                 R = d.mimo_rank, G = d.ngroups;
    const size_t BTH = B * T * H, X = BTH * P * R, BN = BTH * N * R, NH = N / 2;
    const size_t nTB = (T + TBK - 1) / TBK, nTC = (T + TBC - 1) / TBC, nc = (T + kAC - 1) / kAC;
    const bool trap = d.use_trapezoidal != 0;
    const int qb = trap ? chunked_chunk_tokens(d.mimo_rank, true) : 0;
    const size_t bnd = trap && qb > 0 ? B * ((T + qb - 1) / qb) * H * N * R : 0;
    const size_t sizes[26] = {
        X, X, trap ? X : 0, X,                         // gys, gxg, gxb, gxr
        BN, trap ? bnd : 0, BN,                        // gBt, gBb (chunk-start rows), gCt
        BTH, H, H, BTH,                                // gdtc, gAc, gD, gdtx
        BTH * NH, BTH * NH, B * nc * H * NH,           // gphi, Phi, Phi_sum
        B * nTB * H,                                   // gA_part
        B * nTB * H * P * R, B * nTB * H * P * R, B * nTB * H * P * R,  // p_md, p_mz, p_mx
        B * nTC * N * R, B * nTC * N * R,              // p_Bw, p_Cw
        B * nTC * G * N * R, B * nTC * G * N * R,      // p_Bb, p_Cb
        BTH,                                           // p_dtb
        4 * colsum_scratch(d), 4 * colsum_scratch(d), H};  // column-sum passes (4 jobs), dL/dA (x terms)
    Plan p;
    size_t o = 0;
    for (int i = 0; i < 26; ++i) {
        p.off[i] = o;
        o += al(sizes[i] * sizeof(float));
    }
    p.chunk_off = o;
    o += al(chunked_bwd_workspace(d.batch, d.seqlen, d.nheads, d.headdim, d.d_state, d.mimo_rank,
                                  trap, fp32_layer_hs_ok(d)));
    p.total = o;
    return p;
}

// LDS of tb_bc: (2 HS + 8) N R + NTH floats, 2 N R fewer with one head slot (HS = 1 at
// d_state 512), so at most 132 KB (d_state 512, rank 8).
constexpr size_t kBcMaxLds = 160 * 1024;  // gfx950's LDS per workgroup
size_t bc_lds(const m3_layer_desc& d) {
    const size_t NR = (size_t)d.d_state * d.mimo_rank;
    const size_t HS = std::max(1, NTH / (d.d_state / 2));
    return ((2 * HS + (HS > 1 ? 2 : 0) + 6) * NR + NTH) * sizeof(float);
}

// tb_bc<R> with `lds` bytes of dynamic LDS; above 64 KB the kernel's limit is raised first.
template <int R>
int launch_bc(const Args& a, dim3 grid, size_t lds, hipStream_t stream) {
    if (lds > 64 * 1024 &&
        hipFuncSetAttribute(reinterpret_cast<const void*>(&tb_bc<R>),
                            hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) != hipSuccess)
        return 1;
    hipLaunchKernelGGL(tb_bc<R>, grid, dim3(NTH), lds, stream, a);
    return 0;
}


}  // namespace tb

size_t layer_bwd_workspace(const m3_layer_desc& d) {
    if (!fp32_layer_supported(d) || tb::bc_lds(d) > tb::kBcMaxLds || d.mimo_rank > 8) return 0;
    return tb::plan(d).total;
}

int launch_layer_bwd(const m3_layer_desc& d, const m3_layer_params& p, const void* proj,
                     const float* dt_scale, void* fwd_workspace, const float* g_out,
                     const float* g_h, const float* g_angle, const float* g_prev, float* g_proj,
                     const m3_layer_param_grads& g, void* workspace, hipStream_t stream) {
    using namespace tb;
    const Plan pl = plan(d);
    char* ws = reinterpret_cast<char*>(workspace);
    auto part = [&](int i) { return reinterpret_cast<float*>(ws + pl.off[i]); };
    Args a;
    a.B = d.batch, a.T = d.seqlen, a.H = d.nheads, a.P = d.headdim, a.N = d.d_state;
    a.R = d.mimo_rank, a.G = d.ngroups, a.trap = d.use_trapezoidal, a.cplx = d.use_complex;
    a.qb = a.trap ? chunked_chunk_tokens(a.R, true) : 1;
    a.nk = (a.T + a.qb - 1) / a.qb;
    if (a.qb <= 0) return 1;
    a.rs = d.proj_row_stride, a.pl = proj_layout(d), a.eps = d.rms_eps, a.prm = p;
    a.proj = reinterpret_cast<const float*>(proj);
    a.dt_scale = dt_scale;
    a.f = fp32_layer_parts(d, fwd_workspace);
    a.gout = g_out, a.gh = g_h, a.gang = g_angle, a.gprev = g_prev, a.gproj = g_proj, a.out = g;
    a.gys = part(0), a.gxg = part(1), a.gxb = a.trap ? part(2) : nullptr, a.gxr = part(3);
    a.gBt = part(4), a.gBb = a.trap ? part(5) : nullptr, a.gCt = part(6);
    a.gdtc = part(7), a.gAc = part(8), a.gD = part(9), a.gdtx = part(10);
    a.gphi = part(11), a.Phi = part(12), a.Phi_sum = part(13), a.gA_part = part(14);
    a.p_md = part(15), a.p_mz = part(16), a.p_mx = part(17);
    a.p_Bw = part(18), a.p_Cw = part(19), a.p_Bb = part(20), a.p_Cb = part(21), a.p_dtb = part(22);

    const int nTB = (a.T + TBK - 1) / TBK, nTC = (a.T + TBC - 1) / TBC;
    const unsigned gbh = (unsigned)((int64_t)a.B * nTB * a.H);
    switch (a.R) {
        case 1: hipLaunchKernelGGL(tb_gate<1>, dim3(gbh), dim3(NTH), 0, stream, a); break;
        case 2: hipLaunchKernelGGL(tb_gate<2>, dim3(gbh), dim3(NTH), 0, stream, a); break;
        case 3: hipLaunchKernelGGL(tb_gate<3>, dim3(gbh), dim3(NTH), 0, stream, a); break;
        case 4: hipLaunchKernelGGL(tb_gate<4>, dim3(gbh), dim3(NTH), 0, stream, a); break;
        case 5: hipLaunchKernelGGL(tb_gate<5>, dim3(gbh), dim3(NTH), 0, stream, a); break;
        case 6: hipLaunchKernelGGL(tb_gate<6>, dim3(gbh), dim3(NTH), 0, stream, a); break;
        case 7: hipLaunchKernelGGL(tb_gate<7>, dim3(gbh), dim3(NTH), 0, stream, a); break;
        case 8: hipLaunchKernelGGL(tb_gate<8>, dim3(gbh), dim3(NTH), 0, stream, a); break;
        default: return 1;
    }
    if (launch_chunked_bwd(a.B, a.T, a.H, a.P, a.N, a.R, a.f.xg, a.f.xb, a.f.Bt, a.f.Bb, a.f.Ct,
                           a.f.dt, a.f.A, p.D, a.f.xr, nullptr, a.gys, g_h, a.gxg, a.gxb, a.gBt,
                           a.gBb, a.gCt, a.gdtc, a.gAc, a.gD, a.gxr, nullptr,
                           ws + pl.chunk_off, stream, fp32_layer_hs_ok(d) ? a.f.Hs : nullptr,
                           a.trap != 0) != 0)
        return 1;
    switch (a.R) {
        case 1: hipLaunchKernelGGL(tb_x<1>, dim3(gbh), dim3(NTH), 0, stream, a); break;
        case 2: hipLaunchKernelGGL(tb_x<2>, dim3(gbh), dim3(NTH), 0, stream, a); break;
        case 3: hipLaunchKernelGGL(tb_x<3>, dim3(gbh), dim3(NTH), 0, stream, a); break;
        case 4: hipLaunchKernelGGL(tb_x<4>, dim3(gbh), dim3(NTH), 0, stream, a); break;
        case 5: hipLaunchKernelGGL(tb_x<5>, dim3(gbh), dim3(NTH), 0, stream, a); break;
        case 6: hipLaunchKernelGGL(tb_x<6>, dim3(gbh), dim3(NTH), 0, stream, a); break;
        case 7: hipLaunchKernelGGL(tb_x<7>, dim3(gbh), dim3(NTH), 0, stream, a); break;
        case 8: hipLaunchKernelGGL(tb_x<8>, dim3(gbh), dim3(NTH), 0, stream, a); break;
        default: return 1;
    }
    const dim3 gbc((unsigned)((int64_t)a.B * nTC));
    const size_t lbc = bc_lds(d);
    int st = 1;
    switch (a.R) {
        case 1: st = launch_bc<1>(a, gbc, lbc, stream); break;
        case 2: st = launch_bc<2>(a, gbc, lbc, stream); break;
        case 3: st = launch_bc<3>(a, gbc, lbc, stream); break;
        case 4: st = launch_bc<4>(a, gbc, lbc, stream); break;
        case 5: st = launch_bc<5>(a, gbc, lbc, stream); break;
        case 6: st = launch_bc<6>(a, gbc, lbc, stream); break;
        case 7: st = launch_bc<7>(a, gbc, lbc, stream); break;
        case 8: st = launch_bc<8>(a, gbc, lbc, stream); break;
        default: break;
    }
    if (st != 0) return 1;
    if (a.cplx) {
        const int nc = (a.T + kAC - 1) / kAC;
        const int64_t na = (int64_t)a.B * nc * a.H * (a.N / 2);
        const unsigned ga = (unsigned)((na + NTH - 1) / NTH);
        hipLaunchKernelGGL(tb_asum, dim3(ga), dim3(NTH), 0, stream, a);
        hipLaunchKernelGGL(tb_angle, dim3(ga), dim3(NTH), 0, stream, a);
    }
    hipLaunchKernelGGL(tb_tok, dim3((unsigned)((int64_t)a.B * a.T)), dim3(NTH), 0, stream, a);
    float* tmp[2] = {part(23), part(24)};
    const size_t unit = colsum_scratch(d);  // floats per job and pass
    // Column sums of nz partial matrices with K rows: slab sums (kSlab rows), then sums of
    // those, every job in its own scratch region; rows are added in a fixed order.
    auto colsum = [&](int nz, std::initializer_list<const float*> ins, std::initializer_list<float*> outs,
                      std::initializer_list<int> Ms, int64_t K) {
        ColJobs j{};
        int Mmax = 0;
        for (int z = 0; z < nz; ++z) {
            j.in[z] = ins.begin()[z];
            j.M[z] = Ms.begin()[z];
            Mmax = std::max(Mmax, j.M[z]);
        }
        int w = 0;
        while (K > kSlab) {
            const int64_t ks = (K + kSlab - 1) / kSlab;
            for (int z = 0; z < nz; ++z) j.out[z] = tmp[w] + z * unit;
            hipLaunchKernelGGL(tb_colsum, dim3((unsigned)((Mmax + 63) / 64), (unsigned)ks, (unsigned)nz),
                               dim3(NTH), 0, stream, j, K);
            for (int z = 0; z < nz; ++z) j.in[z] = j.out[z];
            w ^= 1;
            K = ks;
        }
        for (int z = 0; z < nz; ++z) j.out[z] = outs.begin()[z];
        hipLaunchKernelGGL(tb_colsum, dim3((unsigned)((Mmax + 63) / 64), 1, (unsigned)nz), dim3(NTH), 0,
                           stream, j, K);
    };
    const int NR = a.N * a.R, HPR = a.H * a.P * a.R;
    const int64_t nbt = (int64_t)a.B * nTB, nbc = (int64_t)a.B * nTC;
    colsum(1, {a.p_dtb}, {g.dt_bias}, {a.H}, (int64_t)a.B * a.T);
    colsum(4, {a.p_Bw, a.p_Cw, a.p_Bb, a.p_Cb}, {g.B_norm_w, g.C_norm_w, g.B_bias, g.C_bias},
           {NR, NR, a.G * NR, a.G * NR}, nbc);
    colsum(4, {a.p_mx, a.p_mz, a.p_md, a.gA_part}, {g.mimo_x, g.mimo_z, g.mimo_down, part(25)},
           {HPR, HPR, HPR, a.H}, nbt);
    hipLaunchKernelGGL(tb_finish, dim3((unsigned)((a.H + NTH - 1) / NTH)), dim3(NTH), 0, stream, a,
                       part(25));
    return hipGetLastError() == hipSuccess ? 0 : 1;
}

}  // namespace m3
