// Fused chunked-SSD prefill on bf16 MFMA for the d_state=128, headdim=64, mimo_rank=2
// layer (the shape of the d_model 768 KulaMamba), gfx950.
//
// Work decomposition
// ------------------
// The sequence of every (batch, head) is cut into S segments of whole 64-token chunks.
// One 512-thread workgroup (8 waves) owns one (batch, head, segment) and walks its
// chunks in order, carrying the (P=64, N=128) fp32 state in MFMA accumulators, so no
// per-chunk state ever goes to HBM. Three launches:
//   1. bc_norm:    per token and group, B^ = RMSNorm(B) * w + bias and C^ likewise in
//                  bf16 (shared by every head, so computed once), pair-packed so that a
//                  RoPE pair (n=2i, n=2i+1) of one rank is one 32-bit word.
//   2. ssd_chunks<false> for segments 0..S-2: only the state update, giving each
//                  segment's end state from a zero start plus its total log-decay and
//                  total RoPE angle increment.
//   3. ssd_chunks<true> for all segments: combines the preceding segments' end states
//                  into the incoming state, then computes every chunk's output.
//
// Per chunk (Q=64 tokens, rows (t,r) = 2t+r, 128 rows) the kernel forms in LDS
//   C~ [(t,r)][n], B~ [(u,r')][n]      bf16, B^/C^ rotated by the RoPE angle
//   B~w[u][n][r'] = B~ * w_u            bf16 (state-update operand)
//   X^T[p][(u,r')] = x * mimo_x         bf16
//   H[p][n]                             bf16 copy of the incoming state
//   Lc[t][u] = [u<=t] exp(c_t-c_u) (a_u + [u<t] b_u)   fp32
// and runs four MFMA contractions (v_mfma_f32_16x16x32_bf16):
//   G3  Y  = diag(e^{c_t}) C~ H^T          inter-chunk output
//   G1  S^T = B~ C~^T, masked by Lc (+D on the diagonal), kept in registers
//   G2  Y += S X                           intra-chunk output, S fed straight from the
//                                          G1 accumulators as the A operand (the k
//                                          order is permuted consistently in X)
//   G4  H^T = e^{c_63} H^T + B~w^T X       state update
// All eight waves share the element-wise preparation. In the MFMA phase waves 0-3 own
// the 16-row output blocks {w, 7-w} (balanced causal work) and waves 4-7 own the state
// update, so each SIMD interleaves one output wave with one state wave.
// The trapezoid is folded into a_u = lambda_u dt_u, b_u = (1-lambda_{u+1}) dt_{u+1}
// (the beta term of token u+1 multiplies B~_u x_u), so the rank is not doubled.
//
// Memory: every global read goes through a buffer descriptor whose size ends at the
// batch row's last token, so reads past the sequence return zero (padding for free).
// The next chunk's reads are issued as soon as a wave finishes its MFMA work.
//
// RoPE frame: inside a segment every angle is taken relative to the segment start.
// Dot products C~.B~ and C~.H are invariant under a common rotation, so outputs are
// unchanged, while sin/cos only see angles accumulated over one segment. Incoming
// segment states are rotated into the local frame when combined, and the final state,
// angle and prev_BX are rotated back to the absolute frame.
#include <algorithm>

#include "m3_common.h"
#include "m3_kernels.h"

namespace m3 {
namespace mf {

constexpr int Q = 64;
constexpr int N = 128;
constexpr int P = 64;
constexpr int R = 2;
constexpr int NR = N * R;
constexpr int NH = N / 2;
constexpr int THREADS = 512;
constexpr int PAD = 8;
constexpr float kLog2e = 1.4426950408889634f;
constexpr int kRsrcFlags = 0x00020000;

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef unsigned u32x2 __attribute__((ext_vector_type(2)));

struct __align__(16) Smem {
    bf16 C[Q * R][N + PAD];    // C~ rows (t,r)
    bf16 B[Q * R][N + PAD];    // B~ rows (u,r')
    bf16 Bw[Q][NR + PAD];      // B~ * w_u, [u][n][r'] order
    bf16 X[P][Q * R + PAD];    // X^T
    bf16 H[P][N + PAD];        // incoming state, bf16
    float L[Q][Q + 8];         // Lc; columns Q, Q+1 hold a_u, b_u
    float c2[Q];               // in-chunk cumulative log2-decay (inclusive)
    float ec[Q];               // exp(c)
    float w[Q];                // exp(c_63 - c_u) (a_u + b_u)
    float dt[Q];
    float tot[8][NH];          // per 8-token group, per pair: sum of dt*theta
    float rot[NH];             // per-pair angle scratch (prologue / epilogue)
    float mzd[P][4];           // mimo_z[p][0..1], mimo_down[p][0..1] of this head
};

struct Args {
    int B, T, H, G, S, cps;
    int trap, cplx;
    int64_t rs;
    ProjLayout pl;
    m3_layer_params prm;
    const bf16* proj;
    const float* dt_scale;
    const bf16* Bn;    // [B*T][G][NR] pair-packed normalised B
    const bf16* Cn;
    float* seg_state;  // [B*H*(S-1)][N][P]
    float* seg_decay;  // [B*H*(S-1)]
    float* seg_angle;  // [B*H*(S-1)][NH]
    bf16* y_out;
    float* h_final;
    float* angle;
    float* prev_bx;
};

__device__ __forceinline__ f32x4 mfma16(const bf16x8& a, const bf16x8& b, const f32x4& c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, int64_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0,
                                             (int)(bytes < 0x7fffffff ? bytes : 0x7fffffff),
                                             kRsrcFlags);
}

__device__ __forceinline__ bf16 ld_bf16(__amdgpu_buffer_rsrc_t r, int off_elems) {
    const unsigned short v = __builtin_amdgcn_raw_buffer_load_b16(r, off_elems * 2, 0, 0);
    return __builtin_bit_cast(bf16, v);
}

__device__ __forceinline__ u32x2 ld_b64(__amdgpu_buffer_rsrc_t r, int off_elems) {
    return __builtin_amdgcn_raw_buffer_load_b64(r, off_elems * 2, 0, 0);
}

// sin and cos of an angle in radians, reduced to [-0.5, 0.5) turns for the hardware.
__device__ __forceinline__ void fast_sincos(float x, float& s, float& c) {
    float rev = x * 0.15915494309189535f;
    rev = rev - rintf(rev);
    s = __builtin_amdgcn_sinf(rev);
    c = __builtin_amdgcn_cosf(rev);
}

__device__ __forceinline__ float fast_exp(float x) { return __builtin_amdgcn_exp2f(x * kLog2e); }

__device__ __forceinline__ float fast_silu(float x) {
    return x * __builtin_amdgcn_rcpf(1.f + fast_exp(-x));
}

__device__ __forceinline__ float fast_softplus(float x) {
    return x > 20.f ? x : __logf(1.f + fast_exp(x));
}

__device__ __forceinline__ float wave_incl_scan(float v, int lane) {
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const float o = __shfl_up(v, off, 64);
        if (lane >= off) v += o;
    }
    return v;
}

__device__ __forceinline__ bf16x2 as_bf16x2(unsigned u) { return __builtin_bit_cast(bf16x2, u); }

__device__ __forceinline__ unsigned pack_bf16x2(float lo, float hi) {
    return __builtin_bit_cast(unsigned, bf16x2{(bf16)lo, (bf16)hi});
}

// ---------------------------------------------------------------------------------
// 1. Normalised B^ / C^ per (token, group): x * rsqrt(mean(x^2) + eps) * w + bias,
//    stored pair-packed: word 2i+r of the row = (value[n=2i][r], value[n=2i+1][r]).
// ---------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void bc_norm(const bf16* __restrict__ proj, int64_t rs,
                                               int64_t offB, int64_t offC, int G,
                                               int64_t ntok_grp, float eps,
                                               const float* __restrict__ wB,
                                               const float* __restrict__ biasB,
                                               const float* __restrict__ wC,
                                               const float* __restrict__ biasC,
                                               bf16* __restrict__ Bn, bf16* __restrict__ Cn) {
    const int lane = threadIdx.x & 63;
    const int64_t tg = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (tg >= ntok_grp) return;
    const int64_t tok = tg / G;
    const int g = (int)(tg % G);
    const bf16* row = proj + tok * rs;
    // lane = pair i; raw order at 4i: (n=2i,r0) (2i,r1) (2i+1,r0) (2i+1,r1)
    const bf16x4 vb = *reinterpret_cast<const bf16x4*>(row + offB + (int64_t)g * NR + 4 * lane);
    const bf16x4 vc = *reinterpret_cast<const bf16x4*>(row + offC + (int64_t)g * NR + 4 * lane);
    float b[4], c[4], sb = 0.f, sc = 0.f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        b[j] = (float)vb[j];
        c[j] = (float)vc[j];
        sb += b[j] * b[j];
        sc += c[j] * c[j];
    }
    sb = group_sum<64>(sb);
    sc = group_sum<64>(sc);
    const float rb = rsqrtf(sb * (1.f / NR) + eps), rc = rsqrtf(sc * (1.f / NR) + eps);
    const int e = 4 * lane;
    float ob[4], oc[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        ob[j] = b[j] * rb * wB[e + j] + biasB[(int64_t)g * NR + e + j];
        oc[j] = c[j] * rc * wC[e + j] + biasC[(int64_t)g * NR + e + j];
    }
    // pair-packed: (e_r0, o_r0, e_r1, o_r1)
    *reinterpret_cast<bf16x4*>(Bn + tg * NR + e) = bf16x4{(bf16)ob[0], (bf16)ob[2], (bf16)ob[1], (bf16)ob[3]};
    *reinterpret_cast<bf16x4*>(Cn + tg * NR + e) = bf16x4{(bf16)oc[0], (bf16)oc[2], (bf16)oc[1], (bf16)oc[3]};
}

// ---------------------------------------------------------------------------------
// 2/3. Segment kernels.
// ---------------------------------------------------------------------------------
template <bool kFull>
__global__ __launch_bounds__(THREADS, 1) void ssd_chunks(Args a) {
    __shared__ Smem sm;
    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int g16 = lane >> 4, l16 = lane & 15;

    const int nseg = kFull ? a.S : a.S - 1;
    // XCD-aware order: consecutive workgroups of one batch row land on one XCD.
    const int nblk = gridDim.x;
    const int blk = (nblk % 8 == 0) ? (blockIdx.x % 8) * (nblk / 8) + blockIdx.x / 8 : blockIdx.x;
    const int seg = blk % nseg;
    const int bh = blk / nseg;
    const int b = bh / a.H, h = bh % a.H;
    const int grp = h / (a.H / a.G);
    const int T = a.T;
    const int K = (T + Q - 1) / Q;
    const int k_begin = seg * a.cps;
    const int k_end = min(K, k_begin + a.cps);
    const int HP = a.H * P;
    const int rs = (int)a.rs;

    const int bnrs = a.G * NR;  // elements between tokens in Bn / Cn

    const float A_h = -__expf(a.prm.A_log[h]);
    const float D_h = a.prm.D[h];
    const float dtb = a.prm.dt_bias[h];

    // Prep role: pair pi = lane (n = 2pi, 2pi+1), tokens 8*wave .. 8*wave+7.
    const int pi = lane;
    const int tq = wave;
    // X role: column p = lane, tokens 8*wave .. 8*wave+7.
    const int xp = lane;
    const float mx0 = a.prm.mimo_x[(h * P + xp) * R], mx1 = a.prm.mimo_x[(h * P + xp) * R + 1];
    // Output role (waves 0-3): gate constants of columns p, kept in LDS.
    if (kFull && tid < P) {
        sm.mzd[tid][0] = a.prm.mimo_z[(h * P + tid) * R];
        sm.mzd[tid][1] = a.prm.mimo_z[(h * P + tid) * R + 1];
        sm.mzd[tid][2] = a.prm.mimo_down[(h * P + tid) * R];
        sm.mzd[tid][3] = a.prm.mimo_down[(h * P + tid) * R + 1];
    }

    // State accumulators: wave w owns the H^T rows n in [16w, 16w+16) (all 64 columns p).
    constexpr int kNT = 1;
    const bool state_wave = true;
    const int nt0 = wave;
    f32x4 hacc[kNT][4];
#pragma unroll
    for (int i = 0; i < kNT; ++i)
#pragma unroll
        for (int pt = 0; pt < 4; ++pt) hacc[i][pt] = f32x4{0.f, 0.f, 0.f, 0.f};

    float phi_start = 0.f;  // absolute angle of pair pi at this segment's start
    if (kFull && seg > 0) {
        // H = sum_i exp(sum_{l=i+1}^{seg-1} D_l) R(-sum_{l=i}^{seg-1} Phi_l) S_i
        const int64_t sbase = (int64_t)bh * (a.S - 1);
        float dsum = 0.f;
        for (int i = seg - 1; i >= 0; --i) {
            __syncthreads();
            if (tid < NH) {
                const float acc = (i == seg - 1) ? 0.f : sm.rot[tid];
                sm.rot[tid] = acc + a.seg_angle[(sbase + i) * NH + tid];
            }
            __syncthreads();
            if (state_wave) {
                const float wgt = __expf(dsum);
                const float* Si = a.seg_state + (sbase + i) * (int64_t)N * P;
#pragma unroll
                for (int i2 = 0; i2 < kNT; ++i2) {
                    const int n0 = 16 * (nt0 + i2) + 4 * g16;
                    float s0, c0, s1, c1;
                    sincosf(-sm.rot[n0 / 2], &s0, &c0);
                    sincosf(-sm.rot[n0 / 2 + 1], &s1, &c1);
#pragma unroll
                    for (int pt = 0; pt < 4; ++pt) {
                        const int p = 16 * pt + l16;
                        const float e0 = Si[(n0 + 0) * P + p], o0 = Si[(n0 + 1) * P + p];
                        const float e1 = Si[(n0 + 2) * P + p], o1 = Si[(n0 + 3) * P + p];
                        hacc[i2][pt][0] += wgt * (e0 * c0 - o0 * s0);
                        hacc[i2][pt][1] += wgt * (e0 * s0 + o0 * c0);
                        hacc[i2][pt][2] += wgt * (e1 * c1 - o1 * s1);
                        hacc[i2][pt][3] += wgt * (e1 * s1 + o1 * c1);
                    }
                }
            }
            dsum += a.seg_decay[sbase + i];
        }
        __syncthreads();
        phi_start = sm.rot[pi];  // sum_{l<seg} Phi_l
    }

    // ---- global reads. A token row gets its own scalar buffer descriptor whose size is
    // zero past the sequence end, so those reads return zero and the per-lane offsets
    // stay loop-invariant.
    const int wv = __builtin_amdgcn_readfirstlane(wave);
    const bf16* proj_b = a.proj + (int64_t)b * T * a.rs;
    const bf16* bn_b = a.Bn + ((int64_t)b * T * a.G + grp) * NR;
    const bf16* cn_b = a.Cn + ((int64_t)b * T * a.G + grp) * NR;
    const int voff_bc = lane * 8;                                   // bytes: 4 bf16 of pair pi
    const int voff_th = ((int)a.pl.theta + lane) * 2;
    const int voff_x = ((int)a.pl.x + h * P + lane) * 2;
    u32x2 rawB[8], rawC[8];
    bf16 rawth[8], rawx[8];
    float dr_a = 0.f, dr_b = 0.f, lr_a = 0.f, lr_b = 0.f;
    auto load_prep = [&](int kk) {
        const int s0 = kk * Q;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int tok = s0 + 8 * wv + j;
            const bool in = tok < T;
            const __amdgpu_buffer_rsrc_t rrow = make_rsrc(proj_b + (int64_t)tok * a.rs, in ? a.rs * 2 : 0);
            const __amdgpu_buffer_rsrc_t rb = make_rsrc(bn_b + (int64_t)tok * bnrs, in ? NR * 2 : 0);
            rawB[j] = __builtin_amdgcn_raw_buffer_load_b64(rb, voff_bc, 0, 0);
            if (kFull) {
                const __amdgpu_buffer_rsrc_t rc = make_rsrc(cn_b + (int64_t)tok * bnrs, in ? NR * 2 : 0);
                rawC[j] = __builtin_amdgcn_raw_buffer_load_b64(rc, voff_bc, 0, 0);
            }
            rawth[j] = a.cplx ? __builtin_bit_cast(bf16, (unsigned short)__builtin_amdgcn_raw_buffer_load_b16(rrow, voff_th, 0, 0))
                              : (bf16)0.f;
            rawx[j] = __builtin_bit_cast(bf16, (unsigned short)__builtin_amdgcn_raw_buffer_load_b16(rrow, voff_x, 0, 0));
        }
        if (wv == 0) {
            // token s0+lane (and s0+64 in every lane, used by lane 63 only)
            const __amdgpu_buffer_rsrc_t rch = make_rsrc(proj_b + (int64_t)s0 * a.rs,
                                                          (int64_t)max(T - s0, 0) * a.rs * 2);
            dr_a = (float)ld_bf16(rch, lane * rs + (int)a.pl.dt + h);
            dr_b = (float)ld_bf16(rch, Q * rs + (int)a.pl.dt + h);
            if (a.trap) {
                lr_a = (float)ld_bf16(rch, lane * rs + (int)a.pl.lam + h);
                lr_b = (float)ld_bf16(rch, Q * rs + (int)a.pl.lam + h);
            }
        }
    };
    load_prep(k_begin);

    float phi_run = 0.f;   // angle of pair pi relative to the segment start
    float logdecay = 0.f;  // total log-decay of the segment (natural log)

    for (int k = k_begin; k < k_end; ++k) {
        const int s0 = k * Q;
        __syncthreads();
        // ---- phase 1: bf16 state copy, token scalars, X^T tile
        if (kFull && state_wave) {
#pragma unroll
            for (int i2 = 0; i2 < kNT; ++i2) {
                const int n0 = 16 * (nt0 + i2) + 4 * g16;
#pragma unroll
                for (int pt = 0; pt < 4; ++pt) {
                    const f32x4 v = hacc[i2][pt];
                    *reinterpret_cast<bf16x4*>(&sm.H[16 * pt + l16][n0]) =
                        bf16x4{(bf16)v[0], (bf16)v[1], (bf16)v[2], (bf16)v[3]};
                }
            }
        }
        if (wave == 0) {
            const int u = lane;
            const int s = s0 + u;
            float sc_a = 1.f, sc_b = 1.f;
            if (a.dt_scale) {
                sc_a = a.dt_scale[((int64_t)b * T + min(s, T - 1)) * a.H + h];
                sc_b = a.dt_scale[((int64_t)b * T + min(s0 + Q, T - 1)) * a.H + h];
            }
            const float dt = s < T ? fast_softplus(dr_a + dtb) * sc_a : 0.f;
            const float lam = a.trap ? __builtin_amdgcn_rcpf(1.f + fast_exp(-lr_a)) : 1.f;
            // token u+1: lanes 0..62 take it from the next lane, lane 63 from token 64
            float dtn = __shfl_down(dt, 1, 64);
            float lamn = __shfl_down(lam, 1, 64);
            if (lane == 63) {
                dtn = s + 1 < T ? fast_softplus(dr_b + dtb) * sc_b : 0.f;
                lamn = a.trap ? __builtin_amdgcn_rcpf(1.f + fast_exp(-lr_b)) : 1.f;
            }
            const float c2 = wave_incl_scan(A_h * kLog2e * dt, lane);
            const float c2_end = __shfl(c2, 63, 64);
            const float av = a.trap ? lam * dt : dt;
            const float bv = a.trap ? (1.f - lamn) * dtn : 0.f;
            sm.c2[u] = c2;
            sm.ec[u] = __builtin_amdgcn_exp2f(c2);
            sm.w[u] = __builtin_amdgcn_exp2f(c2_end - c2) * (av + bv);
            sm.dt[u] = dt;
            sm.L[u][Q] = av;
            sm.L[u][Q + 1] = bv;
        }
        {
            bf16x8 v0, v1;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float x0 = (float)rawx[j], x1 = (float)rawx[4 + j];
                v0[2 * j] = (bf16)(x0 * mx0);
                v0[2 * j + 1] = (bf16)(x0 * mx1);
                v1[2 * j] = (bf16)(x1 * mx0);
                v1[2 * j + 1] = (bf16)(x1 * mx1);
            }
            *reinterpret_cast<bf16x8*>(&sm.X[xp][16 * tq]) = v0;
            *reinterpret_cast<bf16x8*>(&sm.X[xp][16 * tq + 8]) = v1;
        }
        __syncthreads();
        logdecay += sm.c2[Q - 1] * (1.f / kLog2e);

        // ---- phase 2: angle increments per 8-token group; Lc
        float inc[8];
        {
            float tot = 0.f;
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                inc[j] = sm.dt[8 * tq + j] * (float)rawth[j];
                tot += inc[j];
            }
            sm.tot[tq][pi] = tot;
        }
        if (kFull) {
            // Lc[t][u]: thread t = tid/8 fills u = tid%8 + 8j (strided: conflict-free banks)
            const int t = tid >> 3;
            const int u0 = tid & 7;
            const float ct = sm.c2[t];
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int u = u0 + 8 * j;
                float v = 0.f;
                if (u <= t)
                    v = __builtin_amdgcn_exp2f(ct - sm.c2[u]) * (sm.L[u][Q] + (u < t ? sm.L[u][Q + 1] : 0.f));
                sm.L[t][u] = v;
            }
        }
        __syncthreads();

        // ---- phase 3: rotate B^/C^ into B~/C~/B~w
        {
            float excl = 0.f, all = 0.f;
#pragma unroll
            for (int q = 0; q < 8; ++q) {
                const float tq_tot = sm.tot[q][pi];
                if (q < tq) excl += tq_tot;
                all += tq_tot;
            }
            float phi = phi_run - excl;
            phi_run -= all;
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int u = 8 * tq + j;
                phi -= inc[j];
                float sn = 0.f, cs = 1.f;
                if (a.cplx) fast_sincos(phi, sn, cs);
                const bf16x2 k1 = as_bf16x2(pack_bf16x2(cs, -sn));
                const bf16x2 k2 = as_bf16x2(pack_bf16x2(sn, cs));
                const bf16x2 pb0 = as_bf16x2(rawB[j][0]), pb1 = as_bf16x2(rawB[j][1]);
                const float be0 = __builtin_amdgcn_fdot2_f32_bf16(pb0, k1, 0.f, false);
                const float bo0 = __builtin_amdgcn_fdot2_f32_bf16(pb0, k2, 0.f, false);
                const float be1 = __builtin_amdgcn_fdot2_f32_bf16(pb1, k1, 0.f, false);
                const float bo1 = __builtin_amdgcn_fdot2_f32_bf16(pb1, k2, 0.f, false);
                if (kFull) {
                    const bf16x2 pc0 = as_bf16x2(rawC[j][0]), pc1 = as_bf16x2(rawC[j][1]);
                    const float ce0 = __builtin_amdgcn_fdot2_f32_bf16(pc0, k1, 0.f, false);
                    const float co0 = __builtin_amdgcn_fdot2_f32_bf16(pc0, k2, 0.f, false);
                    const float ce1 = __builtin_amdgcn_fdot2_f32_bf16(pc1, k1, 0.f, false);
                    const float co1 = __builtin_amdgcn_fdot2_f32_bf16(pc1, k2, 0.f, false);
                    *reinterpret_cast<unsigned*>(&sm.C[2 * u][2 * pi]) = pack_bf16x2(ce0, co0);
                    *reinterpret_cast<unsigned*>(&sm.C[2 * u + 1][2 * pi]) = pack_bf16x2(ce1, co1);
                    *reinterpret_cast<unsigned*>(&sm.B[2 * u][2 * pi]) = pack_bf16x2(be0, bo0);
                    *reinterpret_cast<unsigned*>(&sm.B[2 * u + 1][2 * pi]) = pack_bf16x2(be1, bo1);
                }
                const float wu = sm.w[u];
                *reinterpret_cast<u32x2*>(&sm.Bw[u][4 * pi]) =
                    u32x2{pack_bf16x2(be0 * wu, be1 * wu), pack_bf16x2(bo0 * wu, bo1 * wu)};
                // keep one token in flight at a time (bounds register pressure)
                __builtin_amdgcn_sched_barrier(0);
            }
        }
        __syncthreads();

        // ---- phase 4: MFMA contractions. Operand addresses derive from an opaque copy
        // of the lane id so they are recomputed per chunk instead of pinned in VGPRs.
        int lane4 = lane;
        asm volatile("" : "+v"(lane4));
        const int g16 = lane4 >> 4, l16 = lane4 & 15;
        if (kFull) {
            {
                // Output block of this wave: SIMD s runs waves s and s+4, which own the
                // 16-row blocks s and 7-s, so causal work is balanced per SIMD.
                const int I = wv < 4 ? wv : 11 - wv;  // uniform: keeps descriptors scalar
                const int ta = 8 * I + 2 * g16;  // tokens of this lane's output rows: ta, ta+1
                // z of this lane's outputs; consumed by the epilogue after the MFMAs.
                const int tblk = s0 + 8 * I;
                const __amdgpu_buffer_rsrc_t rz = make_rsrc(proj_b + (int64_t)tblk * a.rs,
                                                            (int64_t)max(T - tblk, 0) * a.rs * 2);
                bf16 zraw[4][2];
#pragma unroll
                for (int pt = 0; pt < 4; ++pt)
#pragma unroll
                    for (int tt = 0; tt < 2; ++tt)
                        zraw[pt][tt] = ld_bf16(rz, (2 * g16 + tt) * rs + (int)a.pl.z + h * P + 16 * pt + l16);
                bf16x8 cA[4];
#pragma unroll
                for (int s = 0; s < 4; ++s)
                    cA[s] = *reinterpret_cast<const bf16x8*>(&sm.C[16 * I + l16][32 * s + 8 * g16]);
                f32x4 yacc[4];
                // G3: inter-chunk output, then the e^{c_t} row scale.
#pragma unroll
                for (int pt = 0; pt < 4; ++pt) {
                    yacc[pt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                    for (int s = 0; s < 4; ++s)
                        yacc[pt] = mfma16(cA[s],
                                          *reinterpret_cast<const bf16x8*>(&sm.H[16 * pt + l16][32 * s + 8 * g16]),
                                          yacc[pt]);
                }
                const float ea = sm.ec[ta], eb = sm.ec[ta + 1];
#pragma unroll
                for (int pt = 0; pt < 4; ++pt) {
                    yacc[pt][0] *= ea;
                    yacc[pt][1] *= ea;
                    yacc[pt][2] *= eb;
                    yacc[pt][3] *= eb;
                }
                // G1 + mask + G2.
                const int t_col = 8 * I + (l16 >> 1);
                const int r_col = l16 & 1;
                for (int s2 = 0; s2 <= I / 2; ++s2) {
                    bf16x8 aop;
#pragma unroll
                    for (int jj = 0; jj < 2; ++jj) {
                        const int J = 2 * s2 + jj;
                        float m0 = 0.f, m1 = 0.f, m2 = 0.f, m3 = 0.f;
                        if (J <= I) {
                            f32x4 sacc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                            for (int s = 0; s < 4; ++s)
                                sacc = mfma16(*reinterpret_cast<const bf16x8*>(&sm.B[16 * J + l16][32 * s + 8 * g16]),
                                              cA[s], sacc);
                            const int u0 = 8 * J + 2 * g16;
                            const f32x2 lv = *reinterpret_cast<const f32x2*>(&sm.L[t_col][u0]);
                            m0 = sacc[0] * lv[0];
                            m1 = sacc[1] * lv[0];
                            m2 = sacc[2] * lv[1];
                            m3 = sacc[3] * lv[1];
                            if (J == I) {
                                if (u0 == t_col) { if (r_col == 0) m0 += D_h; else m1 += D_h; }
                                if (u0 + 1 == t_col) { if (r_col == 0) m2 += D_h; else m3 += D_h; }
                            }
                        }
                        aop[4 * jj + 0] = (bf16)m0;
                        aop[4 * jj + 1] = (bf16)m1;
                        aop[4 * jj + 2] = (bf16)m2;
                        aop[4 * jj + 3] = (bf16)m3;
                    }
#pragma unroll
                    for (int pt = 0; pt < 4; ++pt) {
                        const bf16* xr = &sm.X[16 * pt + l16][32 * s2];
                        const bf16x4 lo = *reinterpret_cast<const bf16x4*>(xr + 4 * g16);
                        const bf16x4 hi = *reinterpret_cast<const bf16x4*>(xr + 16 + 4 * g16);
                        const bf16x8 bop = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
                        yacc[pt] = mfma16(aop, bop, yacc[pt]);
                    }
                }
                // Epilogue: SiLU(z * mimo_z) gate and MIMO-down sum over r. Stores go
                // through a descriptor that ends at the last token, so padding rows drop.
                const __amdgpu_buffer_rsrc_t ry = make_rsrc(a.y_out + ((int64_t)b * T + tblk) * HP,
                                                            (int64_t)max(T - tblk, 0) * HP * 2);
#pragma unroll
                for (int pt = 0; pt < 4; ++pt) {
                    const int p = 16 * pt + l16;
#pragma unroll
                    for (int tt = 0; tt < 2; ++tt) {
                        const float z = (float)zraw[pt][tt];
                        const float y0 = yacc[pt][2 * tt], y1 = yacc[pt][2 * tt + 1];
                        const f32x4 g = *reinterpret_cast<const f32x4*>(&sm.mzd[p][0]);
                        const float out = g[2] * y0 * fast_silu(z * g[0]) +
                                          g[3] * y1 * fast_silu(z * g[1]);
                        __builtin_amdgcn_raw_buffer_store_b16(
                            __builtin_bit_cast(unsigned short, (bf16)out), ry,
                            ((2 * g16 + tt) * HP + h * P + p) * 2, 0, 0);
                    }
                }
            }
        }
        if (state_wave) {
            // G4: state update H^T = e^{c_63} H^T + B~w^T X.
            const float dch = sm.ec[Q - 1];
#pragma unroll
            for (int i2 = 0; i2 < kNT; ++i2)
#pragma unroll
                for (int pt = 0; pt < 4; ++pt) hacc[i2][pt] *= dch;
#pragma unroll
            for (int s = 0; s < 4; ++s) {
                bf16x8 bop[4];
#pragma unroll
                for (int pt = 0; pt < 4; ++pt)
                    bop[pt] = *reinterpret_cast<const bf16x8*>(&sm.X[16 * pt + l16][32 * s + 8 * g16]);
#pragma unroll
                for (int i2 = 0; i2 < kNT; ++i2) {
                    const int n = 16 * (nt0 + i2) + l16;
                    bf16x8 aop;
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        const bf16x2 v = *reinterpret_cast<const bf16x2*>(&sm.Bw[16 * s + 4 * g16 + j][2 * n]);
                        aop[2 * j] = v[0];
                        aop[2 * j + 1] = v[1];
                    }
#pragma unroll
                    for (int pt = 0; pt < 4; ++pt) hacc[i2][pt] = mfma16(aop, bop[pt], hacc[i2][pt]);
                }
            }
        }
        // Next chunk's element-wise inputs (reads past T return zero); they arrive while
        // the other waves finish this chunk.
        if (k + 1 < k_end) load_prep(k + 1);
    }

    // ---- segment end
    if (!kFull) {
        const int64_t sidx = (int64_t)bh * (a.S - 1) + seg;
        float* out = a.seg_state + sidx * (int64_t)N * P;
#pragma unroll
        for (int i2 = 0; i2 < kNT; ++i2) {
            const int n0 = 16 * (nt0 + i2) + 4 * g16;
#pragma unroll
            for (int pt = 0; pt < 4; ++pt)
#pragma unroll
                for (int v = 0; v < 4; ++v) out[(n0 + v) * P + 16 * pt + l16] = hacc[i2][pt][v];
        }
        if (tid == 0) a.seg_decay[sidx] = logdecay;
        if (wave == 0) a.seg_angle[sidx * NH + pi] = phi_run;
    } else if (seg == a.S - 1) {
        __syncthreads();
        if (wave == 0) {
            sm.rot[pi] = phi_start;
            if (a.angle) a.angle[(int64_t)bh * NH + pi] = a.cplx ? phi_start + phi_run : 0.f;
        }
        __syncthreads();
        if (a.h_final && state_wave) {
            float* hf = a.h_final + (int64_t)bh * P * N;
#pragma unroll
            for (int i2 = 0; i2 < kNT; ++i2) {
                const int n0 = 16 * (nt0 + i2) + 4 * g16;
                float s0, c0, s1, c1;
                sincosf(sm.rot[n0 / 2], &s0, &c0);
                sincosf(sm.rot[n0 / 2 + 1], &s1, &c1);
#pragma unroll
                for (int pt = 0; pt < 4; ++pt) {
                    const f32x4 v = hacc[i2][pt];
                    const f32x4 o = {v[0] * c0 - v[1] * s0, v[0] * s0 + v[1] * c0,
                                     v[2] * c1 - v[3] * s1, v[2] * s1 + v[3] * c1};
                    *reinterpret_cast<f32x4*>(&hf[(16 * pt + l16) * N + n0]) = o;
                }
            }
        }
        if (a.prev_bx) {
            // prev_BX = B~_{T-1} x_{T-1}^T, from the last chunk's tiles (still in LDS),
            // rotated to the absolute frame. Thread: column pair pi, rows p = 8*wave..+7.
            const int ul = (T - 1) - (K - 1) * Q;
            float sn, cs;
            sincosf(sm.rot[pi], &sn, &cs);
            const float be0 = (float)sm.B[2 * ul][2 * pi], bo0 = (float)sm.B[2 * ul][2 * pi + 1];
            const float be1 = (float)sm.B[2 * ul + 1][2 * pi], bo1 = (float)sm.B[2 * ul + 1][2 * pi + 1];
            const float ae0 = be0 * cs - bo0 * sn, ao0 = be0 * sn + bo0 * cs;
            const float ae1 = be1 * cs - bo1 * sn, ao1 = be1 * sn + bo1 * cs;
            float* pb = a.prev_bx + (int64_t)bh * P * N;
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int p = 8 * wave + j;
                const float x0 = (float)sm.X[p][2 * ul], x1 = (float)sm.X[p][2 * ul + 1];
                *reinterpret_cast<f32x2*>(&pb[p * N + 2 * pi]) =
                    f32x2{ae0 * x0 + ae1 * x1, ao0 * x0 + ao1 * x1};
            }
        }
    }
}

}  // namespace mf

bool mfma_prefill_supported(const m3_layer_desc& d, const void* proj) {
    if (d.dtype != M3_DTYPE_BF16) return false;
    if (d.d_state != mf::N || d.headdim != mf::P || d.mimo_rank != mf::R) return false;
    const ProjLayout pl = proj_layout(d);
    if (d.proj_row_stride % 4 != 0 || pl.B % 4 != 0 || pl.C % 4 != 0) return false;
    if (reinterpret_cast<uintptr_t>(proj) % 8 != 0) return false;
    // 32-bit buffer offsets: one batch row of proj (and of B^/C^) stays below 2 GiB.
    if ((int64_t)(d.seqlen + 1) * d.proj_row_stride * 2 >= ((int64_t)1 << 31)) return false;
    if ((int64_t)(d.seqlen + 1) * d.ngroups * mf::NR * 2 >= ((int64_t)1 << 31)) return false;
    return true;
}

// Segments per (batch, head). One workgroup occupies a CU, so the full pass takes
// ceil(B*H*S / 256) rounds of ceil(K/S) chunks, and the state-only pass adds about a third
// of that per segment but the last. Pick the S that minimises this estimate.
static void mfma_segments(const m3_layer_desc& d, int& S, int& cps) {
    const int K = (d.seqlen + mf::Q - 1) / mf::Q;
    const int64_t bh = (int64_t)d.batch * d.nheads;
    const int64_t cus = 256;
    double best = 1e30;
    S = 1;
    for (int s = 1; s <= std::min(K, 64); ++s) {
        const int c = (K + s - 1) / s;
        const int seff = (K + c - 1) / c;
        const double full = (double)((bh * seff + cus - 1) / cus) * c;
        const double part = seff > 1 ? 0.35 * (double)((bh * (seff - 1) + cus - 1) / cus) * c : 0.0;
        const double cost = full + part + 0.5 * seff;  // small per-segment combine cost
        if (cost < best - 1e-9) {
            best = cost;
            S = seff;
        }
    }
    cps = (K + S - 1) / S;
    S = (K + cps - 1) / cps;
}

size_t mfma_prefill_workspace(const m3_layer_desc& d) {
    int S, cps;
    mfma_segments(d, S, cps);
    const size_t ntg = (size_t)d.batch * d.seqlen * d.ngroups;
    const size_t nseg = (size_t)d.batch * d.nheads * (S - 1);
    const size_t bc_bytes = 2 * ntg * mf::NR * sizeof(bf16);
    return bc_bytes + nseg * ((size_t)mf::N * mf::P + 1 + mf::NH) * sizeof(float) + 256;
}

int launch_mfma_prefill(const m3_layer_desc& d, const m3_layer_params& p, const void* proj,
                        const float* dt_scale, void* y_out, float* h_final, float* angle,
                        float* prev_bx, void* workspace, hipStream_t stream) {
    int S, cps;
    mfma_segments(d, S, cps);
    mf::Args a;
    a.B = d.batch; a.T = d.seqlen; a.H = d.nheads; a.G = d.ngroups; a.S = S; a.cps = cps;
    a.trap = d.use_trapezoidal; a.cplx = d.use_complex;
    a.rs = d.proj_row_stride;
    a.pl = proj_layout(d);
    a.prm = p;
    a.proj = reinterpret_cast<const bf16*>(proj);
    a.dt_scale = dt_scale;
    const int64_t ntg = (int64_t)d.batch * d.seqlen * d.ngroups;
    const int64_t nseg = (int64_t)d.batch * d.nheads * (S - 1);
    bf16* bn = reinterpret_cast<bf16*>(workspace);
    bf16* cn = bn + ntg * mf::NR;
    float* ws = reinterpret_cast<float*>(cn + ntg * mf::NR);
    a.Bn = bn;
    a.Cn = cn;
    a.seg_state = ws;
    a.seg_decay = a.seg_state + nseg * mf::N * mf::P;
    a.seg_angle = a.seg_decay + nseg;
    a.y_out = reinterpret_cast<bf16*>(y_out);
    a.h_final = h_final;
    a.angle = angle;
    a.prev_bx = prev_bx;

    hipLaunchKernelGGL(mf::bc_norm, dim3((unsigned)((ntg + 3) / 4)), dim3(256), 0, stream,
                       a.proj, a.rs, a.pl.B, a.pl.C, a.G, ntg, d.rms_eps, p.B_norm_w, p.B_bias,
                       p.C_norm_w, p.C_bias, bn, cn);
    if (S > 1)
        hipLaunchKernelGGL(mf::ssd_chunks<false>, dim3((unsigned)(d.batch * d.nheads * (S - 1))),
                           dim3(mf::THREADS), 0, stream, a);
    hipLaunchKernelGGL(mf::ssd_chunks<true>, dim3((unsigned)(d.batch * d.nheads * S)),
                       dim3(mf::THREADS), 0, stream, a);
    return hipGetLastError() == hipSuccess ? M3_OK : M3_ERR_LAUNCH;
}

}  // namespace m3
