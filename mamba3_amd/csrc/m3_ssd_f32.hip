// Fused chunked-SSD prefill in fp32 for d_state 128 / headdim 64 / rank 2 (the d_model 768
// KulaMamba in fp32), gfx950.
//
// Same algorithm and formulation as the bf16 MFMA kernel (m3_ssd_mfma.hip): the quadratic
// form inside a chunk and the state carried across chunks (mamba3/ssd.py:118-244), with the
// layer's preparation fused (mamba3/mamba3.py:197-256), the trapezoid folded into
// a_u = lambda_u dt_u and b_u = (1 - lambda_{u+1}) dt_{u+1} so the contraction rank stays R.
// Every operand stays fp32: the contractions run on v_mfma_f32_16x16x4_f32 (lane l supplies
// A[l%16][l/16] and B[l/16][l%16]; it holds D[4(l/16)+v][l%16]).
//
// Two launches:
//   1. bc_norm_f32: per (token, group), B^ = RMSNorm(B) * w + bias and C^ likewise, fp32, in
//      the reference's (n, r) order (mamba3/mamba3.py:19-35, 147-157).
//   2. ssd_f32<PB>: one 512-thread workgroup (8 waves) per (batch, head, block of PB of the 64
//      headdim columns) walks the sequence in chunks of Q = 32 tokens (rows (t, r) = 2t + r,
//      64 rows), carrying its columns of the fp32 state H^T [n][p] in MFMA accumulators (wave
//      w owns rows n = 16w .. 16w+15). PB = 32 when the (batch, head) pairs alone leave CUs
//      idle: two workgroups per pair then repeat the scores and the rotation. Per chunk:
//        prep   token scalars; X rows x_u mimo_x[r] and z into LDS; the state copy H;
//               the RoPE angles (a prefix over 8 groups of 4 tokens per pair) and the
//               rotated C~ / B~ tiles (mamba3/mamba3.py:38-45, 160-166)
//        G1     S = (C~ B~^T) * Lc on the 10 causal 16 x 16 blocks, into LDS, with
//               Lc[t][u] = [u<=t] exp(c_t - c_u) (a_u + [u<t] b_u) and D on the diagonal
//        G3+G2  Y = diag(e^{c_t}) C~ H^T + S X (waves: 16-row block w/2, PB/2 columns)
//        G4     H^T = e^{c_end} H^T + (B~ diag(w))^T X, w_u = e^{c_end - c_u} (a_u + b_u)
//        gate   out = sum_r mimo_down_r silu(z mimo_z_r) y_r (mamba3/mamba3.py:233-239)
//      The angles stay absolute (the walk starts at t = 0), so the final state, angle and
//      prev_BX = B~_{T-1} x_r,{T-1}^T need no frame change (mamba3/mamba3.py:241-256).
//      For the training forward (M3_FLAG_FOR_BACKWARD) the walk also stores, from the
//      values it holds, the per-token operands the layer backward reads, in the staged
//      fp32 layer path's layouts (m3_layer_fp32.hip), instead of that path's five launches.
// LDS rows have odd strides (in 32-bit words), so the column reads of the MFMA operands (16
// lanes on 16 rows) hit distinct banks.
#include "m3_common.h"
#include "m3_kernels.h"
#include "m3_mfma.h"

namespace m3 {
namespace f32k {

constexpr int Q = 32;
constexpr int N = 128;
constexpr int P = 64;
constexpr int R = 2;
constexpr int NR = N * R;
constexpr int NH = N / 2;
constexpr int ROWS = Q * R;
constexpr int THREADS = 512;
constexpr int CST = N + 1;
constexpr int SST = ROWS + 1;

template <int PB>
struct Smem {
    float C[ROWS][CST];      // C~ rows (t, r)
    float B[ROWS][CST];      // B~ rows (u, r)
    float X[ROWS][PB + 1];   // x_u mimo_x[p, r], rows (u, r), this block's columns
    float S[ROWS][SST];      // masked scores, rows (t, r), columns (u, r')
    float H[N][PB + 1];      // state H^T at the chunk start, this block's columns
    float Z[Q][PB];          // z
    float part[8][NH];       // per 4-token group: sum of dt theta, per pair
    float phi_run[2][NH];    // pair angles at the end of the previous chunk (by chunk parity)
    float dtv[Q + 1], lamv[Q + 1];  // dt and lambda of the chunk's tokens and the next one
    float c[Q], ec[Q], av[Q], bv[Q], w[Q];
};

struct Args {
    int B, T, H, G;
    int trap, cplx;
    int64_t rs;
    ProjLayout pl;
    m3_layer_params prm;
    const float* proj;
    const float* dt_scale;
    const float* Bn;  // [B*T][G][NR]
    const float* Cn;
    float* y_out;     // [B][T][H*P]
    float* h_final;   // [B][H][P][N] or null
    float* angle;     // [B][H][NH] or null
    float* prev_bx;   // [B][H][P][N] or null
    // With stage set, the per-token operands the layer backward reads (the staged fp32
    // layer's layouts, token row (b T + t) H + h): dt, A, angles, x_r, x_g, x_b, B~, B~ of
    // the previous token, C~ and y before the gate.
    Fp32LayerParts st;
    int stage;
    // With hs_every > 0 the walk also stores its chunk-start states into st.Hs in the layer
    // backward's chunking: the state entering every hs_every-th chunk k at entry k / hs_every
    // of (B, hs_K + 1, H, P, N) (the zero start at entry 0), and the final state at entry hs_K.
    int hs_every, hs_K;
};

__device__ __forceinline__ f32x4 mfma4(float a, float b, const f32x4& c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// exp through the hardware exp2 (relative error ~1e-7 for the arguments here: decays and
// gate inputs), and SiLU on it
__device__ __forceinline__ float exp_hw(float x) { return __builtin_amdgcn_exp2f(x * kLog2e); }
__device__ __forceinline__ float silu_hw(float x) { return x * __builtin_amdgcn_rcpf(1.f + exp_hw(-x)); }

__global__ __launch_bounds__(256) void bc_norm_f32(const float* __restrict__ proj, int64_t rs,
                                                   int64_t offB, int64_t offC, int G,
                                                   int64_t nrows, float eps,
                                                   const float* __restrict__ wB,
                                                   const float* __restrict__ biasB,
                                                   const float* __restrict__ wC,
                                                   const float* __restrict__ biasC,
                                                   float* __restrict__ Bn, float* __restrict__ Cn) {
    const int lane = threadIdx.x & 63;
    const int64_t tg = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (tg >= nrows) return;
    const int64_t tok = tg / G;
    const int g = (int)(tg % G);
    const float* row = proj + tok * rs;
    const int e = 4 * lane;
    const f32x4 vb = *reinterpret_cast<const f32x4*>(row + offB + (int64_t)g * NR + e);
    const f32x4 vc = *reinterpret_cast<const f32x4*>(row + offC + (int64_t)g * NR + e);
    const f32x4 wb = *reinterpret_cast<const f32x4*>(wB + e);
    const f32x4 wc = *reinterpret_cast<const f32x4*>(wC + e);
    const f32x4 bb = *reinterpret_cast<const f32x4*>(biasB + (int64_t)g * NR + e);
    const f32x4 bc = *reinterpret_cast<const f32x4*>(biasC + (int64_t)g * NR + e);
    float sb = 0.f, sc = 0.f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        sb += vb[j] * vb[j];
        sc += vc[j] * vc[j];
    }
    sb = lane_sum<64>(sb);
    sc = lane_sum<64>(sc);
    const float rb = rsqrtf(sb / NR + eps), rc = rsqrtf(sc / NR + eps);
    f32x4 ob, oc;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        ob[j] = vb[j] * rb * wb[j] + bb[j];
        oc[j] = vc[j] * rc * wc[j] + bc[j];
    }
    *reinterpret_cast<f32x4*>(Bn + tg * NR + e) = ob;
    *reinterpret_cast<f32x4*>(Cn + tg * NR + e) = oc;
}

template <int PB>
__global__ __launch_bounds__(THREADS, 1) void ssd_f32(Args a) {
    constexpr int NPT = PB / 16;          // column tiles of the block
    constexpr int TPW = NPT / 2;          // output tiles per wave (row block wave / 2)
    constexpr int XE = PB * Q / THREADS;  // X / Z elements per thread
    constexpr int NPE = PB * N / THREADS; // prev_BX elements per thread
    __shared__ Smem<PB> sm;
    const int tid = threadIdx.x;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lane = tid & 63;
    const int l16 = lane & 15, g4 = lane >> 4;

    // XCD-aware order: consecutive workgroups of one batch row land on one XCD.
    const int nblk = gridDim.x;
    const int blk = (nblk % 8 == 0) ? (blockIdx.x % 8) * (nblk / 8) + blockIdx.x / 8 : blockIdx.x;
    const int bh = blk / (P / PB);
    const int pc = (blk % (P / PB)) * PB;  // first headdim column of the block
    const int b = bh / a.H, h = bh % a.H;
    const int grp = h / (a.H / a.G);
    const int T = a.T;
    const int K = (T + Q - 1) / Q;
    const int HP = a.H * P;

    const float Ah = -expf(a.prm.A_log[h]);
    const float Dh = a.prm.D[h];
    const float dtb = a.prm.dt_bias[h];
    const float* prow = a.proj + (int64_t)b * T * a.rs;

    // prep roles: X / Z element block (token xu, block columns xp .. xp + XE - 1), and the
    // rotation job (tokens 4 wv .. 4 wv + 3 of pair lane)
    const int xu = tid >> 4, xp = XE * (tid & 15);
    float mx0[XE], mx1[XE];
#pragma unroll
    for (int j = 0; j < XE; ++j) {
        mx0[j] = a.prm.mimo_x[(h * P + pc + xp + j) * R];
        mx1[j] = a.prm.mimo_x[(h * P + pc + xp + j) * R + 1];
    }
    // output roles: row block I, block column tiles ptb .. ptb + TPW - 1
    const int I = wv >> 1;
    const int ptb = TPW * (wv & 1);
    float mz[TPW][2], md[TPW][2];
#pragma unroll
    for (int q = 0; q < TPW; ++q)
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int p = pc + 16 * (ptb + q) + l16;
            mz[q][r] = a.prm.mimo_z[(h * P + p) * R + r];
            md[q][r] = a.prm.mimo_down[(h * P + p) * R + r];
        }
    if (tid < NH) sm.phi_run[0][tid] = 0.f;
    const bool st_head = a.stage && pc == 0;  // per-(token, head) operands: one block writes them
    if (st_head && tid == 0) a.st.A[h] = Ah;

    f32x4 hacc[NPT];
#pragma unroll
    for (int pt = 0; pt < NPT; ++pt) hacc[pt] = f32x4{0.f, 0.f, 0.f, 0.f};

    // Raw reads of one chunk (tokens past T read nothing and keep zeros): dt / lambda /
    // dt_scale of token tid (tid <= Q, one past the chunk for b_u), x and z of token xu, and
    // the B^ / C^ rows and theta of tokens 4 wv .. 4 wv + 3, pair lane. Issued a chunk ahead.
    float rdt = 0.f, rlam = 0.f, rsc = 1.f;
    float xv[XE], zv[XE];
    f32x4 rb[4], rc[4];
    float th[4];
    auto load_chunk = [&](int kk) {
        const int s0n = kk * Q;
        if (tid <= Q && s0n + tid < T) {
            const float* pr = prow + (int64_t)(s0n + tid) * a.rs;
            rdt = pr[a.pl.dt + h];
            if (a.trap) rlam = pr[a.pl.lam + h];
            if (a.dt_scale) rsc = a.dt_scale[((int64_t)b * T + s0n + tid) * a.H + h];
        }
#pragma unroll
        for (int j = 0; j < XE; ++j) xv[j] = zv[j] = 0.f;
        if (s0n + xu < T) {
            const float* pr = prow + (int64_t)(s0n + xu) * a.rs + h * P + pc + xp;
#pragma unroll
            for (int j = 0; j < XE; ++j) {
                xv[j] = pr[a.pl.x + j];
                zv[j] = pr[a.pl.z + j];
            }
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int tok = s0n + 4 * wv + j;
            rb[j] = f32x4{0.f, 0.f, 0.f, 0.f};
            rc[j] = f32x4{0.f, 0.f, 0.f, 0.f};
            th[j] = 0.f;
            if (tok < T) {
                const int64_t row = (((int64_t)b * T + tok) * a.G + grp) * NR + 4 * lane;
                rb[j] = *reinterpret_cast<const f32x4*>(a.Bn + row);
                rc[j] = *reinterpret_cast<const f32x4*>(a.Cn + row);
                if (a.cplx) th[j] = prow[(int64_t)tok * a.rs + a.pl.theta + lane];
            }
        }
    };
    load_chunk(0);

    for (int k = 0; k < K; ++k) {
        const int s0 = k * Q;
        const int par = k & 1;
        __syncthreads();  // the previous chunk's tiles are consumed
        // ---- prep 1: token scalars, X / Z rows and the state copy into LDS, from the raw
        // reads issued during the previous chunk's contractions
        if (tid <= Q) {
            float dt = 0.f, lam = 1.f;
            if (s0 + tid < T) {
                dt = softplus_f(rdt + dtb) * rsc;
                if (a.trap) lam = sigmoid_f(rlam);
            }
            sm.dtv[tid] = dt;
            sm.lamv[tid] = lam;
            if (st_head && tid < Q && s0 + tid < T) a.st.dt[((int64_t)b * T + s0 + tid) * a.H + h] = dt;
        }
#pragma unroll
        for (int j = 0; j < XE; ++j) {
            sm.X[2 * xu][xp + j] = xv[j] * mx0[j];
            sm.X[2 * xu + 1][xp + j] = xv[j] * mx1[j];
            sm.Z[xu][xp + j] = zv[j];
        }
#pragma unroll
        for (int pt = 0; pt < NPT; ++pt)
#pragma unroll
            for (int v = 0; v < 4; ++v) sm.H[16 * wv + 4 * g4 + v][16 * pt + l16] = hacc[pt][v];
        if (a.hs_every > 0 && k == 0) {  // the zero start state
            float* hk = a.st.Hs + ((int64_t)b * (a.hs_K + 1) * a.H + h) * (P * N) + (int64_t)pc * N;
#pragma unroll
            for (int pt = 0; pt < NPT; ++pt)
                *reinterpret_cast<f32x4*>(&hk[(16 * pt + l16) * N + 16 * wv + 4 * g4]) = hacc[pt];
        }
        __syncthreads();
        if (a.stage && s0 + xu < T) {
            // x_r, x_g = lambda_t x_r and x_b of the next token = (1 - lambda_{t+1})
            // exp(A dt_{t+1}) x_r (mamba3/mamba3.py:210-224), this thread's X elements
            const int64_t e0 = (((int64_t)b * T + s0 + xu) * a.H + h) * (P * R) + (int64_t)(pc + xp) * R;
            const float lam = sm.lamv[xu];
            const float sbn = a.trap ? (1.f - sm.lamv[xu + 1]) * expf(Ah * sm.dtv[xu + 1]) : 0.f;
#pragma unroll
            for (int j = 0; j < XE; ++j) {
                const f32x2 xr = f32x2{xv[j] * mx0[j], xv[j] * mx1[j]};
                *reinterpret_cast<f32x2*>(a.st.xr + e0 + j * R) = xr;
                *reinterpret_cast<f32x2*>(a.st.xg + e0 + j * R) = xr * lam;
                if (a.trap) {
                    if (s0 + xu + 1 < T) *reinterpret_cast<f32x2*>(a.st.xb + e0 + (int64_t)a.H * P * R + j * R) = xr * sbn;
                    if (s0 + xu == 0) *reinterpret_cast<f32x2*>(a.st.xb + e0 + j * R) = f32x2{0.f, 0.f};
                }
            }
        }
        // ---- prep 2: chunk scalars (wave 0, lane = token: a prefix scan of A dt) and the
        // angle partial sums
        if (wv == 0) {
            const bool in = lane < Q;
            const float dt = in ? sm.dtv[lane] : 0.f;
            const float c = wave_incl_scan(Ah * dt);
            const float cend = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, c), Q - 1));
            if (in) {
                const float av = a.trap ? sm.lamv[lane] * dt : dt;
                const float bv = a.trap ? (1.f - sm.lamv[lane + 1]) * sm.dtv[lane + 1] : 0.f;
                sm.c[lane] = c;
                sm.ec[lane] = exp_hw(c);
                sm.av[lane] = av;
                sm.bv[lane] = bv;
                sm.w[lane] = exp_hw(cend - c) * (av + bv);
            }
        }
        {
            float ps = 0.f;
#pragma unroll
            for (int j = 0; j < 4; ++j) ps += sm.dtv[4 * wv + j] * th[j];
            sm.part[wv][lane] = ps;
        }
        __syncthreads();
        // ---- prep 3: angles and the rotated C~ / B~ rows of tokens 4 wv .. 4 wv + 3, pair lane
        {
            float phi = sm.phi_run[par][lane];
            for (int g = 0; g < wv; ++g) phi -= sm.part[g][lane];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int t = 4 * wv + j;
                phi -= sm.dtv[t] * th[j];
                float sn, cs;
                sincosf(phi, &sn, &cs);
                f32x4 bt, ct;  // (n=2i, r0) (2i, r1) (2i+1, r0) (2i+1, r1)
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    // pair lane holds (n=2i, r0) (2i, r1) (2i+1, r0) (2i+1, r1)
                    const float be = rb[j][r], bo = rb[j][2 + r];
                    const float ce = rc[j][r], co = rc[j][2 + r];
                    bt[r] = be * cs - bo * sn;
                    bt[2 + r] = be * sn + bo * cs;
                    ct[r] = ce * cs - co * sn;
                    ct[2 + r] = ce * sn + co * cs;
                    sm.B[2 * t + r][2 * lane] = bt[r];
                    sm.B[2 * t + r][2 * lane + 1] = bt[2 + r];
                    sm.C[2 * t + r][2 * lane] = ct[r];
                    sm.C[2 * t + r][2 * lane + 1] = ct[2 + r];
                }
                if (st_head && s0 + t < T) {
                    const int64_t tk = ((int64_t)b * T + s0 + t) * a.H + h;
                    *reinterpret_cast<f32x4*>(a.st.Bt + tk * NR + 4 * lane) = bt;
                    *reinterpret_cast<f32x4*>(a.st.Ct + tk * NR + 4 * lane) = ct;
                    if (a.trap) {
                        if (s0 + t + 1 < T) *reinterpret_cast<f32x4*>(a.st.Bb + (tk + a.H) * NR + 4 * lane) = bt;
                        if (s0 + t == 0) *reinterpret_cast<f32x4*>(a.st.Bb + tk * NR + 4 * lane) = f32x4{0.f, 0.f, 0.f, 0.f};
                    }
                    a.st.phi[tk * NH + lane] = phi;
                }
            }
            if (wv == 7) sm.phi_run[par ^ 1][lane] = phi;
        }
        if (k + 1 < K) load_chunk(k + 1);  // consumed by the next chunk's prep
        __syncthreads();
        // ---- G1: masked scores of the causal blocks (I, J), J <= I; wave w takes blocks w
        // and w + 8 of the list (0,0) (1,0) (1,1) (2,0) (2,1) (2,2) (3,0) (3,1) (3,2) (3,3)
        for (int blk = wv; blk < 10; blk += 8) {
            const int bI = blk < 1 ? 0 : blk < 3 ? 1 : blk < 6 ? 2 : 3;
            const int bJ = blk - (bI * (bI + 1)) / 2;
            f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll 8
            for (int k0 = 0; k0 < N; k0 += 4)
                acc = mfma4(sm.C[16 * bI + l16][k0 + g4], sm.B[16 * bJ + l16][k0 + g4], acc);
            const int col = 16 * bJ + l16;
            const int u = col >> 1, rp = col & 1;
            const float cu = sm.c[u], au = sm.av[u], bu = sm.bv[u];
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const int row = 16 * bI + 4 * g4 + v;
                const int t = row >> 1, r = row & 1;
                float s = 0.f;
                if (u <= t) {
                    s = acc[v] * exp_hw(sm.c[t] - cu) * (au + (u < t ? bu : 0.f));
                    if (u == t && r == rp) s += Dh;
                }
                sm.S[row][col] = s;
            }
        }
        __syncthreads();
        // ---- G3 + G2: output rows 16 I .. 16 I + 15, block columns 16 (ptb + q) + l16
        f32x4 yacc[TPW];
#pragma unroll
        for (int q = 0; q < TPW; ++q) yacc[q] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll 4
        for (int k0 = 0; k0 < N; k0 += 4) {
            const float av = sm.C[16 * I + l16][k0 + g4];
#pragma unroll
            for (int q = 0; q < TPW; ++q) yacc[q] = mfma4(av, sm.H[k0 + g4][16 * (ptb + q) + l16], yacc[q]);
        }
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const float e = sm.ec[(16 * I + 4 * g4 + v) >> 1];
#pragma unroll
            for (int q = 0; q < TPW; ++q) yacc[q][v] *= e;
        }
        for (int k0 = 0; k0 < 16 * (I + 1); k0 += 4) {
            const float sv = sm.S[16 * I + l16][k0 + g4];
#pragma unroll
            for (int q = 0; q < TPW; ++q) yacc[q] = mfma4(sv, sm.X[k0 + g4][16 * (ptb + q) + l16], yacc[q]);
        }
        // ---- G4: state update on this wave's rows n = 16 wv .. 16 wv + 15
        {
            const float dec = sm.ec[Q - 1];
#pragma unroll
            for (int pt = 0; pt < NPT; ++pt) hacc[pt] *= dec;
#pragma unroll 4
            for (int k0 = 0; k0 < ROWS; k0 += 4) {
                const float bw = sm.B[k0 + g4][16 * wv + l16] * sm.w[(k0 + g4) >> 1];
#pragma unroll
                for (int pt = 0; pt < NPT; ++pt) hacc[pt] = mfma4(bw, sm.X[k0 + g4][16 * pt + l16], hacc[pt]);
            }
        }
        // ---- the state entering chunk k + 1 for the layer backward. The walk folds the beta
        // term of the next chunk's first token into this chunk (b_{Q-1} B~_{Q-1} x_{Q-1}^T, the
        // last row pair of the tiles); the chunk kernels count it in the next chunk, so it is
        // taken out of the stored state (b = 0 without the trapezoid).
        if (a.hs_every > 0 && (k + 1) % a.hs_every == 0 && k + 1 < K) {
            const float bq = sm.bv[Q - 1];
            float* hk = a.st.Hs + (((int64_t)b * (a.hs_K + 1) + (k + 1) / a.hs_every) * a.H + h) * (P * N) +
                        (int64_t)pc * N;
#pragma unroll
            for (int pt = 0; pt < NPT; ++pt) {
                const int pl = 16 * pt + l16;
                const float x0 = sm.X[2 * (Q - 1)][pl], x1 = sm.X[2 * (Q - 1) + 1][pl];
                f32x4 o;
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    const int n = 16 * wv + 4 * g4 + v;
                    o[v] = hacc[pt][v] - bq * (sm.B[2 * (Q - 1)][n] * x0 + sm.B[2 * (Q - 1) + 1][n] * x1);
                }
                *reinterpret_cast<f32x4*>(&hk[pl * N + 16 * wv + 4 * g4]) = o;
            }
        }
        // ---- gate and MIMO-down; rows 4 g4 + 2 tt + r of the block are (t, r)
#pragma unroll
        for (int q = 0; q < TPW; ++q) {
            const int pl = 16 * (ptb + q) + l16;  // block column
#pragma unroll
            for (int tt = 0; tt < 2; ++tt) {
                const int t = 8 * I + 2 * g4 + tt;
                if (s0 + t < T) {
                    if (a.stage)
                        *reinterpret_cast<f32x2*>(a.st.ys + (((int64_t)b * T + s0 + t) * a.H + h) * (P * R) + (int64_t)(pc + pl) * R) =
                            f32x2{yacc[q][2 * tt], yacc[q][2 * tt + 1]};
                    const float z = sm.Z[t][pl];
                    const float o = md[q][0] * yacc[q][2 * tt] * silu_hw(z * mz[q][0]) +
                                    md[q][1] * yacc[q][2 * tt + 1] * silu_hw(z * mz[q][1]);
                    a.y_out[((int64_t)b * T + s0 + t) * HP + h * P + pc + pl] = o;
                }
            }
        }
    }
    __syncthreads();
    // ---- outputs of the walk
    if (a.hs_every > 0) {
        float* hk = a.st.Hs + (((int64_t)b * (a.hs_K + 1) + a.hs_K) * a.H + h) * (P * N) + (int64_t)pc * N;
#pragma unroll
        for (int pt = 0; pt < NPT; ++pt)
            *reinterpret_cast<f32x4*>(&hk[(16 * pt + l16) * N + 16 * wv + 4 * g4]) = hacc[pt];
    }
    if (a.h_final) {
        float* hf = a.h_final + (int64_t)bh * P * N + (int64_t)pc * N;
#pragma unroll
        for (int pt = 0; pt < NPT; ++pt)
            *reinterpret_cast<f32x4*>(&hf[(16 * pt + l16) * N + 16 * wv + 4 * g4]) = hacc[pt];
    }
    if (a.angle && pc == 0 && tid < NH) a.angle[(int64_t)bh * NH + tid] = a.cplx ? sm.phi_run[K & 1][tid] : 0.f;
    if (a.prev_bx) {
        // B~_{T-1} x_r,{T-1}^T from the last chunk's tiles (still in LDS)
        const int ul = (T - 1) - (K - 1) * Q;
        const int p = tid / (N / NPE), n0 = NPE * (tid % (N / NPE));  // block column p
        const float x0 = sm.X[2 * ul][p], x1 = sm.X[2 * ul + 1][p];
        float* pb = a.prev_bx + (int64_t)bh * P * N + (int64_t)(pc + p) * N + n0;
#pragma unroll
        for (int j = 0; j < NPE; j += 4) {
            f32x4 o;
#pragma unroll
            for (int e = 0; e < 4; ++e) o[e] = sm.B[2 * ul][n0 + j + e] * x0 + sm.B[2 * ul + 1][n0 + j + e] * x1;
            *reinterpret_cast<f32x4*>(pb + j) = o;
        }
    }
}

}  // namespace f32k

static bool fused_fp32_shape_ok(const m3_layer_desc& d, const void* proj, const void* y_out,
                                const void* h_final, const void* prev_bx) {
    if (d.dtype != M3_DTYPE_F32) return false;
    if (d.d_state != f32k::N || d.headdim != f32k::P || d.mimo_rank != f32k::R) return false;
    const ProjLayout pl = proj_layout(d);
    // 16-byte reads of the B / C rows and of x / z
    if (d.proj_row_stride % 4 != 0 || pl.x % 4 != 0 || pl.z % 4 != 0 || pl.B % 4 != 0 || pl.C % 4 != 0)
        return false;
    auto al16 = [](const void* ptr) { return reinterpret_cast<uintptr_t>(ptr) % 16 == 0; };
    if (!al16(proj) || !al16(y_out) || !al16(h_final) || !al16(prev_bx)) return false;
    return true;
}

bool fused_fp32_prefill_supported(const m3_layer_desc& d, const void* proj, const void* y_out,
                                  const void* h_final, const void* prev_bx) {
    return !(d.flags & M3_FLAG_FOR_BACKWARD) && fused_fp32_shape_ok(d, proj, y_out, h_final, prev_bx);
}

bool fused_fp32_train_supported(const m3_layer_desc& d, const void* proj, const void* y_out,
                                const void* h_final, const void* prev_bx) {
    if (!fused_fp32_shape_ok(d, proj, y_out, h_final, prev_bx) || !fp32_layer_supported(d)) return false;
    size_t bytes = 0;
    fp32_layer_scratch(d, nullptr, &bytes);
    return bytes >= fused_fp32_prefill_workspace(d);
}

size_t fused_fp32_prefill_workspace(const m3_layer_desc& d) {
    return 2 * (size_t)d.batch * d.seqlen * d.ngroups * f32k::NR * sizeof(float) + 256;
}

int launch_fused_fp32_prefill(const m3_layer_desc& d, const m3_layer_params& p, const void* proj,
                              const float* dt_scale, void* y_out, float* h_final, float* angle,
                              float* prev_bx, void* workspace, hipStream_t stream,
                              const Fp32LayerParts* stage) {
    const ProjLayout pl = proj_layout(d);
    const int64_t nrows = (int64_t)d.batch * d.seqlen * d.ngroups;
    float* bn = reinterpret_cast<float*>(workspace);
    float* cn = bn + nrows * f32k::NR;
    // Training forward with room for the chunk-start states (workspace = the fp32 layer
    // workspace's chunk-kernel region, whose Hs part is stage->Hs): C^ rows past them.
    const bool hs = stage && stage->Hs && fp32_layer_hs_ok(d);
    int hs_every = 0, hs_K = 0;
    if (hs) {
        const bool trap = d.use_trapezoidal != 0;
        const size_t off = chunked_fwd_hs_offset(d.batch, d.seqlen, d.nheads, d.headdim, d.d_state,
                                                 d.mimo_rank, trap);
        const size_t hsb = (fp32_layer_hs_bytes(d) + 255) & ~(size_t)255;
        cn = reinterpret_cast<float*>(reinterpret_cast<char*>(workspace) + off + hsb);
        const int qb = chunked_chunk_tokens(d.mimo_rank, trap);
        if (qb % f32k::Q != 0) return M3_ERR_UNSUPPORTED;
        hs_every = qb / f32k::Q;
        hs_K = (d.seqlen + qb - 1) / qb;
    }
    hipLaunchKernelGGL(f32k::bc_norm_f32, dim3((unsigned)((nrows + 3) / 4)), dim3(256), 0, stream,
                       reinterpret_cast<const float*>(proj), d.proj_row_stride, pl.B, pl.C, d.ngroups,
                       nrows, d.rms_eps, p.B_norm_w, p.B_bias, p.C_norm_w, p.C_bias, bn, cn);
    f32k::Args a;
    a.B = d.batch; a.T = d.seqlen; a.H = d.nheads; a.G = d.ngroups;
    a.trap = d.use_trapezoidal; a.cplx = d.use_complex;
    a.rs = d.proj_row_stride;
    a.pl = pl;
    a.prm = p;
    a.proj = reinterpret_cast<const float*>(proj);
    a.dt_scale = dt_scale;
    a.Bn = bn;
    a.Cn = cn;
    a.y_out = reinterpret_cast<float*>(y_out);
    a.h_final = h_final;
    a.angle = angle;
    a.prev_bx = prev_bx;
    a.st = stage ? *stage : Fp32LayerParts{};
    a.stage = stage != nullptr;
    a.hs_every = hs_every;
    a.hs_K = hs_K;
    // two 32-column blocks per (batch, head) while the pairs alone leave CUs idle
    const int64_t bh = (int64_t)d.batch * d.nheads;
    if (bh < 256)
        hipLaunchKernelGGL(f32k::ssd_f32<32>, dim3((unsigned)(bh * 2)), dim3(f32k::THREADS), 0, stream, a);
    else
        hipLaunchKernelGGL(f32k::ssd_f32<64>, dim3((unsigned)bh), dim3(f32k::THREADS), 0, stream, a);
    return hipGetLastError() == hipSuccess ? M3_OK : M3_ERR_LAUNCH;
}

}  // namespace m3
