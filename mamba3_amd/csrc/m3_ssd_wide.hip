// bf16 fused chunked-SSD prefill on f16 MFMA for general layer shapes: d_state N in
// {64, 128, 256}, mimo_rank R in {1, 2, 4}, headdim P a multiple of 32 (the d_model 2048
// layer: N=256, P=128, R=4). d_state 128 / headdim 64 / rank 2 has its own kernel
// (m3_ssd_mfma.hip).
//
// Same algorithm as the other prefill kernels: the quadratic form inside a chunk and the
// state carried across chunks (mamba3/ssd.py:118-244), with the layer's preparation fused
// (mamba3/mamba3.py:197-256). It is organised for shapes whose (batch, head) pairs alone
// do not fill the GPU:
//   * a workgroup owns (batch, head, 32 headdim columns), so B*H*P/32 workgroups share
//     the work (256 for the d_model 2048 layer at batch 2); the scores and the RoPE
//     rotation are recomputed by each column block;
//   * a chunk has 64 (t, r) rows, i.e. Q = 64 / R tokens;
//   * sixteen waves (four per SIMD) share both phases of a chunk: contract (waves 0-7 the
//     inter-chunk output of their tile, waves 8-15 the score tiles, all the state update;
//     two score waves compute the next chunk's token scalars and RoPE angles instead of a
//     tile, and output waves 0-1 take their tiles), then output (waves 0-7 the intra-chunk
//     output, gate and store; all the next chunk's B~ / C~ tiles, the score waves its X
//     rows).
//
// Per chunk, in LDS (f16 unless noted):
//   C [(t,r)][n], B [(u,r')][n]       C~ / B~: normalised B^ / C^ (bc_norm_wide) rotated
//                                     by the RoPE angle; row (t,r) = t*R + r
//   XT [p][(u,r')], XwT [p][(u,r')]   x * mimo_x, and the same times the chunk weight w_u
//   S [(t,r)][(u,r')]                 masked scores (fp32 accumulated)
//   H [p][n]                          copy of the incoming state times kHScale
//   tok, phi (fp32)                   token scalars and RoPE angles of the chunk
// The fp32 state H^T lives in MFMA accumulators (wave w owns N/64 tiles of 16 x 16).
// Contractions (v_mfma_f32_16x16x32_f16, fp32 accumulation):
//   G4  H^T = e^{c_end} H^T + B~^T Xw    (A operand by LDS transpose reads of B~)
//   G3  Y   = diag(e^{c_t}) C~ H^T
//   G1  S^T = B~ C~^T per causal 16x16 tile, masked by
//             Lc[t][u] = [u<=t] e^{c_t - c_u} (a_u + [u<t] b_u), plus D on the diagonal
//   G2  Y  += S X
// Output: out[t][p] = sum_r mimo_down[p,r] silu(z[t,p] mimo_z[p,r]) Y[(t,r)][p]
// (mamba3/mamba3.py:233-238). The trapezoid is folded into a_u = lambda_u dt_u and
// b_u = (1 - lambda_{u+1}) dt_{u+1}, as in the other kernels.
#include "m3_common.h"
#include "m3_kernels.h"
#include "m3_mfma.h"

namespace m3 {
namespace wd {

constexpr int ROWS = 64;              // (t, r) rows per chunk
constexpr int PB = 32;                // headdim columns per workgroup
constexpr int THREADS = 1024;         // 16 waves: 0-7 own output tiles, 8-15 score tiles
constexpr int PAD = 8;                // f16 row padding of the S and H tiles
// f16 row padding of the X^T / Xw^T tiles: a row stride of 40 32-bit words (their G2 / G4
// operand reads, 16 rows x 64 bytes per wave, run 1.4-1.8% faster over the whole call than
// at 36; 44, 48 and 52 were no better). The 256 x 1 instantiation has no LDS to spare.
template <int N, int R>
constexpr int padx() { return (N == 256 && R == 1) ? 8 : 16; }
// f16 row padding of the C~ / B~ tiles: a row stride of 8 (mod 16) 32-bit words keeps the
// operand and transpose reads of those tiles free of most bank conflicts (a stride of
// 4 (mod 16) words, padding 8, measured 5% slower at d_state 256).
constexpr int PADCB = 16;
constexpr float kHScale = 1.f / 256.f;  // the f16 state copy holds h * kHScale

struct Tok {
    float c2[ROWS];  // inclusive prefix of A dt over the chunk, log2 units
    float av[ROWS];  // a_u = lambda_u dt_u
    float bv[ROWS];  // b_u = (1 - lambda_{u+1}) dt_{u+1}
    float ec[ROWS];  // exp2(c2_t) / kHScale: inter-chunk output scale
    float w[ROWS];   // exp2(c2_end - c2_u) (a_u + b_u): chunk-state weight
    float dec;       // exp2(c2_end): chunk decay of the state
};

// The R ranks of one token's X row, stored together.
template <int R>
struct __align__(2 * R) XRow {
    f16 v[R];
};

template <int N, int R>
struct __align__(16) Smem {
    static constexpr int Q = ROWS / R;
    f16 C[ROWS][N + PADCB];
    f16 B[ROWS][N + PADCB];
    f16 XT[2][PB][ROWS + padx<N, R>()];  // by chunk parity: G2 of chunk k reads while chunk k+1's is written
    f16 XwT[PB][ROWS + padx<N, R>()];
    f16 S[ROWS][ROWS + PAD];
    f16 H[PB][N + PAD];
    Tok tok[2];           // by chunk parity
    alignas(16) float phi[Q][N / 2];  // RoPE angle of each (token, pair) of the chunk being prepared
    u32x4 th[Q][N / 16];  // theta of that chunk, bf16, 8 pairs per entry
    float mz[PB][R], md[PB][R], mx[PB][R];  // mimo_z, mimo_down * sB sC sX, mimo_x / sX of the block's columns
    F16Scales scl;                          // operand scales of the (group, head)
};

struct Args {
    int B, T, H, G, P, PS;
    int trap, cplx;
    int64_t rs;  // proj row stride (elements)
    ProjLayout pl;
    m3_layer_params prm;
    const bf16* proj;
    const float* dt_scale;
    const f16* Bn;  // [B*T][G][N*R] pair-packed normalised B^
    const f16* Cn;
    bf16* y_out;    // [B*T][H*P]
    float* h_final;
    float* angle;
    float* prev_bx;
};

// Keeps the LDS reads issued above ahead of the LDS writes that follow.
#define M3_LDS_ORDER() asm volatile("" ::: "memory")

__device__ __forceinline__ float readlane(float v, int l) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), l));
}

// ---------------------------------------------------------------------------------
// Normalised B^ / C^ per (token, group) (mamba3/mamba3.py:19-35, 142-157): RMSNorm over
// the N*R row times the weight, plus the bias, in f16, pair-packed: the 32-bit word
// i*R + r holds (value[n=2i][r], value[n=2i+1][r]).
// ---------------------------------------------------------------------------------
constexpr int kWideBcRows = 4;  // (token, group) rows per wave of bc_norm_wide

// The 2R raw bf16 of one RoPE pair of a B / C row as R words (two elements per word, in
// order), by one vector load when the row layout allows it.
template <int R>
__device__ __forceinline__ void load_raw_pair(const bf16* p, bool vec, unsigned (&w)[R]) {
    if (vec) {
        if constexpr (R == 4) {
            const u32x4 v = *reinterpret_cast<const u32x4*>(p);
            w[0] = v[0]; w[1] = v[1]; w[2] = v[2]; w[3] = v[3];
        } else if constexpr (R == 2) {
            const u32x2 v = *reinterpret_cast<const u32x2*>(p);
            w[0] = v[0]; w[1] = v[1];
        } else {
            w[0] = *reinterpret_cast<const unsigned*>(p);
        }
    } else {
        const unsigned short* q = reinterpret_cast<const unsigned short*>(p);
#pragma unroll
        for (int e = 0; e < R; ++e) w[e] = (unsigned)q[2 * e] | ((unsigned)q[2 * e + 1] << 16);
    }
}

// Raw element e of a pair's words, as float.
template <int R>
__device__ __forceinline__ float raw_elem(const unsigned (&w)[R], int e) {
    return __builtin_bit_cast(float, (e & 1) ? (w[e >> 1] & 0xffff0000u) : (w[e >> 1] << 16));
}

// One wave normalises kWideBcRows consecutive (token, group) rows: all their reads are
// issued first, the norm weights are read once, the biases and the operand scales once per
// distinct group of the rows (a scalar branch: a row is one wave's).
template <int N, int R>
__global__ __launch_bounds__(256) void bc_norm_wide(const bf16* __restrict__ proj, int64_t rs,
                                                    int64_t offB, int64_t offC, int G,
                                                    int64_t nrows, float eps, int vec,
                                                    const float* __restrict__ wB,
                                                    const float* __restrict__ biasB,
                                                    const float* __restrict__ wC,
                                                    const float* __restrict__ biasC,
                                                    f16* __restrict__ Bn, f16* __restrict__ Cn) {
    constexpr int NH = N / 2, NR = N * R, PPL = (NH + 63) / 64, KR = kWideBcRows;
    const int lane = threadIdx.x & 63;
    const int64_t l0 = ((int64_t)blockIdx.x * 4 + (threadIdx.x >> 6)) * KR;
    if (l0 >= nrows) return;
    // Lane pairs i = lane + 64 j (j < PPL); pair i covers raw elements 2iR .. 2iR+2R-1:
    // (n=2i, r) at 2iR + r, (n=2i+1, r) at 2iR + R + r. Rows past the end read the last row
    // and store nothing.
    unsigned rwb[KR][PPL][R], rwc[KR][PPL][R];
    int gg[KR];
#pragma unroll
    for (int k = 0; k < KR; ++k) {
        const int64_t tg = l0 + k < nrows ? l0 + k : nrows - 1;
        const int64_t tok = tg / G;
        gg[k] = (int)(tg % G);
        const bf16* rowB = proj + tok * rs + offB + (int64_t)gg[k] * NR;
        const bf16* rowC = proj + tok * rs + offC + (int64_t)gg[k] * NR;
#pragma unroll
        for (int j = 0; j < PPL; ++j) {
            const int i = lane + 64 * j;
            if (i < NH) {
                load_raw_pair<R>(rowB + 2 * i * R, vec, rwb[k][j]);
                load_raw_pair<R>(rowC + 2 * i * R, vec, rwc[k][j]);
            } else {
#pragma unroll
                for (int e = 0; e < R; ++e) rwb[k][j][e] = rwc[k][j][e] = 0u;
            }
        }
    }
    float wvb[PPL][2 * R], wvc[PPL][2 * R];
    float mwb = 0.f, mwc = 0.f;
#pragma unroll
    for (int j = 0; j < PPL; ++j) {
        const int i = lane + 64 * j;
#pragma unroll
        for (int e = 0; e < 2 * R; ++e) {
            wvb[j][e] = i < NH ? wB[2 * i * R + e] : 0.f;
            wvc[j][e] = i < NH ? wC[2 * i * R + e] : 0.f;
            mwb = fmaxf(mwb, fabsf(wvb[j][e]));
            mwc = fmaxf(mwc, fabsf(wvc[j][e]));
        }
    }
    mwb = wave_max(mwb);
    mwc = wave_max(mwc);
    float bvb[PPL][2 * R], bvc[PPL][2 * R];
    float ib = 1.f, ic = 1.f;
    int gcur = -1;
#pragma unroll
    for (int k = 0; k < KR; ++k) {
        const int gk = __builtin_amdgcn_readfirstlane(gg[k]);
        if (gk != gcur) {
            // biases and operand scales of the row's group (1 unless the parameters are large)
            gcur = gk;
            float mbb = 0.f, mbc = 0.f;
#pragma unroll
            for (int j = 0; j < PPL; ++j) {
                const int i = lane + 64 * j;
#pragma unroll
                for (int e = 0; e < 2 * R; ++e) {
                    bvb[j][e] = i < NH ? biasB[(int64_t)gk * NR + 2 * i * R + e] : 0.f;
                    bvc[j][e] = i < NH ? biasC[(int64_t)gk * NR + 2 * i * R + e] : 0.f;
                    mbb = fmaxf(mbb, fabsf(bvb[j][e]));
                    mbc = fmaxf(mbc, fabsf(bvc[j][e]));
                }
            }
            ib = 1.f / bc_row_scale<N, R>(mwb, wave_max(mbb));
            ic = 1.f / bc_row_scale<N, R>(mwc, wave_max(mbc));
        }
        float sb = 0.f, sc = 0.f;
#pragma unroll
        for (int j = 0; j < PPL; ++j)
#pragma unroll
            for (int e = 0; e < 2 * R; ++e) {
                const float vb = raw_elem<R>(rwb[k][j], e), vc = raw_elem<R>(rwc[k][j], e);
                sb += vb * vb;
                sc += vc * vc;
            }
        sb = lane_sum<64>(sb);
        sc = lane_sum<64>(sc);
        const float nb = rsqrtf(sb * (1.f / NR) + eps), nc = rsqrtf(sc * (1.f / NR) + eps);
        if (l0 + k >= nrows) continue;
        const int64_t tg = l0 + k;
#pragma unroll
        for (int j = 0; j < PPL; ++j) {
            const int i = lane + 64 * j;
            if (i >= NH) continue;
            // pair-packed: word r = (value[n=2i][r], value[n=2i+1][r])
            unsigned ob[R], oc[R];
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const int e0 = r, e1 = R + r;
                ob[r] = bits(f16x2{(f16)((raw_elem<R>(rwb[k][j], e0) * nb * wvb[j][e0] + bvb[j][e0]) * ib),
                                   (f16)((raw_elem<R>(rwb[k][j], e1) * nb * wvb[j][e1] + bvb[j][e1]) * ib)});
                oc[r] = bits(f16x2{(f16)((raw_elem<R>(rwc[k][j], e0) * nc * wvc[j][e0] + bvc[j][e0]) * ic),
                                   (f16)((raw_elem<R>(rwc[k][j], e1) * nc * wvc[j][e1] + bvc[j][e1]) * ic)});
            }
            f16* pb = Bn + tg * NR + 2 * i * R;
            f16* pc = Cn + tg * NR + 2 * i * R;
            if constexpr (R == 4) {
                *reinterpret_cast<u32x4*>(pb) = u32x4{ob[0], ob[1], ob[2], ob[3]};
                *reinterpret_cast<u32x4*>(pc) = u32x4{oc[0], oc[1], oc[2], oc[3]};
            } else if constexpr (R == 2) {
                *reinterpret_cast<u32x2*>(pb) = u32x2{ob[0], ob[1]};
                *reinterpret_cast<u32x2*>(pc) = u32x2{oc[0], oc[1]};
            } else {
                *reinterpret_cast<unsigned*>(pb) = ob[0];
                *reinterpret_cast<unsigned*>(pc) = oc[0];
            }
        }
    }
}

// R consecutive 32-bit words (one RoPE pair, all ranks).
template <int R>
__device__ __forceinline__ void load_pair_words(const f16* p, unsigned (&w)[R]) {
    if constexpr (R == 4) {
        const u32x4 v = *reinterpret_cast<const u32x4*>(p);
        w[0] = v[0]; w[1] = v[1]; w[2] = v[2]; w[3] = v[3];
    } else if constexpr (R == 2) {
        const u32x2 v = *reinterpret_cast<const u32x2*>(p);
        w[0] = v[0]; w[1] = v[1];
    } else {
        w[0] = *reinterpret_cast<const unsigned*>(p);
    }
}

// (e, o) rotated by the angle whose (cos, sin) is kA: (e cos - o sin, e sin + o cos).
__device__ __forceinline__ unsigned rotate_pair(unsigned word, f16x2 kA, f16x2 kS) {
    const f16x2 v = as_f16x2(word);
    const f16x2 u = f16x2{v[1], v[1]} * kS;
    return bits(f16x2{v[0], v[0]} * kA + f16x2{-u[0], u[1]});
}

// 8 consecutive bf16 (raw bits): one 128-bit load when the address is 16-byte aligned.
__device__ __forceinline__ u32x4 load8(const bf16* p, bool vec) {
    if (vec) return *reinterpret_cast<const u32x4*>(p);
    const unsigned short* q = reinterpret_cast<const unsigned short*>(p);
    u32x4 v;
#pragma unroll
    for (int j = 0; j < 4; ++j) v[j] = (unsigned)q[2 * j] | ((unsigned)q[2 * j + 1] << 16);
    return v;
}

template <int N, int R>
__global__ __launch_bounds__(THREADS) void ssd_wide(Args a) {
    constexpr int Q = ROWS / R;    // tokens per chunk
    constexpr int NH = N / 2;      // RoPE pairs
    constexpr int NR = N * R;
    constexpr int TPW = N >= 128 ? N / 128 : 1;  // state tiles per wave (N/8 tiles in all)
    constexpr int KN = N / 32;     // k-steps over n
    constexpr int TPL = 4 / R;     // tokens per lane in an output tile
    __shared__ Smem<N, R> sm;

    // wave index in an SGPR, so the role branches below are scalar branches
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int g16 = lane >> 4, l16 = lane & 15;
    // Workgroups go to the 8 XCDs round-robin; renumber them so that consecutive logical
    // workgroups -- the column blocks and heads of one batch row, which read the same
    // normalised B^ / C^ rows -- share an XCD and its L2.
    const int nblk = gridDim.x;
    const int blk = (nblk % 8 == 0) ? (blockIdx.x % 8) * (nblk / 8) + blockIdx.x / 8 : blockIdx.x;
    const int pblk = blk % a.PS;
    const int bh = blk / a.PS;
    const int b = bh / a.H, h = bh % a.H;
    const int grp = h / (a.H / a.G);
    const int p0 = pblk * PB;
    const int T = a.T;
    const int64_t rs = a.rs;
    const bf16* proj = a.proj + (int64_t)b * T * rs;
    const int64_t nrs = (int64_t)a.G * NR;  // B^ / C^ token stride
    const f16* Bn = a.Bn + (int64_t)b * T * nrs + (int64_t)grp * NR;
    const f16* Cn = a.Cn + (int64_t)b * T * nrs + (int64_t)grp * NR;
    const int nchunks = (T + Q - 1) / Q;
    const float Ah = -expf(a.prm.A_log[h]);
    const float dtb = a.prm.dt_bias[h];
    if (wave == 0) {
        const F16Scales sc = layer_f16_scales<N, R>(a.prm, grp, h, a.P, lane);
        if (lane == 0) sm.scl = sc;
    }
    __syncthreads();
    const F16Scales scl = sm.scl.in_sgprs();
    // the skip term D enters the masked scores, which carry 1 / (sB sC)
    const float Dh = a.prm.D[h] * scl.inv_bc;
    const int hp = h * a.P;  // first column of this head in x, z and y

    // Waves 0-7: output tile rows 16 tt .. 16 tt + 15, columns 16 pt .. 16 pt + 15 (G3, G2,
    // gate, store). Waves 8-15: score tiles (G1 and its mask). All waves: state tiles (G4)
    // while there are tiles left, and the next chunk's tiles.
    const bool out_wave = wave < 8;
    const bool g4_wave = wave * TPW < N / 8;
    const int tt = (wave & 7) >> 1, pt = wave & 1;
    const int pe = p0 + 16 * pt + l16;  // this lane's output column
    // X preparation jobs: column xp of tokens xt0 + m * (THREADS / PB) below Q, m < XJ.
    constexpr int XJ = (Q * PB + THREADS - 1) / THREADS;
    // (on the score waves first: the output waves also run G2, the gate and the store in
    // the phase that prepares X)
    const int xtid = Q * PB <= THREADS / 2 ? tid ^ (THREADS / 2) : tid;
    const int xp = xtid % PB, xt0 = xtid / PB;
    if (tid < PB * R) {
        const int c = tid / R, r = tid % R;
        const int64_t e = (int64_t)(hp + p0 + c) * R + r;
        sm.mz[c][r] = a.prm.mimo_z[e];
        sm.md[c][r] = a.prm.mimo_down[e] * scl.out;
        sm.mx[c][r] = a.prm.mimo_x[e] * scl.inv_x;
    }
    // theta staging jobs: units of 8 pairs of one token.
    constexpr int THU = Q * NH / 8;
    constexpr int THJ = (THU + THREADS - 1) / THREADS;
    const bool thvec = a.rs % 8 == 0 && a.pl.theta % 8 == 0 &&
                       reinterpret_cast<uintptr_t>(a.proj) % 16 == 0;

    // ---- per-chunk inputs, read into registers at least a phase before they are used ----
    // Rotation jobs: this thread's two adjacent RoPE pairs 2 ri, 2 ri + 1 at tokens
    // rt0 + m * TSTEP (m < J), so each C~ / B~ row segment goes out as one 64-bit store.
    constexpr int NP2 = NH / 2;
    constexpr int J = (Q * NP2 + THREADS - 1) / THREADS;  // jobs at tokens below Q
    constexpr int TSTEP = THREADS / NP2;
    const int ri = tid % NP2, rt0 = tid / NP2;
    unsigned pwb[J][2][R], pwc[J][2][R];
    auto load_bc = [&](int kk) {
#pragma unroll
        for (int m = 0; m < J; ++m) {
            const int st = kk * Q + rt0 + m * TSTEP;
            const int64_t off = (int64_t)min(st, T - 1) * nrs + 4 * ri * R;  // in range; zeroed when used
#pragma unroll
            for (int e = 0; e < 2; ++e) {
                load_pair_words<R>(Bn + off + 2 * e * R, pwb[m][e]);
                load_pair_words<R>(Cn + off + 2 * e * R, pwc[m][e]);
            }
        }
    };
    // x of the X job (8 columns, raw bf16) and theta of the staging jobs.
    unsigned pxv[XJ];
    u32x4 pth[THJ];
    auto load_xv = [&](int kk) {
#pragma unroll
        for (int m = 0; m < XJ; ++m) {
            const int st = min(kk * Q + xt0 + m * (THREADS / PB), T - 1);
            pxv[m] = __builtin_nontemporal_load(
                reinterpret_cast<const unsigned short*>(proj + (int64_t)st * rs + a.pl.x + hp + p0 + xp));
        }
    };
    auto load_theta = [&](int kk) {
        if (a.cplx) {
#pragma unroll
            for (int m = 0; m < THJ; ++m) {
                const int u = tid + m * THREADS;
                if (u < THU) {
                    const int st = min(kk * Q + u / (NH / 8), T - 1);
                    pth[m] = load8(proj + (int64_t)st * rs + a.pl.theta + 8 * (u % (NH / 8)), thvec);
                }
            }
        }
    };
    auto store_theta = [&]() {
        if (a.cplx) {
#pragma unroll
            for (int m = 0; m < THJ; ++m) {
                const int u = tid + m * THREADS;
                if (u < THU) sm.th[u / (NH / 8)][u % (NH / 8)] = pth[m];
            }
        }
    };
    // Token scalars and RoPE angles (waves 10 .. 10+NWA-1, score waves with one tile each):
    // lane t = token t of the chunk for the scalars, pair ai for the angles.
    constexpr int NWA = (NH + 63) / 64;
    constexpr int kAngleWave0 = 10;
    const bool angle_wave = wave >= kAngleWave0 && wave < kAngleWave0 + NWA;
    const int ai = 64 * (wave - kAngleWave0) + lane;
    float phi_run = 0.f;
    unsigned rdt0 = 0, rlam0 = 0, rdt1 = 0, rlam1 = 0;
    float sc0 = 1.f, sc1 = 1.f;
    auto load_tokens = [&](int kk) {
        if (lane > Q) return;
        const int s0 = kk * Q;
        const int st0 = min(s0 + lane, T - 1), st1 = min(s0 + lane + 1, T - 1);
        const bf16* row0 = proj + (int64_t)st0 * rs;
        const bf16* row1 = proj + (int64_t)st1 * rs;
        rdt0 = *reinterpret_cast<const unsigned short*>(row0 + a.pl.dt + h);
        rdt1 = *reinterpret_cast<const unsigned short*>(row1 + a.pl.dt + h);
        rlam0 = a.trap ? *reinterpret_cast<const unsigned short*>(row0 + a.pl.lam + h) : 0u;
        rlam1 = a.trap ? *reinterpret_cast<const unsigned short*>(row1 + a.pl.lam + h) : 0u;
        sc0 = a.dt_scale ? a.dt_scale[((int64_t)b * T + st0) * a.H + h] : 1.f;
        sc1 = a.dt_scale ? a.dt_scale[((int64_t)b * T + st1) * a.H + h] : 1.f;
    };
    auto bf = [](unsigned u) { return __builtin_bit_cast(float, u << 16); };
    // Token scalars of chunk kk into tok[kk & 1], its RoPE angles into phi.
    auto prep_tokens = [&](int kk) {
        const int s0 = kk * Q;
        const int t = lane;
        const bool v0 = t < Q && s0 + t < T, v1 = t < Q && s0 + t + 1 < T;
        // mamba3/mamba3.py:200-204, 212-216
        // computed for every lane (the clamped reads are finite), then selected
        const float sp_t = fast_softplus_hw(bf(rdt0) + dtb) * sc0;
        const float sp_n = fast_softplus_hw(bf(rdt1) + dtb) * sc1;
        const float sg_t = __builtin_amdgcn_rcpf(1.f + fast_exp(-bf(rlam0)));
        const float sg_n = __builtin_amdgcn_rcpf(1.f + fast_exp(-bf(rlam1)));
        const float dt_t = v0 ? sp_t : 0.f;
        const float dt_n = v1 ? sp_n : 0.f;
        const float lam_t = v0 && a.trap ? sg_t : 1.f;
        const float lam_n = v1 && a.trap ? sg_n : 1.f;
        const float c2 = wave_incl_scan(Ah * dt_t * kLog2e);
        const float c2_end = readlane(c2, Q - 1);
        if (wave == kAngleWave0 + NWA - 1) {
            const float av = a.trap ? lam_t * dt_t : dt_t;
            const float bv = a.trap ? (1.f - lam_n) * dt_n : 0.f;
            Tok& tk = sm.tok[kk & 1];
            if (t < Q) {
                tk.c2[t] = c2;
                tk.av[t] = av;
                tk.bv[t] = bv;
                tk.ec[t] = __builtin_amdgcn_exp2f(c2) * (1.f / kHScale);
                tk.w[t] = __builtin_amdgcn_exp2f(c2_end - c2) * (av + bv);
            }
            if (t == 0) tk.dec = __builtin_amdgcn_exp2f(c2_end);
        }
        if (a.cplx && ai < NH) {
            // phi_t[i] = phi_{t-1}[i] - dt_t theta_t[i] (mamba3/mamba3.py:160-162)
            // 16 theta reads ahead of each group's angle stores (which the reads may not be
            // ordered after)
            const unsigned short* thq = reinterpret_cast<const unsigned short*>(&sm.th[0][0]) + ai;
            float ph = phi_run;
#pragma unroll
            for (int q0 = 0; q0 < Q; q0 += 16) {
                unsigned thv[16];
#pragma unroll
                for (int j = 0; j < 16; ++j) thv[j] = thq[(q0 + j) * NH];
                M3_LDS_ORDER();
#pragma unroll
                for (int j = 0; j < 16; ++j) {
                    ph -= readlane(dt_t, q0 + j) * bf(thv[j]);
                    sm.phi[q0 + j][ai] = ph;
                }
            }
            phi_run = ph;
        }
    };
    // Tiles of chunk kk: rotated C~ / B~ rows, X rows into XT[kk & 1] and XwT.
    auto prep_chunk = [&](int kk) {
        const int s0 = kk * Q;
        const Tok& tk = sm.tok[kk & 1];
#pragma unroll
        for (int m = 0; m < J; ++m) {
            const int t = rt0 + m * TSTEP;
            if (Q * NP2 % THREADS != 0 && t >= Q) break;  // threads past the chunk's jobs (small d_state)
            // Tokens past the end get a zero factor, which zeroes their rows (the clamped
            // words they rotate are finite).
            const bool valid = s0 + t < T;
            f16x2 kA[2], kS[2];
            const f32x2 ph = a.cplx ? *reinterpret_cast<const f32x2*>(&sm.phi[t][2 * ri]) : f32x2{0.f, 0.f};
#pragma unroll
            for (int e = 0; e < 2; ++e) {
                f16x2 k = f16x2{(f16)1.f, (f16)0.f};
                if (a.cplx) {
                    float sn, cs;
                    fast_sincos(ph[e], sn, cs);
                    k = f16x2{(f16)cs, (f16)sn};
                }
                kA[e] = as_f16x2(valid ? bits(k) : 0u);
                kS[e] = __builtin_shufflevector(kA[e], kA[e], 1, 0);
            }
#pragma unroll
            for (int r = 0; r < R; ++r) {
                *reinterpret_cast<u32x2*>(&sm.B[t * R + r][4 * ri]) =
                    u32x2{rotate_pair(pwb[m][0][r], kA[0], kS[0]), rotate_pair(pwb[m][1][r], kA[1], kS[1])};
                *reinterpret_cast<u32x2*>(&sm.C[t * R + r][4 * ri]) =
                    u32x2{rotate_pair(pwc[m][0][r], kA[0], kS[0]), rotate_pair(pwc[m][1][r], kA[1], kS[1])};
            }
        }
        // X rows (t, r) = x_t * mimo_x[p, r] (mamba3/mamba3.py:210), and times w_t.
#pragma unroll
        for (int m = 0; m < XJ; ++m) {
            const int t = xt0 + m * (THREADS / PB);
            if (t >= Q) break;
            const float xval = s0 + t < T ? bf(pxv[m]) : 0.f;
            const float w = tk.w[t];
            XRow<R> xv, xw;
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const float mxr = sm.mx[xp][r];
                xv.v[r] = (f16)(xval * mxr);
                xw.v[r] = (f16)(xval * mxr * w);
            }
            *reinterpret_cast<XRow<R>*>(&sm.XT[kk & 1][xp][t * R]) = xv;
            *reinterpret_cast<XRow<R>*>(&sm.XwT[xp][t * R]) = xw;
        }
    };

    // State tiles of this wave: j -> (n tile, p tile) = ((wave*TPW + j) / 2, (wave*TPW + j) % 2).
    f32x4 hacc[TPW];
#pragma unroll
    for (int j = 0; j < TPW; ++j) hacc[j] = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int idx = tid; idx < PB * (N + PAD) / 2; idx += THREADS)
        reinterpret_cast<unsigned*>(&sm.H[0][0])[idx] = 0u;
    // Prologue: chunk 0's token scalars and tiles; chunk 1's reads and theta.
    load_bc(0);
    load_xv(0);
    load_theta(0);
    if (angle_wave) load_tokens(0);
    store_theta();
    __syncthreads();
    if (angle_wave) {
        prep_tokens(0);
        if (nchunks > 1) load_tokens(1);
    }
    if (nchunks > 1) load_theta(1);
    __syncthreads();
    prep_chunk(0);
    if (nchunks > 1) {
        load_bc(1);
        load_xv(1);
        store_theta();
    }
    __syncthreads();

    // Per chunk k, two phases:
    //   contract: G4, G3, G1 of chunk k; token scalars and RoPE angles of chunk k+1
    //   output:   G2, gate, store of chunk k, its state copy; tiles of chunk k+1
    for (int k = 0; k < nchunks; ++k) {
        const int s0 = k * Q;
        const Tok& tk = sm.tok[k & 1];

        // ---- contract ----
        unsigned zr_bits[TPL];
        if (out_wave) {
#pragma unroll
            for (int q = 0; q < TPL; ++q) {
                const int st = min(s0 + (16 * tt + 4 * g16) / R + q, T - 1);
                zr_bits[q] = __builtin_nontemporal_load(
                    reinterpret_cast<const unsigned short*>(proj + (int64_t)st * rs + a.pl.z + hp + pe));
            }
        }
        if (k + 2 < nchunks) load_theta(k + 2);
        if (angle_wave && k + 1 < nchunks) {
            prep_tokens(k + 1);
            if (k + 2 < nchunks) load_tokens(k + 2);
        }
        if (g4_wave) {
            const float dec = tk.dec;
#pragma unroll
            for (int j = 0; j < TPW; ++j) hacc[j] *= dec;
#pragma unroll
            for (int s = 0; s < 2; ++s) {
#pragma unroll
                for (int j = 0; j < TPW; ++j) {
                    const int jt = wave * TPW + j;
                    const int nt = jt >> 1, ptj = jt & 1;
                    const f16* bp = &sm.B[32 * s + 8 * g16 + (l16 >> 2)][16 * nt + 4 * (l16 & 3)];
                    const f16x4 lo = ld_tr(bp);
                    const f16x4 hi = ld_tr(bp + 4 * (N + PADCB));
                    const f16x8 A = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
                    const f16x8 Bo = *reinterpret_cast<const f16x8*>(&sm.XwT[16 * ptj + l16][32 * s + 8 * g16]);
                    hacc[j] = mfma16(A, Bo, hacc[j]);
                }
            }
        }
        f32x4 yacc = f32x4{0.f, 0.f, 0.f, 0.f};
        if (out_wave) {
#pragma unroll
            for (int s = 0; s < KN; ++s) {
                const f16x8 A = *reinterpret_cast<const f16x8*>(&sm.C[16 * tt + l16][32 * s + 8 * g16]);
                const f16x8 Bo = *reinterpret_cast<const f16x8*>(&sm.H[16 * pt + l16][32 * s + 8 * g16]);
                yacc = mfma16(A, Bo, yacc);
            }
#pragma unroll
            for (int v = 0; v < 4; ++v) yacc[v] *= tk.ec[(16 * tt + 4 * g16 + v) / R];
        }

        // Causal score tiles (ti, ui), ui <= ti, listed row by row as 0..9: waves 8..15 take
        // tile wave-8, waves 8 and 9 also tiles 8 and 9, except the angle waves, whose tiles
        // go to output waves 0.. (which then run a tile and G3, as much as the waves with
        // two tiles). A lane's four u-rows 16 ui + 4 g16 + v cover NU tokens; their mask
        // factors are read (unconditionally: every index is below Q) and formed before the
        // contraction.
        const int tile0 = wave >= 8 ? (angle_wave ? -1 : wave - 8) : (wave < NWA ? kAngleWave0 - 8 + wave : -1);
        const int tile1 = wave == 8 || wave == 9 ? wave : -1;
        for (int c = 0; c < 2; ++c) {
            const int idx = c == 0 ? tile0 : tile1;
            if (idx < 0) break;
            const int ti = idx < 1 ? 0 : idx < 3 ? 1 : idx < 6 ? 2 : 3;
            const int ui = idx - ti * (ti + 1) / 2;
            constexpr int NU = R >= 4 ? 1 : 4 / R;
            const unsigned trow = 16 * ti + l16, t = trow / R;
            const unsigned ub = (unsigned)(16 * ui + 4 * g16) / R;
            // operands one k-step ahead of the MFMA that takes them
            const f16* pa = &sm.B[16 * ui + l16][8 * g16];
            const f16* pb = &sm.C[16 * ti + l16][8 * g16];
            f16x8 A = *reinterpret_cast<const f16x8*>(pa);
            f16x8 Bo = *reinterpret_cast<const f16x8*>(pb);
            const float ct = tk.c2[t];
            float fu[NU];
#pragma unroll
            for (int j = 0; j < NU; ++j) {
                const unsigned u = ub + j;
                const float e = __builtin_amdgcn_exp2f(ct - tk.c2[u]);
                const float ab = fmaf(tk.bv[u], u < t ? 1.f : 0.f, tk.av[u]);
                fu[j] = u <= t ? e * ab : 0.f;
            }
            f32x4 sacc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int s = 0; s < KN; ++s) {
                f16x8 An = A, Bn = Bo;
                if (s + 1 < KN) {
                    An = *reinterpret_cast<const f16x8*>(pa + 32 * (s + 1));
                    Bn = *reinterpret_cast<const f16x8*>(pb + 32 * (s + 1));
                }
                sacc = mfma16(A, Bo, sacc);
                A = An;
                Bo = Bn;
            }
            // lane: u-row 16 ui + 4 g16 + v, t-row 16 ti + l16
            f16x4 sv;
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const float val = sacc[v] * fu[v * NU / 4];
                sv[v] = (f16)(16 * ui + 4 * g16 + v == (int)trow ? val + Dh : val);
            }
            *reinterpret_cast<f16x4*>(&sm.S[trow][16 * ui + 4 * g16]) = sv;
        }
        if (wave == 15) {
            // G2 reads 32 score columns per step: the tiles right of the diagonal in row
            // blocks 0 and 2 are zero.
#pragma unroll
            for (int ti = 0; ti < 4; ti += 2)
                *reinterpret_cast<f16x4*>(&sm.S[16 * ti + l16][16 * (ti + 1) + 4 * g16]) = f16x4{0, 0, 0, 0};
        }
        __syncthreads();

        // ---- output ----
        if (out_wave) {
            // y rows of this chunk; stores past the last token fall outside and are dropped
            const __amdgpu_buffer_rsrc_t ry =
                make_rsrc(a.y_out + ((int64_t)b * T + s0) * a.H * a.P, (int64_t)(T - s0) * a.H * a.P * 2);
            for (int s = 0; s <= tt / 2; ++s) {
                const f16x8 A = *reinterpret_cast<const f16x8*>(&sm.S[16 * tt + l16][32 * s + 8 * g16]);
                const f16x8 Bo = *reinterpret_cast<const f16x8*>(&sm.XT[k & 1][16 * pt + l16][32 * s + 8 * g16]);
                yacc = mfma16(A, Bo, yacc);
            }
#pragma unroll
            for (int q = 0; q < TPL; ++q) {
            const int st = s0 + (16 * tt + 4 * g16) / R + q;
            const float z = bf(zr_bits[q]);
            float o = 0.f;
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const float zr = z * sm.mz[16 * pt + l16][r];
                o += sm.md[16 * pt + l16][r] * zr * __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(-zr * kLog2e)) * yacc[q * R + r];
            }
            __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(unsigned short, (bf16)o), ry,
                                                  ((st - s0) * a.H * a.P + hp + pe) * 2, 0, kStream);
            }
        }
        if (g4_wave) {
#pragma unroll
            for (int j = 0; j < TPW; ++j) {
                const int jt = wave * TPW + j;
                const int nt = jt >> 1, ptj = jt & 1;
                const f16x4 hv = f16x4{(f16)(hacc[j][0] * kHScale), (f16)(hacc[j][1] * kHScale),
                                       (f16)(hacc[j][2] * kHScale), (f16)(hacc[j][3] * kHScale)};
                *reinterpret_cast<f16x4*>(&sm.H[16 * ptj + l16][16 * nt + 4 * g16]) = hv;
            }
        }
        if (k + 1 < nchunks) {
            prep_chunk(k + 1);
            if (k + 2 < nchunks) {
                load_bc(k + 2);
                load_xv(k + 2);
                store_theta();
            }
        }
        __syncthreads();
    }

    // Final state h[p][n] (fp32) from the accumulators: lane holds n = 16 nt + 4 g16 + v.
    if (a.h_final && g4_wave) {
#pragma unroll
        for (int j = 0; j < TPW; ++j) {
            const int jt = wave * TPW + j;
            const int nt = jt >> 1, ptj = jt & 1;
            const int p = p0 + 16 * ptj + l16;
            *reinterpret_cast<f32x4*>(a.h_final + ((int64_t)bh * a.P + p) * N + 16 * nt + 4 * g16) = hacc[j] * scl.state;
        }
    }
    if (a.angle && pblk == 0 && angle_wave && ai < NH)
        a.angle[(int64_t)bh * NH + ai] = a.cplx ? phi_run : 0.f;
    // prev_BX = sum_r B~_{T-1}[n][r] X_{T-1}[p][r] (mamba3/mamba3.py:247-250) from the last
    // chunk's tiles.
    if (a.prev_bx) {
        const int tl = T - 1 - (nchunks - 1) * Q;
        for (int idx = tid; idx < PB * N; idx += THREADS) {
            const int p = idx / N, n = idx % N;
            float v = 0.f;
#pragma unroll
            for (int r = 0; r < R; ++r) v += (float)sm.B[tl * R + r][n] * (float)sm.XT[(nchunks - 1) & 1][p][tl * R + r];
            a.prev_bx[((int64_t)bh * a.P + p0 + p) * N + n] = v * scl.state;
        }
    }
}

template <int N, int R>
int launch(const m3_layer_desc& d, const m3_layer_params& p, const void* proj,
           const float* dt_scale, void* y_out, float* h_final, float* angle, float* prev_bx,
           void* workspace, hipStream_t stream) {
    Args a;
    a.B = d.batch; a.T = d.seqlen; a.H = d.nheads; a.G = d.ngroups; a.P = d.headdim;
    a.PS = d.headdim / PB;
    a.trap = d.use_trapezoidal; a.cplx = d.use_complex;
    a.rs = d.proj_row_stride;
    a.pl = proj_layout(d);
    a.prm = p;
    a.proj = reinterpret_cast<const bf16*>(proj);
    a.dt_scale = dt_scale;
    const int64_t nrows = (int64_t)d.batch * d.seqlen * d.ngroups;
    f16* bn = reinterpret_cast<f16*>(workspace);
    f16* cn = bn + nrows * N * R;
    a.Bn = bn;
    a.Cn = cn;
    a.y_out = reinterpret_cast<bf16*>(y_out);
    a.h_final = h_final;
    a.angle = angle;
    a.prev_bx = prev_bx;
    // vector loads of a pair's 2R raw values when every row offset keeps them aligned
    const int vec = a.rs % (2 * R) == 0 && a.pl.B % (2 * R) == 0 && a.pl.C % (2 * R) == 0 &&
                    reinterpret_cast<uintptr_t>(proj) % (4 * R) == 0;
    constexpr int rows_per_block = 4 * kWideBcRows;
    hipLaunchKernelGGL((bc_norm_wide<N, R>), dim3((unsigned)((nrows + rows_per_block - 1) / rows_per_block)),
                       dim3(256), 0, stream, a.proj, a.rs, a.pl.B, a.pl.C, a.G, nrows, d.rms_eps, vec,
                       p.B_norm_w, p.B_bias, p.C_norm_w, p.C_bias, bn, cn);
    hipLaunchKernelGGL((ssd_wide<N, R>), dim3((unsigned)(d.batch * d.nheads * a.PS)), dim3(THREADS), 0,
                       stream, a);
    return hipGetLastError() == hipSuccess ? M3_OK : M3_ERR_LAUNCH;
}

}  // namespace wd

bool wide_prefill_supported(const m3_layer_desc& d) {
    if (d.dtype != M3_DTYPE_BF16) return false;
    if (d.headdim % wd::PB != 0) return false;
    const int N = d.d_state, R = d.mimo_rank;
    if (N != 64 && N != 128 && N != 256) return false;
    if (R != 1 && R != 2 && R != 4) return false;
    return true;
}

size_t wide_prefill_workspace(const m3_layer_desc& d) {
    const size_t nrows = (size_t)d.batch * d.seqlen * d.ngroups;
    return 2 * nrows * d.d_state * d.mimo_rank * sizeof(f16) + 256;
}

int launch_wide_prefill(const m3_layer_desc& d, const m3_layer_params& p, const void* proj,
                        const float* dt_scale, void* y_out, float* h_final, float* angle,
                        float* prev_bx, void* workspace, hipStream_t stream) {
#define M3_WIDE_CASE(n, r)                                                                      \
    if (d.d_state == n && d.mimo_rank == r)                                                     \
        return wd::launch<n, r>(d, p, proj, dt_scale, y_out, h_final, angle, prev_bx, workspace, \
                                stream);
    M3_WIDE_CASE(64, 1) M3_WIDE_CASE(64, 2) M3_WIDE_CASE(64, 4)
    M3_WIDE_CASE(128, 1) M3_WIDE_CASE(128, 2) M3_WIDE_CASE(128, 4)
    M3_WIDE_CASE(256, 1) M3_WIDE_CASE(256, 2) M3_WIDE_CASE(256, 4)
#undef M3_WIDE_CASE
    return M3_ERR_UNSUPPORTED;
}

}  // namespace m3
