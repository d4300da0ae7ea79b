// Fused chunked-SSD prefill on MFMA for bf16 layers with d_state=128, headdim=64,
// mimo_rank=2 (the shape of the d_model 768 KulaMamba), gfx950.
//
// Work decomposition
// ------------------
// The sequence of every (batch, head) is cut into S segments of whole 64-token chunks
// (mfma_plan: one segment, equal segments, or a short first and a long second segment
// when the pairs leave CUs free). One 1024-thread workgroup (16 waves) owns one (batch,
// head, segment) and walks its chunks in order, carrying the (P=64, N=128) fp32 state in
// MFMA accumulators, so no per-chunk state ever goes to HBM. Three launches:
//   1. bc_norm:    per token and group, B^ = RMSNorm(B) * w + bias and C^ likewise in
//                  f16 (shared by every head, so computed once), pair-packed so that a
//                  RoPE pair (n=2i, n=2i+1) of one rank is one 32-bit word.
//   2. ssd_chunks<false> for segments 0..S-2: only the state update, giving each
//                  segment's end state from a zero start plus its total log-decay and
//                  total RoPE angle increment. When its workgroups leave CUs idle, launch
//                  1 covers only the tokens this pass reads and spare workgroups of this
//                  launch normalise the other tokens' B^ / C^ (read only by launch 3).
//   3. ssd_chunks<true> for all segments: combines the preceding segments' end states
//                  into the incoming state, then computes every chunk's output.
//
// Per chunk (Q=64 tokens, rows (t,r) = 2t+r, 128 rows) the kernel forms in LDS
//   C~ [(t,r)][n], B~ [(u,r')][n]      f16, B^/C^ rotated by the RoPE angle
//   X^T[p][(u,r')] = x * mimo_x         f16 (columns permuted for the G2 operand reads)
//   Xw [p][(u,r')] = X^T * w_u          f16 (state-update operand, w_u the chunk weight)
//   H[p][n]                             f16 copy of the incoming state, scaled by 1/256
// and runs four MFMA contractions (v_mfma_f32_16x16x32_f16, fp32 accumulation):
//   G3  Y  = diag(e^{c_t}) C~ H^T          inter-chunk output
//   G1  S^T = B~ C~^T, masked by Lc[t][u] = [u<=t] exp(c_t-c_u) (a_u + [u<t] b_u)
//       (+D on the diagonal), kept in registers
//   G2  Y += S X                           intra-chunk output, S fed straight from the
//                                          G1 accumulators as the A operand (the k
//                                          order is permuted consistently in X^T)
//   G4  H^T = e^{c_63} H^T + B~^T Xw       state update (A operand by LDS transpose
//                                          reads of the B~ tile)
// Roles: SIMD s runs waves s and s+4. Every wave holds 16 state rows and runs its share
// of G4; wave s then computes output block s and wave s+4 output block 7-s (so each
// SIMD carries the same causal work), wave s prepares the RoPE rotation of pairs
// 16s..16s+15 for the next chunk and wave s+4 a quarter of X^T / Xw.
// The trapezoid is folded into a_u = lambda_u dt_u, b_u = (1-lambda_{u+1}) dt_{u+1}
// (the beta term of token u+1 multiplies B~_u x_u), so the rank is not doubled.
//
// Memory: every global read goes through a buffer descriptor whose size ends at the
// batch row's last token, so reads past the sequence return zero (padding for free).
// The next chunk's reads are issued right after the state update.
//
// RoPE frame: inside a segment every angle is taken relative to the segment start.
// Dot products C~.B~ and C~.H are invariant under a common rotation, so outputs are
// unchanged, while sin/cos only see angles accumulated over one segment. Incoming
// segment states are rotated into the local frame when combined, and the final state,
// angle and prev_BX are rotated back to the absolute frame.
#include <algorithm>
#include <type_traits>

#include "m3_common.h"
#include "m3_kernels.h"
#include "m3_mfma.h"

namespace m3 {
namespace mf {

constexpr int Q = 64;
constexpr int N = 128;
constexpr int P = 64;
constexpr int R = 2;
constexpr int NR = N * R;
constexpr int NH = N / 2;
constexpr int THREADS = 1024;  // 8 MFMA waves + 8 helper waves, four per SIMD
constexpr int NMW = 8;          // waves 0..7 run the MFMA work, 8..15 are helpers
// f16 row padding of the C~, B~ and H tiles: a row stride of 72 32-bit words. Their MFMA
// operand reads (ds_read_b128, 16 rows x 64 bytes per wave) run at 1.5x the LDS throughput
// of a 68-word stride (16 waves per CU, all CUs busy), and the transposed B~ reads and the
// tile stores stay conflict-free.
constexpr int PAD = 16;


constexpr int NSLOT = 3;
// The f16 copy of the state used by G3 holds h * kHScale (|h| up to ~1.6e7 fits); the
// G3 row scale multiplies by 1/kHScale.
constexpr float kHScale = 1.f / 256.f;  // token-scalar ring: chunks k, k+1 read while k+2 is written

// Per-chunk token scalars (index = token within the chunk), written by MFMA wave 0.
struct Tok {
    float c2[Q];   // inclusive prefix of A*dt over the chunk, log2 units
    float av[Q];   // a_u = lambda_u dt_u
    float bv[Q];   // b_u = (1 - lambda_{u+1}) dt_{u+1}
    float ec[Q];   // exp2(c2_u)
    float hb[Q];   // exp2(c2[8*(u/8)+7] - c2_u) (a_u + b_u): decay to the end of u's 8-block
    float dtr[Q];  // dt_u / (2 pi): RoPE angle increment per unit theta, in turns
    f16 w16[Q];    // exp2(c2[63] - c2_u) (a_u + b_u): chunk-state weight
};

struct __align__(16) Smem {
    f16 C[Q * R][N + PAD];    // C~ rows (t,r) = 2t+r; 16-byte column chunks swizzled (sw_cb)
    f16 B[Q * R][N + PAD];    // B~ rows (u,r'), same swizzle
    f16 X[2][Q * R][P];       // X rows (u,r') = x_u * mimo_x[r'], columns p swizzled (xsw);
                              // double-buffered by chunk parity
    f16 H[P][N + PAD];        // incoming state times kHScale
    bf16 Zt[2][Q][P];         // z of the chunk per (t, p), columns swizzled (zsw); each entry
                              // is replaced in place by the gated output. Double-buffered by
                              // chunk parity.
    Tok tok[NSLOT];
    float rot[NH];            // per-pair angle scratch (prologue / epilogue)
    F16Scales scl;            // operand scales of the (group, head)
    f32x4 mzd[P];             // per p: -mimo_z[0] log2e, -mimo_z[1] log2e, mimo_down*mimo_z [0], [1]
    f16 mxT[R][P];            // mimo_x per rank and p
};

// The (token, group) rows of tokens [lo, hi) of every batch row, numbered consecutively:
// logical row l is batch row l / per_b, physical row (b T + lo) G + l % per_b.
struct BcRows {
    const bf16* proj;
    int64_t rs, offB, offC;
    int G;
    float eps;
    const float *wB, *biasB, *wC, *biasC;
    f16 *Bn, *Cn;
    int64_t nrows;  // logical rows: batch * (hi - lo) * G
    int64_t per_b;  // (hi - lo) * G
    int64_t skip;   // (T - (hi - lo)) * G: physical rows between batch rows' ranges
    int64_t lo_g;   // lo * G
    __device__ __forceinline__ int64_t phys(int64_t l) const {
        if (skip == 0) return l + lo_g;  // the whole sequence
        const int64_t b = l / per_b;
        return l + b * skip + lo_g;
    }
};

struct Args {
    int B, T, H, G, S, cps;
    int first;  // chunks of segment 0 (segments 1.. have cps chunks, the last may be shorter)
    int order;  // 1: two segments, dispatched long-first per XCD (ssd_chunks<true>)
    int trap, cplx;
    int64_t rs;
    ProjLayout pl;
    m3_layer_params prm;
    const bf16* proj;
    const float* dt_scale;
    const f16* Bn;    // [B*T][G][NR] pair-packed normalised B
    const f16* Cn;
    float* seg_state;  // [B*H*(S-1)][N][P]
    float* seg_decay;  // [B*H*(S-1)]
    float* seg_angle;  // [B*H*(S-1)][NH]
    bf16* y_out;
    float* h_final;
    float* angle;
    float* prev_bx;
    // ssd_chunks<false>: workgroups past the nstate state-pass ones normalise bcr's rows
    // (the tokens the state pass does not read) on the CUs the state pass leaves idle.
    int nstate;
    BcRows bcr;
};





// C~ / B~ tiles: 64-byte column groups of a row are XOR-swizzled by the row's 16-row
// block, so the preparation's 64-bit stores (lanes 16 rows apart) hit distinct banks.
// MFMA operand reads cover 16 rows of one block, so their pattern is only permuted.
__device__ __forceinline__ int sw_cb(int row, int col) { return col ^ (32 * ((row >> 4) & 3)); }
// X tile [(u,r)][p] (128-byte rows): 16-column groups XOR-swizzled by (row/2)%4, so the
// transpose reads of the MFMA operands (4 rows x 16 columns per 16 lanes, 8 rows per
// 32-lane pass) and the 128-bit row writes are free of bank conflicts.
__device__ __forceinline__ int xsw(int row, int col) { return col ^ (16 * ((row >> 1) & 3)); }
// z tile [t][p] of bf16: 16-column groups XOR-swizzled by (t/2)%4, so the MFMA waves'
// 16-bit accesses (16 consecutive columns per 16-lane group, the four groups on rows 2
// apart) use distinct banks; the helpers' 128-bit row accesses stay contiguous.
__device__ __forceinline__ int zsw(int t, int p) { return p ^ (16 * ((t >> 1) & 3)); }



// ---------------------------------------------------------------------------------
// 1. Normalised B^ / C^ per (token, group): x * rsqrt(mean(x^2) + eps) * w + bias,
//    stored pair-packed: word 2i+r of the row = (value[n=2i][r], value[n=2i+1][r]).
// ---------------------------------------------------------------------------------
constexpr int kBcTok = 4;  // (token, group) rows per wave of bc_norm

// A wave normalises KR consecutive logical rows starting at l0: all their reads go out
// together, the weights are read once (rows past the end read the last row and store
// nothing). Lane = pair i; raw order at 4i: (n=2i,r0) (2i,r1) (2i+1,r0) (2i+1,r1).
template <int KR>
__device__ __forceinline__ void bc_norm_rows(const BcRows& c, int64_t l0, int lane) {
    const int e = 4 * lane;
    bf16x4 vb[KR], vc[KR];
    int gg[KR];
    int64_t tgp[KR];
#pragma unroll
    for (int k = 0; k < KR; ++k) {
        const int64_t tg = c.phys(l0 + k < c.nrows ? l0 + k : c.nrows - 1);
        tgp[k] = tg;
        const int64_t tok = tg / c.G;
        gg[k] = (int)(tg % c.G);
        const bf16* row = c.proj + tok * c.rs;
        vb[k] = *reinterpret_cast<const bf16x4*>(row + c.offB + (int64_t)gg[k] * NR + e);
        vc[k] = *reinterpret_cast<const bf16x4*>(row + c.offC + (int64_t)gg[k] * NR + e);
    }
    const f32x4 wb4 = *reinterpret_cast<const f32x4*>(c.wB + e);
    const f32x4 wc4 = *reinterpret_cast<const f32x4*>(c.wC + e);
    auto absmax4 = [](f32x4 v) { return fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3]))); };
    // Operand scales of a group (1 unless the parameters are large): those of the first
    // row's group, recomputed for a row of another group (a scalar branch: a row is one
    // wave's).
    const float mwb = wave_max(absmax4(wb4)), mwc = wave_max(absmax4(wc4));
    auto scales_of = [&](int g, float& ib, float& ic) {
        const f32x4 bb4 = *reinterpret_cast<const f32x4*>(c.biasB + (int64_t)g * NR + e);
        const f32x4 bc4 = *reinterpret_cast<const f32x4*>(c.biasC + (int64_t)g * NR + e);
        ib = 1.f / bc_row_scale<N, R>(mwb, wave_max(absmax4(bb4)));
        ic = 1.f / bc_row_scale<N, R>(mwc, wave_max(absmax4(bc4)));
    };
    const int g0 = __builtin_amdgcn_readfirstlane(gg[0]);
    float ib0, ic0;
    scales_of(g0, ib0, ic0);
#pragma unroll
    for (int k = 0; k < KR; ++k) {
        const f32x4 bb4 = *reinterpret_cast<const f32x4*>(c.biasB + (int64_t)gg[k] * NR + e);
        const f32x4 bc4 = *reinterpret_cast<const f32x4*>(c.biasC + (int64_t)gg[k] * NR + e);
        float ib = ib0, ic = ic0;
        const int gk = __builtin_amdgcn_readfirstlane(gg[k]);
        if (gk != g0) scales_of(gk, ib, ic);
        float b[4], cc[4], sb = 0.f, sc = 0.f;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            b[j] = (float)vb[k][j];
            cc[j] = (float)vc[k][j];
            sb += b[j] * b[j];
            sc += cc[j] * cc[j];
        }
        sb = lane_sum<64>(sb);
        sc = lane_sum<64>(sc);
        const float rb = rsqrtf(sb * (1.f / NR) + c.eps), rc = rsqrtf(sc * (1.f / NR) + c.eps);
        float ob[4], oc[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            ob[j] = (b[j] * rb * wb4[j] + bb4[j]) * ib;
            oc[j] = (cc[j] * rc * wc4[j] + bc4[j]) * ic;
        }
        // pair-packed: (e_r0, o_r0, e_r1, o_r1)
        if (l0 + k < c.nrows) {
            *reinterpret_cast<f16x4*>(c.Bn + tgp[k] * NR + e) = f16x4{(f16)ob[0], (f16)ob[2], (f16)ob[1], (f16)ob[3]};
            *reinterpret_cast<f16x4*>(c.Cn + tgp[k] * NR + e) = f16x4{(f16)oc[0], (f16)oc[2], (f16)oc[1], (f16)oc[3]};
        }
    }
}

__global__ __launch_bounds__(256) void bc_norm(BcRows c) {
    const int64_t l0 = ((int64_t)blockIdx.x * 4 + (threadIdx.x >> 6)) * kBcTok;
    if (l0 >= c.nrows) return;
    bc_norm_rows<kBcTok>(c, l0, threadIdx.x & 63);
}

// ---------------------------------------------------------------------------------
// 2/3. Segment kernels.
// ---------------------------------------------------------------------------------

// Output rows of one 16-row block I of the chunk (tokens 8I .. 8I+7, rows (t,r) = 2t+r),
// computed by one MFMA wave:
//   G3  Y  = diag(e^{c_t}) C~ H^T                       (inter-chunk)
//   G1  S^T = B~ C~^T for the causal column blocks J <= I, two blocks at a time; each pair
//       is scaled by Lc[t][u] = [u<=t] exp(c_t-c_u) (a_u + [u<t] b_u) (+D on the
//       diagonal) and fed straight into
//   G2  Y += S X as the A operand. The pair's accumulator rows give this lane the k values
//       (u,r') = 32 s2 + 4 g + v and 32 s2 + 16 + 4 g + v (g = lane/16, v < 4); the X
//       operand is read with transpose reads in the same row order.
// Then out[t][p] = sum_r mimo_down_r silu(z mimo_z_r) y_r from z in the z tile; the bf16
// result replaces z there.
template <int I>
__device__ __forceinline__ void out_block(Smem& sm, const Tok& tk, int par, int g16, int l16, float D_h) {
    constexpr int NP = I / 2 + 1;  // column-block pairs
    // Token scalars this lane needs (rows t_col, columns u = 8J + 2 g16 + {0,1}).
    const int t_col = 8 * I + (l16 >> 1);
    const int r_col = l16 & 1;
    const int u0d = 8 * I + 2 * g16;
    const float ct = tk.c2[t_col];
    // e^{c_t}, times 1/kHScale for the scaled f16 state copy
    const f32x2 ecv = *reinterpret_cast<const f32x2*>(&tk.ec[u0d]) * (1.f / kHScale);

    // C~ rows of this block (logical column 32s + 8 g16 sits at 32 (s ^ (I&3)) + 8 g16)
    // and the first H operand group.
    f16x8 cA[4], hop[2][4];
#pragma unroll
    for (int s = 0; s < 4; ++s)
        cA[s] = *reinterpret_cast<const f16x8*>(&sm.C[16 * I + l16][8 * g16 + 32 * (s ^ (I & 3))]);
#pragma unroll
    for (int s = 0; s < 4; ++s)
        hop[0][s] = *reinterpret_cast<const f16x8*>(&sm.H[l16][32 * s + 8 * g16]);
    M3_FENCE();
    // G3: Y = C~ H^T (scaled by e^{c_t} below)
    f32x4 yacc[4];
#pragma unroll
    for (int pt = 0; pt < 4; ++pt) {
        if (pt + 1 < 4) {
#pragma unroll
            for (int s = 0; s < 4; ++s)
                hop[(pt + 1) & 1][s] = *reinterpret_cast<const f16x8*>(&sm.H[16 * (pt + 1) + l16][32 * s + 8 * g16]);
        }
        M3_FENCE();
        yacc[pt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < 4; ++s) yacc[pt] = mfma16(cA[s], hop[pt & 1][s], yacc[pt]);
        M3_FENCE();
    }
#pragma unroll
    for (int pt = 0; pt < 4; ++pt) {
        yacc[pt][0] *= ecv[0];
        yacc[pt][1] *= ecv[0];
        yacc[pt][2] *= ecv[1];
        yacc[pt][3] *= ecv[1];
    }

    // Fused G1 / mask / G2 over pairs of causal column blocks.
    // X transpose reads: rows 32 s2 + 16 h + 4 g16 + jr share (row/2)%4 = (2 g16 + jr/2)%4,
    // so one pointer per column group pt serves every (s2, h) with a constant offset.
    const int jr = l16 >> 2, jc = 4 * (l16 & 3);
    const int xm = (2 * g16 + (jr >> 1)) & 3;
    const f16* xp[4];
#pragma unroll
    for (int pt = 0; pt < 4; ++pt) xp[pt] = &sm.X[par][4 * g16 + jr][16 * (pt ^ xm) + jc];
#pragma unroll
    for (int s2 = 0; s2 < NP; ++s2) {
        f16x8 bop[4];
        f16x4 xlo[4], xhi[4];
#pragma unroll
        for (int s = 0; s < 4; ++s)
            bop[s] = *reinterpret_cast<const f16x8*>(&sm.B[32 * s2 + l16][8 * g16 + 32 * (s ^ ((2 * s2) & 3))]);
#pragma unroll
        for (int pt = 0; pt < 4; ++pt) {
            xlo[pt] = ld_tr(xp[pt] + (32 * s2) * P);
            xhi[pt] = ld_tr(xp[pt] + (32 * s2 + 16) * P);
        }
        M3_FENCE();
        f32x4 sacc[2];
        sacc[0] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < 4; ++s) sacc[0] = mfma16(bop[s], cA[s], sacc[0]);
        M3_FENCE();
        sacc[1] = f32x4{0.f, 0.f, 0.f, 0.f};
        if (2 * s2 + 1 <= I) {
#pragma unroll
            for (int s = 0; s < 4; ++s)
                bop[s] = *reinterpret_cast<const f16x8*>(
                    &sm.B[32 * s2 + 16 + l16][8 * g16 + 32 * (s ^ ((2 * s2 + 1) & 3))]);
            M3_FENCE();
#pragma unroll
            for (int s = 0; s < 4; ++s) sacc[1] = mfma16(bop[s], cA[s], sacc[1]);
            M3_FENCE();
        }
        // This lane's S^T values of block J: rows (u, r') = (8J + 2 g16 + v/2, v&1),
        // column (t_col, r_col).
        f16x8 aop;
#pragma unroll
        for (int jj = 0; jj < 2; ++jj) {
            const int J = 2 * s2 + jj;
            float m0 = 0.f, m1 = 0.f, m2 = 0.f, m3 = 0.f;
            if (J < I) {
                // u < t: exp(c_t - c_u)(a_u + b_u), split at the end of u's 8-block so
                // both factors are at most one.
                const float gt = __builtin_amdgcn_exp2f(ct - tk.c2[8 * J + 7]);
                const f32x2 hj = *reinterpret_cast<const f32x2*>(&tk.hb[8 * J + 2 * g16]);
                const float l0 = gt * hj[0], l1 = gt * hj[1];
                m0 = sacc[jj][0] * l0;
                m1 = sacc[jj][1] * l0;
                m2 = sacc[jj][2] * l1;
                m3 = sacc[jj][3] * l1;
            } else if (J == I) {
                const f32x2 cud = *reinterpret_cast<const f32x2*>(&tk.c2[u0d]);
                const f32x2 aud = *reinterpret_cast<const f32x2*>(&tk.av[u0d]);
                const f32x2 bud = *reinterpret_cast<const f32x2*>(&tk.bv[u0d]);
                const float e0 = __builtin_amdgcn_exp2f(ct - cud[0]);
                const float e1 = __builtin_amdgcn_exp2f(ct - cud[1]);
                const float l0 = u0d <= t_col ? e0 * (aud[0] + (u0d < t_col ? bud[0] : 0.f)) : 0.f;
                const float l1 = u0d + 1 <= t_col ? e1 * (aud[1] + (u0d + 1 < t_col ? bud[1] : 0.f)) : 0.f;
                m0 = sacc[jj][0] * l0;
                m1 = sacc[jj][1] * l0;
                m2 = sacc[jj][2] * l1;
                m3 = sacc[jj][3] * l1;
                if (u0d == t_col) { if (r_col == 0) m0 += D_h; else m1 += D_h; }
                if (u0d + 1 == t_col) { if (r_col == 0) m2 += D_h; else m3 += D_h; }
            }
            aop[4 * jj + 0] = (f16)m0;
            aop[4 * jj + 1] = (f16)m1;
            aop[4 * jj + 2] = (f16)m2;
            aop[4 * jj + 3] = (f16)m3;
        }
#pragma unroll
        for (int pt = 0; pt < 4; ++pt) yacc[pt] = mfma16(aop, cat8(xlo[pt], xhi[pt]), yacc[pt]);
        M3_FENCE();
    }

    // Gate and MIMO down-projection, out = sum_r mimo_down_r silu(z mimo_z_r) y_r
    // = z sum_r (mimo_down_r mimo_z_r y_r) sigmoid(z mimo_z_r).
#pragma unroll
    for (int pt = 0; pt < 4; ++pt) {
        const int p = 16 * pt + l16;
        const f32x4 m = sm.mzd[p];
#pragma unroll
        for (int tt = 0; tt < 2; ++tt) {
            const int t = 8 * I + 2 * g16 + tt;
            bf16* zp = &sm.Zt[par][t][zsw(t, p)];
            const float z = (float)*zp;
            // sigmoid(z mimo_z_r) = 1 / (1 + e_r), 0 where e_r overflows to inf
            const float s0 = __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(z * m[0]));
            const float s1 = __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(z * m[1]));
            const float w1 = yacc[pt][2 * tt + 1] * m[3];
            *zp = (bf16)(z * __builtin_fmaf(yacc[pt][2 * tt] * m[2], s0, w1 * s1));
        }
    }
}

// Pipelined chunk walk, per chunk k:
//   barrier A -> M(k): MFMA waves: state update G4 on chunk k's tiles, output block of
//                chunk k, gated from the z tile. Helper waves: chunk k-1's output to HBM,
//                then RoPE rotation, X rows and z of chunk k+1 (X rows and z straight into
//                the buffers of the other parity), reads of chunk k+2 issued as registers
//                free up.
//   barrier B -> W(k+1): MFMA waves write the f16 state copy H_{k+1}; helper waves write
//                the C~ / B~ tiles of chunk k+1.
// Roles (SIMD s runs waves s, s+4, s+8, s+12):
//   MFMA wave w < 8: state rows n = 16w .. 16w+15; output block w (w < 4) or 11-w, so
//                each SIMD carries blocks {s, 7-s} (the same causal work); wave 0 also
//                computes the token scalars two chunks ahead.
//   helper wave 8+h: RoPE pairs 16 (h%4) + 2 (lane%8) + {0, 1} for tokens 8 (lane/8) +
//                4 (h/4) + {0..3}; X rows and z of token 8h + lane/8, columns
//                8 (lane%8) .. +7. Helpers issue every global read and store, so the MFMA
//                waves never wait on memory.
template <bool kFull>
__global__ __launch_bounds__(THREADS, 1) void ssd_chunks(Args a) {
    __shared__ Smem sm;
    const int tid = threadIdx.x;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);

    const int nseg = kFull ? a.S : a.S - 1;
    if (!kFull && (int)blockIdx.x >= a.nstate) {
        // Spare workgroup of the state pass: B^ / C^ of the tokens past the state pass
        // (read only by the full pass), eight rows per wave and flight. No barrier, no LDS.
        const int nw = (gridDim.x - a.nstate) * (THREADS / 64);
        const int gw = (blockIdx.x - a.nstate) * (THREADS / 64) + wv;
        for (int64_t l0 = (int64_t)gw * 8; l0 < a.bcr.nrows; l0 += (int64_t)nw * 8)
            bc_norm_rows<8>(a.bcr, l0, tid & 63);
        return;
    }
    // Workgroup i runs on XCD i % 8. Consecutive (batch, head) pairs (one batch row shares
    // B^ / C^) are kept on one XCD. Split plan (a.order): each XCD first gets the long second
    // segments of its pairs, one per CU, then the short first segments, which cycle through
    // the remaining CUs while the long ones run.
    const int nblk = kFull ? (int)gridDim.x : a.nstate;
    int seg, bh;
    if (kFull && a.order) {
        const int L = nblk / 16;  // pairs per XCD
        const int i = blockIdx.x / 8;
        seg = i < L ? 1 : 0;
        bh = (blockIdx.x % 8) * L + (i < L ? i : i - L);
    } else {
        const int blk = (nblk % 8 == 0) ? (blockIdx.x % 8) * (nblk / 8) + blockIdx.x / 8 : blockIdx.x;
        seg = blk % nseg;
        bh = blk / nseg;
    }
    const int b = bh / a.H, h = bh % a.H;
    const int grp = h / (a.H / a.G);
    const int T = a.T;
    const int K = (T + Q - 1) / Q;
    const int k_begin = seg == 0 ? 0 : a.first + (seg - 1) * a.cps;
    const int k_end = min(K, seg == 0 ? a.first : k_begin + a.cps);
    const int rs = (int)a.rs;
    const int bnrs = a.G * NR;  // elements between tokens in Bn / Cn

    const float A2 = -__expf(a.prm.A_log[h]) * kLog2e;
    const float dtb = a.prm.dt_bias[h];

    const int lane0 = tid & 63;
    if (wv == 0) {
        // the state pass only forms X operands (its states stay in the scaled frame)
        const F16Scales sc = kFull ? layer_f16_scales<N, R>(a.prm, grp, h, P, lane0)
                                   : F16Scales{1.f / mimo_x_scale<R>(a.prm, h, P, lane0), 1.f, 1.f, 1.f};
        if (lane0 == 0) sm.scl = sc;
    }
    __syncthreads();
    const F16Scales scl = sm.scl.in_sgprs();
    // the skip term D enters the masked scores, which carry 1 / (sB sC)
    const float D_h = a.prm.D[h] * scl.inv_bc;
    if (kFull && tid < P) {
        const float z0 = a.prm.mimo_z[(h * P + tid) * R], z1 = a.prm.mimo_z[(h * P + tid) * R + 1];
        sm.mzd[tid] = f32x4{-z0 * kLog2e, -z1 * kLog2e, a.prm.mimo_down[(h * P + tid) * R] * z0 * scl.out,
                            a.prm.mimo_down[(h * P + tid) * R + 1] * z1 * scl.out};
    }
    if (tid < P) {
        sm.mxT[0][tid] = (f16)(a.prm.mimo_x[(h * P + tid) * R] * scl.inv_x);
        sm.mxT[1][tid] = (f16)(a.prm.mimo_x[(h * P + tid) * R + 1] * scl.inv_x);
    }

    // State accumulators of the MFMA waves: wave w owns the H^T rows n in [16w, 16w+16),
    // all 64 columns p.
    f32x4 hacc[4];
#pragma unroll
    for (int pt = 0; pt < 4; ++pt) hacc[pt] = f32x4{0.f, 0.f, 0.f, 0.f};

    // Helper lanes: hw = helper index, q = token octet, c8 = column slot.
    const int hw = wv - NMW;
    const int q8 = lane0 >> 3, c8 = lane0 & 7;
    // RoPE pairs of helper lanes (pa0, pa0+1); pair lanes (helpers 0-3, lanes 0-7) own the
    // per-pair outputs. phi_start: absolute angles (radians) of the pairs at the segment start.
    const int pa0 = 16 * (hw & 3) + 2 * c8;
    const bool pair_lane = wv >= NMW && hw < 4 && q8 == 0;
    float phi_start0 = 0.f, phi_start1 = 0.f;
    if (kFull && seg > 0) {
        // H = sum_i exp(sum_{l=i+1}^{seg-1} D_l) R(-sum_{l=i}^{seg-1} Phi_l) S_i over the
        // preceding segments i < seg. The suffix sums (per-pair angles, log-weights) are
        // taken in the order of a walk from seg-1 down, from reads issued eight at a time,
        // into the C~ tile (unused until the first tiles are written); the MFMA waves then
        // read the segment states two at a time. Index clamps and zero weights keep every
        // read unconditional.
        const int g16 = lane0 >> 4, l16 = lane0 & 15;
        const int64_t sbase = (int64_t)bh * (a.S - 1);
        float* rotA = reinterpret_cast<float*>(&sm.C[0][0]);  // [i][pair], i < seg <= 63
        float* lw = rotA + 64 * NH;                          // [i]
        if (tid < NH) {
            float acc = 0.f;
            for (int i0 = seg - 1; i0 >= 0; i0 -= 8) {
                float v[8];
#pragma unroll
                for (int u = 0; u < 8; ++u) v[u] = a.seg_angle[(sbase + max(i0 - u, 0)) * NH + tid];
#pragma unroll
                for (int u = 0; u < 8; ++u) {
                    acc += i0 - u >= 0 ? v[u] : 0.f;
                    if (i0 - u >= 0) rotA[(i0 - u) * NH + tid] = acc;
                }
            }
        } else if (tid == 64) {
            float acc = 0.f;
            for (int i0 = seg - 1; i0 >= 0; i0 -= 8) {
                float v[8];
#pragma unroll
                for (int u = 0; u < 8; ++u) v[u] = a.seg_decay[sbase + max(i0 - u, 0)];
#pragma unroll
                for (int u = 0; u < 8; ++u) {
                    if (i0 - u >= 0) lw[i0 - u] = acc;
                    acc += i0 - u >= 0 ? v[u] : 0.f;
                }
            }
        }
        __syncthreads();
        if (wv < NMW) {
            const int n0 = 16 * wv + 4 * g16;
            for (int i0 = seg - 1; i0 >= 0; i0 -= 2) {
                float sv[2][4][4];  // [segment][pt][n0 + e]
#pragma unroll
                for (int u = 0; u < 2; ++u) {
                    const float* Si = a.seg_state + (sbase + max(i0 - u, 0)) * (int64_t)N * P;
#pragma unroll
                    for (int pt = 0; pt < 4; ++pt)
#pragma unroll
                        for (int e = 0; e < 4; ++e) sv[u][pt][e] = Si[(n0 + e) * P + 16 * pt + l16];
                }
#pragma unroll
                for (int u = 0; u < 2; ++u) {
                    const int i = max(i0 - u, 0);
                    const float wgt = i0 - u >= 0 ? __expf(lw[i]) : 0.f;
                    float s0, c0, s1, c1;
                    sincosf(-rotA[i * NH + n0 / 2], &s0, &c0);
                    sincosf(-rotA[i * NH + n0 / 2 + 1], &s1, &c1);
#pragma unroll
                    for (int pt = 0; pt < 4; ++pt) {
                        const float e0 = sv[u][pt][0], o0 = sv[u][pt][1];
                        const float e1 = sv[u][pt][2], o1 = sv[u][pt][3];
                        hacc[pt][0] += wgt * (e0 * c0 - o0 * s0);
                        hacc[pt][1] += wgt * (e0 * s0 + o0 * c0);
                        hacc[pt][2] += wgt * (e1 * c1 - o1 * s1);
                        hacc[pt][3] += wgt * (e1 * s1 + o1 * c1);
                    }
                }
            }
        }
        if (pair_lane) {
            phi_start0 = rotA[pa0];  // sum_{l<seg} Phi_l
            phi_start1 = rotA[pa0 + 1];
        }
        __syncthreads();  // the C~ tile is written after this
    }

    const bf16* proj_b = a.proj + (int64_t)b * T * a.rs;
    const f16* bn_b = a.Bn + ((int64_t)b * T * a.G + grp) * NR;
    const f16* cn_b = a.Cn + ((int64_t)b * T * a.G + grp) * NR;

    float logdecay = 0.f;  // total log-decay of the segment (natural log)
    float phi_run0 = 0.f, phi_run1 = 0.f;  // pair angles relative to the segment start, turns

    if (wv < NMW) {
        // ======================= MFMA waves =======================
        // ---- G4: H^T = e^{c_63} H^T + (B~ diag(w))^T X on chunk k's tiles
        auto state_update = [&](const Tok& tk, int par) {
            const int lane = opaque(threadIdx.x & 63);
            const int g16 = lane >> 4, l16 = lane & 15;
            const float dch = tk.ec[Q - 1];
#pragma unroll
            for (int pt = 0; pt < 4; ++pt) hacc[pt] *= dch;
            // Operand k order (u,r) = 32 s + 16 half + 4 g16 + m. A operand (B~^T, rows
            // n = 16 wave + lane%16) and B operand (X, columns p) both come from transpose
            // reads: lane j of a 16-lane group addresses row k0 + j/4, columns c0 + 4 (j%4).
            const int jr = l16 >> 2, jc = 4 * (l16 & 3);
            const int n0 = 16 * wv;
            // Rows 32 s + 16 h + 4 g16 + jr: the B~ swizzle depends only on (2s + h)%4 and the
            // X swizzle only on the lane, so a few pointers serve every (s, h) with constant
            // offsets.
            const int xm = (2 * g16 + (jr >> 1)) & 3;
            const f16* xp[4];
            const f16* bp[4];
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                xp[c] = &sm.X[par][4 * g16 + jr][16 * (c ^ xm) + jc];
                bp[c] = &sm.B[4 * g16 + jr][(n0 + jc) ^ (32 * c)];
            }
#pragma unroll
            for (int s = 0; s < 4; ++s) {
                const f16x4 alo = ld_tr(bp[(2 * s) & 3] + (32 * s) * (N + PAD));
                const f16x4 ahi = ld_tr(bp[(2 * s + 1) & 3] + (32 * s + 16) * (N + PAD));
                f16x4 xlo[4], xhi[4];
#pragma unroll
                for (int pt = 0; pt < 4; ++pt) {
                    xlo[pt] = ld_tr(xp[pt] + (32 * s) * P);
                    xhi[pt] = ld_tr(xp[pt] + (32 * s + 16) * P);
                }
                // chunk-state weights of tokens 16s + 2 g16 + {0,1} and 16s + 8 + 2 g16 + {0,1}
                const f16x2 wlo = *reinterpret_cast<const f16x2*>(&tk.w16[16 * s + 2 * g16]);
                const f16x2 whi = *reinterpret_cast<const f16x2*>(&tk.w16[16 * s + 8 + 2 * g16]);
                M3_FENCE();
                const f16x8 aop = {alo[0] * wlo[0], alo[1] * wlo[0], alo[2] * wlo[1], alo[3] * wlo[1],
                                   ahi[0] * whi[0], ahi[1] * whi[0], ahi[2] * whi[1], ahi[3] * whi[1]};
#pragma unroll
                for (int pt = 0; pt < 4; ++pt) hacc[pt] = mfma16(aop, cat8(xlo[pt], xhi[pt]), hacc[pt]);
                M3_FENCE();
            }
            logdecay += tk.c2[Q - 1] * (1.f / kLog2e);
        };
        // ---- f16 copy of the state for G3 (W phase)
        auto write_state = [&]() {
            const int lane = opaque(threadIdx.x & 63);
            const int g16 = lane >> 4, l16 = lane & 15;
            const int n0 = 16 * wv + 4 * g16;
#pragma unroll
            for (int pt = 0; pt < 4; ++pt) {
                const f32x4 v = hacc[pt] * kHScale;
                *reinterpret_cast<f16x4*>(&sm.H[16 * pt + l16][n0]) =
                    f16x4{(f16)v[0], (f16)v[1], (f16)v[2], (f16)v[3]};
            }
        };
        // ---- token scalars (wave 0)
        unsigned sdt = 0u, sdt64 = 0u, slam = 0u, slam64 = 0u;
        float ssc = 1.f, ssc64 = 1.f;
        auto load_sc = [&](int kk) {
            const int lane = opaque(threadIdx.x & 63);
            const int s0 = kk * Q;
            const __amdgpu_buffer_rsrc_t rp = make_rsrc(proj_b + (int64_t)s0 * a.rs, (int64_t)max(T - s0, 0) * a.rs * 2);
            sdt = ld_u16(rp, (__mul24(lane, rs) + (int)a.pl.dt + h) * 2);
            sdt64 = ld_u16(rp, (Q * rs + (int)a.pl.dt + h) * 2);
            if (a.trap) {
                slam = ld_u16(rp, (__mul24(lane, rs) + (int)a.pl.lam + h) * 2);
                slam64 = ld_u16(rp, (Q * rs + (int)a.pl.lam + h) * 2);
            }
            if (a.dt_scale) {
                ssc = a.dt_scale[((int64_t)b * T + min(s0 + lane, T - 1)) * a.H + h];
                ssc64 = a.dt_scale[((int64_t)b * T + min(s0 + Q, T - 1)) * a.H + h];
            }
        };
        // token scalars of chunk kk into its ring slot (mamba3/mamba3.py:200-216)
        auto tok_scalars = [&](int kk) {
            const int lane = opaque(threadIdx.x & 63);
            const int s0 = kk * Q;
            Tok& tk = sm.tok[kk % NSLOT];
            const float dt = s0 + lane < T ? fast_softplus(bf16_f32(sdt) + dtb) * ssc : 0.f;
            const float lam = a.trap ? __builtin_amdgcn_rcpf(1.f + fast_exp(-bf16_f32(slam))) : 1.f;
            float dtn = bperm(dt, lane + 1);
            float lamn = bperm(lam, lane + 1);
            if (lane == 63) {
                dtn = s0 + Q < T ? fast_softplus(bf16_f32(sdt64) + dtb) * ssc64 : 0.f;
                lamn = a.trap ? __builtin_amdgcn_rcpf(1.f + fast_exp(-bf16_f32(slam64))) : 1.f;
            }
            const float c2 = wave_incl_scan(A2 * dt);
            const float c2e = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, c2), 63));
            const float c2b = bperm(c2, lane | 7);
            const float av = a.trap ? lam * dt : dt;
            const float bv = a.trap ? (1.f - lamn) * dtn : 0.f;
            tk.c2[lane] = c2;
            tk.av[lane] = av;
            tk.bv[lane] = bv;
            tk.ec[lane] = __builtin_amdgcn_exp2f(c2);
            tk.hb[lane] = __builtin_amdgcn_exp2f(c2b - c2) * (av + bv);
            tk.dtr[lane] = dt * 0.15915494309189535f;
            tk.w16[lane] = (f16)(__builtin_amdgcn_exp2f(c2e - c2) * (av + bv));
        };

        // prologue: token scalars of the first two chunks
        if (wv == 0) {
            load_sc(k_begin);
            tok_scalars(k_begin);
            if (k_begin + 1 < k_end) {
                load_sc(k_begin + 1);
                tok_scalars(k_begin + 1);
            }
            if (k_begin + 2 < k_end) load_sc(k_begin + 2);
        }
        __syncthreads();
        if (kFull) write_state();

        for (int k = k_begin; k < k_end; ++k) {
            const bool more = k + 1 < k_end;
            const int par = k & 1;
            __syncthreads();
            const Tok& tk = sm.tok[k % NSLOT];
            state_update(tk, par);
            if (kFull) {
                const int lane = opaque(threadIdx.x & 63);
                const int g16 = lane >> 4, l16 = lane & 15;
                switch (wv) {
                    case 0: out_block<0>(sm, tk, par, g16, l16, D_h); break;
                    case 1: out_block<1>(sm, tk, par, g16, l16, D_h); break;
                    case 2: out_block<2>(sm, tk, par, g16, l16, D_h); break;
                    case 3: out_block<3>(sm, tk, par, g16, l16, D_h); break;
                    case 4: out_block<7>(sm, tk, par, g16, l16, D_h); break;
                    case 5: out_block<6>(sm, tk, par, g16, l16, D_h); break;
                    case 6: out_block<5>(sm, tk, par, g16, l16, D_h); break;
                    default: out_block<4>(sm, tk, par, g16, l16, D_h); break;
                }
            }
            if (wv == 0) {
                if (k + 2 < k_end) tok_scalars(k + 2);
                if (k + 3 < k_end) load_sc(k + 3);
            }
            __syncthreads();
            if (kFull && more) write_state();  // H_{k+1}, read by G3 of chunk k+1
        }
        // ---- segment end (MFMA waves: state outputs)
        __syncthreads();
        const int g16 = lane0 >> 4, l16 = lane0 & 15;
        if (!kFull) {
            const int64_t sidx = (int64_t)bh * (a.S - 1) + seg;
            float* out = a.seg_state + sidx * (int64_t)N * P;
            const int n0 = 16 * wv + 4 * g16;
#pragma unroll
            for (int pt = 0; pt < 4; ++pt)
#pragma unroll
                for (int v = 0; v < 4; ++v) out[(n0 + v) * P + 16 * pt + l16] = hacc[pt][v];
            if (tid == 0) a.seg_decay[sidx] = logdecay;
        } else if (seg == a.S - 1) {
            __syncthreads();  // absolute start angles of every pair in sm.rot
            if (a.h_final) {
                float* hf = a.h_final + (int64_t)bh * P * N;
                const int n0 = 16 * wv + 4 * g16;
                float s0, c0, s1, c1;
                sincosf(sm.rot[n0 / 2], &s0, &c0);
                sincosf(sm.rot[n0 / 2 + 1], &s1, &c1);
#pragma unroll
                for (int pt = 0; pt < 4; ++pt) {
                    const f32x4 v = hacc[pt] * scl.state;
                    const f32x4 o = {v[0] * c0 - v[1] * s0, v[0] * s0 + v[1] * c0,
                                     v[2] * c1 - v[3] * s1, v[2] * s1 + v[3] * c1};
                    *reinterpret_cast<f32x4*>(&hf[(16 * pt + l16) * N + n0]) = o;
                }
            }
            if (a.prev_bx) {
                // prev_BX = B~_{T-1} x_{T-1}^T, from the last chunk's tiles (still in LDS),
                // rotated to the absolute frame. Thread: column pair lane, rows p = 8*wave..+7.
                const int ul = (T - 1) - (K - 1) * Q;
                const int pp = lane0;
                float sn, cs;
                sincosf(sm.rot[pp], &sn, &cs);
                const int c0 = sw_cb(2 * ul, 2 * pp);  // rows 2ul and 2ul+1 share the 16-row block
                const float be0 = (float)sm.B[2 * ul][c0], bo0 = (float)sm.B[2 * ul][c0 + 1];
                const float be1 = (float)sm.B[2 * ul + 1][c0], bo1 = (float)sm.B[2 * ul + 1][c0 + 1];
                const float ae0 = be0 * cs - bo0 * sn, ao0 = be0 * sn + bo0 * cs;
                const float ae1 = be1 * cs - bo1 * sn, ao1 = be1 * sn + bo1 * cs;
                float* pb = a.prev_bx + (int64_t)bh * P * N;
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const int p = 8 * wv + j;
                    const float x0 = (float)sm.X[(K - 1) & 1][2 * ul][xsw(2 * ul, p)];
                    const float x1 = (float)sm.X[(K - 1) & 1][2 * ul + 1][xsw(2 * ul + 1, p)];
                    *reinterpret_cast<f32x2*>(&pb[p * N + 2 * pp]) =
                        f32x2{ae0 * x0 + ae1 * x1, ao0 * x0 + ao1 * x1} * scl.state;
                }
            }
        }
    } else {
        // ======================= helper waves =======================
        const int th = hw >> 2;        // which four tokens of the octet this lane rotates
        u32x4 rawB[4], rawC[4], xr, zr;
        unsigned rawth[8];
        u32x2 outB[4][2], outC[4][2];

        // ---- reads of chunk kk (past the sequence end the descriptors return zero). Each
        // group is issued right after its registers' previous contents are consumed, so the
        // reads spread over the M phase and have a whole chunk step to arrive.
        auto rsrc_proj = [&](int kk) {
            const int s0 = kk * Q;
            return make_rsrc(proj_b + (int64_t)s0 * a.rs, (int64_t)max(T - s0, 0) * a.rs * 2);
        };
        auto load_x = [&](int kk) {
            const int lane = opaque(threadIdx.x & 63);
            const int t = 8 * hw + (lane >> 3), p = 8 * (lane & 7);
            xr = __builtin_amdgcn_raw_buffer_load_b128(rsrc_proj(kk), (__mul24(t, rs) + (int)a.pl.x + h * P + p) * 2, 0, kStream);
        };
        auto load_z = [&](int kk) {
            const int lane = opaque(threadIdx.x & 63);
            const int t = 8 * hw + (lane >> 3), p = 8 * (lane & 7);
            zr = __builtin_amdgcn_raw_buffer_load_b128(rsrc_proj(kk), (__mul24(t, rs) + (int)a.pl.z + h * P + p) * 2, 0, kStream);
        };
        auto load_th = [&](int kk) {
            const int lane = opaque(threadIdx.x & 63);
            const int q = lane >> 3;
            const int pa = 16 * (hw & 3) + 2 * (lane & 7);
            const int s0 = kk * Q;
            // theta through a descriptor of size zero when the layer has no RoPE (reads give
            // 0, so the angles stay zero): no branch, so the reads stay where they are written.
            const __amdgpu_buffer_rsrc_t rth =
                make_rsrc(proj_b + (int64_t)s0 * a.rs, a.cplx ? (int64_t)max(T - s0, 0) * a.rs * 2 : 0);
            const int vth = (__mul24(8 * q, rs) + (a.cplx ? (int)a.pl.theta : 0) + pa) * 2;
#pragma unroll
            for (int j = 0; j < 8; ++j) rawth[j] = __builtin_amdgcn_raw_buffer_load_b32(rth, vth, j * rs * 2, 0);
        };
        // the four tokens' B^ / C^ words of this lane: one offset, the token step in soffset
        auto load_bc4 = [&](int kk) {
            const int lane = opaque(threadIdx.x & 63);
            const int q = lane >> 3;
            const int pa = 16 * (hw & 3) + 2 * (lane & 7);
            const int s0 = kk * Q;
            const int left = max(T - s0, 0);
            const int64_t bcbytes = left > 0 ? ((int64_t)(left - 1) * bnrs + NR) * 2 : 0;
            const int vbc = (__mul24(8 * q + 4 * th, bnrs) + 4 * pa) * 2;
            const __amdgpu_buffer_rsrc_t rb = make_rsrc(bn_b + (int64_t)s0 * bnrs, bcbytes);
            const __amdgpu_buffer_rsrc_t rc = make_rsrc(cn_b + (int64_t)s0 * bnrs, bcbytes);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                rawB[j] = __builtin_amdgcn_raw_buffer_load_b128(rb, vbc, j * bnrs * 2, 0);
                if (kFull) rawC[j] = __builtin_amdgcn_raw_buffer_load_b128(rc, vbc, j * bnrs * 2, 0);
            }
        };
        auto load_all = [&](int kk) {
            load_x(kk);
            if (kFull) load_z(kk);
            load_th(kk);
            load_bc4(kk);
        };
        // ---- RoPE rotation of this lane's four tokens, two pairs, both ranks
        // kn: chunk whose theta reads are issued once the prefix has used this chunk's.
        auto prep = [&](int kk, int kn) {
            const int lane = opaque(threadIdx.x & 63);
            const int q = lane >> 3;
            const Tok& tk = sm.tok[kk % NSLOT];
            const f32x4 d0 = *reinterpret_cast<const f32x4*>(&tk.dtr[8 * q]);
            const f32x4 d1 = *reinterpret_cast<const f32x4*>(&tk.dtr[8 * q + 4]);
            // RoPE angle increments (turns) dt_u theta_u of tokens 8q..8q+7 for both pairs:
            // totals of the first and second four; the prefix of the per-lane totals over q
            // (lanes 8 apart) gives each lane's starting angles.
            float lo0 = 0.f, lo1 = 0.f, hi0 = 0.f, hi1 = 0.f;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                lo0 += d0[j] * __builtin_bit_cast(float, rawth[j] << 16);
                lo1 += d0[j] * __builtin_bit_cast(float, rawth[j] & 0xffff0000u);
                hi0 += d1[j] * __builtin_bit_cast(float, rawth[4 + j] << 16);
                hi1 += d1[j] * __builtin_bit_cast(float, rawth[4 + j] & 0xffff0000u);
            }
            const float tot0 = lo0 + hi0, tot1 = lo1 + hi1;
            // inclusive prefix over q (lanes 8 apart; the step-8 partner of an even q is in
            // the previous 16-lane row, so every step goes through bpermute)
            float incl0 = tot0, incl1 = tot1;
#pragma unroll
            for (int off = 8; off < 64; off <<= 1) {
                const float o0 = bperm(incl0, lane - off);
                const float o1 = bperm(incl1, lane - off);
                if (lane >= off) {
                    incl0 += o0;
                    incl1 += o1;
                }
            }
            const float ctot0 = bperm(incl0, 56 + (lane & 7));
            const float ctot1 = bperm(incl1, 56 + (lane & 7));
            float phi0 = phi_run0 - (incl0 - tot0);
            float phi1 = phi_run1 - (incl1 - tot1);
            phi_run0 -= ctot0;
            phi_run1 -= ctot1;
            // tokens 8q .. 8q+3 precede this lane's four when th = 1
            phi0 -= th ? lo0 : 0.f;
            phi1 -= th ? lo1 : 0.f;
            // this lane's four tokens: dt and theta words
            float dsel[4];
            unsigned tsel[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                dsel[j] = th ? d1[j] : d0[j];
                tsel[j] = th ? rawth[4 + j] : rawth[j];
            }
            M3_FENCE();
            load_th(kn);
            M3_FENCE();
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float dt = dsel[j];
                const unsigned thw = tsel[j];
                phi0 -= dt * __builtin_bit_cast(float, thw << 16);
                phi1 -= dt * __builtin_bit_cast(float, thw & 0xffff0000u);
                f16x2 rb[2][2];  // [pair][rank]: rotated (even, odd) of B^
#pragma unroll
                for (int pr = 0; pr < 2; ++pr) {
                    const float phi = pr == 0 ? phi0 : phi1;
                    const float rev = __builtin_amdgcn_fractf(phi);
                    const float sn = __builtin_amdgcn_sinf(rev), cs = __builtin_amdgcn_cosf(rev);
                    // (e, o) -> (e cos - o sin, e sin + o cos) = e (cos, sin) + (-u0, u1) with
                    // u = o (sin, cos): one packed multiply and one packed fma (the negation
                    // is a source modifier)
                    const f16x2 kA = f16x2{(f16)cs, (f16)sn};
                    const f16x2 kS = __builtin_shufflevector(kA, kA, 1, 0);
#pragma unroll
                    for (int r = 0; r < 2; ++r) {
                        const f16x2 v = as_f16x2(rawB[j][2 * pr + r]);
                        const f16x2 u = f16x2{v[1], v[1]} * kS;
                        rb[pr][r] = f16x2{v[0], v[0]} * kA + f16x2{-u[0], u[1]};
                        if (kFull) {
                            const f16x2 c = as_f16x2(rawC[j][2 * pr + r]);
                            const f16x2 uc = f16x2{c[1], c[1]} * kS;
                            outC[j][r][pr] = bits(f16x2{c[0], c[0]} * kA + f16x2{-uc[0], uc[1]});
                        }
                    }
                }
                outB[j][0] = u32x2{bits(rb[0][0]), bits(rb[1][0])};
                outB[j][1] = u32x2{bits(rb[0][1]), bits(rb[1][1])};
            }
        };
        // ---- X rows (u,r) = x_u mimo_x[r], columns 8 (lane%8) .. +7, of token 8 hw + lane/8,
        // straight into X buffer par (not read in this M phase)
        auto prep_x = [&](int par) {
            const int lane = opaque(threadIdx.x & 63);
            const int p = 8 * (lane & 7);
            const f16x8 mx0 = *reinterpret_cast<const f16x8*>(&sm.mxT[0][p]);
            const f16x8 mx1 = *reinterpret_cast<const f16x8*>(&sm.mxT[1][p]);
            f16x8 xv;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                xv[2 * i] = (f16)bf16_f32(xr[i] & 0xffffu);
                xv[2 * i + 1] = (f16)__builtin_bit_cast(float, xr[i] & 0xffff0000u);
            }
            const int t = 8 * hw + (lane >> 3);
            *reinterpret_cast<f16x8*>(&sm.X[par][2 * t][xsw(2 * t, p)]) = xv * mx0;
            *reinterpret_cast<f16x8*>(&sm.X[par][2 * t + 1][xsw(2 * t + 1, p)]) = xv * mx1;
        };
        // ---- z of token 8 hw + lane/8, columns 8 (lane%8) .. +7, into z tile par (the MFMA
        // waves apply the gate in their output epilogue)
        auto stage_z = [&](int par) {
            const int lane = opaque(threadIdx.x & 63);
            const int t = 8 * hw + (lane >> 3), p = 8 * (lane & 7);
            *reinterpret_cast<u32x4*>(&sm.Zt[par][t][zsw(t, p)]) = zr;
        };
        // ---- W phase: tiles of the prepared chunk
        auto write_tiles = [&]() {
            const int lane = opaque(threadIdx.x & 63);
            const int q = lane >> 3;
            const int pa = 16 * (hw & 3) + 2 * (lane & 7);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int row = 2 * (8 * q + 4 * th + j);
                const int col = sw_cb(row, 2 * pa);  // rows row, row+1 share the swizzle
                const int off = __mul24(row, (N + PAD) * 2) + col * 2;  // bytes
                char* cbase = reinterpret_cast<char*>(&sm.C[0][0]) + off;
                char* bbase = reinterpret_cast<char*>(&sm.B[0][0]) + off;
                // The fences keep these as single 64-bit stores.
                if (kFull) {
                    *reinterpret_cast<u32x2*>(cbase) = outC[j][0];
                    M3_LDS_FENCE();
                    *reinterpret_cast<u32x2*>(cbase + (N + PAD) * 2) = outC[j][1];
                    M3_LDS_FENCE();
                }
                *reinterpret_cast<u32x2*>(bbase) = outB[j][0];
                M3_LDS_FENCE();
                *reinterpret_cast<u32x2*>(bbase + (N + PAD) * 2) = outB[j][1];
                M3_LDS_FENCE();
            }
        };
        // ---- chunk kk's output (its z tile, overwritten by the MFMA waves) to HBM
        auto store_out = [&](int kk) {
            const int lane = opaque(threadIdx.x & 63);
            const int t = 8 * hw + (lane >> 3), p = 8 * (lane & 7);
            const u32x4 o = *reinterpret_cast<const u32x4*>(&sm.Zt[kk & 1][t][zsw(t, p)]);
            const int s0 = kk * Q;
            const int HP = a.H * P;
            const __amdgpu_buffer_rsrc_t ry =
                make_rsrc(a.y_out + ((int64_t)b * T + s0) * HP, (int64_t)max(T - s0, 0) * HP * 2);
            __builtin_amdgcn_raw_buffer_store_b128(o, ry, (__mul24(t, HP) + h * P + p) * 2, 0, kStream);
        };

        // prologue: first chunk's tiles and z, reads of the second chunk
        load_all(k_begin);
        __syncthreads();
        prep_x(k_begin & 1);
        M3_FENCE();  // each read group after the last use of its registers
        load_x(k_begin + 1);
        M3_FENCE();
        if (kFull) {
            stage_z(k_begin & 1);
            M3_FENCE();
            load_z(k_begin + 1);
            M3_FENCE();
        }
        prep(k_begin, k_begin + 1);
        write_tiles();

        for (int k = k_begin; k < k_end; ++k) {
            const bool more = k + 1 < k_end;
            __syncthreads();
            // chunk k-1's output (gated in its z tile by the MFMA waves in M(k-1)) to HBM,
            // first thing in M(k): stage_z below then overwrites the same lane's entries of
            // that z tile with chunk k+1's z
            if (kFull && k > k_begin) store_out(k - 1);
            if (more) {
                // B^ / C^ of chunk k+1 (shared by all heads of the batch row, mostly L2
                // hits) are read now and rotated last; x, z and theta are a chunk ahead.
                load_bc4(k + 1);
                prep_x((k + 1) & 1);
                M3_FENCE();
                load_x(k + 2);
                M3_FENCE();
                if (kFull) {
                    stage_z((k + 1) & 1);
                    M3_FENCE();
                    load_z(k + 2);
                    M3_FENCE();
                }
                prep(k + 1, k + 2);
            }
            __syncthreads();
            if (more) write_tiles();
        }
        // ---- segment end (helper waves: the last chunk's output, per-pair angles)
        __syncthreads();
        if (kFull) store_out(k_end - 1);
        if (!kFull) {
            const int64_t sidx = (int64_t)bh * (a.S - 1) + seg;
            if (pair_lane) {
                a.seg_angle[sidx * NH + pa0] = phi_run0 * 6.283185307179586f;
                a.seg_angle[sidx * NH + pa0 + 1] = phi_run1 * 6.283185307179586f;
            }
        } else if (seg == a.S - 1) {
            if (pair_lane) {
                sm.rot[pa0] = phi_start0;
                sm.rot[pa0 + 1] = phi_start1;
                if (a.angle) {
                    a.angle[(int64_t)bh * NH + pa0] = a.cplx ? phi_start0 + phi_run0 * 6.283185307179586f : 0.f;
                    a.angle[(int64_t)bh * NH + pa0 + 1] = a.cplx ? phi_start1 + phi_run1 * 6.283185307179586f : 0.f;
                }
            }
            __syncthreads();
        }
    }

}

}  // namespace mf

bool mfma_prefill_supported(const m3_layer_desc& d, const void* proj, const void* y_out) {
    if (d.dtype != M3_DTYPE_BF16) return false;
    if (d.d_state != mf::N || d.headdim != mf::P || d.mimo_rank != mf::R) return false;
    const ProjLayout pl = proj_layout(d);
    // 128-bit x / z loads and y stores, 32-bit theta loads.
    if (d.proj_row_stride % 8 != 0 || pl.x % 8 != 0 || pl.z % 8 != 0 || pl.theta % 2 != 0) return false;
    if (reinterpret_cast<uintptr_t>(proj) % 16 != 0 || reinterpret_cast<uintptr_t>(y_out) % 16 != 0)
        return false;
    // Row offsets are formed with 24-bit multiplies (v_mul_i32_i24): the row strides stay
    // below 2^23 elements.
    if (d.proj_row_stride >= (1 << 23) || (int64_t)d.ngroups * mf::NR >= (1 << 23) ||
        (int64_t)d.nheads * d.headdim >= (1 << 23))
        return false;
    // 32-bit buffer offsets: one batch row of proj (and of B^/C^) stays below 2 GiB.
    if ((int64_t)(d.seqlen + 1) * d.proj_row_stride * 2 >= ((int64_t)1 << 31)) return false;
    if ((int64_t)(d.seqlen + 1) * d.ngroups * mf::NR * 2 >= ((int64_t)1 << 31)) return false;
    return true;
}

// Work plan of the chunk walk: every (batch, head) sequence is cut into S segments, segment 0
// of `first` chunks and the others of `cps` chunks (the last may be shorter). Segments after
// the first need their predecessors' end states, from a state-only pass over segments
// 0..S-2 launched before the full pass.
struct SegPlan {
    int S, cps, first, order;
};

// Costs in chunk-times of one full-pass workgroup (one workgroup fills a CU). The state-only
// pass takes 0.45 of that per chunk (measured at (8, 8192): 2.17 us against 4.85 us). Every
// workgroup also pays a fixed cost for its pipeline fill and drain (1.5 chunk-times in the
// full pass, 1.0 in the state pass: fitted to (4, 2048), where two equal segments beat one,
// eight and long-first splits); a split plan pays one more launch and each segment's
// combine of earlier states.
constexpr double kStatePassCost = 0.45;
constexpr double kSegFixed = 1.5, kStateSegFixed = 1.0;
constexpr int kXcds = 8, kCusPerXcd = 32;

// Makespan of workgroups of the given lengths dispatched in order onto the CUs of one XCD,
// each to the CU that frees first.
static double xcd_makespan(const double* len, int n) {
    double cu[kCusPerXcd] = {};
    double end = 0.0;
    for (int i = 0; i < n; ++i) {
        double* c = std::min_element(cu, cu + kCusPerXcd);
        *c += len[i];
        end = std::max(end, *c);
    }
    return end;
}

// Uniform plans (S equal segments, workgroups of a launch spread evenly over the XCDs) and,
// when the (batch, head) pairs fill at most one CU each and divide evenly over the XCDs, the
// long-first split: segment 0 short, segment 1 long, the long segments start at once and the
// short ones cycle through the CUs left over. Pick the cheapest.
static SegPlan mfma_plan(const m3_layer_desc& d) {
    const int K = (d.seqlen + mf::Q - 1) / mf::Q;
    const int64_t bh = (int64_t)d.batch * d.nheads;
    // The search below costs tens of microseconds of host time; the workspace query and the
    // launch of one call ask for the same shape, so the last plan is kept per thread.
    thread_local int64_t memo_bh = -1;
    thread_local int memo_K = -1;
    thread_local SegPlan memo{1, 1, 1, 0};
    if (bh == memo_bh && K == memo_K) return memo;
    const int64_t cus = (int64_t)kXcds * kCusPerXcd;
    auto rounds = [&](int64_t n) { return (double)((n + cus - 1) / cus); };
    SegPlan best{1, K, K, 0};
    double best_cost = rounds(bh) * (K + kSegFixed);
    for (int s = 2; s <= std::min(K, 64); ++s) {
        const int c = (K + s - 1) / s;
        const int seff = (K + c - 1) / c;
        if (seff != s) continue;
        const double cost = rounds(bh * s) * (c + kSegFixed) +
                            rounds(bh * (s - 1)) * (kStatePassCost * c + kStateSegFixed) + 1.0 + 0.25 * (s - 1);
        if (cost < best_cost - 1e-9) {
            best_cost = cost;
            best = SegPlan{s, c, c, 0};
        }
    }
    if (bh % kXcds == 0 && bh <= cus && K >= 2) {
        const int L = (int)(bh / kXcds);
        double len[2 * kCusPerXcd];
        for (int f = 1; f <= K / 2; ++f) {
            for (int i = 0; i < L; ++i) {
                len[i] = K - f + kSegFixed;
                len[L + i] = f + kSegFixed;
            }
            const double cost = kStatePassCost * f + kStateSegFixed + xcd_makespan(len, 2 * L) + 1.0 + 0.25;
            if (cost < best_cost - 1e-9) {
                best_cost = cost;
                best = SegPlan{2, K - f, f, 1};
            }
        }
    }
    memo_bh = bh;
    memo_K = K;
    memo = best;
    return best;
}

// The (token, group) rows of tokens [lo, hi) of every batch row.
static mf::BcRows bc_rows(const m3_layer_desc& d, const m3_layer_params& p, const void* proj,
                          f16* bn, f16* cn, int64_t lo, int64_t hi) {
    const ProjLayout pl = proj_layout(d);
    mf::BcRows c;
    c.proj = reinterpret_cast<const bf16*>(proj);
    c.rs = d.proj_row_stride;
    c.offB = pl.B;
    c.offC = pl.C;
    c.G = d.ngroups;
    c.eps = d.rms_eps;
    c.wB = p.B_norm_w;
    c.biasB = p.B_bias;
    c.wC = p.C_norm_w;
    c.biasC = p.C_bias;
    c.Bn = bn;
    c.Cn = cn;
    c.per_b = (hi - lo) * d.ngroups;
    c.nrows = (int64_t)d.batch * c.per_b;
    c.skip = (int64_t)d.seqlen * d.ngroups - c.per_b;
    c.lo_g = lo * d.ngroups;
    return c;
}

static void launch_bc_rows(const mf::BcRows& c, hipStream_t stream) {
    const int64_t rows_per_block = 4 * mf::kBcTok;
    if (c.nrows > 0)
        hipLaunchKernelGGL(mf::bc_norm, dim3((unsigned)((c.nrows + rows_per_block - 1) / rows_per_block)),
                           dim3(256), 0, stream, c);
}

// B^ / C^ rows of every (token, group) of the layer, pair-packed f16 (bc_norm).
void launch_bc_norm(const m3_layer_desc& d, const m3_layer_params& p, const void* proj,
                    f16* bn, f16* cn, hipStream_t stream) {
    launch_bc_rows(bc_rows(d, p, proj, bn, cn, 0, d.seqlen), stream);
}

size_t mfma_prefill_workspace(const m3_layer_desc& d) {
    const int S = mfma_plan(d).S;
    const size_t ntg = (size_t)d.batch * d.seqlen * d.ngroups;
    const size_t nseg = (size_t)d.batch * d.nheads * (S - 1);
    const size_t bc_bytes = 2 * ntg * mf::NR * sizeof(f16);
    return bc_bytes + nseg * ((size_t)mf::N * mf::P + 1 + mf::NH) * sizeof(float) + 256;
}

int launch_mfma_prefill(const m3_layer_desc& d, const m3_layer_params& p, const void* proj,
                        const float* dt_scale, void* y_out, float* h_final, float* angle,
                        float* prev_bx, void* workspace, hipStream_t stream) {
    const SegPlan plan = mfma_plan(d);
    const int S = plan.S;
    mf::Args a;
    a.B = d.batch; a.T = d.seqlen; a.H = d.nheads; a.G = d.ngroups;
    a.S = S; a.cps = plan.cps; a.first = plan.first; a.order = plan.order;
    a.trap = d.use_trapezoidal; a.cplx = d.use_complex;
    a.rs = d.proj_row_stride;
    a.pl = proj_layout(d);
    a.prm = p;
    a.proj = reinterpret_cast<const bf16*>(proj);
    a.dt_scale = dt_scale;
    const int64_t ntg = (int64_t)d.batch * d.seqlen * d.ngroups;
    const int64_t nseg = (int64_t)d.batch * d.nheads * (S - 1);
    f16* bn = reinterpret_cast<f16*>(workspace);
    f16* cn = bn + ntg * mf::NR;
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

    // With a state pass that leaves CUs idle, the B^ / C^ of the tokens it reads are
    // normalised first and those of the other tokens by spare workgroups of the state pass.
    a.nstate = (int)nseg;
    const int ncu = kXcds * kCusPerXcd;
    const int64_t t_state = S > 1 ? std::min<int64_t>(d.seqlen, (int64_t)(plan.first + (S - 2) * plan.cps) * mf::Q) : 0;
    const int nspare = (S > 1 && nseg < ncu && t_state < d.seqlen) ? ncu - (int)nseg : 0;
    if (nspare > 0) {
        launch_bc_rows(bc_rows(d, p, proj, bn, cn, 0, t_state), stream);
        a.bcr = bc_rows(d, p, proj, bn, cn, t_state, d.seqlen);
    } else {
        launch_bc_norm(d, p, proj, bn, cn, stream);
        a.bcr = bc_rows(d, p, proj, bn, cn, 0, 0);
    }
    if (S > 1)
        hipLaunchKernelGGL(mf::ssd_chunks<false>, dim3((unsigned)(nseg + nspare)), dim3(mf::THREADS), 0,
                           stream, a);
    hipLaunchKernelGGL(mf::ssd_chunks<true>, dim3((unsigned)(d.batch * d.nheads * S)),
                       dim3(mf::THREADS), 0, stream, a);
    return hipGetLastError() == hipSuccess ? M3_OK : M3_ERR_LAUNCH;
}

}  // namespace m3
