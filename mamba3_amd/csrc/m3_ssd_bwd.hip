// fp32-MFMA chunk kernels of the chunked SSD on pre-processed inputs (the op of
// m3_chunked_ssd_fwd): its backward, and (with Args::fwd set) its fp32 forward, which reuses
// the chunk-state, scan and score kernels (their gradient halves skipped) and adds the output
// tiles fwd_out (y = (W o G) Xf + exp(c_t) C H_k^T + D x_raw).
//
// The backward replaces, under autograd, the reference's chunked_ssd (mamba3/ssd.py:118-244): the custom
// backward of _IntraChunkFn (ssd.py:67-115), the scan backward (mamba3/scan.py:101-141,
// mamba3/csrc/scan.cu:52-126) and ATen's backward of the bmm / cumsum / exp around them. The
// reference differentiates through the materialised per-token outer products
// BX_total (B,K,H,Q,P,N); this file never forms them.
//
// Per (batch b, head h) and chunk k of Qb tokens (positions t, s in [0, Qb)), with
// c_t = sum_{j<=t} A dt_j, W[t,s] = exp(c_t - c_s) for s <= t (else 0), the R2 = R or 2R
// factor columns Xf[s,p,j] = dt_s x[s,p,j] (x_g, then x_b) and Bf[s,n,j] (B_g, then B_b):
//   h at token t     = exp(c_t) H_k + sum_{s<=t} W[t,s] sum_j Xf[s,:,j] Bf[s,:,j]^T
//   y[t,p,r]         = sum_n C[t,n,r] h_t[p,n] + D x_raw[t,p,r]
//   H_{k+1}          = exp(c_end) H_k + sum_s exp(c_end - c_s) sum_j Xf[s,:,j] Bf[s,:,j]^T
// Gradients, with dH = dL/dH_{k+1} (from the reverse scan), G[(t,r),(s,j)] = C_t.Bf_s and
// DX[(t,r),(s,j)] = dy_t.Xf_s, M = W o G, DM = W o DX:
//   dXf[s,p,j] = sum_{t,r} M[(t,r),(s,j)] dy[t,p,r] + exp(c_end - c_s) sum_n Bf[s,n,j] dH[p,n]
//   dBf[s,n,j] = sum_{t,r} DM[(t,r),(s,j)] C[t,n,r] + exp(c_end - c_s) sum_p Xf[s,p,j] dH[p,n]
//   dC[t,n,r]  = sum_{s,j} DM[(t,r),(s,j)] Bf[s,n,j] + exp(c_t) sum_p dy[t,p,r] H_k[p,n]
//   dc_t       = sum_s W Z[t,s] - sum_{t'} W Z[t',t] + sum_{p,r} dy[t,p,r] y_inter[t,p,r]
//                - q_t + [t = Qb-1] (sum_s q_s + exp(c_end) <dH, H_k>),
//                Z = sum_{r,j} G o DX,  q_s = sum_{p,j} Xf[s,p,j] (state term of dXf)[s,p,j]
//   d(A dt_t)  = sum_{t'>=t} dc_t';  ddt_t = A d(A dt_t) + sum_{p,j} dXf[s,p,j] x[s,p,j]
// Qb = min(64, 128 / R2), so that the score tiles are at most 128 x 128; with the beta terms
// they are one 64 x 128 tile, which bwd_fused keeps in LDS (M and DM never reach memory),
// otherwise bwd_scores writes M and DM for bwd_dxf / bwd_dbf / bwd_dc. R here is the rank
// of the tiles, a power of two: ranks 3, 5, 6 and 7 run on tiles of rank 4 or 8 whose extra
// slots read as zero (their rows and columns of G, DX, M and DM are zero). The chunk
// states H_k and dH come from the state scan kernels over K+1 chunks, the last one carrying
// dL/dh_final. Every sum runs in a fixed order: results are deterministic.
#include <hip/hip_runtime.h>

#include "m3_kernels.h"
#include "m3_mfma.h"

namespace m3 {
namespace bw {

constexpr int TT = 64;    // output tile edge
constexpr int KT = 16;    // contraction step
constexpr int NTH = 256;  // threads per tile block
constexpr int TW = 128;   // wide output tile (columns over N or the score columns)

// R: the arrays' rank; RT: the rank of the tiles (R rounded up to 1, 2, 4 or 8).
struct Shape {
    int B, T, H, P, N, R, RT, R2, Qb, K, nPt, nNt;
    int64_t PN;
    int QR() const { return Qb * RT; }
    int QR2() const { return Qb * R2; }
};

// Chunk of QB = min(64, 128 / R2) tokens for rank R (R2 = 2R with the beta terms): score
// tiles (t,r) x (s,j) of QR x QR2 <= 128 x 128.
#define BW_CONSTS                                   \
    constexpr int R2 = BETA ? 2 * R : R;            \
    constexpr int QB = 128 / R2 >= 64 ? 64 : 128 / R2; \
    constexpr int QR = QB * R, QR2 = QB * R2;       \
    (void)QR;                                        \
    (void)QR2;

struct Args {
    Shape s;
    const float *xg, *xb, *Bg, *Bb, *C, *dt, *A, *D, *xr, *hinit, *dy, *dhf;
    float *dxg, *dxb, *dBg, *dBb, *dC, *ddt, *dA, *dD, *dxr, *dhinit;
    // workspace
    float *cum, *dec, *ddec, *hext, *Hs, *gext, *dch, *M, *DM, *dcI, *pInter, *pState, *pDt,
        *pA, *pD;
    // forward (fwd = 1): the chunk-state and score kernels skip their gradient halves
    int fwd;
    // have_hs = 1: the chunk-start states Hs come from the forward (the chunk-local states and
    // the forward scan are skipped)
    int have_hs;
    // comb_b = 1 (the layer's backward, with the beta terms): dBg receives dB_g[t] + dB_b[t + 1]
    // (B_b of a token is the rotated B of the token before it) and dBb only the b part of
    // each chunk's first token, as (B, K, H, N, R) rows, which belong to the previous chunk's
    // last token
    int comb_b;
    float *y, *hfin;
};

// Chunk ch = (b K + k) H + h (the scan's (B,K,H) order); its position in the (B,K+1,H)
// arrays of the extended scan.
__device__ __forceinline__ int64_t chx(const Shape& s, int b, int k, int h) {
    return ((int64_t)b * (s.K + 1) + k) * s.H + h;
}
// Chunk and tile of a block of a kernel with `tiles` output tiles per chunk, launched as one
// dimension of tile_grid(nch, tiles) blocks: the tiles of a chunk are 8 block indices apart, so
// they run on one XCD (workgroups are dealt round-robin over the 8 XCDs) at about the same
// time and share the chunk's operands through that XCD's L2. False for the padding blocks.
constexpr int kXcds = 8;
__device__ __forceinline__ bool chunk_tile(int nch, int tiles, int& ch, int& tile) {
    const int L = blockIdx.x, rest = L / kXcds;
    tile = rest % tiles;
    ch = (rest / tiles) * kXcds + L % kXcds;
    return ch < nch;
}
inline unsigned tile_grid(int64_t nch, int tiles) {
    return (unsigned)((nch + kXcds - 1) / kXcds * kXcds * tiles);
}

// Offset of token row (b, tg, h) of a (B,T,H,X,R) tensor, in units of X*R elements.
__device__ __forceinline__ int64_t row(const Shape& s, int b, int tg, int h) {
    return ((int64_t)b * s.T + tg) * s.H + h;
}

// Rows padded to a stride of 17 (mod 32) floats: the MFMA operand reads (16 lanes per k-row,
// 4 k-rows) and the stores of k-fastest fetches (16 k-rows per column) spread over the banks.
template <int TN>
struct Lds {
    float A[KT][TT + 17];
    float B[KT][TN + 17];
};

// Tile layout of the fp32 MFMA accumulators (v_mfma_f32_16x16x4_f32: lane l holds rows
// 4 (l / 16) + v, v < 4, of column l % 16 of a 16 x 16 block): wave w owns rows 16w..16w+15 of
// the 64-row tile, so thread (tx, ty) = (tid % 16, tid / 16) holds rows 4 ty + v of the columns
// tcol(tx, j) = tx + 16 j; its accumulator acc[j][v].
__device__ __forceinline__ int tcol(int tx, int j) { return tx + 16 * j; }

// threadIdx.x through an empty asm: values derived from it are formed where they are used and
// cannot be hoisted out of the GEMM or tile that uses them (a kernel running several GEMMs in
// sequence would otherwise keep every GEMM's per-thread addresses live from its entry).
__device__ __forceinline__ int opaque_tid() {
    int t = threadIdx.x;
    asm volatile("" : "+v"(t));
    return t;
}

// acc[j][v] += sum_k A(4 ty + v, k) B(k, tcol(tx, j)) over k < kdim, for the 64 x TN tile of
// a 256-thread block, on fp32 MFMA. Each operand comes as a load and a finish: la(m, k) /
// lb(k, n) read element (m, k) / (k, n) from an address that is in bounds for every row
// m < 64 (column n < TN) and k < kdim, without a branch; fa(m, k, v) / fb(k, n, v) turn the
// loaded value into the operand's (zero outside the operand, scaled) once it has arrived,
// also without a branch. The loads of step k0 + KT are issued while step k0 is multiplied and
// finished as they are stored to LDS, so no load waits inside the step that issues it. AK / BK
// pick the order in which consecutive threads fetch an operand: k fastest (for operands
// contiguous along k in memory) or row / column fastest.
template <int TN, bool AK, bool BK, class LA, class FA, class LB, class FB>
__device__ __forceinline__ void gemm_acc(f32x4 (&acc)[TN / 16], int kdim, LA la, FA fa, LB lb,
                                         FB fb, Lds<TN>& l) {
    constexpr int NA = KT * TT / NTH;  // A elements per thread and step
    constexpr int NB = KT * TN / NTH;  // B elements per thread and step
    const int tid = opaque_tid(), lane = tid & 63, wave = tid >> 6;
    auto ak = [](int e) { return AK ? e % KT : e / TT; };
    auto am = [](int e) { return AK ? e / KT : e % TT; };
    auto bk = [](int e) { return BK ? e % KT : e / TN; };
    auto bn = [](int e) { return BK ? e / KT : e % TN; };
    float ra[NA], rb[NB];
    auto fetch = [&](int k0) {
#pragma unroll
        for (int i = 0; i < NA; ++i) {
            const int e = tid + NTH * i;
            ra[i] = la(am(e), min(k0 + ak(e), kdim - 1));
        }
#pragma unroll
        for (int i = 0; i < NB; ++i) {
            const int e = tid + NTH * i;
            rb[i] = lb(min(k0 + bk(e), kdim - 1), bn(e));
        }
    };
    fetch(0);
#pragma unroll 1
    for (int k0 = 0; k0 < kdim; k0 += KT) {
#pragma unroll
        for (int i = 0; i < NA; ++i) {
            const int e = tid + NTH * i, k = k0 + ak(e);
            const float v = fa(am(e), min(k, kdim - 1), ra[i]);
            l.A[ak(e)][am(e)] = k < kdim ? v : 0.f;
        }
#pragma unroll
        for (int i = 0; i < NB; ++i) {
            const int e = tid + NTH * i, k = k0 + bk(e);
            const float v = fb(min(k, kdim - 1), bn(e), rb[i]);
            l.B[bk(e)][bn(e)] = k < kdim ? v : 0.f;
        }
        __syncthreads();
        if (k0 + KT < kdim) fetch(k0 + KT);
#pragma unroll
        for (int k4 = 0; k4 < KT; k4 += 4) {
            const float av = l.A[k4 + (lane >> 4)][16 * wave + (lane & 15)];
#pragma unroll
            for (int j = 0; j < TN / 16; ++j) {
                const float bv = l.B[k4 + (lane >> 4)][16 * j + (lane & 15)];
                acc[j] = __builtin_amdgcn_mfma_f32_16x16x4f32(av, bv, acc[j], 0, 0, 0);
            }
        }
        __syncthreads();
    }
}

// As gemm_acc<TN, true, BK>, with each A element the sum of two finished loads:
// A(m, k) = fa(m, k, la(m, k)) + fa2(m, k, la2(m, k)).
template <int TN, bool BK, class LA, class FA, class LA2, class FA2, class LB, class FB>
__device__ __forceinline__ void gemm_acc_a2(f32x4 (&acc)[TN / 16], int kdim, LA la, FA fa, LA2 la2,
                                            FA2 fa2, LB lb, FB fb, Lds<TN>& l) {
    constexpr int NA = KT * TT / NTH;
    constexpr int NB = KT * TN / NTH;
    const int tid = opaque_tid(), lane = tid & 63, wave = tid >> 6;
    auto ak = [](int e) { return e % KT; };
    auto am = [](int e) { return e / KT; };
    auto bk = [](int e) { return BK ? e % KT : e / TN; };
    auto bn = [](int e) { return BK ? e / KT : e % TN; };
    float ra[NA], ra2[NA], rb[NB];
    auto fetch = [&](int k0) {
#pragma unroll
        for (int i = 0; i < NA; ++i) {
            const int e = tid + NTH * i, k = min(k0 + ak(e), kdim - 1);
            ra[i] = la(am(e), k);
            ra2[i] = la2(am(e), k);
        }
#pragma unroll
        for (int i = 0; i < NB; ++i) {
            const int e = tid + NTH * i;
            rb[i] = lb(min(k0 + bk(e), kdim - 1), bn(e));
        }
    };
    fetch(0);
#pragma unroll 1
    for (int k0 = 0; k0 < kdim; k0 += KT) {
#pragma unroll
        for (int i = 0; i < NA; ++i) {
            const int e = tid + NTH * i, k = k0 + ak(e), kc = min(k, kdim - 1);
            const float v = fa(am(e), kc, ra[i]) + fa2(am(e), kc, ra2[i]);
            l.A[ak(e)][am(e)] = k < kdim ? v : 0.f;
        }
#pragma unroll
        for (int i = 0; i < NB; ++i) {
            const int e = tid + NTH * i, k = k0 + bk(e);
            const float v = fb(min(k, kdim - 1), bn(e), rb[i]);
            l.B[bk(e)][bn(e)] = k < kdim ? v : 0.f;
        }
        __syncthreads();
        if (k0 + KT < kdim) fetch(k0 + KT);
#pragma unroll
        for (int k4 = 0; k4 < KT; k4 += 4) {
            const float av = l.A[k4 + (lane >> 4)][16 * wave + (lane & 15)];
#pragma unroll
            for (int j = 0; j < TN / 16; ++j) {
                const float bv = l.B[k4 + (lane >> 4)][16 * j + (lane & 15)];
                acc[j] = __builtin_amdgcn_mfma_f32_16x16x4f32(av, bv, acc[j], 0, 0, 0);
            }
        }
        __syncthreads();
    }
}

// As gemm_acc, with the A operand read by the MFMA steps straight from an LDS matrix:
// A(m, k) = as(m, k) for m < 64 and k < kdim (a multiple of KT); only B is staged.
template <int TN, bool BK, class AS, class LB, class FB>
__device__ __forceinline__ void gemm_lds_a(f32x4 (&acc)[TN / 16], int kdim, AS as, LB lb, FB fb,
                                           Lds<TN>& l) {
    constexpr int NB = KT * TN / NTH;
    const int tid = opaque_tid(), lane = tid & 63, wave = tid >> 6;
    auto bk = [](int e) { return BK ? e % KT : e / TN; };
    auto bn = [](int e) { return BK ? e / KT : e % TN; };
    float rb[NB];
    auto fetch = [&](int k0) {
#pragma unroll
        for (int i = 0; i < NB; ++i) {
            const int e = tid + NTH * i;
            rb[i] = lb(k0 + bk(e), bn(e));
        }
    };
    fetch(0);
#pragma unroll 1
    for (int k0 = 0; k0 < kdim; k0 += KT) {
#pragma unroll
        for (int i = 0; i < NB; ++i) {
            const int e = tid + NTH * i;
            l.B[bk(e)][bn(e)] = fb(k0 + bk(e), bn(e), rb[i]);
        }
        __syncthreads();
        if (k0 + KT < kdim) fetch(k0 + KT);
#pragma unroll
        for (int k4 = 0; k4 < KT; k4 += 4) {
            const float av = as(16 * wave + (lane & 15), k0 + k4 + (lane >> 4));
#pragma unroll
            for (int j = 0; j < TN / 16; ++j) {
                const float bv = l.B[k4 + (lane >> 4)][16 * j + (lane & 15)];
                acc[j] = __builtin_amdgcn_mfma_f32_16x16x4f32(av, bv, acc[j], 0, 0, 0);
            }
        }
        __syncthreads();
    }
}

template <int NJ>
__device__ __forceinline__ void zero(f32x4 (&acc)[NJ]) {
#pragma unroll
    for (int j = 0; j < NJ; ++j) acc[j] = f32x4{0.f, 0.f, 0.f, 0.f};
}

// Accessors of chunk (b, k, h). Token positions at or past T read as 0. R is the rank of
// the tiles; with PADR the arrays hold a smaller rank s.R (3 for R = 4; 5, 6 or 7 for R = 8)
// and the tile slots of the missing ranks read as 0, so every score, state and output term
// of the real ranks is the unpadded one, and the kernels store nothing for those slots.
template <int R, bool BETA, bool PADR>
struct Chunk {
    static constexpr int R2 = BETA ? 2 * R : R;
    static constexpr int QB = 128 / R2 >= 64 ? 64 : 128 / R2;
    const Args* a;
    int b, k, h;
    // Token 0 of the chunk in every per-token array, the 32-bit element strides between
    // consecutive tokens and the number of tokens below T: the GEMM operand fetches (one
    // element each) are then a compare and two 24-bit multiply-adds.
    int nt, tsP, tsN, tsH, ra;
    const float *xg0, *xb0, *bg0, *bb0, *c0, *dy0, *dt0, *xr0;
    __device__ Chunk(const Args* a_, int b_, int k_, int h_) : a(a_), b(b_), k(k_), h(h_) {
        const Shape& s = a->s;
        ra = PADR ? s.R : R;
        nt = min(QB, s.T - k * QB);
        tsP = s.H * s.P * rk();
        tsN = s.H * s.N * rk();
        tsH = s.H;
        const int64_t r0 = row(s, b, k * QB, h);
        const int64_t oP = r0 * s.P * rk(), oN = r0 * s.N * rk();
        xg0 = a->xg + oP;
        bg0 = a->Bg + oN;
        xb0 = BETA ? a->xb + oP : nullptr;
        bb0 = BETA ? a->Bb + oN : nullptr;
        c0 = a->C + oN;
        dy0 = a->dy ? a->dy + oP : nullptr;
        dt0 = a->dt + r0;
        xr0 = a->xr + oP;
    }
    // The arrays' rank (R unless PADR).
    __device__ int rk() const {
        if constexpr (PADR) return ra;
        return R;
    }
    // Whether rank slot r (< R) of the tiles holds a real rank.
    __device__ bool has(int r) const { return !PADR || r < rk(); }
    __device__ bool real(int t) const { return t < nt; }
    // Loads without a branch: the token is clamped into the chunk's real tokens and the rank
    // slot into the array's ranks, so the address is in bounds for any t < QB + 64 and column
    // below P (N); ok() / okj() say whether the loaded value is a real element (the operands
    // are zero where it is not).
    __device__ int tcl(int t) const { return min(t, nt - 1); }
    __device__ int rcl(int r) const {
        if constexpr (PADR) return min(r, ra - 1);
        return r;
    }
    __device__ bool ok(int t, int r) const { return real(t) && has(r); }
    __device__ bool okj(int t, int j) const { return ok(t, j < R ? j : j - R); }
    __device__ float lx(int t, int p, int j) const {
        const bool g = !BETA || j < R;
        return (g ? xg0 : xb0)[tcl(t) * tsP + p * rk() + rcl(g ? j : j - R)];
    }
    __device__ float lbf(int t, int n, int j) const {
        const bool g = !BETA || j < R;
        return (g ? bg0 : bb0)[tcl(t) * tsN + n * rk() + rcl(g ? j : j - R)];
    }
    __device__ float lc(int t, int n, int r) const { return c0[tcl(t) * tsN + n * rk() + rcl(r)]; }
    __device__ float ldy(int t, int p, int r) const { return dy0[tcl(t) * tsP + p * rk() + rcl(r)]; }
    __device__ float lxr(int t, int p, int r) const { return xr0[tcl(t) * tsP + p * rk() + rcl(r)]; }
    __device__ float ldt(int t) const { return dt0[tcl(t) * tsH]; }
    __device__ float dtv(int t) const { return real(t) ? dt0[t * tsH] : 0.f; }
    // x factor j of token t (x_g rank j for j < R, else x_b rank j - R), without dt.
    __device__ float x(int t, int p, int j) const {
        const int r = j < R ? j : j - R;
        if (!real(t) || !has(r)) return 0.f;
        return (j < R ? xg0 : xb0)[t * tsP + p * rk() + r];
    }
    __device__ float bf(int t, int n, int j) const {
        const int r = j < R ? j : j - R;
        if (!real(t) || !has(r)) return 0.f;
        return (j < R ? bg0 : bb0)[t * tsN + n * rk() + r];
    }
    __device__ float c(int t, int n, int r) const {
        return real(t) && has(r) ? c0[t * tsN + n * rk() + r] : 0.f;
    }
    __device__ float dy(int t, int p, int r) const {
        return real(t) && has(r) ? dy0[t * tsP + p * rk() + r] : 0.f;
    }
};

// ---- K0: c_t (inclusive cumsum of A dt within the chunk) and the chunk decays.
template <int R, bool BETA, bool PADR>
__global__ __launch_bounds__(64) void bwd_cum(Args a) {
    BW_CONSTS
    const Shape& s = a.s;
    const int ch = blockIdx.x, h = ch % s.H, k = (ch / s.H) % s.K, b = ch / (s.H * s.K);
    const int t = threadIdx.x, tg = k * QB + t;
    const float l = (t < QB && tg < s.T) ? a.A[h] * a.dt[row(s, b, tg, h)] : 0.f;
    const float c = wave_incl_scan(l);
    if (t < QB) a.cum[(int64_t)ch * QB + t] = c;
    if (t == QB - 1) {
        a.dec[chx(s, b, k, h)] = __expf(c);
        if (k == s.K - 1) a.dec[chx(s, b, s.K, h)] = 1.f;
    }
}

// ---- K2: chunk-local states (scan input) and the y_inter gradient of each chunk state:
//   hext[k][p,n] = sum_{s,j} exp(c_end - c_s) Xf[s,p,j] Bf[s,n,j]
//   gext[k][p,n] = sum_{t,r} exp(c_t) dy[t,p,r] C[t,n,r]
// plus the extra chunk K: hext = 0, gext = dL/dh_final (or 0). Tiles of 64 p x 128 n.
template <int R, bool BETA, bool PADR>
__global__ __launch_bounds__(NTH) void bwd_states(Args a) {
    BW_CONSTS
    __shared__ Lds<TW> l;
    __shared__ float cs[64], wx[64], ec[64];
    const Shape& s = a.s;
    int ch, tile;
    if (!chunk_tile(s.B * s.K * s.H, s.nPt * s.nNt, ch, tile)) return;
    const int h = ch % s.H, k = (ch / s.H) % s.K, b = ch / (s.H * s.K);
    const int pt = tile / s.nNt, nt = tile % s.nNt;
    const int p0 = pt * TT, n0 = nt * TW;
    const Chunk<R, BETA, PADR> q{&a, b, k, h};
    if (threadIdx.x < QB) cs[threadIdx.x] = a.cum[(int64_t)ch * QB + threadIdx.x];
    __syncthreads();
    if (threadIdx.x < QB) {  // per-token weights of the two contractions
        const int t = threadIdx.x;
        wx[t] = __expf(cs[QB - 1] - cs[t]) * q.dtv(t);
        ec[t] = __expf(cs[t]);
    }
    __syncthreads();
    const int tx = threadIdx.x & 15, ty = threadIdx.x >> 4;
    constexpr int NJ = TW / 16;
    f32x4 acc[NJ];
    const int pmax = s.P - 1, nmax = s.N - 1;
    if (!a.have_hs) {
    zero(acc);
    gemm_acc<TW, false, false>(acc, QB * R2,
                 [&](int mm, int j) { return q.lx(j / R2, min(p0 + mm, pmax), j % R2); },
                 [&](int mm, int j, float v) {
                     const int t = j / R2;
                     const float w = wx[t];
                     return p0 + mm < s.P && q.okj(t, j % R2) ? w * v : 0.f;
                 },
                 [&](int j, int nn) { return q.lbf(j / R2, min(n0 + nn, nmax), j % R2); },
                 [&](int j, int nn, float v) { return n0 + nn < s.N && q.okj(j / R2, j % R2) ? v : 0.f; },
                 l);
    float* ho = a.hext + chx(s, b, k, h) * s.PN;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
            const int p = p0 + 4 * ty + i, n = n0 + tcol(tx, j);
            if (p < s.P && n < s.N) ho[(int64_t)p * s.N + n] = acc[j][i];
        }
    }
    if (!a.fwd) {
    zero(acc);
    gemm_acc<TW, false, false>(acc, QB * R,
                 [&](int mm, int j) { return q.ldy(j / R, min(p0 + mm, pmax), j % R); },
                 [&](int mm, int j, float v) {
                     const int t = j / R;
                     const float w = ec[t];
                     return p0 + mm < s.P && q.ok(t, j % R) ? w * v : 0.f;
                 },
                 [&](int j, int nn) { return q.lc(j / R, min(n0 + nn, nmax), j % R); },
                 [&](int j, int nn, float v) { return n0 + nn < s.N && q.ok(j / R, j % R) ? v : 0.f; },
                 l);
    float* go = a.gext + chx(s, b, k, h) * s.PN;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
            const int p = p0 + 4 * ty + i, n = n0 + tcol(tx, j);
            if (p < s.P && n < s.N) go[(int64_t)p * s.N + n] = acc[j][i];
        }
    }
    if (k == s.K - 1) {
        float* he = a.hext + chx(s, b, s.K, h) * s.PN;
        float* ge = a.gext + chx(s, b, s.K, h) * s.PN;
        const float* df = a.dhf ? a.dhf + ((int64_t)b * s.H + h) * s.PN : nullptr;
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < NJ; ++j) {
                const int p = p0 + 4 * ty + i, n = n0 + tcol(tx, j);
                if (p < s.P && n < s.N) {
                    const int64_t o = (int64_t)p * s.N + n;
                    if (!a.have_hs) he[o] = 0.f;
                    if (!a.fwd) ge[o] = df ? df[o] : 0.f;
                }
            }
    }
}

// ---- K1: masked scores M = W o G and DM = W o DX of the chunk, and the intra-chunk part of
// dc: sum_s W Z[t,s] - sum_t' W Z[t',t]. One block per chunk, looping over its 64 x 128 tiles;
// W o G waits in LDS while DX is formed.
template <int R, bool BETA, bool PADR>
__global__ __launch_bounds__(NTH) void bwd_scores(Args a) {
    BW_CONSTS
    __shared__ Lds<TW> l;
    __shared__ float zp[TT][TW + 1];
    __shared__ float cs[64], dts[64], rowacc[64], colacc[64];
    __shared__ float rowp[4][TT], colp[2][TW];
    const Shape& s = a.s;
    const int ch = blockIdx.x, h = ch % s.H, k = (ch / s.H) % s.K, b = ch / (s.H * s.K);
    const Chunk<R, BETA, PADR> q{&a, b, k, h};
    const int tid = threadIdx.x, tx = tid & 15, ty = tid >> 4;
    if (tid < 64) {
        cs[tid] = tid < QB ? a.cum[(int64_t)ch * QB + tid] : 0.f;
        dts[tid] = tid < QB ? q.dtv(tid) : 0.f;
        rowacc[tid] = 0.f;
        colacc[tid] = 0.f;
    }
    __syncthreads();
    float* Mo = a.M + (int64_t)ch * QR * QR2;
    float* DMo = a.DM + (int64_t)ch * QR * QR2;
    constexpr int NJ = TW / 16;
    for (int m0 = 0; m0 < QR; m0 += TT) {
        for (int c0 = 0; c0 < QR2; c0 += TW) {
            f32x4 g[NJ];
            zero(g);
            // G[(t,r),(s,j)] = sum_n C[t,n,r] Bf[s,n,j]
            gemm_acc<TW, true, true>(g, s.N,
                         [&](int mm, int n) { const int m = m0 + mm; return q.lc(m / R, n, m % R); },
                         [&](int mm, int n, float v) { const int m = m0 + mm; return q.ok(m / R, m % R) ? v : 0.f; },
                         [&](int n, int cc) { const int c = c0 + cc; return q.lbf(c / R2, n, c % R2); },
                         [&](int n, int cc, float v) {
                             const int c = c0 + cc;
                             return c < QR2 && q.okj(c / R2, c % R2) ? v : 0.f;
                         },
                         l);
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < NJ; ++j) {
                    const int m = m0 + 4 * ty + i, c = c0 + tcol(tx, j);
                    const int t = m / R, u = c / R2;
                    const float w = c < QR2 && u <= t ? __expf(cs[t] - cs[u]) : 0.f;
                    if (c < QR2) Mo[(int64_t)m * QR2 + c] = w * g[j][i];
                    zp[4 * ty + i][tcol(tx, j)] = w * g[j][i];
                }
            if (a.fwd) continue;
            // DX[(t,r),(s,j)] = sum_p dy[t,p,r] dt_s x[s,p,j]; gemm_acc's first barrier orders
            // the zp writes above before the reads below
            zero(g);
            gemm_acc<TW, true, true>(g, s.P,
                         [&](int mm, int p) { const int m = m0 + mm; return q.ldy(m / R, p, m % R); },
                         [&](int mm, int p, float v) { const int m = m0 + mm; return q.ok(m / R, m % R) ? v : 0.f; },
                         [&](int p, int cc) { const int c = c0 + cc; return q.lx(c / R2, p, c % R2); },
                         [&](int p, int cc, float v) {
                             const int c = c0 + cc, t = min(c / R2, 63);
                             const float d = dts[t];
                             return c < QR2 && q.okj(c / R2, c % R2) ? d * v : 0.f;
                         },
                         l);
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < NJ; ++j) {
                    const int m = m0 + 4 * ty + i, c = c0 + tcol(tx, j);
                    const int t = m / R, u = c / R2;
                    const float w = c < QR2 && u <= t ? __expf(cs[t] - cs[u]) : 0.f;
                    if (c < QR2) DMo[(int64_t)m * QR2 + c] = w * g[j][i];
                    zp[4 * ty + i][tcol(tx, j)] *= g[j][i];
                }
            __syncthreads();
            // Z over the (r, j) blocks of the tile, summed into rows (t) and columns (s): first
            // every thread sums 32 entries of one row (a quarter of it) and 32 of one column
            // (half of it), then the token totals add those partials, all in a fixed order.
            const int nt = TT / R, nc = min(TW, QR2 - c0), ns = nc / R2;
            {
                const int rr = tid & 63, c4 = 32 * (tid >> 6);
                float v = 0.f;
#pragma unroll 8
                for (int i = 0; i < 32; ++i) v += c4 + i < nc ? zp[rr][c4 + i] : 0.f;
                rowp[tid >> 6][rr] = v;
                const int cc = tid & 127, r2 = 32 * (tid >> 7);
                float w = 0.f;
#pragma unroll 8
                for (int i = 0; i < 32; ++i) w += zp[r2 + i][cc];
                colp[tid >> 7][cc] = w;
            }
            __syncthreads();
            if (tid < nt) {
                float v = 0.f;
#pragma unroll
                for (int r = 0; r < R; ++r)
                    for (int qq = 0; qq < 4; ++qq) v += rowp[qq][tid * R + r];
                rowacc[m0 / R + tid] += v;
            } else if (tid >= 128 && tid < 128 + ns) {
                const int u = tid - 128;
                float v = 0.f;
                for (int j = 0; j < R2; ++j) v += colp[0][u * R2 + j] + colp[1][u * R2 + j];
                colacc[c0 / R2 + u] += v;
            }
            __syncthreads();
        }
    }
    if (!a.fwd && tid < QB) a.dcI[(int64_t)ch * QB + tid] = rowacc[tid] - colacc[tid];
}

// Sums v over the rows of the 64 x 64 tile that belong to one token (R2 consecutive rows per
// token, `per` of them) and over the 16 column groups, in a fixed order; token u of the tile
// gets the sum in out[u] (threads tid < 64 / per). `red` holds 64 x 16 floats.
__device__ __forceinline__ void tile_token_sums(const float (&v)[4], int per, float (*red)[17],
                                                float* out) {
    const int tid = threadIdx.x, tx = tid & 15, ty = tid >> 4;
#pragma unroll
    for (int i = 0; i < 4; ++i) red[4 * ty + i][tx] = v[i];
    __syncthreads();
    if (tid < TT / per) {
        float acc = 0.f;
        for (int r = 0; r < per; ++r)
            for (int x = 0; x < 16; ++x) acc += red[tid * per + r][x];
        out[tid] = acc;
    }
    __syncthreads();
}

// Score elements (row (t,r), column (s,j)) for the consumer tiles below: the chunk's W o G /
// W o DX scratch in global memory (row stride QR2), or the fused kernel's LDS tile.
struct ScoresGlobal {
    static constexpr bool kLds = false;
    const float* p;
    int stride;
    __device__ __forceinline__ float operator()(int m, int c) const { return p[m * stride + c]; }
};
struct ScoresLds {
    static constexpr bool kLds = true;
    float (*S)[TW + 1];
    __device__ __forceinline__ float operator()(int m, int c) const { return S[m][c]; }
};

// ---- K3: dXf rows (s,j) x columns p; writes dx_g / dx_b = dt_s dXf and the per-token
// partials q_s (state term . Xf) and sum_{p,j} dXf x. M(m, c) gives W o G; cs holds c of
// the chunk's tokens.
template <int R, bool BETA, bool PADR, class SM>
__device__ __forceinline__ void dxf_tile(const Args& a, const Chunk<R, BETA, PADR>& q, int ch,
                                         int rt, int pt, SM M, Lds<TT>& l, float (*red)[17],
                                         const float* cs, float* outv) {
    BW_CONSTS
    const Shape& s = a.s;
    const int b = q.b, k = q.k, h = q.h;
    const int m0 = rt * TT, p0 = pt * TT;
    const int tid = opaque_tid(), tx = tid & 15, ty = tid >> 4;
    const float cend = cs[QB - 1];
    const float* dH = a.dch + chx(s, b, k, h) * s.PN;
    f32x4 acc[4];
    zero(acc);
    const int pmax = s.P - 1;
    // this thread's x factors and dt, read in one batch ahead of the contraction (clamped
    // addresses; masked below)
    float xv[4][4], dv[4], rv[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int m = m0 + 4 * ty + i, t = m / R2, j = m % R2;
        dv[i] = q.ldt(t);
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) xv[i][jj] = q.lx(t, min(p0 + tcol(tx, jj), pmax), j);
    }
    gemm_acc<TT, true, true>(acc, s.N,
             [&](int mm, int n) { const int m = m0 + mm; return q.lbf(m / R2, n, m % R2); },
             [&](int mm, int n, float v) { const int m = m0 + mm; return q.okj(m / R2, m % R2) ? v : 0.f; },
             [&](int n, int pp) { return dH[min(p0 + pp, pmax) * s.N + n]; },
             [&](int n, int pp, float v) { return p0 + pp < s.P ? v : 0.f; },
             l);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int m = m0 + 4 * ty + i, t = m / R2, j = m % R2;
        const bool okr = q.okj(t, j);
        dv[i] = okr ? dv[i] : 0.f;
        const float e = __expf(cend - cs[t]), d = dv[i];
        rv[i] = 0.f;
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
            xv[i][jj] = okr && p0 + tcol(tx, jj) < s.P ? xv[i][jj] : 0.f;
            acc[jj][i] *= e;
            rv[i] += d * xv[i][jj] * acc[jj][i];
        }
    }
    const int per = R2, nts = TT / per;
    tile_token_sums(rv, per, red, outv);
    if (tid < nts) a.pState[((int64_t)ch * s.nPt + pt) * QB + m0 / per + tid] = outv[tid];
    {
        auto lb = [&](int jr, int pp) { return q.ldy(jr / R, min(p0 + pp, pmax), jr % R); };
        auto fb = [&](int jr, int pp, float v) { return p0 + pp < s.P && q.ok(jr / R, jr % R) ? v : 0.f; };
        if constexpr (SM::kLds)
            gemm_lds_a<TT, false>(acc, QR, [&](int mm, int jr) { return M(jr, m0 + mm); }, lb, fb, l);
        else
            gemm_acc<TT, false, false>(acc, QR, [&](int mm, int jr) { return M(jr, m0 + mm); },
                                       [&](int mm, int jr, float v) { return v; }, lb, fb, l);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int m = m0 + 4 * ty + i, t = m / R2, j = m % R2;
        const float d = dv[i];
        rv[i] = 0.f;
        const int jr = j < R ? j : j - R;
        const bool w = q.real(t) && q.has(jr);
        float* out = j < R ? a.dxg : a.dxb;
        const int64_t base = row(s, b, k * QB + t, h) * s.P * q.rk() + jr;
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
            const int p = p0 + tcol(tx, jj);
            rv[i] += acc[jj][i] * xv[i][jj];
            if (w && p < s.P) out[base + (int64_t)p * q.rk()] = d * acc[jj][i];
        }
    }
    tile_token_sums(rv, per, red, outv);
    if (tid < nts) a.pDt[((int64_t)ch * s.nPt + pt) * QB + m0 / per + tid] = outv[tid];
}

template <int R, bool BETA, bool PADR>
__global__ __launch_bounds__(NTH, 4) void bwd_dxf(Args a) {
    BW_CONSTS
    __shared__ Lds<TT> l;
    __shared__ float red[TT][17];
    __shared__ float cs[64], outv[64];
    const Shape& s = a.s;
    int ch, tile;
    if (!chunk_tile(s.B * s.K * s.H, QR2 / TT * s.nPt, ch, tile)) return;
    const int h = ch % s.H, k = (ch / s.H) % s.K, b = ch / (s.H * s.K);
    const Chunk<R, BETA, PADR> q{&a, b, k, h};
    if (threadIdx.x < QB) cs[threadIdx.x] = a.cum[(int64_t)ch * QB + threadIdx.x];
    __syncthreads();
    dxf_tile(a, q, ch, tile / s.nPt, tile % s.nPt, ScoresGlobal{a.M + (int64_t)ch * QR * QR2, QR2},
             l, red, cs, outv);
}

// ---- K4: dBf rows (s,j) x columns n; writes dB_g / dB_b. DM(m, c) gives W o DX.
template <int R, bool BETA, bool PADR, class SM>
__device__ __forceinline__ void dbf_tile(const Args& a, const Chunk<R, BETA, PADR>& q, int rt,
                                         int nt, SM DM, Lds<TW>& l, const float* cs,
                                         const float* dts) {
    BW_CONSTS
    const Shape& s = a.s;
    const int b = q.b, k = q.k, h = q.h;
    const int m0 = rt * TT, n0 = nt * TW;
    constexpr int NJ = TW / 16;
    const int tid = opaque_tid(), ty = tid >> 4, tx = tid & 15;
    const float cend = cs[QB - 1];
    const float* dH = a.dch + chx(s, b, k, h) * s.PN;
    f32x4 acc[NJ];
    zero(acc);
    const int nmax = s.N - 1;
    gemm_acc<TW, true, false>(acc, s.P,
             [&](int mm, int p) { const int m = m0 + mm; return q.lx(m / R2, p, m % R2); },
             [&](int mm, int p, float v) {
                 const int m = m0 + mm, t = m / R2;
                 const float d = dts[t];
                 return q.okj(t, m % R2) ? d * v : 0.f;
             },
             [&](int p, int nn) { return dH[p * s.N + min(n0 + nn, nmax)]; },
             [&](int p, int nn, float v) { return n0 + nn < s.N ? v : 0.f; },
             l);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float e = __expf(cend - cs[(m0 + 4 * ty + i) / R2]);
#pragma unroll
        for (int j = 0; j < NJ; ++j) acc[j][i] *= e;
    }
    {
        auto lb = [&](int jr, int nn) { return q.lc(jr / R, min(n0 + nn, nmax), jr % R); };
        auto fb = [&](int jr, int nn, float v) { return n0 + nn < s.N && q.ok(jr / R, jr % R) ? v : 0.f; };
        if constexpr (SM::kLds)
            gemm_lds_a<TW, false>(acc, QR, [&](int mm, int jr) { return DM(jr, m0 + mm); }, lb, fb, l);
        else
            gemm_acc<TW, false, false>(acc, QR, [&](int mm, int jr) { return DM(jr, m0 + mm); },
                                       [&](int mm, int jr, float v) { return v; }, lb, fb, l);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int m = m0 + 4 * ty + i, t = m / R2, j = m % R2;
        const int jr = j < R ? j : j - R;
        if (!q.real(t) || !q.has(jr)) continue;
        float* out = j < R ? a.dBg : a.dBb;
        const int64_t base = row(s, b, k * QB + t, h) * s.N * q.rk() + jr;
#pragma unroll
        for (int jj = 0; jj < NJ; ++jj) {
            const int n = n0 + tcol(tx, jj);
            if (n < s.N) out[base + (int64_t)n * q.rk()] = acc[jj][i];
        }
    }
}

template <int R, bool BETA, bool PADR>
__global__ __launch_bounds__(NTH, 4) void bwd_dbf(Args a) {
    BW_CONSTS
    __shared__ Lds<TW> l;
    __shared__ float cs[64], dts[64];
    const Shape& s = a.s;
    int ch, tile;
    if (!chunk_tile(s.B * s.K * s.H, QR2 / TT * s.nNt, ch, tile)) return;
    const int h = ch % s.H, k = (ch / s.H) % s.K, b = ch / (s.H * s.K);
    const Chunk<R, BETA, PADR> q{&a, b, k, h};
    if (threadIdx.x < QB) {
        cs[threadIdx.x] = a.cum[(int64_t)ch * QB + threadIdx.x];
        dts[threadIdx.x] = q.dtv(threadIdx.x);
    }
    __syncthreads();
    dbf_tile(a, q, tile / s.nNt, tile % s.nNt, ScoresGlobal{a.DM + (int64_t)ch * QR * QR2, QR2}, l,
             cs, dts);
}

// ---- K5: dC rows (t,r) x columns n, and the per-token partials sum_{n,r} C dC_inter.
// DM(m, c) gives W o DX.
template <int R, bool BETA, bool PADR, class SM>
__device__ __forceinline__ void dc_tile(const Args& a, const Chunk<R, BETA, PADR>& q, int ch,
                                        int rt, int nt, SM DM, Lds<TW>& l, float (*red)[17],
                                        const float* cs, float* outv) {
    BW_CONSTS
    const Shape& s = a.s;
    const int b = q.b, k = q.k, h = q.h;
    const int m0 = rt * TT, n0 = nt * TW;
    constexpr int NJ = TW / 16;
    const int tid = opaque_tid(), tx = tid & 15, ty = tid >> 4;
    const float* Hk = a.Hs + chx(s, b, k, h) * s.PN;
    f32x4 acc[NJ];
    zero(acc);
    const int nmax = s.N - 1;
    gemm_acc<TW, true, false>(acc, s.P,
             [&](int mm, int p) { const int m = m0 + mm; return q.ldy(m / R, p, m % R); },
             [&](int mm, int p, float v) { const int m = m0 + mm; return q.ok(m / R, m % R) ? v : 0.f; },
             [&](int p, int nn) { return Hk[p * s.N + min(n0 + nn, nmax)]; },
             [&](int p, int nn, float v) { return n0 + nn < s.N ? v : 0.f; },
             l);
    float rv[4];
    {
        // C of this thread's rows, read in one batch (clamped addresses, masked below)
        float cv[4][NJ];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int m = m0 + 4 * ty + i;
#pragma unroll
            for (int j = 0; j < NJ; ++j) cv[i][j] = q.lc(m / R, min(n0 + tcol(tx, j), nmax), m % R);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int m = m0 + 4 * ty + i, t = m / R, r = m % R;
            const bool okr = q.ok(t, r);
            const float e = __expf(cs[t]);
            rv[i] = 0.f;
#pragma unroll
            for (int j = 0; j < NJ; ++j) {
                acc[j][i] *= e;
                if (okr && n0 + tcol(tx, j) < s.N) rv[i] += cv[i][j] * acc[j][i];
            }
        }
    }
    const int per = R, nts = TT / per;
    tile_token_sums(rv, per, red, outv);
    if (tid < nts) a.pInter[((int64_t)ch * s.nNt + nt) * QB + m0 / per + tid] = outv[tid];
    {
        auto lb = [&](int jc, int nn) { return q.lbf(jc / R2, min(n0 + nn, nmax), jc % R2); };
        auto fb = [&](int jc, int nn, float v) { return n0 + nn < s.N && q.okj(jc / R2, jc % R2) ? v : 0.f; };
        if constexpr (SM::kLds) {
            if constexpr (BETA && QR == TT) {
                if (a.comb_b) {
                    // B_b of token s is B_g of token s - 1: the contraction runs over the Qb R
                    // columns (s, r) of B_g, with DM's two columns that meet each summed, and
                    // token 0's B_b enters below as a rank-R update
                    gemm_lds_a<TW, false>(acc, QR,
                             [&](int mm, int kc) {
                                 const int u = kc / R, r = kc % R;
                                 const float g = DM(m0 + mm, u * R2 + r);
                                 return u + 1 < QB ? g + DM(m0 + mm, (u + 1) * R2 + R + r) : g;
                             },
                             [&](int kc, int nn) { return q.lbf(kc / R, min(n0 + nn, nmax), kc % R); },
                             [&](int kc, int nn, float v) { return n0 + nn < s.N && q.okj(kc / R, kc % R) ? v : 0.f; },
                             l);
#pragma unroll 1
                    for (int r = 0; r < R; ++r) {
                        float bb[NJ];
#pragma unroll
                        for (int j = 0; j < NJ; ++j) {
                            const int n = n0 + tcol(tx, j);
                            const float v = q.lbf(0, min(n, nmax), R + r);
                            bb[j] = n < s.N && q.okj(0, R + r) ? v : 0.f;
                        }
#pragma unroll
                        for (int i = 0; i < 4; ++i) {
                            const float d = DM(m0 + 4 * ty + i, R + r);
#pragma unroll
                            for (int j = 0; j < NJ; ++j) acc[j][i] += d * bb[j];
                        }
                    }
                } else {
                    gemm_lds_a<TW, false>(acc, QR2, [&](int mm, int jc) { return DM(m0 + mm, jc); }, lb, fb, l);
                }
            } else {
                gemm_lds_a<TW, false>(acc, QR2, [&](int mm, int jc) { return DM(m0 + mm, jc); }, lb, fb, l);
            }
        } else {
            gemm_acc<TW, true, false>(acc, QR2, [&](int mm, int jc) { return DM(m0 + mm, jc); },
                                      [&](int mm, int jc, float v) { return v; }, lb, fb, l);
        }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int m = m0 + 4 * ty + i, t = m / R, r = m % R;
        if (!q.real(t) || !q.has(r)) continue;
        const int64_t base = row(s, b, k * QB + t, h) * s.N * q.rk() + r;
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
            const int n = n0 + tcol(tx, j);
            if (n < s.N) a.dC[base + (int64_t)n * q.rk()] = acc[j][i];
        }
    }
}

template <int R, bool BETA, bool PADR>
__global__ __launch_bounds__(NTH) void bwd_dc(Args a) {
    BW_CONSTS
    __shared__ Lds<TW> l;
    __shared__ float red[TT][17];
    __shared__ float cs[64], outv[64];
    const Shape& s = a.s;
    int ch, tile;
    if (!chunk_tile(s.B * s.K * s.H, QR / TT * s.nNt, ch, tile)) return;
    const int h = ch % s.H, k = (ch / s.H) % s.K, b = ch / (s.H * s.K);
    const Chunk<R, BETA, PADR> q{&a, b, k, h};
    if (threadIdx.x < QB) cs[threadIdx.x] = a.cum[(int64_t)ch * QB + threadIdx.x];
    __syncthreads();
    dc_tile(a, q, ch, tile / s.nNt, tile % s.nNt, ScoresGlobal{a.DM + (int64_t)ch * QR * QR2, QR2},
            l, red, cs, outv);
}

// ---- K4 with the B factor gradients combined (Args::comb_b): rows (t, r) of the chunk's
// tokens get dB_g[t] + dB_b[t + 1]. The b part of token t + 1 enters through the operands
// (DM^T rows and e dt x rows of the two factors summed), so the tile has Qb R rows instead of
// 2 Qb R. Token 0's b part goes to its own row block (dBb, (B, K, H, N, R)), formed on the
// VALU. ed[t] = exp(c_end - c_t) dt_t.
template <int R, bool BETA, bool PADR>
__device__ __forceinline__ void dbf_comb_tile(const Args& a, const Chunk<R, BETA, PADR>& q, int ch,
                                              int nt, ScoresLds DM, Lds<TW>& l, const float* ed) {
    BW_CONSTS
    static_assert(BETA && QR == TT, "rows (t, r) of one tile");
    const Shape& s = a.s;
    const int b = q.b, k = q.k, h = q.h;
    const int n0 = nt * TW;
    constexpr int NJ = TW / 16;
    const int tid = opaque_tid(), ty = tid >> 4, tx = tid & 15;
    const float* dH = a.dch + chx(s, b, k, h) * s.PN;
    f32x4 acc[NJ];
    zero(acc);
    const int nmax = s.N - 1;
    auto lbh = [&](int p, int nn) { return dH[p * s.N + min(n0 + nn, nmax)]; };
    auto fbh = [&](int p, int nn, float v) { return n0 + nn < s.N ? v : 0.f; };
    // e dt x_g of token t plus e dt x_b of token t + 1
    gemm_acc_a2<TW, false>(acc, s.P,
             [&](int m, int p) { return q.lx(m / R, p, m % R); },
             [&](int m, int p, float v) { const int t = m / R; return q.ok(t, m % R) ? ed[t] * v : 0.f; },
             [&](int m, int p) { return q.lx(m / R + 1, p, R + m % R); },
             [&](int m, int p, float v) {
                 const int t = min(m / R + 1, QB - 1);
                 return m / R + 1 < QB && q.ok(t, m % R) ? ed[t] * v : 0.f;
             },
             lbh, fbh, l);
    gemm_lds_a<TW, false>(acc, QR,
             [&](int m, int kk) {
                 const int t = m / R, r = m % R;
                 const float g = DM(kk, t * R2 + r);
                 return t + 1 < QB ? g + DM(kk, (t + 1) * R2 + R + r) : g;
             },
             [&](int jr, int nn) { return q.lc(jr / R, min(n0 + nn, nmax), jr % R); },
             [&](int jr, int nn, float v) { return n0 + nn < s.N && q.ok(jr / R, jr % R) ? v : 0.f; },
             l);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int m = 4 * ty + i, t = m / R, r = m % R;
        if (!q.real(t) || !q.has(r)) continue;
        const int64_t base = row(s, b, k * QB + t, h) * s.N * q.rk() + r;
#pragma unroll
        for (int jj = 0; jj < NJ; ++jj) {
            const int n = n0 + tcol(tx, jj);
            if (n < s.N) a.dBg[base + (int64_t)n * q.rk()] = acc[jj][i];
        }
    }
    // token 0's b part: sum_{(t,r')} DM[(t,r'),(0,R+r)] C[t,n,r'] + ed[0] sum_p x_b[0,p,r] dH[p,n]
    for (int e = tid; e < TW * R; e += NTH) {
        const int n = n0 + e / R, r = e % R;
        if (n >= s.N || !q.has(r)) continue;
        float v = 0.f;
#pragma unroll 16
        for (int kk = 0; kk < QR; ++kk) {
            const float cv = q.lc(kk / R, n, kk % R);  // clamped load, masked after it arrives
            v += DM(kk, R + r) * (q.ok(kk / R, kk % R) ? cv : 0.f);
        }
        float w = 0.f;
#pragma unroll 16
        for (int p = 0; p < s.P; ++p) w += q.lx(0, p, R + r) * dH[p * s.N + n];
        a.dBb[((int64_t)ch * s.N + n) * q.rk() + r] = v + ed[0] * w;
    }
}

// ---- K3-5 fused, for chunks whose score tiles are one 64 x 128 tile (every rank with the
// beta terms: QR = Qb R = 64, QR2 = Qb 2R = 128). One block per chunk forms W o G in an LDS
// tile, runs the dXf tiles on it, forms DX, takes the Z sums of (W o G) o DX element by
// element while it replaces the tile by W o DX, then runs the dC and dBf tiles on that. W o G
// and W o DX never reach HBM. (The chunk's operands are still read about three times over its
// ten GEMMs; with 96 blocks per XCD in flight those re-reads mostly miss the L2.)
template <int R, bool BETA, bool PADR>
__global__ __launch_bounds__(NTH, 3) void bwd_fused(Args a) {
    BW_CONSTS
    static_assert(QR == TT && QR2 == TW, "one 64 x 128 score tile per chunk");
    __shared__ Lds<TW> l;
    __shared__ float S[TT][TW + 1];
    __shared__ float red[TT][17];
    __shared__ float cs[64], dts[64], outv[64], zrow[64], zcol[64], ed[64];
    const Shape& s = a.s;
    const int ch = blockIdx.x, h = ch % s.H, k = (ch / s.H) % s.K, b = ch / (s.H * s.K);
    const Chunk<R, BETA, PADR> q{&a, b, k, h};
    const int tid = threadIdx.x, tx = tid & 15, ty = tid >> 4;
    if (tid < 64) {
        cs[tid] = tid < QB ? a.cum[(int64_t)ch * QB + tid] : 0.f;
        dts[tid] = tid < QB ? q.dtv(tid) : 0.f;
    }
    __syncthreads();
    if (tid < 64) ed[tid] = tid < QB ? __expf(cs[QB - 1] - cs[tid]) * dts[tid] : 0.f;
    constexpr int NJ = TW / 16;
    const ScoresLds Sat{S};
    f32x4 g[NJ];
    // W o G -> S: G[(t,r),(s,j)] = sum_n C[t,n,r] Bf[s,n,j]
    if (a.comb_b) {
        // B_b of token s is B_g of token s - 1, so the b columns of G are its g columns one
        // token later: a 64 x (Qb R) GEMM whose values are stored twice (each with its own
        // W), and token 0's b columns (B_b of token 0) on the VALU
        f32x4 gg[4];
        zero(gg);
        gemm_acc<TT, true, true>(gg, s.N,
                     [&](int m, int n) { return q.lc(m / R, n, m % R); },
                     [&](int m, int n, float v) { return q.ok(m / R, m % R) ? v : 0.f; },
                     [&](int n, int c) { return q.lbf(c / R, n, c % R); },
                     [&](int n, int c, float v) { return q.okj(c / R, c % R) ? v : 0.f; },
                     reinterpret_cast<Lds<TT>&>(l));
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int m = 4 * ty + i, c = tcol(tx, j), t = m / R, u = c / R, r = c % R;
                S[m][u * R2 + r] = u <= t ? __expf(cs[t] - cs[u]) * gg[j][i] : 0.f;
                if (u + 1 < QB)
                    S[m][(u + 1) * R2 + R + r] = u + 1 <= t ? __expf(cs[t] - cs[u + 1]) * gg[j][i] : 0.f;
            }
        for (int e = tid; e < TT * R; e += NTH) {
            const int m = e / R, r = e % R, t = m / R;
            float v = 0.f;
#pragma unroll 16
            for (int n = 0; n < s.N; ++n) {
                const float cv = q.lc(t, n, m % R), bv = q.lbf(0, n, R + r);
                v += cv * bv;
            }
            S[m][R + r] = q.ok(t, m % R) && q.okj(0, R + r) ? __expf(cs[t] - cs[0]) * v : 0.f;
        }
    } else {
        zero(g);
        gemm_acc<TW, true, true>(g, s.N,
                     [&](int m, int n) { return q.lc(m / R, n, m % R); },
                     [&](int m, int n, float v) { return q.ok(m / R, m % R) ? v : 0.f; },
                     [&](int n, int c) { return q.lbf(c / R2, n, c % R2); },
                     [&](int n, int c, float v) { return q.okj(c / R2, c % R2) ? v : 0.f; },
                     l);
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < NJ; ++j) {
                const int m = 4 * ty + i, c = tcol(tx, j), t = m / R, u = c / R2;
                S[m][c] = u <= t ? __expf(cs[t] - cs[u]) * g[j][i] : 0.f;
            }
    }
    __syncthreads();
#pragma unroll 1
    for (int rt = 0; rt < QR2 / TT; ++rt)
#pragma unroll 1
        for (int pt = 0; pt < s.nPt; ++pt)
            dxf_tile(a, q, ch, rt, pt, Sat, reinterpret_cast<Lds<TT>&>(l), red, cs, outv);
    // DX[(t,r),(s,j)] = sum_p dy[t,p,r] dt_s x[s,p,j]
    zero(g);
    gemm_acc<TW, true, true>(g, s.P,
                 [&](int m, int p) { return q.ldy(m / R, p, m % R); },
                 [&](int m, int p, float v) { return q.ok(m / R, m % R) ? v : 0.f; },
                 [&](int p, int c) { return q.lx(c / R2, p, c % R2); },
                 [&](int p, int c, float v) { return q.okj(c / R2, c % R2) ? dts[c / R2] * v : 0.f; },
                 l);
    {
        // Z = (W o G) o DX at this thread's elements (each thread reads and then overwrites
        // only its own elements of S), summed over its columns per row and over its rows per
        // column; the 16 partials of each row and column are then added in a fixed order.
        float zr[4], zc[NJ];
#pragma unroll
        for (int j = 0; j < NJ; ++j) zc[j] = 0.f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            zr[i] = 0.f;
#pragma unroll
            for (int j = 0; j < NJ; ++j) {
                const int m = 4 * ty + i, c = tcol(tx, j), t = m / R, u = c / R2;
                const float z = S[m][c] * g[j][i];
                zr[i] += z;
                zc[j] += z;
                S[m][c] = u <= t ? __expf(cs[t] - cs[u]) * g[j][i] : 0.f;
            }
        }
        float(*cp)[TW] = reinterpret_cast<float(*)[TW]>(&l.B[0][0]);  // 16 x 128 of l.B's 16 x 145
#pragma unroll
        for (int i = 0; i < 4; ++i) red[4 * ty + i][tx] = zr[i];
#pragma unroll
        for (int j = 0; j < NJ; ++j) cp[ty][tcol(tx, j)] = zc[j];
        __syncthreads();
        if (tid < QB) {
            float v = 0.f;
            for (int r = 0; r < R; ++r)
                for (int x = 0; x < 16; ++x) v += red[tid * R + r][x];
            zrow[tid] = v;
        } else if (tid >= 128 && tid < 128 + QB) {
            const int u = tid - 128;
            float v = 0.f;
            for (int j = 0; j < R2; ++j)
                for (int y = 0; y < 16; ++y) v += cp[y][u * R2 + j];
            zcol[u] = v;
        }
        __syncthreads();
        if (tid < QB) a.dcI[(int64_t)ch * QB + tid] = zrow[tid] - zcol[tid];
    }
#pragma unroll 1
    for (int nt = 0; nt < s.nNt; ++nt) dc_tile(a, q, ch, 0, nt, Sat, l, red, cs, outv);
    if (a.comb_b) {
#pragma unroll 1
        for (int nt = 0; nt < s.nNt; ++nt) dbf_comb_tile(a, q, ch, nt, Sat, l, ed);
    } else {
#pragma unroll 1
        for (int rt = 0; rt < QR2 / TT; ++rt)
#pragma unroll 1
            for (int nt = 0; nt < s.nNt; ++nt) dbf_tile(a, q, rt, nt, Sat, l, cs, dts);
    }
}

// ---- K6: per chunk: dc -> d(A dt) (suffix sums), ddt, the chunk's partials of dA and dD,
// and dx_raw = D dy.
template <int R, bool BETA, bool PADR>
__global__ __launch_bounds__(NTH) void bwd_tokens(Args a) {
    BW_CONSTS
    __shared__ float dcs[64], part[NTH];
    const Shape& s = a.s;
    const int ch = blockIdx.x, h = ch % s.H, k = (ch / s.H) % s.K, b = ch / (s.H * s.K);
    const Chunk<R, BETA, PADR> q{&a, b, k, h};
    const int tid = threadIdx.x;
    if (tid < 64) {
        const int t = tid;
        float dc = 0.f, qs = 0.f;
        if (t < QB) {
            dc = a.dcI[(int64_t)ch * QB + t];
            for (int nt = 0; nt < s.nNt; ++nt) dc += a.pInter[((int64_t)ch * s.nNt + nt) * QB + t];
            for (int pt = 0; pt < s.nPt; ++pt) qs += a.pState[((int64_t)ch * s.nPt + pt) * QB + t];
            dc -= qs;
        }
        const float qtot = __builtin_bit_cast(float, __builtin_amdgcn_readlane(
                                                         __builtin_bit_cast(int, wave_incl_scan(qs)), 63));
        if (t == QB - 1) dc += qtot + a.dec[chx(s, b, k, h)] * a.ddec[chx(s, b, k, h)];
        dcs[t] = dc;
    }
    __syncthreads();
    if (tid < 64) {
        const int t = tid;
        float dl = 0.f;
        for (int u = QB - 1; u >= t; --u) dl += dcs[u];
        float contrib = 0.f;
        if (t < QB && q.real(t)) {
            float pd = 0.f;
            for (int pt = 0; pt < s.nPt; ++pt) pd += a.pDt[((int64_t)ch * s.nPt + pt) * QB + t];
            a.ddt[row(s, b, k * QB + t, h)] = a.A[h] * dl + pd;
            contrib = q.dtv(t) * dl;
        }
        const float tot = __builtin_bit_cast(float, __builtin_amdgcn_readlane(
                                                        __builtin_bit_cast(int, wave_incl_scan(contrib)), 63));
        if (t == 0) a.pA[ch] = tot;
    }
    // dD partial and dx_raw over the chunk's real tokens.
    const float Dh = a.D[h];
    const int nreal = min(QB, s.T - k * QB);
    const int per_tok = s.P * q.rk();
    float v = 0.f;
    const float* __restrict__ dy = a.dy;
    const float* __restrict__ xr = a.xr;
    float* __restrict__ dxr = a.dxr;
    const bool vec = per_tok % 4 == 0 &&
                     ((reinterpret_cast<uintptr_t>(dy) | reinterpret_cast<uintptr_t>(xr) |
                       reinterpret_cast<uintptr_t>(dxr)) & 15) == 0;
    if (vec) {  // 16-byte pieces of each token's row
        const int q4 = per_tok / 4;
        for (int e = tid; e < nreal * q4; e += NTH) {
            const int t = e / q4, pr = e % q4;
            const int64_t o = row(s, b, k * QB + t, h) * per_tok + 4 * pr;
            const f32x4 g = *reinterpret_cast<const f32x4*>(dy + o);
            const f32x4 x = *reinterpret_cast<const f32x4*>(xr + o);
            v += g[0] * x[0];
            v += g[1] * x[1];
            v += g[2] * x[2];
            v += g[3] * x[3];
            *reinterpret_cast<f32x4*>(dxr + o) = g * Dh;
        }
    } else {
        for (int e = tid; e < nreal * per_tok; e += NTH) {
            const int t = e / per_tok, pr = e % per_tok;
            const int64_t o = row(s, b, k * QB + t, h) * per_tok + pr;
            const float g = dy[o];
            v += g * xr[o];
            dxr[o] = Dh * g;
        }
    }
    part[tid] = v;
    __syncthreads();
    for (int w = NTH / 2; w > 0; w >>= 1) {
        if (tid < w) part[tid] += part[tid + w];
        __syncthreads();
    }
    if (tid == 0) a.pD[ch] = part[0];
}

// ---- K7: dA[h], dD[h] = sums of the chunk partials over (b, k), in a fixed order.
__global__ __launch_bounds__(NTH) void bwd_reduce(Args a) {
    __shared__ float pa[NTH], pd[NTH];
    const Shape& s = a.s;
    const int h = blockIdx.x, tid = threadIdx.x;
    const int n = s.B * s.K;
    float va = 0.f, vd = 0.f;
    for (int i = tid; i < n; i += NTH) {
        va += a.pA[(int64_t)i * s.H + h];
        vd += a.pD[(int64_t)i * s.H + h];
    }
    pa[tid] = va;
    pd[tid] = vd;
    __syncthreads();
    for (int w = NTH / 2; w > 0; w >>= 1) {
        if (tid < w) {
            pa[tid] += pa[tid + w];
            pd[tid] += pd[tid + w];
        }
        __syncthreads();
    }
    if (tid == 0) {
        a.dA[h] = pa[0];
        a.dD[h] = pd[0];
    }
}

// ---- forward output: y rows (t,r) x columns p of the chunk,
//   y = (W o G) Xf + exp(c_t) C H_k^T + D x_raw   (M = W o G from bwd_scores in forward mode)
template <int R, bool BETA, bool PADR>
__global__ __launch_bounds__(NTH, 4) void fwd_out(Args a) {
    BW_CONSTS
    __shared__ Lds<TT> l;
    __shared__ float cs[64], dts[64];
    const Shape& s = a.s;
    int ch, tile;
    if (!chunk_tile(s.B * s.K * s.H, QR / TT * s.nPt, ch, tile)) return;
    const int h = ch % s.H, k = (ch / s.H) % s.K, b = ch / (s.H * s.K);
    const int rt = tile / s.nPt, pt = tile % s.nPt;
    const int m0 = rt * TT, p0 = pt * TT;
    const Chunk<R, BETA, PADR> q{&a, b, k, h};
    const int tid = threadIdx.x, tx = tid & 15, ty = tid >> 4;
    if (tid < QB) {
        cs[tid] = a.cum[(int64_t)ch * QB + tid];
        dts[tid] = q.dtv(tid);
    }
    __syncthreads();
    const float* Hk = a.Hs + chx(s, b, k, h) * s.PN;
    f32x4 acc[4];
    zero(acc);
    const int pmax = s.P - 1;
    // x_raw of this thread's outputs, read in one batch ahead of the contractions
    float xrv[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int m = m0 + 4 * ty + i;
#pragma unroll
        for (int j = 0; j < 4; ++j) xrv[i][j] = q.lxr(m / R, min(p0 + tcol(tx, j), pmax), m % R);
    }
    gemm_acc<TT, true, true>(acc, s.N,
                             [&](int mm, int n) { const int m = m0 + mm; return q.lc(m / R, n, m % R); },
                             [&](int mm, int n, float v) { const int m = m0 + mm; return q.ok(m / R, m % R) ? v : 0.f; },
                             [&](int n, int pp) { return Hk[min(p0 + pp, pmax) * s.N + n]; },
                             [&](int n, int pp, float v) { return p0 + pp < s.P ? v : 0.f; },
                             l);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float e = __expf(cs[(m0 + 4 * ty + i) / R]);
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[j][i] *= e;
    }
    const float* Mi = a.M + (int64_t)ch * QR * QR2;
    gemm_acc<TT, true, false>(acc, QR2,
                              [&](int mm, int jc) { return Mi[(m0 + mm) * QR2 + jc]; },
                              [&](int mm, int jc, float v) { return v; },
                              [&](int jc, int pp) { return q.lx(jc / R2, min(p0 + pp, pmax), jc % R2); },
                              [&](int jc, int pp, float v) {
                                  const int u = jc / R2;
                                  const float d = dts[u];
                                  return p0 + pp < s.P && q.okj(u, jc % R2) ? d * v : 0.f;
                              },
                              l);
    const float Dh = a.D[h];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int m = m0 + 4 * ty + i, t = m / R, r = m % R;
        if (!q.real(t) || !q.has(r)) continue;
        const int64_t base = row(s, b, k * QB + t, h) * s.P * q.rk() + r;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int p = p0 + tcol(tx, j);
            if (p < s.P) a.y[base + (int64_t)p * q.rk()] = acc[j][i] + Dh * xrv[i][j];
        }
    }
}

// h_final = the state after the last chunk (entry K of the extended scan output).
__global__ __launch_bounds__(NTH) void fwd_final(Args a) {
    const Shape& s = a.s;
    const int bh = blockIdx.x, b = bh / s.H, h = bh % s.H;
    const float* src = a.Hs + chx(s, b, s.K, h) * s.PN;
    float* dst = a.hfin + (int64_t)bh * s.PN;
    for (int64_t i = threadIdx.x; i < s.PN; i += NTH) dst[i] = src[i];
}

// Workspace carve-up (all fp32, each part 256-byte aligned).
struct Plan {
    Shape s;
    size_t off[16];
    size_t scan_off, total;
};

inline size_t al(size_t x) { return (x + 255) & ~(size_t)255; }

bool make_shape(int B, int T, int H, int P, int N, int R, bool beta, Shape& s) {
    if (R < 1 || R > 8) return false;
    const int RT = R <= 2 ? R : R <= 4 ? 4 : 8;
    s.B = B, s.T = T, s.H = H, s.P = P, s.N = N, s.R = R, s.RT = RT, s.R2 = beta ? 2 * RT : RT;
    s.Qb = 128 / s.R2 >= 64 ? 64 : 128 / s.R2;  // as BW_CONSTS
    s.K = (T + s.Qb - 1) / s.Qb;
    s.nPt = (P + TT - 1) / TT;
    s.nNt = (N + TW - 1) / TW;
    s.PN = (int64_t)P * N;
    return true;
}

// hs_given: the chunk-start states come from the forward, so the chunk-local states hext and
// the scanned states Hs take no space. The reverse scan runs in place: dch is gext. With the
// beta terms the score scratch M / DM takes no space either.
Plan make_plan(const Shape& s, bool hs_given) {
    Plan pl;
    pl.s = s;
    const size_t BKH = (size_t)s.B * s.K * s.H, BK1H = (size_t)s.B * (s.K + 1) * s.H;
    const size_t states = hs_given ? 0 : BK1H * s.PN;
    // with the beta terms one fused kernel keeps W o G / W o DX in LDS (bwd_fused)
    const size_t scores = s.R2 == 2 * s.RT ? 0 : BKH * s.QR() * s.QR2();
    const size_t sizes[15] = {
        BKH * s.Qb,                              // cum
        BK1H,                                    // dec
        BK1H,                                    // ddec
        states, states, BK1H * s.PN,             // hext, Hs, gext
        0,                                       // dch (= gext)
        scores,                                  // M
        scores,                                  // DM
        BKH * s.Qb,                              // dcI
        BKH * s.nNt * s.Qb,                      // pInter
        BKH * s.nPt * s.Qb, BKH * s.nPt * s.Qb,  // pState, pDt
        BKH, BKH};                               // pA, pD
    size_t o = 0;
    for (int i = 0; i < 15; ++i) {
        pl.off[i] = o;
        o += al(sizes[i] * sizeof(float));
    }
    pl.scan_off = o;
    o += al(scan_bwd_workspace(s.B, s.K + 1, s.H, s.PN));
    pl.total = o;
    return pl;
}

template <int R, bool BETA, bool PADR>
int launch(const Args& a, const float* h_init, float* dh_init, float* scan_ws, hipStream_t stream) {
    BW_CONSTS
    const Shape& s = a.s;
    const unsigned nch = (unsigned)((int64_t)s.B * s.K * s.H);
    constexpr int nRt = QR / TT, nRt2 = QR2 / TT;
    hipLaunchKernelGGL((bwd_cum<R, BETA, PADR>), dim3(nch), dim3(64), 0, stream, a);
    hipLaunchKernelGGL((bwd_states<R, BETA, PADR>), dim3(tile_grid(nch, s.nPt * s.nNt)), dim3(NTH), 0, stream, a);
    if (!a.have_hs &&
        launch_scan_fwd(a.dec, a.hext, h_init, a.Hs, s.B, s.K + 1, s.H, s.PN, stream) != 0)
        return 1;
    if (launch_scan_bwd(a.dec, a.Hs, a.gext, a.ddec, a.dch, dh_init, scan_ws, s.B, s.K + 1, s.H,
                        s.PN, stream) != 0)
        return 1;
    if constexpr (QR == TT && QR2 == TW) {
        hipLaunchKernelGGL((bwd_fused<R, BETA, PADR>), dim3(nch), dim3(NTH), 0, stream, a);
    } else {
        hipLaunchKernelGGL((bwd_scores<R, BETA, PADR>), dim3(nch), dim3(NTH), 0, stream, a);
        hipLaunchKernelGGL((bwd_dxf<R, BETA, PADR>), dim3(tile_grid(nch, nRt2 * s.nPt)), dim3(NTH), 0, stream, a);
        hipLaunchKernelGGL((bwd_dbf<R, BETA, PADR>), dim3(tile_grid(nch, nRt2 * s.nNt)), dim3(NTH), 0, stream, a);
        hipLaunchKernelGGL((bwd_dc<R, BETA, PADR>), dim3(tile_grid(nch, nRt * s.nNt)), dim3(NTH), 0, stream, a);
    }
    hipLaunchKernelGGL((bwd_tokens<R, BETA, PADR>), dim3(nch), dim3(NTH), 0, stream, a);
    hipLaunchKernelGGL(bwd_reduce, dim3(s.H), dim3(NTH), 0, stream, a);
    return hipGetLastError() == hipSuccess ? 0 : 1;
}

// Forward workspace: c, chunk decays, chunk-local states, scanned states, W o G.
Plan make_plan_fwd(const Shape& s) {
    Plan pl;
    pl.s = s;
    const size_t BKH = (size_t)s.B * s.K * s.H, BK1H = (size_t)s.B * (s.K + 1) * s.H;
    const size_t sizes[5] = {BKH * s.Qb, BK1H, BK1H * s.PN, BK1H * s.PN, BKH * s.QR() * s.QR2()};
    size_t o = 0;
    for (int i = 0; i < 5; ++i) {
        pl.off[i] = o;
        o += al(sizes[i] * sizeof(float));
    }
    pl.scan_off = o;
    pl.total = o;
    return pl;
}

template <int R, bool BETA, bool PADR>
int launch_fwd(const Args& a, const float* h_init, hipStream_t stream) {
    BW_CONSTS
    const Shape& s = a.s;
    const unsigned nch = (unsigned)((int64_t)s.B * s.K * s.H);
    constexpr int nRt = QR / TT;
    hipLaunchKernelGGL((bwd_cum<R, BETA, PADR>), dim3(nch), dim3(64), 0, stream, a);
    hipLaunchKernelGGL((bwd_states<R, BETA, PADR>), dim3(tile_grid(nch, s.nPt * s.nNt)), dim3(NTH), 0, stream, a);
    if (launch_scan_fwd(a.dec, a.hext, h_init, a.Hs, s.B, s.K + 1, s.H, s.PN, stream) != 0) return 1;
    hipLaunchKernelGGL((bwd_scores<R, BETA, PADR>), dim3(nch), dim3(NTH), 0, stream, a);
    hipLaunchKernelGGL((fwd_out<R, BETA, PADR>), dim3(tile_grid(nch, nRt * s.nPt)), dim3(NTH), 0, stream, a);
    if (a.hfin) hipLaunchKernelGGL(fwd_final, dim3(s.B * s.H), dim3(NTH), 0, stream, a);
    return hipGetLastError() == hipSuccess ? 0 : 1;
}

}  // namespace bw

size_t chunked_fwd_mfma_workspace(int B, int T, int H, int P, int N, int R, bool beta) {
    bw::Shape s;
    if (!chunked_bwd_shape_ok(B, T, H, P, N, R, beta) || !bw::make_shape(B, T, H, P, N, R, beta, s))
        return 0;
    return bw::make_plan_fwd(s).total;
}

int launch_chunked_fwd_mfma(int B, int T, int H, int P, int N, int R, const float* x_g,
                            const float* x_b, const float* B_g, const float* B_b, const float* C,
                            const float* dt, const float* A, const float* D, const float* x_raw,
                            const float* h_init, float* y, float* h_final, void* workspace,
                            hipStream_t stream) {
    using namespace bw;
    Shape s;
    if (!make_shape(B, T, H, P, N, R, x_b != nullptr, s)) return 1;
    const Plan pl = make_plan_fwd(s);
    char* ws = reinterpret_cast<char*>(workspace);
    auto part = [&](int i) { return reinterpret_cast<float*>(ws + pl.off[i]); };
    Args a = {};
    a.s = s;
    a.xg = x_g, a.xb = x_b, a.Bg = B_g, a.Bb = B_b, a.C = C, a.dt = dt, a.A = A, a.D = D;
    a.xr = x_raw, a.hinit = h_init;
    a.cum = part(0), a.dec = part(1), a.hext = part(2), a.Hs = part(3), a.M = part(4);
    a.fwd = 1, a.y = y, a.hfin = h_final;
    const bool pad = s.RT != s.R;
    switch (s.RT * 4 + (x_b != nullptr ? 2 : 0) + (pad ? 1 : 0)) {
        case 4: return launch_fwd<1, false, false>(a, h_init, stream);
        case 6: return launch_fwd<1, true, false>(a, h_init, stream);
        case 8: return launch_fwd<2, false, false>(a, h_init, stream);
        case 10: return launch_fwd<2, true, false>(a, h_init, stream);
        case 16: return launch_fwd<4, false, false>(a, h_init, stream);
        case 17: return launch_fwd<4, false, true>(a, h_init, stream);
        case 18: return launch_fwd<4, true, false>(a, h_init, stream);
        case 19: return launch_fwd<4, true, true>(a, h_init, stream);
        case 32: return launch_fwd<8, false, false>(a, h_init, stream);
        case 33: return launch_fwd<8, false, true>(a, h_init, stream);
        case 34: return launch_fwd<8, true, false>(a, h_init, stream);
        case 35: return launch_fwd<8, true, true>(a, h_init, stream);
        default: return 1;
    }
}

size_t chunked_fwd_hs_offset(int B, int T, int H, int P, int N, int R, bool beta) {
    bw::Shape s;
    if (!bw::make_shape(B, T, H, P, N, R, beta, s)) return 0;
    return bw::make_plan_fwd(s).off[3];
}

int chunked_chunk_tokens(int R, bool beta) {
    bw::Shape s;
    return bw::make_shape(1, 1, 1, 1, 2, R, beta, s) ? s.Qb : 0;
}

bool chunked_bwd_shape_ok(int B, int T, int H, int P, int N, int R, bool beta) {
    bw::Shape s;
    if (!bw::make_shape(B, T, H, P, N, R, beta, s)) return false;
    return true;
}

size_t chunked_bwd_workspace(int B, int T, int H, int P, int N, int R, bool beta, bool hs_given) {
    bw::Shape s;
    if (!bw::make_shape(B, T, H, P, N, R, beta, s)) return 0;
    return bw::make_plan(s, hs_given).total;
}

int launch_chunked_bwd(int B, int T, int H, int P, int N, int R, const float* x_g,
                       const float* x_b, const float* B_g, const float* B_b, const float* C,
                       const float* dt, const float* A, const float* D, const float* x_raw,
                       const float* h_init, const float* dy, const float* dh_final, float* dx_g,
                       float* dx_b, float* dB_g, float* dB_b, float* dC, float* ddt, float* dA,
                       float* dD, float* dx_raw, float* dh_init, void* workspace,
                       hipStream_t stream, const float* hs_pre, bool comb_b) {
    using namespace bw;
    Shape s;
    if (!make_shape(B, T, H, P, N, R, x_b != nullptr, s)) return 1;
    if (comb_b && x_b == nullptr) return 1;
    const Plan pl = make_plan(s, hs_pre != nullptr);
    char* ws = reinterpret_cast<char*>(workspace);
    auto part = [&](int i) { return reinterpret_cast<float*>(ws + pl.off[i]); };
    Args a;
    a.s = s;
    a.xg = x_g, a.xb = x_b, a.Bg = B_g, a.Bb = B_b, a.C = C, a.dt = dt, a.A = A, a.D = D;
    a.xr = x_raw, a.hinit = h_init, a.dy = dy, a.dhf = dh_final;
    a.dxg = dx_g, a.dxb = dx_b, a.dBg = dB_g, a.dBb = dB_b, a.dC = dC, a.ddt = ddt, a.dA = dA;
    a.dD = dD, a.dxr = dx_raw, a.dhinit = dh_init;
    a.cum = part(0), a.dec = part(1), a.ddec = part(2), a.hext = part(3), a.Hs = part(4);
    a.gext = part(5), a.dch = a.gext, a.M = part(7), a.DM = part(8), a.dcI = part(9);
    a.pInter = part(10), a.pState = part(11), a.pDt = part(12), a.pA = part(13), a.pD = part(14);
    float* scan_ws = reinterpret_cast<float*>(ws + pl.scan_off);
    a.fwd = 0, a.y = nullptr, a.hfin = nullptr;
    a.have_hs = hs_pre != nullptr;
    if (hs_pre) a.Hs = const_cast<float*>(hs_pre);  // read only
    a.comb_b = comb_b ? 1 : 0;

    const bool beta = x_b != nullptr, pad = s.RT != s.R;
    switch (s.RT * 4 + (beta ? 2 : 0) + (pad ? 1 : 0)) {
        case 4: return launch<1, false, false>(a, h_init, dh_init, scan_ws, stream);
        case 6: return launch<1, true, false>(a, h_init, dh_init, scan_ws, stream);
        case 8: return launch<2, false, false>(a, h_init, dh_init, scan_ws, stream);
        case 10: return launch<2, true, false>(a, h_init, dh_init, scan_ws, stream);
        case 16: return launch<4, false, false>(a, h_init, dh_init, scan_ws, stream);
        case 17: return launch<4, false, true>(a, h_init, dh_init, scan_ws, stream);
        case 18: return launch<4, true, false>(a, h_init, dh_init, scan_ws, stream);
        case 19: return launch<4, true, true>(a, h_init, dh_init, scan_ws, stream);
        case 32: return launch<8, false, false>(a, h_init, dh_init, scan_ws, stream);
        case 33: return launch<8, false, true>(a, h_init, dh_init, scan_ws, stream);
        case 34: return launch<8, true, false>(a, h_init, dh_init, scan_ws, stream);
        case 35: return launch<8, true, true>(a, h_init, dh_init, scan_ws, stream);
        default: return 1;
    }
}

}  // namespace m3
