// Small-batch projections of the decode step (gfx950): at most 8 rows of bf16 activations
// times a bf16 weight of N rows x K (nn.Linear's layout), bound by the weight read. For
// decode batches they replace the block step's projections and the element-wise work
// around them (mamba3/block.py:94-100, 182-183; mamba3/mamba3.py:19-35, 275-316;
// mamba3/block.py:16-26), one kernel each:
//   small_linear:  out = [res +] s * (n W^T)            (in_proj, out_proj, w_down, lm_head)
//   small_swiglu:  out = silu(n Wg^T) * (n Wu^T)         (w_gate, w_up)
// where n = RMSNorm(x; w_n) when a norm weight is given (else n = x) and res / s apply
// only when a residual is given (s = 1 without one). RMSNorm follows the reference's
// arithmetic: fp32 mean of squares, the scale and x * scale rounded to bf16, times the bf16
// weight, rounded to bf16.
//
// LPR consecutive lanes (8, 16, 32 or 64, chosen from K so that each lane holds at most 8
// pieces) share an output row and split K into 16-byte pieces (lane s reads
// k = 8 s + 8 LPR j), so the lanes of a row read contiguous bytes, and every lane issues all
// its pieces before it uses them, ahead of the activations' staging: one memory round trip
// per kernel, spread over N * LPR / 256 blocks of 256 threads. The (normalised) activations
// are staged once per block in LDS as bf16 (with the norm weight), so larger blocks stage
// them fewer times (256 threads: +8% LM decode against 128; 512 is slower), padded to MM rows
// with zeros and followed by one zero piece that
// stands in for the steps past K in the last group of 8 (whose weight reads are clamped to
// the last piece of the row). Every row group reads the same LDS addresses (broadcast). Dot
// products accumulate in fp32 (v_dot2_f32_bf16); DPP steps (and lane shuffles beyond 16
// lanes) sum the lanes of a row, and lane m of the row writes output m.
#include "m3_common.h"
#include "m3_kernels.h"
#include "m3_mfma.h"

namespace m3 {

constexpr int kGvThreads = 256;
constexpr int kGvU = 8;  // weight pieces in flight per lane
constexpr int kGvStage = 4;  // activation pieces staged per thread and pass

typedef unsigned gv_u32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 gv_bf16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 gv_bf16x8 __attribute__((ext_vector_type(8)));

struct GemvArgs {
    const bf16* x;    // [M][K], rows contiguous
    const bf16* nw;   // [K] RMSNorm weight, or nullptr
    float eps;
    const bf16* w0;   // [N][K]
    const bf16* w1;   // [N][K] SwiGLU's up weight (small_swiglu only)
    const bf16* res;  // [M][N] or nullptr
    float scale;
    bf16* out;        // [M][N]
    int M, N, K;
};

// Sum over aligned groups of LPR lanes: lane ^ 1 and lane ^ 2 within the quad, the mirror
// lane 7 - i within the half-row (the other quad), the mirror lane 15 - i within the row
// (the other half-row), then lane ^ 16 and lane ^ 32 across rows.
template <int LPR>
__device__ __forceinline__ float sum_lanes(float v) {
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, false));
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, false));
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x141, 0xF, 0xF, false));
    if constexpr (LPR >= 16)
        v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x140, 0xF, 0xF, false));
    if constexpr (LPR >= 32) v += __shfl_xor(v, 16, kWave);
    if constexpr (LPR >= 64) v += __shfl_xor(v, 32, kWave);
    return v;
}

// The pairs are taken with __builtin_shufflevector: bit-casting the 32-bit components of a
// uint4 to bf16x2 made this compiler pass the first component to all four instructions.
__device__ __forceinline__ float dot8(gv_bf16x8 a, gv_bf16x8 b, float c) {
    c = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(a, a, 0, 1), __builtin_shufflevector(b, b, 0, 1), c, false);
    c = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(a, a, 2, 3), __builtin_shufflevector(b, b, 2, 3), c, false);
    c = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(a, a, 4, 5), __builtin_shufflevector(b, b, 4, 5), c, false);
    c = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(a, a, 6, 7), __builtin_shufflevector(b, b, 6, 7), c, false);
    return c;
}

template <int MM, bool kNorm, bool kSwiglu, int LPR>
__global__ __launch_bounds__(kGvThreads) void gemv_small(GemvArgs a) {
    constexpr int kRows = kGvThreads / LPR;  // output rows per block
    extern __shared__ __align__(16) unsigned char gv_smem[];
    bf16* sx = reinterpret_cast<bf16*>(gv_smem);  // [MM][K], one zero piece, [K] norm weight
    __shared__ float sss[kGvThreads / 64][MM];    // per-wave sums of squares
    const int tid = threadIdx.x;
    const int K = a.K, M = a.M;
    const int kv = K / 8;  // 16-byte pieces per row

    const int ls = tid % LPR;  // lane within the row
    const int n = blockIdx.x * kRows + tid / LPR;
    const int nr = n < a.N ? n : a.N - 1;  // rows past N read the last row and store nothing
    const bf16* wr0 = a.w0 + (int64_t)nr * K + ls * 8;
    const bf16* wr1 = kSwiglu ? a.w1 + (int64_t)nr * K + ls * 8 : nullptr;
    // pieces of this lane: k = 8 ls + 8 LPR j for j < nj (the row's K / 8 pieces are split
    // evenly when LPR divides them; otherwise the last lanes' final piece is past K)
    const int nj = (kv + LPR - 1) / LPR;

    gv_bf16x8 wq0[kGvU], wq1[kGvU];
    auto load_group = [&](int j0) {
#pragma unroll
        for (int u = 0; u < kGvU; ++u) {
            // clamped to this lane's last piece inside the row
            int j = j0 + u < nj ? j0 + u : nj - 1;
            j = ls + LPR * j < kv ? j : (kv - 1 - ls) / LPR;
            wq0[u] = *reinterpret_cast<const gv_bf16x8*>(wr0 + j * 8 * LPR);
            if constexpr (kSwiglu) wq1[u] = *reinterpret_cast<const gv_bf16x8*>(wr1 + j * 8 * LPR);
        }
        __builtin_amdgcn_sched_barrier(0);  // every piece in flight before the first use
    };
    // The first group of weight pieces goes out before anything else, so its round trip
    // overlaps the staging (and normalisation) of the activations.
    load_group(0);

    // Stage the activations (rows past M and the trailing piece are zero) and the norm weight.
    // Buffer reads past the M rows (and past the weight) return zero, so every read of a
    // pass is issued unconditionally, before the pass's stores: one round trip per pass.
    // With the norm, each thread also sums the squares of its pieces per row (fp32) while
    // they are in registers.
    const __amdgpu_buffer_rsrc_t rx = make_rsrc(a.x, (int64_t)M * K * 2);
    const int nstage = MM * kv + 1;
    // the norm weight's first pass is read ahead of the activations
    const __amdgpu_buffer_rsrc_t rw = make_rsrc(a.nw, kNorm ? (int64_t)K * 2 : 0);
    gv_u32x4 wv0[kGvStage];
    if constexpr (kNorm) {
#pragma unroll
        for (int u = 0; u < kGvStage; ++u)
            wv0[u] = __builtin_amdgcn_raw_buffer_load_b128(rw, (u * kGvThreads + tid) * 16, 0, 0);
    }
    float ss[MM];
#pragma unroll
    for (int m = 0; m < MM; ++m) ss[m] = 0.f;
    for (int i0 = 0; i0 < nstage; i0 += kGvThreads * kGvStage) {
        gv_u32x4 v[kGvStage];
#pragma unroll
        for (int u = 0; u < kGvStage; ++u)
            v[u] = __builtin_amdgcn_raw_buffer_load_b128(rx, (i0 + u * kGvThreads + tid) * 16, 0, 0);
#pragma unroll
        for (int u = 0; u < kGvStage; ++u) {
            const int i = i0 + u * kGvThreads + tid;
            if (i < nstage) *reinterpret_cast<gv_u32x4*>(sx + (int64_t)i * 8) = v[u];
            if constexpr (kNorm) {
                // pieces past the M rows read zero and add nothing
                const gv_bf16x8 xv = __builtin_bit_cast(gv_bf16x8, v[u]);
                float q = 0.f;
#pragma unroll
                for (int e = 0; e < 8; ++e) q += (float)xv[e] * (float)xv[e];
                const int m = i / kv;
#pragma unroll
                for (int mm = 0; mm < MM; ++mm) ss[mm] += m == mm ? q : 0.f;
            }
        }
    }
    bf16* snw = sx + (MM * kv + 1) * 8;
    if constexpr (kNorm) {
        for (int i0 = 0; i0 < kv; i0 += kGvThreads * kGvStage) {
            gv_u32x4 v[kGvStage];
#pragma unroll
            for (int u = 0; u < kGvStage; ++u)
                v[u] = i0 == 0 ? wv0[u] : __builtin_amdgcn_raw_buffer_load_b128(rw, (i0 + u * kGvThreads + tid) * 16, 0, 0);
#pragma unroll
            for (int u = 0; u < kGvStage; ++u) {
                const int i = i0 + u * kGvThreads + tid;
                if (i < kv) *reinterpret_cast<gv_u32x4*>(snw + i * 8) = v[u];
            }
        }
    } else {
        __syncthreads();
    }
    if constexpr (kNorm) {
        // fp32 sum of squares per row: the threads' partials, a wave sum, the waves' partials
        // in order; then x * s and the weight, rounded as the reference's RMSNorm
#pragma unroll
        for (int m = 0; m < MM; ++m) {
            const float t = sum_lanes<64>(ss[m]);
            if ((tid & 63) == 0) sss[tid >> 6][m] = t;
        }
        __syncthreads();
        for (int i = tid; i < MM * kv; i += kGvThreads) {
            const int m = i / kv, c = i - m * kv;
            float sq = 0.f;
#pragma unroll
            for (int w = 0; w < kGvThreads / 64; ++w) sq += sss[w][m];
            const float sc = (float)(bf16)rsqrtf(sq / (float)K + a.eps);
            gv_bf16x8 xv = *reinterpret_cast<const gv_bf16x8*>(sx + (int64_t)i * 8);
            const gv_bf16x8 wv = *reinterpret_cast<const gv_bf16x8*>(snw + c * 8);
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float xs = (float)(bf16)((float)xv[e] * sc);
                xv[e] = (bf16)(xs * (float)wv[e]);
            }
            *reinterpret_cast<gv_bf16x8*>(sx + (int64_t)i * 8) = xv;
        }
        __syncthreads();
    }

    float acc0[MM], acc1[MM];
#pragma unroll
    for (int m = 0; m < MM; ++m) acc0[m] = acc1[m] = 0.f;
    for (int j0 = 0; j0 < nj; j0 += kGvU) {
        if (j0 > 0) load_group(j0);
#pragma unroll
        for (int u = 0; u < kGvU; ++u) {
            const bool live = j0 + u < nj && ls + LPR * (j0 + u) < kv;
#pragma unroll
            for (int m = 0; m < MM; ++m) {
                const int xo = live ? m * K + ls * 8 + (j0 + u) * 8 * LPR : MM * K;
                const gv_bf16x8 xv = *reinterpret_cast<const gv_bf16x8*>(sx + xo);
                acc0[m] = dot8(xv, wq0[u], acc0[m]);
                if constexpr (kSwiglu) acc1[m] = dot8(xv, wq1[u], acc1[m]);
            }
        }
    }

    float v = 0.f;
#pragma unroll
    for (int m = 0; m < MM; ++m) {
        const float s0 = sum_lanes<LPR>(acc0[m]);
        float r = s0;
        if constexpr (kSwiglu) r = silu_f(s0) * sum_lanes<LPR>(acc1[m]);
        v = ls == m ? r : v;
    }
    if (n < a.N && ls < M) {
        const int64_t o = (int64_t)ls * a.N + n;
        if (a.res) v = (float)a.res[o] + a.scale * v;
        a.out[o] = (bf16)v;
    }
}

int gemv_small_lds_bytes(int m, int k, bool norm) {
    const int mm = m <= 1 ? 1 : m <= 2 ? 2 : m <= 4 ? 4 : 8;
    return (mm * k + 8 + (norm ? k : 0)) * 2;
}

template <int MM, int LPR>
static void launch_gemv_ml(const GemvArgs& a, bool norm, bool swiglu, hipStream_t stream) {
    constexpr int rows = kGvThreads / LPR;
    const dim3 grid((unsigned)((a.N + rows - 1) / rows));
    const size_t lds = (size_t)gemv_small_lds_bytes(MM, a.K, norm);
    if (norm && swiglu) hipLaunchKernelGGL((gemv_small<MM, true, true, LPR>), grid, dim3(kGvThreads), lds, stream, a);
    else if (norm) hipLaunchKernelGGL((gemv_small<MM, true, false, LPR>), grid, dim3(kGvThreads), lds, stream, a);
    else if (swiglu) hipLaunchKernelGGL((gemv_small<MM, false, true, LPR>), grid, dim3(kGvThreads), lds, stream, a);
    else hipLaunchKernelGGL((gemv_small<MM, false, false, LPR>), grid, dim3(kGvThreads), lds, stream, a);
}

// Lanes per row: the fewest (at least 8) that leave each lane at most 8 pieces of 8 values.
template <int MM>
static void launch_gemv_m(const GemvArgs& a, bool norm, bool swiglu, hipStream_t stream) {
    const int pieces = a.K / 8;
    if (pieces <= 64) launch_gemv_ml<MM, 8>(a, norm, swiglu, stream);
    else if (pieces <= 128) launch_gemv_ml<MM, 16>(a, norm, swiglu, stream);
    else if (pieces <= 256) launch_gemv_ml<MM, 32>(a, norm, swiglu, stream);
    else launch_gemv_ml<MM, 64>(a, norm, swiglu, stream);
}

int launch_gemv_small(const void* x, const void* norm_w, float eps, const void* w0, const void* w1,
                      const void* res, float scale, void* out, int m, int n, int k,
                      hipStream_t stream) {
    GemvArgs a;
    a.x = reinterpret_cast<const bf16*>(x);
    a.nw = reinterpret_cast<const bf16*>(norm_w);
    a.eps = eps;
    a.w0 = reinterpret_cast<const bf16*>(w0);
    a.w1 = reinterpret_cast<const bf16*>(w1);
    a.res = reinterpret_cast<const bf16*>(res);
    a.scale = res ? scale : 1.f;
    a.out = reinterpret_cast<bf16*>(out);
    a.M = m, a.N = n, a.K = k;
    const bool norm = norm_w != nullptr, swiglu = w1 != nullptr;
    if (m <= 1) launch_gemv_m<1>(a, norm, swiglu, stream);
    else if (m <= 2) launch_gemv_m<2>(a, norm, swiglu, stream);
    else if (m <= 4) launch_gemv_m<4>(a, norm, swiglu, stream);
    else launch_gemv_m<8>(a, norm, swiglu, stream);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

}  // namespace m3
