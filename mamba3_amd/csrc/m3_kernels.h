// Host-side launchers of the Mamba-3 kernels. Arguments are validated by the C-ABI
// layer (m3_api.cpp) before any of these is called.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "../../include/mamba3_amd.h"

namespace m3 {

// Column offsets of one in_proj row: [z | x | B | C | dt | lambda | theta].
struct ProjLayout {
    int64_t z, x, B, C, dt, lam, theta, width;
};

inline ProjLayout proj_layout(const m3_layer_desc& d) {
    ProjLayout L;
    const int64_t d_inner = (int64_t)d.nheads * d.headdim;
    const int64_t d_bc = (int64_t)d.ngroups * d.d_state * d.mimo_rank;
    L.z = 0;
    L.x = d_inner;
    L.B = 2 * d_inner;
    L.C = L.B + d_bc;
    L.dt = L.C + d_bc;
    int64_t o = L.dt + d.nheads;
    L.lam = d.use_trapezoidal ? o : -1;
    if (d.use_trapezoidal) o += d.nheads;
    L.theta = d.use_complex ? o : -1;
    if (d.use_complex) o += d.d_state / 2;
    L.width = o;
    return L;
}

int launch_scan_fwd(const float* decay, const float* h_chunk, const float* h_init,
                    float* h_states, int64_t B, int64_t K, int64_t H, int64_t PN,
                    hipStream_t stream);

// Backward of the scan: workspace bytes (0 when PN % 256 != 0) and launcher. grad and
// d_chunk may be the same array (in place).
size_t scan_bwd_workspace(int64_t B, int64_t K, int64_t H, int64_t PN);
int launch_scan_bwd(const float* decay, const float* h_states, const float* grad,
                    float* d_decay, float* d_chunk, float* d_h_init, float* workspace,
                    int64_t B, int64_t K, int64_t H, int64_t PN, hipStream_t stream);

// Generic (fp32 VALU) fused layer prefill: any supported shape, any dtype.
size_t generic_prefill_workspace(const m3_layer_desc& d);
int launch_generic_prefill(const m3_layer_desc& d, const m3_layer_params& p, const void* proj,
                           const float* dt_scale, void* y_out, float* h_final, float* angle,
                           float* prev_bx, void* workspace, hipStream_t stream);

int launch_generic_chunked(int B, int T, int H, int P, int N, int R, int dtype,
                           const void* x_g, const void* x_b, const void* B_g, const void* B_b,
                           const void* C, const void* dt, const float* A, const float* D,
                           const void* x_raw, const float* h_init, void* y, float* h_final,
                           float* state_ws, hipStream_t stream);

// bf16 MFMA fused prefill for d_state 128, headdim 64, mimo_rank 2.
bool mfma_prefill_supported(const m3_layer_desc& d, const void* proj, const void* y_out);
// Normalised B^ / C^ rows (RMSNorm * weight + bias) per (token, group), pair-packed f16
// (N*R values per row; word R*i + r holds the pair (2i, 2i+1) of rank r).
void launch_bc_norm(const m3_layer_desc& d, const m3_layer_params& p, const void* proj,
                    _Float16* bn, _Float16* cn, hipStream_t stream);
size_t mfma_prefill_workspace(const m3_layer_desc& d);
int launch_mfma_prefill(const m3_layer_desc& d, const m3_layer_params& p, const void* proj,
                        const float* dt_scale, void* y_out, float* h_final, float* angle,
                        float* prev_bx, void* workspace, hipStream_t stream);

// bf16 MFMA fused prefill for d_state 64/128/256, mimo_rank 1/2/4, headdim % 32 == 0.
bool wide_prefill_supported(const m3_layer_desc& d);
size_t wide_prefill_workspace(const m3_layer_desc& d);
int launch_wide_prefill(const m3_layer_desc& d, const m3_layer_params& p, const void* proj,
                        const float* dt_scale, void* y_out, float* h_final, float* angle,
                        float* prev_bx, void* workspace, hipStream_t stream);

// Backward of the chunked SSD (fp32): shape support, workspace bytes and launcher.
bool chunked_bwd_shape_ok(int B, int T, int H, int P, int N, int R, bool beta);
// fp32 chunked SSD forward on the same chunk kernels (fp32 MFMA); 0 bytes = not supported.
size_t chunked_fwd_mfma_workspace(int B, int T, int H, int P, int N, int R, bool beta);
int launch_chunked_fwd_mfma(int B, int T, int H, int P, int N, int R, const float* x_g,
                            const float* x_b, const float* B_g, const float* B_b, const float* C,
                            const float* dt, const float* A, const float* D, const float* x_raw,
                            const float* h_init, float* y, float* h_final, void* workspace,
                            hipStream_t stream);
// Workspace of launch_chunked_bwd; hs_given: the call passes hs_pre (less space).
size_t chunked_bwd_workspace(int B, int T, int H, int P, int N, int R, bool beta,
                             bool hs_given = false);
// Byte offset, in the fp32-MFMA chunk forward's workspace, of its chunk-start states
// (B, K+1, H, P, N): the hs_pre a backward of the same shape may take.
size_t chunked_fwd_hs_offset(int B, int T, int H, int P, int N, int R, bool beta);
// Tokens per chunk of the fp32-MFMA chunk kernels (0 for shapes they do not take).
int chunked_chunk_tokens(int R, bool beta);
int launch_chunked_bwd(int B, int T, int H, int P, int N, int R, const float* x_g,
                       const float* x_b, const float* B_g, const float* B_b, const float* C,
                       const float* dt, const float* A, const float* D, const float* x_raw,
                       const float* h_init, const float* dy, const float* dh_final, float* dx_g,
                       float* dx_b, float* dB_g, float* dB_b, float* dC, float* ddt, float* dA,
                       float* dD, float* dx_raw, float* dh_init, void* workspace,
                       hipStream_t stream, const float* hs_pre = nullptr, bool comb_b = false);
// comb_b (needs the beta terms): dB_g receives dB_g[t] + dB_b[t + 1] and dB_b only the b part
// of each chunk's first token, as (B, K, H, N, R) rows with K chunks of
// chunked_chunk_tokens(R, true) tokens (they belong to the previous chunk's last token).

// fp32 layer prefill on the fp32-MFMA chunk kernels (preparation, chunked SSD, gate).
// Its workspace holds chunked_ssd's inputs and the SSD output, which the layer backward reads.
// The training forward's per-token operands of the layer backward, and Hs: the chunk-start
// states (B, K+1, H, P, N) in the fp32 chunk kernels' chunking (entry 0 the zero start,
// entry K the final state), which the backward reads instead of recomputing them.
struct Fp32LayerParts {
    float *dt, *A, *phi, *xg, *xb, *xr, *Bt, *Bb, *Ct, *ys, *Hs;
};
Fp32LayerParts fp32_layer_parts(const m3_layer_desc& d, void* workspace);
// Whether the training forward leaves valid chunk-start states in Fp32LayerParts::Hs (then the
// fused fp32 forward keeps its B^ rows at the chunk-kernel region's start and its C^ rows
// lp::al(fp32_layer_hs_bytes) past Hs), and their size.
bool fp32_layer_hs_ok(const m3_layer_desc& d);
size_t fp32_layer_hs_bytes(const m3_layer_desc& d);
bool fp32_layer_supported(const m3_layer_desc& d);
// Fused fp32 prefill (m3_ssd_f32.hip): d_state 128, headdim 64, rank 2, without
// M3_FLAG_FOR_BACKWARD; 16-byte aligned rows of proj and y_out, h_final and prev_bx.
bool fused_fp32_prefill_supported(const m3_layer_desc& d, const void* proj, const void* y_out,
                                  const void* h_final, const void* prev_bx);
// The same kernel for the training forward (M3_FLAG_FOR_BACKWARD): it also writes the staged
// per-token operands the layer backward reads (fp32_layer_parts of the fp32 layer workspace)
// and keeps its B^ / C^ rows in that workspace's chunk-kernel region.
bool fused_fp32_train_supported(const m3_layer_desc& d, const void* proj, const void* y_out,
                                const void* h_final, const void* prev_bx);
// The chunk-kernel region of the fp32 layer workspace (pointer into ws, and its size).
void* fp32_layer_scratch(const m3_layer_desc& d, void* ws, size_t* bytes);
size_t fused_fp32_prefill_workspace(const m3_layer_desc& d);
int launch_fused_fp32_prefill(const m3_layer_desc& d, const m3_layer_params& p, const void* proj,
                              const float* dt_scale, void* y_out, float* h_final, float* angle,
                              float* prev_bx, void* workspace, hipStream_t stream,
                              const Fp32LayerParts* stage = nullptr);
size_t fp32_layer_workspace(const m3_layer_desc& d);
int launch_fp32_layer(const m3_layer_desc& d, const m3_layer_params& p, const void* proj,
                      const float* dt_scale, void* y_out, float* h_final, float* angle,
                      float* prev_bx, void* workspace, hipStream_t stream);

// Backward of the fp32 layer prefill (gate, chunked SSD, preparation) from the forward's
// workspace: workspace bytes and launcher.
size_t layer_bwd_workspace(const m3_layer_desc& d);
int launch_layer_bwd(const m3_layer_desc& d, const m3_layer_params& p, const void* proj,
                     const float* dt_scale, void* fwd_workspace, const float* g_out,
                     const float* g_h, const float* g_angle, const float* g_prev, float* g_proj,
                     const m3_layer_param_grads& g, void* workspace, hipStream_t stream);

// Backward of the decode step (m3_step_bwd.hip): supported shapes, workspace bytes and
// launcher (fp32 proj, states and gradients).
bool step_bwd_supported(const m3_layer_desc& d);
size_t step_bwd_workspace(const m3_layer_desc& d);
int launch_step_bwd(const m3_layer_desc& d, const m3_layer_params& p, const float* proj,
                    const float* dt_scale, const float* h, const float* prev, const float* ang,
                    const float* gy, const float* gH, const float* gP, const float* gA,
                    float* g_proj, float* g_h, float* g_prev, float* g_ang,
                    const m3_layer_param_grads& out, void* workspace, hipStream_t stream);

// Block RMSNorm (m3_norm.hip): forward, and backward workspace bytes and launcher.
int launch_rmsnorm_fwd(const void* x, int xdtype, const void* w, int wdtype, void* y,
                       int ydtype, float* rstd, int64_t rows, int d, float eps,
                       hipStream_t stream);
size_t rmsnorm_bwd_workspace(int64_t rows, int d);

// out (rows x d_ff) = silu(gu[:, :d_ff]) * gu[:, d_ff:2 d_ff], bf16 (m3_norm.hip).
int launch_silu_mul(const void* gu, void* out, int64_t rows, int dff, int64_t stride,
                    hipStream_t stream);

// Small-batch decode projections (m3_gemv.hip): out = [res +] s (n W0^T), or with W1
// silu(n W0^T) * (n W1^T); n = RMSNorm(x; norm_w) when norm_w is given. bf16, m <= 8,
// k % 64 == 0, gemv_small_lds_bytes(m, k, norm) <= 65536.
int gemv_small_lds_bytes(int m, int k, bool norm);
int launch_gemv_small(const void* x, const void* norm_w, float eps, const void* w0, const void* w1,
                      const void* res, float scale, void* out, int m, int n, int k,
                      hipStream_t stream);
int launch_rmsnorm_bwd(const void* x, int xdtype, const void* w, int wdtype, const float* rstd,
                       const void* g, int gdtype, void* dx, void* dw, void* workspace,
                       int64_t rows, int d, hipStream_t stream);

// Returns 1 when the step kernel supports (N, R), else 0.
int step_supported(int N, int R);
int launch_step(const m3_layer_desc& d, const m3_layer_params& p, const void* proj,
                const float* dt_scale, const float* h_in, const float* prev_in,
                const void* angle_in, int angle_dtype, void* y_out, float* h_out,
                float* prev_out, void* angle_out, hipStream_t stream);

}  // namespace m3
