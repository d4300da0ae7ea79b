/*
 * mamba3_amd.h — C-ABI of the MI355X (gfx950) Mamba-3 chunked-SSD forward path.
 *
 * Every entry point takes plain device pointers, sizes and a HIP stream passed as
 * `void*` (a hipStream_t; NULL means the null stream). Nothing here allocates or
 * synchronises the host: outputs and workspaces are owned by the caller, and every call
 * is reentrant on distinct buffers. The one exception to "no global state" is
 * m3_prefill_fwd_noalloc, whose workspace is a static per-device array of the library. Each call
 * returns M3_OK (0) or an m3_status code; m3_status_string() names it. Arguments
 * are validated on the host before any launch, so a rejected call launches nothing.
 *
 * Layouts are row-major and contiguous. Shape letters: B batch, T sequence length,
 * H heads, P headdim, N d_state, R mimo_rank, G ngroups, K number of chunks,
 * d_in_proj = 2*H*P + 2*G*N*R + H (+H if trapezoidal) (+N/2 if complex).
 * The in_proj row is split as [z | x | B | C | dt | lambda | theta]; inside B and C
 * the flat index is g*N*R + n*R + r (rank fastest); inside z and x it is h*P + p.
 */
#ifndef MAMBA3_AMD_H
#define MAMBA3_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Element types of activations (the in_proj output, the gated output). */
enum m3_dtype {
    M3_DTYPE_F32 = 0,
    M3_DTYPE_BF16 = 1
};

enum m3_status {
    M3_OK = 0,
    M3_ERR_NULL_POINTER = 1,      /* a required pointer is NULL */
    M3_ERR_INVALID_SHAPE = 2,     /* a size is non-positive or inconsistent */
    M3_ERR_UNSUPPORTED = 3,       /* shape/dtype outside what the kernels handle */
    M3_ERR_WORKSPACE = 4,         /* workspace missing or smaller than required */
    M3_ERR_MISALIGNED = 5,        /* a pointer violates the documented alignment */
    M3_ERR_LAUNCH = 6,            /* the HIP runtime rejected a kernel launch */
    M3_ERR_DEVICE = 7,            /* device query failed (no device / wrong arch) */
    M3_ERR_SCRATCH_LIMIT = 8      /* m3_prefill_fwd_noalloc: workspace need exceeds its scratch */
};

/* Size of the static per-device scratch of m3_prefill_fwd_noalloc (64 MiB). */
#define M3_NOALLOC_SCRATCH_BYTES ((size_t)64 << 20)

/* Static description of one KulaMamba layer and of the activation tensor it reads.
 * Mirrors the constructor of KulaMamba (mamba3/mamba3.py:50-112). */
typedef struct m3_layer_desc {
    int32_t batch;            /* B */
    int32_t seqlen;           /* T (1 for step) */
    int32_t nheads;           /* H */
    int32_t headdim;          /* P */
    int32_t d_state;          /* N (even) */
    int32_t mimo_rank;        /* R */
    int32_t ngroups;          /* G (divides H) */
    int32_t use_trapezoidal;  /* 0/1: lambda columns present, two-term update */
    int32_t use_complex;      /* 0/1: theta columns present, data-dependent RoPE */
    int32_t dtype;            /* m3_dtype of proj and of the gated output */
    int64_t proj_row_stride;  /* elements between consecutive tokens of proj (>= d_in_proj) */
    float rms_eps;            /* RMSNorm epsilon of B_norm / C_norm (1e-5 in the reference) */
    int32_t flags;            /* M3_FLAG_* bits (0 by default) */
} m3_layer_desc;

/* The bf16 MFMA prefill kernels hold the normalised B^ / C^ values, x * mimo_x, the
 * decay-masked scores and a copy of the state as f16 MFMA operands. They bring large
 * parameters into the f16 range themselves: B^, C^ and x * mimo_x are held divided by
 * powers of two derived from the parameters (one rank's B^ row norm sqrt(N R) max|w| +
 * sqrt(N) max|bias| to at most 128, |mimo_x| to at most 256) and the fp32 epilogues undo
 * them, so any checkpoint runs on them. Left to the caller: activations of ordinary size
 * (|x * mimo_x| / 2^k below 65504, dt below ~4). This flag forces the fp32 generic kernel
 * instead (VALU, about 100x slower), for callers that want no f16 operand at all. */
#define M3_FLAG_NO_F16_OPERANDS 1
/* fp32 layers: m3_prefill_fwd keeps the intermediates m3_layer_bwd differentiates through in
 * its workspace (the fp32 layer workspace; for d_state 128, headdim 64, mimo_rank 2 the fused
 * fp32 kernel writes them as it walks the sequence, other shapes run the staged fp32 layer
 * path). Without it an fp32 layer of that shape runs the fused fp32 kernel alone, whose
 * workspace holds only the normalised B^ / C^. */
#define M3_FLAG_FOR_BACKWARD 2

/* Small per-layer parameters, all fp32 device arrays. Names follow the reference's
 * parameters (mamba3/mamba3.py:95-111). */
typedef struct m3_layer_params {
    const float* A_log;      /* [H] */
    const float* D;          /* [H] */
    const float* dt_bias;    /* [H] */
    const float* B_norm_w;   /* [N*R] */
    const float* C_norm_w;   /* [N*R] */
    const float* B_bias;     /* [G,N,R] */
    const float* C_bias;     /* [G,N,R] */
    const float* mimo_x;     /* [H,P,R] */
    const float* mimo_z;     /* [H,P,R] */
    const float* mimo_down;  /* [H,P,R] */
} m3_layer_params;

/* Gradients of the small per-layer parameters (fp32 device arrays, same shapes as
 * m3_layer_params; written, not accumulated), and of the optional dt_scale input
 * ([B,T,H] fp32, dt = softplus(dt_raw + dt_bias) * dt_scale, mamba3/mamba3.py:200-202;
 * NULL when not wanted). */
typedef struct m3_layer_param_grads {
    float* A_log;
    float* D;
    float* dt_bias;
    float* B_norm_w;
    float* C_norm_w;
    float* B_bias;
    float* C_bias;
    float* mimo_x;
    float* mimo_z;
    float* mimo_down;
    float* dt_scale;
} m3_layer_param_grads;

const char* m3_status_string(int status);

/* Library version as major*10000 + minor*100 + patch. 0.2.0 (200): m3_layer_param_grads
 * gained its dt_scale field and m3_prefill_kernel_name was added; 0.1.0 (100) had neither. */
int m3_version(void);

/*
 * Name of the prefill kernel m3_prefill_fwd would run for these arguments (the dispatch
 * depends on the shape, dtype, flags and the pointers' alignment): "mfma_d128_p64_r2",
 * "mfma_general", "fp32_fused", "fp32_fused_train", "fp32_layer" or "generic"; NULL for an
 * invalid descriptor. No counterpart in the reference (one ATen path). A static string.
 */
const char* m3_prefill_kernel_name(const m3_layer_desc* desc, const void* proj,
                                   const void* y_out, const float* h_final,
                                   const float* prev_bx);

/*
 * Inter-chunk state scan. Replaces the reference's native `scan_forward`
 * (mamba3/csrc/scan.cu:128-166, bound at scan.cu:214-216) and its torch fallback
 * (mamba3/scan.py:34-44):
 *     h_states[b,0,h,:]   = h_init[b,h,:]  (or 0 when h_init is NULL)
 *     h_states[b,k+1,h,:] = decay[b,k,h] * h_states[b,k,h,:] + h_chunk[b,k,h,:]
 * decay [B,K,H], h_chunk [B,K,H,PN], h_init [B,H,PN] (nullable), h_states [B,K,H,PN];
 * all fp32. Unlike the reference, PN is not limited to 16384.
 * Pointers must be 16-byte aligned when PN % 4 == 0 (the vectorised path).
 */
int m3_scan_fwd(const float* decay, const float* h_chunk, const float* h_init,
                float* h_states, int64_t batch, int64_t nchunks, int64_t nheads,
                int64_t pn, void* stream);

/*
 * Backward of the inter-chunk state scan. Replaces the reference's native
 * `scan_backward` (mamba3/csrc/scan.cu:168-211, kernel at scan.cu:52-126, bound at
 * scan.cu:217-219) and its torch fallback `_scan_backward_torch` (mamba3/scan.py:47-62).
 * With G[K-1] = grad[K-1] and G[k] = grad[k] + decay[b,k,h] G[k+1]:
 *     d_chunk[b,k,h,:] = G[k+1] for k < K-1, 0 for k = K-1
 *     d_decay[b,k,h]   = sum_j G[k+1][j] h_states[b,k,h,j] for k < K-1, 0 for k = K-1
 *     d_h_init[b,h,:]  = G[0]   (not written when d_h_init is NULL)
 * decay, d_decay [B,K,H]; h_states, grad, d_chunk [B,K,H,PN]; d_h_init [B,H,PN]; all fp32.
 * d_decay sums are formed in a fixed order (deterministic). Any PN and any pointer
 * alignment (PN a multiple of 256 with 16-byte aligned arrays takes the vectorised path).
 * workspace: m3_scan_bwd_workspace_size() bytes (0 is possible), 256-byte aligned.
 */
int m3_scan_bwd_workspace_size(int64_t batch, int64_t nchunks, int64_t nheads, int64_t pn,
                               size_t* bytes);
int m3_scan_bwd(const float* decay, const float* h_states, const float* grad, float* d_decay,
                float* d_chunk, float* d_h_init, void* workspace, size_t workspace_bytes,
                int64_t batch, int64_t nchunks, int64_t nheads, int64_t pn, void* stream);

/*
 * Backward of m3_prefill_fwd for fp32 layers (desc->dtype fp32, mimo_rank 1..8), from the
 * workspace of that forward call, which holds its intermediates (the per-token operands and,
 * for most shapes, the chunk-start states the backward then does not recompute; pass the same buffer, unchanged,
 * with its size; that forward ran with M3_FLAG_FOR_BACKWARD in desc->flags, as does this call). Replaces the reference's autograd through mamba3/mamba3.py:197-256 (ATen's
 * backward of the dt softplus, the B/C RMSNorm + bias, the RoPE rotation and its angle cumsum,
 * the MIMO and trapezoid terms and the SiLU gate) and through chunked_ssd (see
 * m3_chunked_ssd_bwd). Inputs: g_out [B,T,H*P] = dL/d(gated output), and nullable g_h
 * [B,H,P,N], g_angle [B,H,N/2], g_prev [B,H,P,N] for the prefill state; outputs g_proj
 * [B,proj_row_stride] (every column of the in_proj layout written) and the parameter
 * gradients `grads` (written, not accumulated). fp32 throughout; deterministic.
 * workspace: m3_layer_bwd_workspace_size() bytes, 256-byte aligned.
 */
int m3_layer_bwd_workspace_size(const m3_layer_desc* desc, size_t* bytes);
int m3_layer_bwd(const m3_layer_desc* desc, const m3_layer_params* params, const void* proj,
                 const float* dt_scale, void* fwd_workspace, size_t fwd_workspace_bytes,
                 const float* g_out, const float* g_h, const float* g_angle, const float* g_prev,
                 float* g_proj, const m3_layer_param_grads* grads, void* workspace,
                 size_t workspace_bytes, void* stream);

/*
 * Bytes of device workspace m3_prefill_fwd needs for `desc` (0 is possible).
 * No counterpart in the reference, which allocates inside ATen.
 */
int m3_prefill_workspace_size(const m3_layer_desc* desc, size_t* bytes);

/*
 * Fused chunked-SSD prefill of one KulaMamba layer, from the in_proj output to the
 * gated, rank-reduced activation that feeds out_proj. Replaces the reference region
 * mamba3/mamba3.py:199-256 (dt/decay prep, _process_BC_train, MIMO/trapezoid prep,
 * chunked_ssd of mamba3/ssd.py:118-244 with _IntraChunkFn ssd.py:30-65 and ssd_scan,
 * the SiLU gate and MIMO-down sum) and the prefill state of mamba3.py:241-256.
 *   proj      [B,T,proj_row_stride] in desc->dtype
 *   dt_scale  [B,T,H] fp32 or NULL (multiplies softplus(dt), mamba3.py:200-202)
 *   y_out     [B,T,H*P] in desc->dtype (input of out_proj)
 *   h_final   [B,H,P,N] fp32 or NULL   (state 'h')
 *   angle     [B,H,N/2] fp32 or NULL   (state 'angle' = cumulative RoPE angle at T-1)
 *   prev_bx   [B,H,P,N] fp32 or NULL   (state 'prev_BX' = B~_{T-1} x_{T-1}^T)
 *   workspace of at least m3_prefill_workspace_size() bytes, 256-byte aligned.
 */
int m3_prefill_fwd(const m3_layer_desc* desc, const m3_layer_params* params,
                   const void* proj, const float* dt_scale, void* y_out,
                   float* h_final, float* angle, float* prev_bx,
                   void* workspace, size_t workspace_bytes, void* stream);

/*
 * m3_prefill_fwd without a caller workspace: no counterpart in the reference. For callers
 * that cannot allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc). Same arguments, dispatch, kernels and results as
 * m3_prefill_fwd, but the workspace is a static array of the library on each GPU
 * (M3_NOALLOC_SCRATCH_BYTES, held from the first call on that GPU until the process
 * ends); calls needing more return M3_ERR_SCRATCH_LIMIT and launch nothing. It calls no
 * allocator. M3_FLAG_FOR_BACKWARD is refused (M3_ERR_UNSUPPORTED): the backward's operands
 * would be left in the shared scratch, which the next call overwrites. The scratch keeps the last call's contents and needs no clearing (every
 * kernel writes what it later reads). All calls on one GPU share the array: calls that
 * overlap in time on one GPU (other streams or threads) race and must be serialised by
 * the caller.
 */
int m3_prefill_fwd_noalloc(const m3_layer_desc* desc, const m3_layer_params* params,
                           const void* proj, const float* dt_scale, void* y_out,
                           float* h_final, float* angle, float* prev_bx, void* stream);

/*
 * O(1) decode step of one KulaMamba layer for B tokens. Replaces
 * mamba3/mamba3.py:275-316 (everything in KulaMamba.step between in_proj and
 * out_proj, including _process_BC_step mamba3.py:170-190). Out of place, like the
 * reference (which returns a new state dict, mamba3.py:322):
 *   proj [B,proj_row_stride] in desc->dtype; dt_scale [B,H] fp32 or NULL;
 *   h_in, prev_bx_in [B,H,P,N] fp32; angle_in [B,H,N/2] of angle_dtype;
 *   y_out [B,H*P] desc->dtype; h_out, prev_bx_out [B,H,P,N] fp32;
 *   angle_out [B,H,N/2] of angle_dtype. Output buffers must not alias inputs.
 * desc->seqlen is ignored (one token per batch row).
 */
int m3_step_fwd(const m3_layer_desc* desc, const m3_layer_params* params,
                const void* proj, const float* dt_scale,
                const float* h_in, const float* prev_bx_in, const void* angle_in,
                int angle_dtype, void* y_out, float* h_out, float* prev_bx_out,
                void* angle_out, void* stream);

/*
 * Backward of m3_step_fwd. Replaces ATen's autograd through KulaMamba.step between in_proj
 * and out_proj (mamba3/mamba3.py:275-322, with _process_BC_step :170-190), which the
 * reference differentiates like any other torch code. fp32 only (desc->dtype F32; a bf16
 * caller upcasts): proj [B,proj_row_stride], dt_scale [B,H] or NULL, h_in, prev_bx_in
 * [B,H,P,N], angle_in [B,H,N/2] as passed to the forward; g_y [B,H*P] = dL/dy (the gated
 * output); g_h_out, g_prev_bx_out [B,H,P,N] and g_angle_out [B,H,N/2] = dL/d(new state), each
 * NULL for zero. Outputs: g_proj (the in_proj columns of each row written), g_h_in,
 * g_prev_bx_in, g_angle_in, and the parameter gradients `grads` (written, not accumulated;
 * grads->dt_scale [B,H] when not NULL). Deterministic. Supported: every layer the API takes
 * (even d_state <= 512, headdim <= 256, mimo_rank <= 8; at most 100 KiB of LDS per head).
 * workspace: m3_step_bwd_workspace_size() bytes, 256-byte aligned.
 */
int m3_step_bwd_workspace_size(const m3_layer_desc* desc, size_t* bytes);
int m3_step_bwd(const m3_layer_desc* desc, const m3_layer_params* params, const float* proj,
                const float* dt_scale, const float* h_in, const float* prev_bx_in,
                const float* angle_in, const float* g_y, const float* g_h_out,
                const float* g_prev_bx_out, const float* g_angle_out, float* g_proj,
                float* g_h_in, float* g_prev_bx_in, float* g_angle_in,
                const m3_layer_param_grads* grads, void* workspace, size_t workspace_bytes,
                void* stream);

/*
 * Chunked SSD on pre-processed, head-expanded inputs: the public op
 * chunked_ssd (mamba3/ssd.py:118-244). All tensors are in `dtype` except h_init,
 * h_final (fp32) and A, D (fp32 [H]).
 *   x_g, x_raw [B,T,H,P,R]; x_b [B,T,H,P,R] or NULL (then B_b must be NULL);
 *   B_g, C [B,T,H,N,R]; B_b [B,T,H,N,R] or NULL; dt [B,T,H];
 *   h_init [B,H,P,N] fp32 or NULL; y [B,T,H,P,R] in dtype; h_final [B,H,P,N] or NULL.
 * state_ws: [B,H,P,N] fp32 scratch owned by the caller (may equal h_final), used by the
 * generic kernel. workspace (256-byte aligned, m3_chunked_ssd_fwd_workspace_size() bytes, or
 * NULL): with it, fp32 inputs run on the fp32-MFMA chunk kernels shared with
 * m3_chunked_ssd_bwd (chunk states, state scan, masked scores, output tiles).
 */
int m3_chunked_ssd_fwd(int32_t batch, int32_t seqlen, int32_t nheads, int32_t headdim,
                       int32_t d_state, int32_t mimo_rank, int32_t dtype,
                       const void* x_g, const void* x_b, const void* B_g, const void* B_b,
                       const void* C, const void* dt, const float* A, const float* D,
                       const void* x_raw, const float* h_init, void* y, float* h_final,
                       float* state_ws, void* workspace, size_t workspace_bytes, void* stream);

/*
 * Bytes of device workspace with which m3_chunked_ssd_fwd runs fp32 inputs on its fp32-MFMA
 * chunk kernels (mimo_rank 1, 2, 4 or 8; headdim * d_state a multiple of 256 or at most
 * 16384). 0: that path does not apply (bf16, other shapes); m3_chunked_ssd_fwd then runs the
 * generic kernel, as it also does when no workspace (or too small a one) is passed. No
 * counterpart in the reference, which allocates inside ATen.
 */
int m3_chunked_ssd_fwd_workspace_size(int32_t batch, int32_t seqlen, int32_t nheads,
                                      int32_t headdim, int32_t d_state, int32_t mimo_rank,
                                      int32_t dtype, int32_t has_beta, size_t* bytes);

/*
 * Backward of m3_chunked_ssd_fwd, all tensors fp32 (the caller upcasts bf16). Replaces the
 * reference's autograd through chunked_ssd (mamba3/ssd.py:118-244): _IntraChunkFn.backward
 * (ssd.py:67-115), SSDScanFn.backward (mamba3/scan.py:101-141) with the native
 * scan_backward (mamba3/csrc/scan.cu:168-211), and ATen's backward of the bmm / cumsum /
 * exp / cat around them, without the per-token (P,N) outer products.
 * Inputs are the forward's (same shapes; x_b / B_b NULL for no beta terms; h_init
 * nullable) plus dy [B,T,H,P,R] = dL/dy and dh_final [B,H,P,N] = dL/dh_final (nullable).
 * Outputs (all written, not accumulated): dx_g, dx_b, dB_g, dB_b, dC, dx_raw like their
 * inputs (dx_b / dB_b NULL exactly when x_b is), ddt [B,T,H], dA [H], dD [H],
 * dh_init [B,H,P,N] (nullable: not written). mimo_rank must be 1, 2, 4 or 8. Sums run in a
 * fixed order
 * (deterministic). workspace: m3_chunked_ssd_bwd_workspace_size() bytes, 256-byte aligned.
 */
int m3_chunked_ssd_bwd_workspace_size(int32_t batch, int32_t seqlen, int32_t nheads,
                                      int32_t headdim, int32_t d_state, int32_t mimo_rank,
                                      int32_t has_beta, size_t* bytes);
int m3_chunked_ssd_bwd(int32_t batch, int32_t seqlen, int32_t nheads, int32_t headdim,
                       int32_t d_state, int32_t mimo_rank, const float* x_g, const float* x_b,
                       const float* B_g, const float* B_b, const float* C, const float* dt,
                       const float* A, const float* D, const float* x_raw, const float* h_init,
                       const float* dy, const float* dh_final, float* dx_g, float* dx_b,
                       float* dB_g, float* dB_b, float* dC, float* ddt, float* dA, float* dD,
                       float* dx_raw, float* dh_init, void* workspace, size_t workspace_bytes,
                       void* stream);

/*
 * RMSNorm of the residual blocks in one pass over the activations. Replaces the reference's
 * RMSNorm.forward (mamba3/mamba3.py:19-35) as used by KulaMambaBlock / KulaMambaLM
 * (mamba3/block.py:45-72, 138-140, 182), which runs it as several element-wise ATen ops.
 *   s[r] = rsqrt(mean_j x[r,j]^2 + eps)            (fp32)
 *   y[r,j] = (x[r,j] * s[r]) * weight[j]            the scale and x*s rounded to x's dtype,
 *                                                  as the reference does
 * x [rows, d] in x_dtype; weight [d] in w_dtype; y [rows, d] in y_dtype, which must be bf16
 * when both x and weight are bf16 and fp32 otherwise (the promotion of the two); rstd [rows]
 * fp32 or NULL (s, kept for the backward). 0 < rows < 2^33, 0 < d <= 2^24.
 */
int m3_rmsnorm_fwd(const void* x, int x_dtype, const void* weight, int w_dtype, void* y,
                   int y_dtype, float* rstd, int64_t rows, int32_t d, float eps, void* stream);

/*
 * Backward of m3_rmsnorm_fwd (the reference differentiates it through ATen), fp32
 * arithmetic: with g = dL/dy (grad_dtype = the forward's y_dtype) and a = sum_j w_j g_j x_j,
 *   dx = s w g - x s^3 a / d   (x_dtype)     dweight = sum_rows g x s   (w_dtype)
 * dweight is summed in a fixed order (deterministic). workspace:
 * m3_rmsnorm_bwd_workspace_size() bytes, 256-byte aligned.
 */
int m3_rmsnorm_bwd_workspace_size(int64_t rows, int32_t d, size_t* bytes);
int m3_rmsnorm_bwd(const void* x, int x_dtype, const void* weight, int w_dtype,
                   const float* rstd, const void* grad, int grad_dtype, void* dx, void* dweight,
                   void* workspace, size_t workspace_bytes, int64_t rows, int32_t d,
                   void* stream);

/*
 * SwiGLU's element-wise step (mamba3/block.py:16-26: silu(w_gate x) * w_up x) on the output of
 * one GEMM over the concatenated [w_gate; w_up] weight: gate_up [rows, row_stride] bf16 with
 * the gate in columns [0, d_ff) and up in [d_ff, 2 d_ff); out [rows, d_ff] bf16 =
 * silu(gate) * up, computed in fp32 and rounded once. out must not alias gate_up.
 */
int m3_silu_mul(const void* gate_up, int64_t rows, int32_t d_ff, int64_t row_stride, void* out,
                void* stream);

/*
 * Small-batch projections of the decode step, bf16, bound by the weight read. For decode
 * batches of at most 8 rows they replace, each in one kernel, the block step's projections
 * with the work around them (mamba3/block.py:94-100: ssm_norm + in_proj, out_proj + residual,
 * mlp_norm + SwiGLU, w_down + residual; mamba3/mamba3.py:275-316 in_proj / out_proj of
 * KulaMamba.step; mamba3/block.py:182-183 the final norm + lm_head).
 *   m3_small_linear:  out = n W^T, or res + scale * (n W^T) when residual is given
 *   m3_small_swiglu:  out = silu(n W_gate^T) * (n W_up^T)   (mamba3/block.py:16-26)
 * with n = RMSNorm(x; norm_w, eps) (mamba3/mamba3.py:19-35, the reference's bf16 roundings)
 * when norm_w is given, else n = x. x [m, k], weights [n, k] (nn.Linear's layout), norm_w
 * [k], residual and out [m, n]; all bf16, rows contiguous. 1 <= m <= 8, k % 64 == 0,
 * (m' k + 8) * 2 <= 65536 bytes of staged rows (m' = m rounded up to 1, 2, 4 or 8); x and the
 * weights 16-byte aligned. out may alias residual (each element is read and written by one
 * thread), not x or the weights. Accumulation in fp32; one bf16 rounding of the result.
 */
int m3_small_linear(const void* x, const void* norm_w, float eps, const void* weight,
                    const void* residual, float scale, void* out, int32_t m, int32_t n, int32_t k,
                    void* stream);
int m3_small_swiglu(const void* x, const void* norm_w, float eps, const void* w_gate,
                    const void* w_up, void* out, int32_t m, int32_t n, int32_t k, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MAMBA3_AMD_H */
