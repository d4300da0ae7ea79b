// C-ABI entry points (declared in include/mamba3_amd.h). Validates every argument on
// the host, then calls the launchers. Never throws, never allocates, never syncs. The one
// piece of global state is the static scratch of m3_prefill_fwd_noalloc (below).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <mutex>

#include "m3_kernels.h"

namespace {

using m3::proj_layout;

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

bool aligned(const void* p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

int check_desc(const m3_layer_desc* d) {
    if (!d) return M3_ERR_NULL_POINTER;
    if (d->batch <= 0 || d->seqlen <= 0 || d->nheads <= 0 || d->headdim <= 0 ||
        d->d_state <= 0 || d->mimo_rank <= 0 || d->ngroups <= 0)
        return M3_ERR_INVALID_SHAPE;
    if (d->d_state % 2 != 0) return M3_ERR_INVALID_SHAPE;
    if (d->nheads % d->ngroups != 0) return M3_ERR_INVALID_SHAPE;
    if (d->dtype != M3_DTYPE_F32 && d->dtype != M3_DTYPE_BF16) return M3_ERR_UNSUPPORTED;
    if (d->use_trapezoidal != 0 && d->use_trapezoidal != 1) return M3_ERR_INVALID_SHAPE;
    if (d->use_complex != 0 && d->use_complex != 1) return M3_ERR_INVALID_SHAPE;
    if (d->proj_row_stride < proj_layout(*d).width) return M3_ERR_INVALID_SHAPE;
    if (!(d->rms_eps >= 0.f)) return M3_ERR_INVALID_SHAPE;
    if (d->flags & ~(M3_FLAG_NO_F16_OPERANDS | M3_FLAG_FOR_BACKWARD)) return M3_ERR_INVALID_SHAPE;
    // Kernel limits: headdim <= 256, d_state <= 512, rank <= 8.
    if (d->headdim > 256 || d->d_state > 512 || d->mimo_rank > 8) return M3_ERR_UNSUPPORTED;
    return M3_OK;
}

int check_params(const m3_layer_params* p) {
    if (!p) return M3_ERR_NULL_POINTER;
    if (!p->A_log || !p->D || !p->dt_bias || !p->B_norm_w || !p->C_norm_w || !p->B_bias ||
        !p->C_bias || !p->mimo_x || !p->mimo_z || !p->mimo_down)
        return M3_ERR_NULL_POINTER;
    return M3_OK;
}

int check_scan_bwd_shape(int64_t batch, int64_t nchunks, int64_t nheads, int64_t pn) {
    if (batch <= 0 || nchunks <= 0 || nheads <= 0 || pn <= 0) return M3_ERR_INVALID_SHAPE;
    if (batch * nheads * pn > ((int64_t)1 << 40) || nchunks > (1 << 30)) return M3_ERR_UNSUPPORTED;
    if (batch * nheads > 0x7fffffff) return M3_ERR_UNSUPPORTED;
    return M3_OK;
}

// Which prefill kernel a call dispatches to: the d_state 128 / headdim 64 / rank 2 MFMA
// kernel (bf16, aligned rows, 16-byte aligned proj / y_out), the general MFMA kernel
// (bf16, d_state 64/128/256, rank 1/2/4, headdim % 32 == 0, 16-byte aligned h_final) --
// both with f16 operands (scaled by powers of two for large parameters), so not under
// M3_FLAG_NO_F16_OPERANDS, which a caller may set to force the generic fp32 kernel -- the
// fused fp32 kernel
// (fp32, d_state 128 / headdim 64 / rank 2; under M3_FLAG_FOR_BACKWARD it also writes the
// staged operands of the layer backward into the fp32 layer workspace), the fp32 layer path
// on the fp32-MFMA chunk kernels (fp32, rank 1..8) or the generic one.
enum class PrefillPath { kMfma, kWide, kFp32Fused, kFp32FusedTrain, kFp32, kGeneric };

PrefillPath prefill_path(const m3_layer_desc& d, const void* proj, const void* y_out,
                         const void* h_final, const void* prev_bx) {
    const bool f16_ok = !(d.flags & M3_FLAG_NO_F16_OPERANDS);
    if (f16_ok && m3::mfma_prefill_supported(d, proj, y_out)) return PrefillPath::kMfma;
    if (f16_ok && m3::wide_prefill_supported(d) && aligned(h_final, 16)) return PrefillPath::kWide;
    if (m3::fused_fp32_prefill_supported(d, proj, y_out, h_final, prev_bx)) return PrefillPath::kFp32Fused;
    if ((d.flags & M3_FLAG_FOR_BACKWARD) && m3::fused_fp32_train_supported(d, proj, y_out, h_final, prev_bx))
        return PrefillPath::kFp32FusedTrain;
    if (m3::fp32_layer_supported(d)) return PrefillPath::kFp32;
    return PrefillPath::kGeneric;
}

size_t prefill_path_workspace(const m3_layer_desc& d, PrefillPath path) {
    switch (path) {
        case PrefillPath::kMfma: return m3::mfma_prefill_workspace(d);
        case PrefillPath::kWide: return m3::wide_prefill_workspace(d);
        case PrefillPath::kFp32Fused: return m3::fused_fp32_prefill_workspace(d);
        case PrefillPath::kFp32FusedTrain:
        case PrefillPath::kFp32: return m3::fp32_layer_workspace(d);
        default: return m3::generic_prefill_workspace(d);
    }
}

int check_prefill_args(const m3_layer_desc* desc, const m3_layer_params* params,
                       const void* proj, const void* y_out) {
    int st = check_desc(desc);
    if (st != M3_OK) return st;
    st = check_params(params);
    if (st != M3_OK) return st;
    if (!proj || !y_out) return M3_ERR_NULL_POINTER;
    return M3_OK;
}

int launch_prefill_path(PrefillPath path, const m3_layer_desc& d, const m3_layer_params& p,
                        const void* proj, const float* dt_scale, void* y_out, float* h_final,
                        float* angle, float* prev_bx, void* ws, hipStream_t stream) {
    switch (path) {
        case PrefillPath::kMfma:
            return m3::launch_mfma_prefill(d, p, proj, dt_scale, y_out, h_final, angle, prev_bx,
                                           ws, stream);
        case PrefillPath::kWide:
            return m3::launch_wide_prefill(d, p, proj, dt_scale, y_out, h_final, angle, prev_bx,
                                           ws, stream);
        case PrefillPath::kFp32Fused:
            return m3::launch_fused_fp32_prefill(d, p, proj, dt_scale, y_out, h_final, angle,
                                                 prev_bx, ws, stream);
        case PrefillPath::kFp32FusedTrain: {
            const m3::Fp32LayerParts parts = m3::fp32_layer_parts(d, ws);
            size_t bytes = 0;
            void* scratch_rows = m3::fp32_layer_scratch(d, ws, &bytes);
            return m3::launch_fused_fp32_prefill(d, p, proj, dt_scale, y_out, h_final, angle,
                                                 prev_bx, scratch_rows, stream, &parts);
        }
        case PrefillPath::kFp32:
            return m3::launch_fp32_layer(d, p, proj, dt_scale, y_out, h_final, angle, prev_bx,
                                         ws, stream) == 0
                       ? M3_OK
                       : M3_ERR_LAUNCH;
        default:
            return m3::launch_generic_prefill(d, p, proj, dt_scale, y_out, h_final, angle,
                                              prev_bx, ws, stream);
    }
}

// ---- static scratch of m3_prefill_fwd_noalloc
// One copy of this array exists on every GPU the library runs on, from the first call on
// that GPU until the process ends. Host code never uses the array's name as an address:
// its device address is looked up once per device (hipGetSymbolAddress, with that device
// current) and kept in g_scratch.
static __device__ __align__(256) unsigned char scratch[M3_NOALLOC_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch[kMaxDevices];

int scratch_for_stream(hipStream_t stream, void** out) {
    int cur = -1;
    if (hipGetDevice(&cur) != hipSuccess) return M3_ERR_DEVICE;
    int dev = cur;
    if (stream != nullptr) {
        hipDevice_t sd;
        if (hipStreamGetDevice(stream, &sd) != hipSuccess) return M3_ERR_DEVICE;
        dev = static_cast<int>(sd);
    }
    if (dev < 0 || dev >= kMaxDevices) return M3_ERR_DEVICE;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (g_scratch[dev] == nullptr) {
        if (dev != cur && hipSetDevice(dev) != hipSuccess) return M3_ERR_DEVICE;
        void* ptr = nullptr;
        const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (dev != cur) (void)hipSetDevice(cur);
        if (e != hipSuccess || ptr == nullptr) return M3_ERR_DEVICE;
        g_scratch[dev] = ptr;
    }
    *out = g_scratch[dev];
    return M3_OK;
}

}  // namespace

extern "C" {

const char* m3_status_string(int status) {
    switch (status) {
        case M3_OK: return "ok";
        case M3_ERR_NULL_POINTER: return "a required pointer is NULL";
        case M3_ERR_INVALID_SHAPE: return "invalid or inconsistent shape";
        case M3_ERR_UNSUPPORTED: return "shape or dtype not supported by the kernels";
        case M3_ERR_WORKSPACE: return "workspace missing or too small";
        case M3_ERR_MISALIGNED: return "pointer alignment violated";
        case M3_ERR_LAUNCH: return "kernel launch failed";
        case M3_ERR_DEVICE: return "device query failed";
        case M3_ERR_SCRATCH_LIMIT:
            return "workspace need exceeds the static scratch of m3_prefill_fwd_noalloc "
                   "(M3_NOALLOC_SCRATCH_BYTES); use m3_prefill_fwd with a caller workspace";
        default: return "unknown status";
    }
}

int m3_version(void) { return 200; }

const char* m3_prefill_kernel_name(const m3_layer_desc* desc, const void* proj, const void* y_out,
                                   const float* h_final, const float* prev_bx) {
    if (check_desc(desc) != M3_OK) return nullptr;
    switch (prefill_path(*desc, proj, y_out, h_final, prev_bx)) {
        case PrefillPath::kMfma: return "mfma_d128_p64_r2";
        case PrefillPath::kWide: return "mfma_general";
        case PrefillPath::kFp32Fused: return "fp32_fused";
        case PrefillPath::kFp32FusedTrain: return "fp32_fused_train";
        case PrefillPath::kFp32: return "fp32_layer";
        default: return "generic";
    }
}

int m3_scan_fwd(const float* decay, const float* h_chunk, const float* h_init,
                float* h_states, int64_t batch, int64_t nchunks, int64_t nheads, int64_t pn,
                void* stream) {
    if (!decay || !h_chunk || !h_states) return M3_ERR_NULL_POINTER;
    if (batch <= 0 || nchunks <= 0 || nheads <= 0 || pn <= 0) return M3_ERR_INVALID_SHAPE;
    if (batch * nheads * pn > ((int64_t)1 << 40)) return M3_ERR_UNSUPPORTED;
    if (nchunks > (1 << 30)) return M3_ERR_UNSUPPORTED;
    return m3::launch_scan_fwd(decay, h_chunk, h_init, h_states, batch, nchunks, nheads, pn,
                               as_stream(stream)) == 0
               ? M3_OK
               : M3_ERR_LAUNCH;
}

int m3_scan_bwd_workspace_size(int64_t batch, int64_t nchunks, int64_t nheads, int64_t pn,
                               size_t* bytes) {
    if (!bytes) return M3_ERR_NULL_POINTER;
    const int st = check_scan_bwd_shape(batch, nchunks, nheads, pn);
    if (st != M3_OK) return st;
    *bytes = m3::scan_bwd_workspace(batch, nchunks, nheads, pn);
    return M3_OK;
}

int m3_scan_bwd(const float* decay, const float* h_states, const float* grad, float* d_decay,
                float* d_chunk, float* d_h_init, void* workspace, size_t workspace_bytes,
                int64_t batch, int64_t nchunks, int64_t nheads, int64_t pn, void* stream) {
    if (!decay || !h_states || !grad || !d_decay || !d_chunk) return M3_ERR_NULL_POINTER;
    const int st = check_scan_bwd_shape(batch, nchunks, nheads, pn);
    if (st != M3_OK) return st;
    const size_t need = m3::scan_bwd_workspace(batch, nchunks, nheads, pn);
    if (need > 0 && (!workspace || workspace_bytes < need)) return M3_ERR_WORKSPACE;
    if (workspace && !aligned(workspace, 256)) return M3_ERR_MISALIGNED;
    return m3::launch_scan_bwd(decay, h_states, grad, d_decay, d_chunk, d_h_init,
                               reinterpret_cast<float*>(workspace), batch, nchunks, nheads, pn,
                               as_stream(stream)) == 0
               ? M3_OK
               : M3_ERR_LAUNCH;
}

// Workspace for whichever prefill kernel the shape may dispatch to (the pointers' alignment
// is not known here, so the largest of the candidates).
static size_t prefill_workspace(const m3_layer_desc& d) {
    size_t n = m3::generic_prefill_workspace(d);
    n = std::max(n, m3::fp32_layer_workspace(d));
    if (m3::fused_fp32_prefill_supported(d, nullptr, nullptr, nullptr, nullptr))
        n = std::max(n, m3::fused_fp32_prefill_workspace(d));
    if (m3::mfma_prefill_supported(d, nullptr, nullptr)) n = std::max(n, m3::mfma_prefill_workspace(d));
    if (m3::wide_prefill_supported(d)) n = std::max(n, m3::wide_prefill_workspace(d));
    return n;
}

int m3_prefill_workspace_size(const m3_layer_desc* desc, size_t* bytes) {
    if (!bytes) return M3_ERR_NULL_POINTER;
    const int st = check_desc(desc);
    if (st != M3_OK) return st;
    *bytes = prefill_workspace(*desc);
    return M3_OK;
}

int m3_prefill_fwd(const m3_layer_desc* desc, const m3_layer_params* params, const void* proj,
                   const float* dt_scale, void* y_out, float* h_final, float* angle,
                   float* prev_bx, void* workspace, size_t workspace_bytes, void* stream) {
    int st = check_prefill_args(desc, params, proj, y_out);
    if (st != M3_OK) return st;
    const PrefillPath path = prefill_path(*desc, proj, y_out, h_final, prev_bx);
    const size_t need = prefill_path_workspace(*desc, path);
    if (need > 0 && (!workspace || workspace_bytes < need)) return M3_ERR_WORKSPACE;
    if (workspace && !aligned(workspace, 256)) return M3_ERR_MISALIGNED;
    return launch_prefill_path(path, *desc, *params, proj, dt_scale, y_out, h_final, angle,
                               prev_bx, workspace, as_stream(stream));
}

int m3_prefill_fwd_noalloc(const m3_layer_desc* desc, const m3_layer_params* params,
                           const void* proj, const float* dt_scale, void* y_out, float* h_final,
                           float* angle, float* prev_bx, void* stream) {
    int st = check_prefill_args(desc, params, proj, y_out);
    if (st != M3_OK) return st;
    // The backward's operands would land in the shared scratch, which the next call
    // overwrites and no caller can hand to m3_layer_bwd.
    if (desc->flags & M3_FLAG_FOR_BACKWARD) return M3_ERR_UNSUPPORTED;
    const PrefillPath path = prefill_path(*desc, proj, y_out, h_final, prev_bx);
    const size_t need = prefill_path_workspace(*desc, path);
    if (need > M3_NOALLOC_SCRATCH_BYTES) return M3_ERR_SCRATCH_LIMIT;
    void* ws = nullptr;
    if (need > 0) {
        st = scratch_for_stream(as_stream(stream), &ws);
        if (st != M3_OK) return st;
    }
    return launch_prefill_path(path, *desc, *params, proj, dt_scale, y_out, h_final, angle,
                               prev_bx, ws, as_stream(stream));
}

int m3_layer_bwd_workspace_size(const m3_layer_desc* desc, size_t* bytes) {
    if (!bytes) return M3_ERR_NULL_POINTER;
    const int st = check_desc(desc);
    if (st != M3_OK) return st;
    *bytes = m3::layer_bwd_workspace(*desc);
    return *bytes > 0 ? M3_OK : M3_ERR_UNSUPPORTED;
}

int m3_layer_bwd(const m3_layer_desc* desc, const m3_layer_params* params, const void* proj,
                 const float* dt_scale, void* fwd_workspace, size_t fwd_workspace_bytes,
                 const float* g_out, const float* g_h, const float* g_angle, const float* g_prev,
                 float* g_proj, const m3_layer_param_grads* grads, void* workspace,
                 size_t workspace_bytes, void* stream) {
    int st = check_desc(desc);
    if (st != M3_OK) return st;
    st = check_params(params);
    if (st != M3_OK) return st;
    if (!proj || !fwd_workspace || !g_out || !g_proj || !grads) return M3_ERR_NULL_POINTER;
    if (!grads->A_log || !grads->D || !grads->dt_bias || !grads->B_norm_w || !grads->C_norm_w ||
        !grads->B_bias || !grads->C_bias || !grads->mimo_x || !grads->mimo_z || !grads->mimo_down)
        return M3_ERR_NULL_POINTER;
    const size_t need = m3::layer_bwd_workspace(*desc);
    if (need == 0) return M3_ERR_UNSUPPORTED;
    if (fwd_workspace_bytes < m3::fp32_layer_workspace(*desc)) return M3_ERR_WORKSPACE;
    if (!workspace || workspace_bytes < need) return M3_ERR_WORKSPACE;
    if (!aligned(workspace, 256) || !aligned(fwd_workspace, 256)) return M3_ERR_MISALIGNED;
    return m3::launch_layer_bwd(*desc, *params, proj, dt_scale, fwd_workspace, g_out, g_h,
                                g_angle, g_prev, g_proj, *grads, workspace,
                                as_stream(stream)) == 0
               ? M3_OK
               : M3_ERR_LAUNCH;
}

int m3_step_fwd(const m3_layer_desc* desc, const m3_layer_params* params, const void* proj,
                const float* dt_scale, const float* h_in, const float* prev_bx_in,
                const void* angle_in, int angle_dtype, void* y_out, float* h_out,
                float* prev_bx_out, void* angle_out, void* stream) {
    int st = check_desc(desc);
    if (st != M3_OK) return st;
    st = check_params(params);
    if (st != M3_OK) return st;
    if (!proj || !h_in || !prev_bx_in || !angle_in || !y_out || !h_out || !prev_bx_out ||
        !angle_out)
        return M3_ERR_NULL_POINTER;
    if (angle_dtype != M3_DTYPE_F32 && angle_dtype != M3_DTYPE_BF16) return M3_ERR_UNSUPPORTED;
    if (!m3::step_supported(desc->d_state, desc->mimo_rank)) return M3_ERR_UNSUPPORTED;
    if (!aligned(h_in, 16) || !aligned(prev_bx_in, 16) || !aligned(h_out, 16) ||
        !aligned(prev_bx_out, 16))
        return M3_ERR_MISALIGNED;
    if (h_in == h_out || prev_bx_in == prev_bx_out || h_in == prev_bx_out ||
        prev_bx_in == h_out)
        return M3_ERR_INVALID_SHAPE;
    return m3::launch_step(*desc, *params, proj, dt_scale, h_in, prev_bx_in, angle_in,
                           angle_dtype, y_out, h_out, prev_bx_out, angle_out,
                           as_stream(stream));
}

int m3_step_bwd_workspace_size(const m3_layer_desc* desc, size_t* bytes) {
    if (!bytes) return M3_ERR_NULL_POINTER;
    const int st = check_desc(desc);
    if (st != M3_OK) return st;
    *bytes = m3::step_bwd_workspace(*desc);
    return *bytes > 0 ? M3_OK : M3_ERR_UNSUPPORTED;
}

int m3_step_bwd(const m3_layer_desc* desc, const m3_layer_params* params, const float* proj,
                const float* dt_scale, const float* h_in, const float* prev_bx_in,
                const float* angle_in, const float* g_y, const float* g_h_out,
                const float* g_prev_bx_out, const float* g_angle_out, float* g_proj,
                float* g_h_in, float* g_prev_bx_in, float* g_angle_in,
                const m3_layer_param_grads* grads, void* workspace, size_t workspace_bytes,
                void* stream) {
    int st = check_desc(desc);
    if (st != M3_OK) return st;
    st = check_params(params);
    if (st != M3_OK) return st;
    if (desc->dtype != M3_DTYPE_F32) return M3_ERR_UNSUPPORTED;
    if (!proj || !h_in || !prev_bx_in || !angle_in || !g_y || !g_proj || !g_h_in ||
        !g_prev_bx_in || !g_angle_in || !grads)
        return M3_ERR_NULL_POINTER;
    if (!grads->A_log || !grads->D || !grads->dt_bias || !grads->B_norm_w || !grads->C_norm_w ||
        !grads->B_bias || !grads->C_bias || !grads->mimo_x || !grads->mimo_z || !grads->mimo_down)
        return M3_ERR_NULL_POINTER;
    const size_t need = m3::step_bwd_workspace(*desc);
    if (need == 0) return M3_ERR_UNSUPPORTED;
    if (!workspace || workspace_bytes < need) return M3_ERR_WORKSPACE;
    if (!aligned(workspace, 256)) return M3_ERR_MISALIGNED;
    return m3::launch_step_bwd(*desc, *params, proj, dt_scale, h_in, prev_bx_in, angle_in, g_y,
                               g_h_out, g_prev_bx_out, g_angle_out, g_proj, g_h_in, g_prev_bx_in,
                               g_angle_in, *grads, workspace, as_stream(stream)) == 0
               ? M3_OK
               : M3_ERR_LAUNCH;
}

static bool norm_dtypes_ok(int xd, int wd, int yd) {
    auto ok = [](int t) { return t == M3_DTYPE_F32 || t == M3_DTYPE_BF16; };
    if (!ok(xd) || !ok(wd) || !ok(yd)) return false;
    // the output dtype is the promotion of the activation and weight dtypes
    return yd == ((xd == M3_DTYPE_BF16 && wd == M3_DTYPE_BF16) ? M3_DTYPE_BF16 : M3_DTYPE_F32);
}

// Grid limits of the norm kernels: rows / 4 blocks (x) forward, d / 256 column blocks (y)
// for the dweight partials.
static bool norm_shape_ok(int64_t rows, int32_t d) {
    return rows > 0 && rows < ((int64_t)1 << 33) && d > 0 && d <= (1 << 24);
}

int m3_rmsnorm_fwd(const void* x, int x_dtype, const void* weight, int w_dtype, void* y,
                   int y_dtype, float* rstd, int64_t rows, int32_t d, float eps, void* stream) {
    if (!x || !weight || !y) return M3_ERR_NULL_POINTER;
    if (!norm_shape_ok(rows, d) || !(eps >= 0.f)) return M3_ERR_INVALID_SHAPE;
    if (!norm_dtypes_ok(x_dtype, w_dtype, y_dtype)) return M3_ERR_UNSUPPORTED;
    return m3::launch_rmsnorm_fwd(x, x_dtype, weight, w_dtype, y, y_dtype, rstd, rows, d, eps,
                                  as_stream(stream)) == 0
               ? M3_OK
               : M3_ERR_LAUNCH;
}

int m3_rmsnorm_bwd_workspace_size(int64_t rows, int32_t d, size_t* bytes) {
    if (!bytes) return M3_ERR_NULL_POINTER;
    if (!norm_shape_ok(rows, d)) return M3_ERR_INVALID_SHAPE;
    *bytes = m3::rmsnorm_bwd_workspace(rows, d);
    return M3_OK;
}

int m3_rmsnorm_bwd(const void* x, int x_dtype, const void* weight, int w_dtype,
                   const float* rstd, const void* grad, int grad_dtype, void* dx, void* dweight,
                   void* workspace, size_t workspace_bytes, int64_t rows, int32_t d,
                   void* stream) {
    if (!x || !weight || !rstd || !grad || !dx || !dweight) return M3_ERR_NULL_POINTER;
    if (!norm_shape_ok(rows, d)) return M3_ERR_INVALID_SHAPE;
    if (!norm_dtypes_ok(x_dtype, w_dtype, grad_dtype)) return M3_ERR_UNSUPPORTED;
    if (!workspace || workspace_bytes < m3::rmsnorm_bwd_workspace(rows, d)) return M3_ERR_WORKSPACE;
    if (!aligned(workspace, 256)) return M3_ERR_MISALIGNED;
    return m3::launch_rmsnorm_bwd(x, x_dtype, weight, w_dtype, rstd, grad, grad_dtype, dx,
                                  dweight, workspace, rows, d, as_stream(stream)) == 0
               ? M3_OK
               : M3_ERR_LAUNCH;
}

int m3_silu_mul(const void* gate_up, int64_t rows, int32_t d_ff, int64_t row_stride, void* out,
                void* stream) {
    if (!gate_up || !out) return M3_ERR_NULL_POINTER;
    if (rows <= 0 || d_ff <= 0 || row_stride < 2 * (int64_t)d_ff) return M3_ERR_INVALID_SHAPE;
    if (rows * (int64_t)d_ff >= ((int64_t)1 << 39)) return M3_ERR_INVALID_SHAPE;  // 32-bit grid
    return m3::launch_silu_mul(gate_up, out, rows, d_ff, row_stride, as_stream(stream)) == 0
               ? M3_OK
               : M3_ERR_LAUNCH;
}

// Shapes the small-batch projection kernels take: at most 8 activation rows, K a multiple
// of 64 whose staged rows (and norm weight) fit 64 KB of LDS, 16-byte aligned activation,
// norm-weight and weight rows.
static int small_proj_check(const void* x, const void* nw, const void* w0, const void* w1,
                            const void* out, int32_t m, int32_t n, int32_t k) {
    if (!x || !w0 || !out) return M3_ERR_NULL_POINTER;
    if (m < 1 || m > 8 || n < 1 || k < 64 || k % 64 != 0) return M3_ERR_INVALID_SHAPE;
    if (m3::gemv_small_lds_bytes(m, k, nw != nullptr) > 65536) return M3_ERR_UNSUPPORTED;
    if (!aligned(x, 16) || !aligned(w0, 16) || (w1 && !aligned(w1, 16)) || (nw && !aligned(nw, 16)))
        return M3_ERR_MISALIGNED;
    return M3_OK;
}

int m3_small_linear(const void* x, const void* norm_w, float eps, const void* weight,
                    const void* residual, float scale, void* out, int32_t m, int32_t n, int32_t k,
                    void* stream) {
    const int st = small_proj_check(x, norm_w, weight, nullptr, out, m, n, k);
    if (st != M3_OK) return st;
    if (norm_w && !(eps >= 0.f)) return M3_ERR_INVALID_SHAPE;
    return m3::launch_gemv_small(x, norm_w, eps, weight, nullptr, residual, scale, out, m, n, k,
                                 as_stream(stream)) == 0
               ? M3_OK
               : M3_ERR_LAUNCH;
}

int m3_small_swiglu(const void* x, const void* norm_w, float eps, const void* w_gate,
                    const void* w_up, void* out, int32_t m, int32_t n, int32_t k, void* stream) {
    if (!w_up) return M3_ERR_NULL_POINTER;
    const int st = small_proj_check(x, norm_w, w_gate, w_up, out, m, n, k);
    if (st != M3_OK) return st;
    if (norm_w && !(eps >= 0.f)) return M3_ERR_INVALID_SHAPE;
    return m3::launch_gemv_small(x, norm_w, eps, w_gate, w_up, nullptr, 1.f, out, m, n, k,
                                 as_stream(stream)) == 0
               ? M3_OK
               : M3_ERR_LAUNCH;
}

int m3_chunked_ssd_fwd_workspace_size(int32_t batch, int32_t seqlen, int32_t nheads,
                                      int32_t headdim, int32_t d_state, int32_t mimo_rank,
                                      int32_t dtype, int32_t has_beta, size_t* bytes) {
    if (!bytes) return M3_ERR_NULL_POINTER;
    if (batch <= 0 || seqlen <= 0 || nheads <= 0 || headdim <= 0 || d_state <= 0 ||
        mimo_rank <= 0 || (has_beta != 0 && has_beta != 1))
        return M3_ERR_INVALID_SHAPE;
    if (dtype != M3_DTYPE_F32 && dtype != M3_DTYPE_BF16) return M3_ERR_UNSUPPORTED;
    *bytes = dtype == M3_DTYPE_F32 ? m3::chunked_fwd_mfma_workspace(batch, seqlen, nheads, headdim,
                                                                    d_state, mimo_rank, has_beta)
                                   : 0;
    return M3_OK;
}

int m3_chunked_ssd_fwd(int32_t batch, int32_t seqlen, int32_t nheads, int32_t headdim,
                       int32_t d_state, int32_t mimo_rank, int32_t dtype, const void* x_g,
                       const void* x_b, const void* B_g, const void* B_b, const void* C,
                       const void* dt, const float* A, const float* D, const void* x_raw,
                       const float* h_init, void* y, float* h_final, float* state_ws,
                       void* workspace, size_t workspace_bytes, void* stream) {
    if (batch <= 0 || seqlen <= 0 || nheads <= 0 || headdim <= 0 || d_state <= 0 ||
        mimo_rank <= 0)
        return M3_ERR_INVALID_SHAPE;
    if (dtype != M3_DTYPE_F32 && dtype != M3_DTYPE_BF16) return M3_ERR_UNSUPPORTED;
    if (headdim > 256 || d_state > 512 || mimo_rank > 8) return M3_ERR_UNSUPPORTED;
    if (!x_g || !B_g || !C || !dt || !A || !D || !x_raw || !y) return M3_ERR_NULL_POINTER;
    if ((x_b == nullptr) != (B_b == nullptr)) return M3_ERR_NULL_POINTER;
    const size_t need = dtype == M3_DTYPE_F32
                            ? m3::chunked_fwd_mfma_workspace(batch, seqlen, nheads, headdim,
                                                             d_state, mimo_rank, x_b != nullptr)
                            : 0;
    if (need > 0 && workspace && workspace_bytes >= need) {
        if (!aligned(workspace, 256)) return M3_ERR_MISALIGNED;
        auto fp = [](const void* v) { return reinterpret_cast<const float*>(v); };
        return m3::launch_chunked_fwd_mfma(batch, seqlen, nheads, headdim, d_state, mimo_rank,
                                           fp(x_g), fp(x_b), fp(B_g), fp(B_b), fp(C), fp(dt), A, D,
                                           fp(x_raw), h_init, reinterpret_cast<float*>(y),
                                           h_final, workspace, as_stream(stream)) == 0
                   ? M3_OK
                   : M3_ERR_LAUNCH;
    }
    if (!h_final && !state_ws) return M3_ERR_WORKSPACE;
    return m3::launch_generic_chunked(batch, seqlen, nheads, headdim, d_state, mimo_rank, dtype,
                                      x_g, x_b, B_g, B_b, C, dt, A, D, x_raw, h_init, y, h_final,
                                      state_ws, as_stream(stream));
}

int m3_chunked_ssd_bwd_workspace_size(int32_t batch, int32_t seqlen, int32_t nheads,
                                      int32_t headdim, int32_t d_state, int32_t mimo_rank,
                                      int32_t has_beta, size_t* bytes) {
    if (!bytes) return M3_ERR_NULL_POINTER;
    if (batch <= 0 || seqlen <= 0 || nheads <= 0 || headdim <= 0 || d_state <= 0 ||
        mimo_rank <= 0 || (has_beta != 0 && has_beta != 1))
        return M3_ERR_INVALID_SHAPE;
    if (!m3::chunked_bwd_shape_ok(batch, seqlen, nheads, headdim, d_state, mimo_rank, has_beta))
        return M3_ERR_UNSUPPORTED;
    *bytes = m3::chunked_bwd_workspace(batch, seqlen, nheads, headdim, d_state, mimo_rank, has_beta);
    return M3_OK;
}

int m3_chunked_ssd_bwd(int32_t batch, int32_t seqlen, int32_t nheads, int32_t headdim,
                       int32_t d_state, int32_t mimo_rank, const float* x_g, const float* x_b,
                       const float* B_g, const float* B_b, const float* C, const float* dt,
                       const float* A, const float* D, const float* x_raw, const float* h_init,
                       const float* dy, const float* dh_final, float* dx_g, float* dx_b,
                       float* dB_g, float* dB_b, float* dC, float* ddt, float* dA, float* dD,
                       float* dx_raw, float* dh_init, void* workspace, size_t workspace_bytes,
                       void* stream) {
    if (batch <= 0 || seqlen <= 0 || nheads <= 0 || headdim <= 0 || d_state <= 0 ||
        mimo_rank <= 0)
        return M3_ERR_INVALID_SHAPE;
    if (!x_g || !B_g || !C || !dt || !A || !D || !x_raw || !dy || !dx_g || !dB_g || !dC ||
        !ddt || !dA || !dD || !dx_raw)
        return M3_ERR_NULL_POINTER;
    const bool beta = x_b != nullptr;
    if ((B_b != nullptr) != beta || (dx_b != nullptr) != beta || (dB_b != nullptr) != beta)
        return M3_ERR_NULL_POINTER;
    if (!m3::chunked_bwd_shape_ok(batch, seqlen, nheads, headdim, d_state, mimo_rank, beta))
        return M3_ERR_UNSUPPORTED;
    const size_t need =
        m3::chunked_bwd_workspace(batch, seqlen, nheads, headdim, d_state, mimo_rank, beta);
    if (!workspace || workspace_bytes < need) return M3_ERR_WORKSPACE;
    if (!aligned(workspace, 256)) return M3_ERR_MISALIGNED;
    return m3::launch_chunked_bwd(batch, seqlen, nheads, headdim, d_state, mimo_rank, x_g, x_b,
                                  B_g, B_b, C, dt, A, D, x_raw, h_init, dy, dh_final, dx_g, dx_b,
                                  dB_g, dB_b, dC, ddt, dA, dD, dx_raw, dh_init, workspace,
                                  as_stream(stream)) == 0
               ? M3_OK
               : M3_ERR_LAUNCH;
}

}  // extern "C"
