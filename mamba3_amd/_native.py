"""ctypes binding of `lib/libmamba3_amd.so` (C-ABI declared in include/mamba3_amd.h).

PyTorch supplies device memory and the current HIP stream; every compute call goes
through the native library. There is no CPU or eager fallback: a CPU tensor or a
missing library raises.
"""

from __future__ import annotations

import ctypes
import threading
from pathlib import Path

import torch

LIB_PATH = Path(__file__).resolve().parent / "lib" / "libmamba3_amd.so"

M3_DTYPE_F32 = 0
M3_DTYPE_BF16 = 1

_DTYPE_CODE = {torch.float32: M3_DTYPE_F32, torch.bfloat16: M3_DTYPE_BF16}

# Exported symbols, kept in step with include/mamba3_amd.h.
EXPORTED_SYMBOLS = (
    "m3_status_string",
    "m3_version",
    "m3_scan_fwd",
    "m3_scan_bwd_workspace_size",
    "m3_scan_bwd",
    "m3_prefill_workspace_size",
    "m3_prefill_fwd",
    "m3_step_fwd",
    "m3_chunked_ssd_fwd",
    "m3_chunked_ssd_fwd_workspace_size",
    "m3_chunked_ssd_bwd_workspace_size",
    "m3_chunked_ssd_bwd",
    "m3_layer_bwd_workspace_size",
    "m3_layer_bwd",
    "m3_prefill_fwd_noalloc",
    "m3_rmsnorm_fwd",
    "m3_rmsnorm_bwd_workspace_size",
    "m3_rmsnorm_bwd",
    "m3_small_linear",
    "m3_small_swiglu",
    "m3_silu_mul",
    "m3_step_bwd_workspace_size",
    "m3_step_bwd",
    "m3_prefill_kernel_name",
)

M3_ERR_UNSUPPORTED = 3
M3_ERR_SCRATCH_LIMIT = 8
NOALLOC_SCRATCH_BYTES = 64 << 20


class NativeError(RuntimeError):
    """A native entry point returned a non-zero m3_status."""


class LayerDesc(ctypes.Structure):
    _fields_ = [
        ("batch", ctypes.c_int32),
        ("seqlen", ctypes.c_int32),
        ("nheads", ctypes.c_int32),
        ("headdim", ctypes.c_int32),
        ("d_state", ctypes.c_int32),
        ("mimo_rank", ctypes.c_int32),
        ("ngroups", ctypes.c_int32),
        ("use_trapezoidal", ctypes.c_int32),
        ("use_complex", ctypes.c_int32),
        ("dtype", ctypes.c_int32),
        ("proj_row_stride", ctypes.c_int64),
        ("rms_eps", ctypes.c_float),
        ("flags", ctypes.c_int32),
    ]


M3_FLAG_NO_F16_OPERANDS = 1
M3_FLAG_FOR_BACKWARD = 2


class LayerParams(ctypes.Structure):
    _fields_ = [(name, ctypes.c_void_p) for name in (
        "A_log", "D", "dt_bias", "B_norm_w", "C_norm_w", "B_bias", "C_bias",
        "mimo_x", "mimo_z", "mimo_down")]


class LayerParamGrads(ctypes.Structure):
    _fields_ = LayerParams._fields_ + [("dt_scale", ctypes.c_void_p)]


_lib = None
_lib_lock = threading.Lock()

_vp = ctypes.c_void_p
_i32 = ctypes.c_int32
_i64 = ctypes.c_int64


def _declare(lib: ctypes.CDLL) -> None:
    lib.m3_status_string.restype = ctypes.c_char_p
    lib.m3_status_string.argtypes = [ctypes.c_int]
    lib.m3_version.restype = ctypes.c_int
    lib.m3_version.argtypes = []
    lib.m3_scan_fwd.restype = ctypes.c_int
    lib.m3_scan_fwd.argtypes = [_vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _vp]
    lib.m3_scan_bwd_workspace_size.restype = ctypes.c_int
    lib.m3_scan_bwd_workspace_size.argtypes = [_i64, _i64, _i64, _i64, ctypes.POINTER(ctypes.c_size_t)]
    lib.m3_scan_bwd.restype = ctypes.c_int
    lib.m3_scan_bwd.argtypes = [_vp, _vp, _vp, _vp, _vp, _vp, _vp, ctypes.c_size_t,
                                _i64, _i64, _i64, _i64, _vp]
    lib.m3_prefill_kernel_name.restype = ctypes.c_char_p
    lib.m3_prefill_kernel_name.argtypes = [ctypes.POINTER(LayerDesc), _vp, _vp, _vp, _vp]
    lib.m3_prefill_workspace_size.restype = ctypes.c_int
    lib.m3_prefill_workspace_size.argtypes = [ctypes.POINTER(LayerDesc),
                                              ctypes.POINTER(ctypes.c_size_t)]
    lib.m3_prefill_fwd.restype = ctypes.c_int
    lib.m3_prefill_fwd.argtypes = [ctypes.POINTER(LayerDesc), ctypes.POINTER(LayerParams),
                                   _vp, _vp, _vp, _vp, _vp, _vp, _vp, ctypes.c_size_t, _vp]
    lib.m3_prefill_fwd_noalloc.restype = ctypes.c_int
    lib.m3_prefill_fwd_noalloc.argtypes = [ctypes.POINTER(LayerDesc), ctypes.POINTER(LayerParams),
                                           _vp, _vp, _vp, _vp, _vp, _vp, _vp]
    lib.m3_rmsnorm_fwd.restype = ctypes.c_int
    lib.m3_rmsnorm_fwd.argtypes = [_vp, ctypes.c_int, _vp, ctypes.c_int, _vp, ctypes.c_int, _vp,
                                   _i64, _i32, ctypes.c_float, _vp]
    lib.m3_rmsnorm_bwd_workspace_size.restype = ctypes.c_int
    lib.m3_rmsnorm_bwd_workspace_size.argtypes = [_i64, _i32, ctypes.POINTER(ctypes.c_size_t)]
    lib.m3_rmsnorm_bwd.restype = ctypes.c_int
    lib.m3_rmsnorm_bwd.argtypes = [_vp, ctypes.c_int, _vp, ctypes.c_int, _vp, _vp, ctypes.c_int,
                                   _vp, _vp, _vp, ctypes.c_size_t, _i64, _i32, _vp]
    lib.m3_small_linear.restype = ctypes.c_int
    lib.m3_small_linear.argtypes = [_vp, _vp, ctypes.c_float, _vp, _vp, ctypes.c_float, _vp,
                                    _i32, _i32, _i32, _vp]
    lib.m3_silu_mul.restype = ctypes.c_int
    lib.m3_silu_mul.argtypes = [_vp, _i64, _i32, _i64, _vp, _vp]
    lib.m3_small_swiglu.restype = ctypes.c_int
    lib.m3_small_swiglu.argtypes = [_vp, _vp, ctypes.c_float, _vp, _vp, _vp, _i32, _i32, _i32, _vp]
    lib.m3_step_fwd.restype = ctypes.c_int
    lib.m3_step_fwd.argtypes = [ctypes.POINTER(LayerDesc), ctypes.POINTER(LayerParams),
                                _vp, _vp, _vp, _vp, _vp, ctypes.c_int, _vp, _vp, _vp, _vp, _vp]
    lib.m3_chunked_ssd_fwd.restype = ctypes.c_int
    lib.m3_chunked_ssd_fwd.argtypes = [_i32, _i32, _i32, _i32, _i32, _i32, _i32,
                                       _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                                       _vp, _vp, _vp, _vp, ctypes.c_size_t, _vp]
    lib.m3_chunked_ssd_fwd_workspace_size.restype = ctypes.c_int
    lib.m3_chunked_ssd_fwd_workspace_size.argtypes = [_i32] * 8 + [ctypes.POINTER(ctypes.c_size_t)]
    lib.m3_layer_bwd_workspace_size.restype = ctypes.c_int
    lib.m3_layer_bwd_workspace_size.argtypes = [ctypes.POINTER(LayerDesc), ctypes.POINTER(ctypes.c_size_t)]
    lib.m3_layer_bwd.restype = ctypes.c_int
    lib.m3_layer_bwd.argtypes = ([ctypes.POINTER(LayerDesc), ctypes.POINTER(LayerParams)]
                                 + [_vp] * 3 + [ctypes.c_size_t] + [_vp] * 5
                                 + [ctypes.POINTER(LayerParamGrads), _vp, ctypes.c_size_t, _vp])
    lib.m3_step_bwd_workspace_size.restype = ctypes.c_int
    lib.m3_step_bwd_workspace_size.argtypes = [ctypes.POINTER(LayerDesc), ctypes.POINTER(ctypes.c_size_t)]
    lib.m3_step_bwd.restype = ctypes.c_int
    lib.m3_step_bwd.argtypes = ([ctypes.POINTER(LayerDesc), ctypes.POINTER(LayerParams)]
                                + [_vp] * 13
                                + [ctypes.POINTER(LayerParamGrads), _vp, ctypes.c_size_t, _vp])
    lib.m3_chunked_ssd_bwd_workspace_size.restype = ctypes.c_int
    lib.m3_chunked_ssd_bwd_workspace_size.argtypes = [_i32] * 7 + [ctypes.POINTER(ctypes.c_size_t)]
    lib.m3_chunked_ssd_bwd.restype = ctypes.c_int
    lib.m3_chunked_ssd_bwd.argtypes = [_i32] * 6 + [_vp] * 23 + [ctypes.c_size_t, _vp]


def lib() -> ctypes.CDLL:
    """Load the native library (once). Raises if it has not been built."""
    global _lib
    if _lib is None:
        with _lib_lock:
            if _lib is None:
                if not LIB_PATH.exists():
                    raise RuntimeError(
                        f"mamba3_amd native library not found at {LIB_PATH}; "
                        "build it with `python -m mamba3_amd.build`")
                handle = ctypes.CDLL(str(LIB_PATH))
                _declare(handle)
                _lib = handle
    return _lib


def check(status: int, what: str) -> None:
    if status != 0:
        msg = lib().m3_status_string(status).decode()
        raise NativeError(f"{what}: {msg} (m3_status {status})")


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return _DTYPE_CODE[dtype]
    except KeyError:
        raise TypeError(f"mamba3_amd kernels support float32 and bfloat16, got {dtype}") from None


def require_gpu(*tensors: torch.Tensor) -> None:
    for t in tensors:
        if t is not None and not t.is_cuda:
            raise RuntimeError(
                "mamba3_amd runs its SSD path only as HIP kernels on an AMD GPU; "
                f"got a tensor on {t.device}. Move the module and inputs to the GPU.")


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def stream_of(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def scan_fwd(decay: torch.Tensor, h_chunk: torch.Tensor, h_init: torch.Tensor | None,
             out: torch.Tensor) -> None:
    B, K, H, PN = h_chunk.shape
    check(lib().m3_scan_fwd(ptr(decay), ptr(h_chunk), ptr(h_init), ptr(out), B, K, H, PN,
                            stream_of(h_chunk)), "m3_scan_fwd")


def scan_bwd(decay: torch.Tensor, h_states: torch.Tensor, grad: torch.Tensor,
             d_decay: torch.Tensor, d_chunk: torch.Tensor, d_h_init: torch.Tensor | None) -> None:
    """m3_scan_bwd on contiguous fp32 tensors (B,K,H) / (B,K,H,PN) / (B,H,PN)."""
    B, K, H, PN = h_states.shape
    n = ctypes.c_size_t(0)
    check(lib().m3_scan_bwd_workspace_size(B, K, H, PN, ctypes.byref(n)), "m3_scan_bwd_workspace_size")
    ws = torch.empty(max(n.value, 1), dtype=torch.uint8, device=h_states.device)
    check(lib().m3_scan_bwd(ptr(decay), ptr(h_states), ptr(grad), ptr(d_decay), ptr(d_chunk),
                            ptr(d_h_init), ptr(ws), n.value, B, K, H, PN, stream_of(h_states)),
          "m3_scan_bwd")


def prefill_workspace_bytes(desc: LayerDesc) -> int:
    n = ctypes.c_size_t(0)
    check(lib().m3_prefill_workspace_size(ctypes.byref(desc), ctypes.byref(n)),
          "m3_prefill_workspace_size")
    return n.value


def prefill_kernel_name(desc: LayerDesc, proj=None, y_out=None, h_final=None, prev_bx=None) -> str:
    """Name of the prefill kernel m3_prefill_fwd runs for these arguments."""
    name = lib().m3_prefill_kernel_name(ctypes.byref(desc), ptr(proj), ptr(y_out), ptr(h_final),
                                        ptr(prev_bx))
    if name is None:
        raise NativeError("m3_prefill_kernel_name: invalid layer descriptor")
    return name.decode()


def prefill_fwd(desc: LayerDesc, params: LayerParams, proj, dt_scale, y_out, h_final, angle,
                prev_bx, workspace, workspace_bytes: int) -> None:
    check(lib().m3_prefill_fwd(ctypes.byref(desc), ctypes.byref(params), ptr(proj),
                               ptr(dt_scale), ptr(y_out), ptr(h_final), ptr(angle),
                               ptr(prev_bx), ptr(workspace), workspace_bytes,
                               stream_of(proj)), "m3_prefill_fwd")


def prefill_fwd_noalloc(desc: LayerDesc, params: LayerParams, proj, dt_scale, y_out, h_final,
                        angle, prev_bx) -> None:
    """m3_prefill_fwd_noalloc: m3_prefill_fwd on the library's static per-device scratch."""
    check(lib().m3_prefill_fwd_noalloc(ctypes.byref(desc), ctypes.byref(params), ptr(proj),
                                       ptr(dt_scale), ptr(y_out), ptr(h_final), ptr(angle),
                                       ptr(prev_bx), stream_of(proj)), "m3_prefill_fwd_noalloc")


def step_fwd(desc: LayerDesc, params: LayerParams, proj, dt_scale, h_in, prev_in, angle_in,
             y_out, h_out, prev_out, angle_out) -> None:
    check(lib().m3_step_fwd(ctypes.byref(desc), ctypes.byref(params), ptr(proj),
                            ptr(dt_scale), ptr(h_in), ptr(prev_in), ptr(angle_in),
                            dtype_code(angle_in.dtype), ptr(y_out), ptr(h_out), ptr(prev_out),
                            ptr(angle_out), stream_of(proj)), "m3_step_fwd")


def chunked_fwd_mfma_applies(B, T, H, P, N, R, has_beta: bool) -> bool:
    """True when m3_chunked_ssd_fwd runs fp32 inputs of this shape on its fp32-MFMA path."""
    n = ctypes.c_size_t(0)
    check(lib().m3_chunked_ssd_fwd_workspace_size(B, T, H, P, N, R, 0, int(has_beta),
                                                  ctypes.byref(n)),
          "m3_chunked_ssd_fwd_workspace_size")
    return n.value > 0


def chunked_fwd(B, T, H, P, N, R, dtype, x_g, x_b, B_g, B_b, C, dt, A, D, x_raw, h_init, y,
                h_final, state_ws, use_workspace: bool = True) -> None:
    """m3_chunked_ssd_fwd; allocates the workspace of the fp32-MFMA path when it applies
    (use_workspace=False runs the generic kernel)."""
    n = ctypes.c_size_t(0)
    check(lib().m3_chunked_ssd_fwd_workspace_size(B, T, H, P, N, R, dtype_code(dtype),
                                                  int(x_b is not None), ctypes.byref(n)),
          "m3_chunked_ssd_fwd_workspace_size")
    if not use_workspace:
        n.value = 0
    ws = torch.empty(n.value, dtype=torch.uint8, device=x_g.device) if n.value else None
    check(lib().m3_chunked_ssd_fwd(B, T, H, P, N, R, dtype_code(dtype), ptr(x_g), ptr(x_b),
                                   ptr(B_g), ptr(B_b), ptr(C), ptr(dt), ptr(A), ptr(D),
                                   ptr(x_raw), ptr(h_init), ptr(y), ptr(h_final),
                                   ptr(state_ws), ptr(ws), n.value, stream_of(x_g)),
          "m3_chunked_ssd_fwd")


def chunked_bwd_workspace_bytes(B, T, H, P, N, R, has_beta: bool) -> int:
    n = ctypes.c_size_t(0)
    check(lib().m3_chunked_ssd_bwd_workspace_size(B, T, H, P, N, R, int(has_beta), ctypes.byref(n)),
          "m3_chunked_ssd_bwd_workspace_size")
    return n.value


def chunked_bwd(B, T, H, P, N, R, x_g, x_b, B_g, B_b, C, dt, A, D, x_raw, h_init, dy, dh_final,
                dx_g, dx_b, dB_g, dB_b, dC, ddt, dA, dD, dx_raw, dh_init) -> None:
    """m3_chunked_ssd_bwd on contiguous fp32 tensors; allocates the workspace."""
    n = chunked_bwd_workspace_bytes(B, T, H, P, N, R, x_b is not None)
    ws = torch.empty(max(n, 1), dtype=torch.uint8, device=x_g.device)
    check(lib().m3_chunked_ssd_bwd(B, T, H, P, N, R, ptr(x_g), ptr(x_b), ptr(B_g), ptr(B_b),
                                   ptr(C), ptr(dt), ptr(A), ptr(D), ptr(x_raw), ptr(h_init),
                                   ptr(dy), ptr(dh_final), ptr(dx_g), ptr(dx_b), ptr(dB_g),
                                   ptr(dB_b), ptr(dC), ptr(ddt), ptr(dA), ptr(dD), ptr(dx_raw),
                                   ptr(dh_init), ptr(ws), n, stream_of(x_g)),
          "m3_chunked_ssd_bwd")


def layer_bwd_supported(desc: LayerDesc) -> bool:
    """True when m3_layer_bwd covers this (fp32) layer shape."""
    n = ctypes.c_size_t(0)
    st = lib().m3_layer_bwd_workspace_size(ctypes.byref(desc), ctypes.byref(n))
    return st == 0 and n.value > 0


def layer_bwd_workspace_bytes(desc: LayerDesc) -> int:
    n = ctypes.c_size_t(0)
    check(lib().m3_layer_bwd_workspace_size(ctypes.byref(desc), ctypes.byref(n)),
          "m3_layer_bwd_workspace_size")
    return n.value


def layer_bwd(desc: LayerDesc, params: LayerParams, proj, dt_scale, fwd_ws, g_out, g_h, g_angle,
              g_prev, g_proj, grads: LayerParamGrads) -> None:
    """m3_layer_bwd; allocates its workspace."""
    n = layer_bwd_workspace_bytes(desc)
    ws = torch.empty(n, dtype=torch.uint8, device=proj.device)
    check(lib().m3_layer_bwd(ctypes.byref(desc), ctypes.byref(params), ptr(proj), ptr(dt_scale),
                             ptr(fwd_ws), fwd_ws.numel(), ptr(g_out), ptr(g_h), ptr(g_angle),
                             ptr(g_prev), ptr(g_proj), ctypes.byref(grads), ptr(ws), n,
                             stream_of(proj)),
          "m3_layer_bwd")


def step_bwd_supported(desc: LayerDesc) -> bool:
    """True when m3_step_bwd covers this (fp32) layer shape."""
    n = ctypes.c_size_t(0)
    st = lib().m3_step_bwd_workspace_size(ctypes.byref(desc), ctypes.byref(n))
    return st == 0 and n.value > 0


def step_bwd(desc: LayerDesc, params: LayerParams, proj, dt_scale, h_in, prev_in, angle_in, g_y,
             g_h, g_prev, g_angle, g_proj, g_h_in, g_prev_in, g_angle_in,
             grads: LayerParamGrads) -> None:
    """m3_step_bwd; allocates its workspace."""
    n = ctypes.c_size_t(0)
    check(lib().m3_step_bwd_workspace_size(ctypes.byref(desc), ctypes.byref(n)),
          "m3_step_bwd_workspace_size")
    ws = torch.empty(n.value, dtype=torch.uint8, device=proj.device)
    check(lib().m3_step_bwd(ctypes.byref(desc), ctypes.byref(params), ptr(proj), ptr(dt_scale),
                            ptr(h_in), ptr(prev_in), ptr(angle_in), ptr(g_y), ptr(g_h),
                            ptr(g_prev), ptr(g_angle), ptr(g_proj), ptr(g_h_in), ptr(g_prev_in),
                            ptr(g_angle_in), ctypes.byref(grads), ptr(ws), n.value,
                            stream_of(proj)),
          "m3_step_bwd")


def rmsnorm_fwd(x, weight, y, rstd, eps: float) -> None:
    """m3_rmsnorm_fwd on contiguous x (rows, d)."""
    rows, d = x.shape
    check(lib().m3_rmsnorm_fwd(ptr(x), dtype_code(x.dtype), ptr(weight), dtype_code(weight.dtype),
                               ptr(y), dtype_code(y.dtype), ptr(rstd), rows, d, eps,
                               stream_of(x)), "m3_rmsnorm_fwd")


SMALL_PROJ_MAX_ROWS = 8


def small_proj_ok(m: int, k: int, norm: bool = False) -> bool:
    """The shapes m3_small_linear / m3_small_swiglu take: m <= 8 rows, k a multiple of 64
    whose staged rows (m rounded up to 1, 2, 4 or 8) and, with a norm, the norm weight fit
    64 KB of LDS."""
    mm = 1 if m <= 1 else 2 if m <= 2 else 4 if m <= 4 else 8
    need = (mm * k + 8 + (k if norm else 0)) * 2
    return 1 <= m <= SMALL_PROJ_MAX_ROWS and k >= 64 and k % 64 == 0 and need <= 65536


def small_linear(x, norm_w, eps, weight, residual, scale, out) -> None:
    """m3_small_linear on contiguous bf16 x (m, k), weight (n, k), out (m, n)."""
    m, k = x.shape
    check(lib().m3_small_linear(ptr(x), ptr(norm_w), eps, ptr(weight), ptr(residual), scale,
                                ptr(out), m, weight.shape[0], k, stream_of(x)), "m3_small_linear")


def small_swiglu(x, norm_w, eps, w_gate, w_up, out) -> None:
    """m3_small_swiglu on contiguous bf16 x (m, k), weights (n, k), out (m, n)."""
    m, k = x.shape
    check(lib().m3_small_swiglu(ptr(x), ptr(norm_w), eps, ptr(w_gate), ptr(w_up), ptr(out), m,
                                w_gate.shape[0], k, stream_of(x)), "m3_small_swiglu")


def silu_mul(gate_up, d_ff, out) -> None:
    """m3_silu_mul on bf16 gate_up (rows, >= 2 d_ff) with unit column stride."""
    check(lib().m3_silu_mul(ptr(gate_up), gate_up.shape[0], d_ff, gate_up.stride(0), ptr(out),
                            stream_of(gate_up)), "m3_silu_mul")


def rmsnorm_bwd(x, weight, rstd, grad, dx, dweight) -> None:
    """m3_rmsnorm_bwd on contiguous (rows, d) tensors; allocates the workspace."""
    rows, d = x.shape
    n = ctypes.c_size_t(0)
    check(lib().m3_rmsnorm_bwd_workspace_size(rows, d, ctypes.byref(n)), "m3_rmsnorm_bwd_workspace_size")
    ws = torch.empty(max(n.value, 1), dtype=torch.uint8, device=x.device)
    check(lib().m3_rmsnorm_bwd(ptr(x), dtype_code(x.dtype), ptr(weight), dtype_code(weight.dtype),
                               ptr(rstd), ptr(grad), dtype_code(grad.dtype), ptr(dx), ptr(dweight),
                               ptr(ws), n.value, rows, d, stream_of(x)), "m3_rmsnorm_bwd")
