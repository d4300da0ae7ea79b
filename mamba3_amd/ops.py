"""torch.library custom ops over the C-ABI library (include/mamba3_amd.h).

Every native entry point the Python API uses is a registered op in the `mamba3_amd`
namespace with a fake (meta) kernel, and the differentiable ones with an autograd
formula, so that `torch.compile(fullgraph=True)` traces a KulaMamba layer, `chunked_ssd`
and `ssd_scan` without graph breaks, forward and backward (the reference keeps the same
property, mamba3/scan.py:5, tests/test_mamba3.py:584-616). The op bodies allocate
outputs and workspace with the caching allocator, take the current stream and call the
library through ctypes (`_native`); no op has a CPU or eager fallback.

Layer ops take the layer's shape as plain integers and its ten small parameters as
tensors in the order (A_log, D, dt_bias, B_norm.weight, C_norm.weight, B_bias, C_bias,
mimo_x, mimo_z, mimo_down); the kernels read fp32 copies of them, which are cached per
source tensor and version.
"""

from __future__ import annotations

import weakref
from collections import OrderedDict
from typing import Optional

import torch

from . import _native

NS = "mamba3_amd"

# ---------------------------------------------------------------------------- helpers
_F32_CACHE: "OrderedDict[tuple, list]" = OrderedDict()
_F32_CACHE_MAX = 256

def _cache_entry(params) -> list:
    """[LayerParams, fp32 tensors, weak refs] for the ten layer parameters. An entry is
    used only while every source tensor is the same live object at the same version."""
    key = tuple((t.data_ptr(), t._version, t.dtype, t.device) for t in params)
    hit = _F32_CACHE.get(key)
    if hit is not None and all(r() is t for r, t in zip(hit[2], params)):
        _F32_CACHE.move_to_end(key)
        return hit
    with torch.no_grad():
        f32 = [t.detach().float().contiguous() for t in params]
    entry = [_native.LayerParams(*[t.data_ptr() for t in f32]), f32,
             [weakref.ref(t) for t in params]]
    _F32_CACHE[key] = entry
    while len(_F32_CACHE) > _F32_CACHE_MAX:
        _F32_CACHE.popitem(last=False)
    return entry


def _f32_params(params) -> tuple:
    """(LayerParams, fp32 tensors) for the ten layer parameters (cached)."""
    entry = _cache_entry(params)
    return entry[0], entry[1]


def _desc(batch, seqlen, nheads, headdim, d_state, mimo_rank, ngroups, trap, cplx, eps,
          dtype, row_stride) -> _native.LayerDesc:
    return _native.LayerDesc(
        batch=batch, seqlen=seqlen, nheads=nheads, headdim=headdim, d_state=d_state,
        mimo_rank=mimo_rank, ngroups=ngroups, use_trapezoidal=int(trap), use_complex=int(cplx),
        dtype=_native.dtype_code(dtype), proj_row_stride=row_stride, rms_eps=float(eps))


def _state_shapes(B, nheads, headdim, d_state):
    return (B, nheads, headdim, d_state), (B, nheads, d_state // 2)


# ---------------------------------------------------------------------------- prefill
@torch.library.custom_op(f"{NS}::prefill", mutates_args=())
def prefill(proj: torch.Tensor, A_log: torch.Tensor, D: torch.Tensor, dt_bias: torch.Tensor,
            B_norm_w: torch.Tensor, C_norm_w: torch.Tensor, B_bias: torch.Tensor,
            C_bias: torch.Tensor, mimo_x: torch.Tensor, mimo_z: torch.Tensor,
            mimo_down: torch.Tensor, dt_scale: Optional[torch.Tensor], nheads: int,
            headdim: int, d_state: int, mimo_rank: int, ngroups: int, trap: bool, cplx: bool,
            eps: float, return_state: bool) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor,
                                                     torch.Tensor]:
    """m3_prefill_fwd: in_proj output (B,T,W) -> (y (B,T,H*P) in proj.dtype, h, angle,
    prev_BX). Without return_state the three state tensors are empty."""
    _native.require_gpu(proj)
    proj = proj.contiguous()
    Bat, T, _ = proj.shape
    desc = _desc(Bat, T, nheads, headdim, d_state, mimo_rank, ngroups, trap, cplx, eps,
                 proj.dtype, proj.stride(-2))
    params = (A_log, D, dt_bias, B_norm_w, C_norm_w, B_bias, C_bias, mimo_x, mimo_z, mimo_down)
    pack, _ = _f32_params(params)
    dev = proj.device
    y = torch.empty(Bat, T, nheads * headdim, device=dev, dtype=proj.dtype)
    if return_state:
        hs, as_ = _state_shapes(Bat, nheads, headdim, d_state)
        h = torch.empty(hs, device=dev, dtype=torch.float32)
        angle = torch.empty(as_, device=dev, dtype=torch.float32)
        prev = torch.empty(hs, device=dev, dtype=torch.float32)
    else:
        h = angle = prev = None
    ws_bytes = _native.prefill_workspace_bytes(desc)
    ws = torch.empty(max(ws_bytes, 1), device=dev, dtype=torch.uint8)
    _native.prefill_fwd(desc, pack, proj, dt_scale, y, h, angle, prev, ws, ws_bytes)
    if not return_state:  # three distinct empty tensors: outputs of an op may not alias
        h, angle, prev = (torch.empty(0, device=dev, dtype=torch.float32) for _ in range(3))
    return y, h, angle, prev


@prefill.register_fake
def _(proj, A_log, D, dt_bias, B_norm_w, C_norm_w, B_bias, C_bias, mimo_x, mimo_z, mimo_down,
      dt_scale, nheads, headdim, d_state, mimo_rank, ngroups, trap, cplx, eps, return_state):
    Bat, T, _ = proj.shape
    y = proj.new_empty(Bat, T, nheads * headdim)
    if not return_state:
        e = proj.new_empty(0, dtype=torch.float32)
        return y, e, e.clone(), e.clone()
    hs, as_ = _state_shapes(Bat, nheads, headdim, d_state)
    return (y, proj.new_empty(hs, dtype=torch.float32), proj.new_empty(as_, dtype=torch.float32),
            proj.new_empty(hs, dtype=torch.float32))


# ------------------------------------------------------------ prefill for training
def _train_desc(proj, nheads, headdim, d_state, mimo_rank, ngroups, trap, cplx, eps):
    """fp32 descriptor of the training forward and of m3_layer_bwd: the forward keeps the
    intermediates the backward reads (M3_FLAG_FOR_BACKWARD)."""
    Bat, T, W = proj.shape
    desc = _desc(Bat, T, nheads, headdim, d_state, mimo_rank, ngroups, trap, cplx, eps,
                 torch.float32, W)
    desc.flags |= _native.M3_FLAG_FOR_BACKWARD
    return desc


@torch.library.custom_op(f"{NS}::prefill_train", mutates_args=())
def prefill_train(proj: torch.Tensor, A_log: torch.Tensor, D: torch.Tensor,
                  dt_bias: torch.Tensor, B_norm_w: torch.Tensor, C_norm_w: torch.Tensor,
                  B_bias: torch.Tensor, C_bias: torch.Tensor, mimo_x: torch.Tensor,
                  mimo_z: torch.Tensor, mimo_down: torch.Tensor,
                  dt_scale: Optional[torch.Tensor], nheads: int, headdim: int, d_state: int,
                  mimo_rank: int, ngroups: int, trap: bool, cplx: bool,
                  eps: float) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor,
                                       torch.Tensor]:
    """The prefill in fp32 arithmetic (bf16 inputs upcast) on the fp32 layer path, whose
    workspace (last output) holds the activations m3_layer_bwd differentiates through.
    Raises for shapes m3_layer_bwd does not cover."""
    _native.require_gpu(proj)
    proj32 = proj.detach().float().contiguous()
    desc = _train_desc(proj32, nheads, headdim, d_state, mimo_rank, ngroups, trap, cplx, eps)
    if not _native.layer_bwd_supported(desc):
        raise _native.NativeError(
            f"training through KulaMamba(d_state={d_state}, headdim={headdim}, "
            f"mimo_rank={mimo_rank}, ngroups={ngroups}) is not supported by m3_layer_bwd "
            "(the rank exceeds 8 or the shape exceeds the kernels' limits); "
            "run this layer without gradients")
    pack, _ = _f32_params((A_log, D, dt_bias, B_norm_w, C_norm_w, B_bias, C_bias, mimo_x,
                           mimo_z, mimo_down))
    Bat, T, _ = proj32.shape
    dev = proj.device
    ws_bytes = _native.prefill_workspace_bytes(desc)
    ws = torch.empty(max(ws_bytes, 1), device=dev, dtype=torch.uint8)
    y = torch.empty(Bat, T, nheads * headdim, device=dev, dtype=torch.float32)
    hs, as_ = _state_shapes(Bat, nheads, headdim, d_state)
    h = torch.empty(hs, device=dev, dtype=torch.float32)
    angle = torch.empty(as_, device=dev, dtype=torch.float32)
    prev = torch.empty(hs, device=dev, dtype=torch.float32)
    _native.prefill_fwd(desc, pack, proj32, dt_scale, y, h, angle, prev, ws, ws_bytes)
    return y.to(proj.dtype), h, angle, prev, ws


def _train_ws_bytes(proj, nheads, headdim, d_state, mimo_rank, ngroups, trap, cplx, eps) -> int:
    desc = _train_desc(proj, nheads, headdim, d_state, mimo_rank, ngroups, trap, cplx, eps)
    return max(_native.prefill_workspace_bytes(desc), 1)


@prefill_train.register_fake
def _(proj, A_log, D, dt_bias, B_norm_w, C_norm_w, B_bias, C_bias, mimo_x, mimo_z, mimo_down,
      dt_scale, nheads, headdim, d_state, mimo_rank, ngroups, trap, cplx, eps):
    Bat, T, _ = proj.shape
    hs, as_ = _state_shapes(Bat, nheads, headdim, d_state)
    n = _train_ws_bytes(proj, nheads, headdim, d_state, mimo_rank, ngroups, trap, cplx, eps)
    return (proj.new_empty(Bat, T, nheads * headdim), proj.new_empty(hs, dtype=torch.float32),
            proj.new_empty(as_, dtype=torch.float32), proj.new_empty(hs, dtype=torch.float32),
            proj.new_empty(n, dtype=torch.uint8))


@torch.library.custom_op(f"{NS}::layer_bwd", mutates_args=())
def layer_bwd(proj: torch.Tensor, A_log: torch.Tensor, D: torch.Tensor, dt_bias: torch.Tensor,
              B_norm_w: torch.Tensor, C_norm_w: torch.Tensor, B_bias: torch.Tensor,
              C_bias: torch.Tensor, mimo_x: torch.Tensor, mimo_z: torch.Tensor,
              mimo_down: torch.Tensor, dt_scale: Optional[torch.Tensor], fwd_ws: torch.Tensor,
              g_y: torch.Tensor, g_h: Optional[torch.Tensor], g_angle: Optional[torch.Tensor],
              g_prev: Optional[torch.Tensor], nheads: int, headdim: int, d_state: int,
              mimo_rank: int, ngroups: int, trap: bool, cplx: bool,
              eps: float) -> list[torch.Tensor]:
    """m3_layer_bwd: gradients of prefill_train's outputs with respect to proj (fp32), the
    ten parameters (fp32, their shapes) and dt_scale (fp32 (B,T,H); zeros when dt_scale
    is None)."""
    proj32 = proj.detach().float().contiguous()
    desc = _train_desc(proj32, nheads, headdim, d_state, mimo_rank, ngroups, trap, cplx, eps)
    params = (A_log, D, dt_bias, B_norm_w, C_norm_w, B_bias, C_bias, mimo_x, mimo_z, mimo_down)
    pack, f32 = _f32_params(params)

    def f32c(t):
        return None if t is None else t.float().contiguous()

    g_proj = torch.empty_like(proj32)
    grads = [torch.empty_like(t) for t in f32]
    Bat, T, _ = proj32.shape
    g_dts = torch.zeros(Bat, T, nheads, device=proj.device, dtype=torch.float32)
    _native.layer_bwd(desc, pack, proj32, dt_scale, fwd_ws, f32c(g_y), f32c(g_h), f32c(g_angle),
                      f32c(g_prev), g_proj,
                      _native.LayerParamGrads(*[t.data_ptr() for t in grads],
                                              g_dts.data_ptr() if dt_scale is not None else None))
    return [g_proj, *grads, g_dts]


@layer_bwd.register_fake
def _(proj, A_log, D, dt_bias, B_norm_w, C_norm_w, B_bias, C_bias, mimo_x, mimo_z, mimo_down,
      dt_scale, fwd_ws, g_y, g_h, g_angle, g_prev, nheads, headdim, d_state, mimo_rank, ngroups,
      trap, cplx, eps):
    params = (A_log, D, dt_bias, B_norm_w, C_norm_w, B_bias, C_bias, mimo_x, mimo_z, mimo_down)
    Bat, T, _ = proj.shape
    return [proj.new_empty(proj.shape, dtype=torch.float32),
            *[t.new_empty(t.shape, dtype=torch.float32) for t in params],
            proj.new_empty(Bat, T, nheads, dtype=torch.float32)]


def _prefill_train_setup(ctx, inputs, output):
    *tensors, dt_scale, nheads, headdim, d_state, mimo_rank, ngroups, trap, cplx, eps = inputs
    ctx.cfg = (nheads, headdim, d_state, mimo_rank, ngroups, trap, cplx, eps)
    ctx.has_scale = dt_scale is not None
    ctx.save_for_backward(*tensors, dt_scale, output[4])
    ctx.set_materialize_grads(False)


def _prefill_train_backward(ctx, g_y, g_h, g_angle, g_prev, g_ws):
    *tensors, dt_scale, ws = ctx.saved_tensors
    proj, params = tensors[0], tensors[1:]
    if g_y is None:
        g_y = proj.new_zeros(proj.shape[0], proj.shape[1], ctx.cfg[0] * ctx.cfg[1],
                             dtype=torch.float32)
    out = layer_bwd(proj, *params, dt_scale, ws, g_y, g_h, g_angle, g_prev, *ctx.cfg)
    g_proj, g_params, g_dts = out[0], out[1:11], out[11]
    grads = [g_proj.to(proj.dtype)] + [g.to(p.dtype) for g, p in zip(g_params, params)]
    grads.append(g_dts if ctx.has_scale else None)
    return (*grads, None, None, None, None, None, None, None, None)


prefill_train.register_autograd(_prefill_train_backward, setup_context=_prefill_train_setup)


# ---------------------------------------------------------------------------- step
def _step_eager(proj: torch.Tensor, A_log: torch.Tensor, D: torch.Tensor, dt_bias: torch.Tensor,
         B_norm_w: torch.Tensor, C_norm_w: torch.Tensor, B_bias: torch.Tensor,
         C_bias: torch.Tensor, mimo_x: torch.Tensor, mimo_z: torch.Tensor,
         mimo_down: torch.Tensor, dt_scale: Optional[torch.Tensor], h: torch.Tensor,
         prev_bx: torch.Tensor, angle: torch.Tensor, nheads: int, headdim: int, d_state: int,
         mimo_rank: int, ngroups: int, trap: bool, cplx: bool,
         eps: float) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
    """m3_step_fwd on one token per row: proj (B,W) and the state -> (y (B,H*P), new h,
    new prev_BX, new angle). The state comes back in new tensors (h and prev_BX fp32,
    angle in its input dtype). Its autograd formula is m3_step_bwd."""
    out = [torch.empty(proj.shape[0], nheads * headdim, device=proj.device, dtype=proj.dtype),
           torch.empty_like(h, dtype=torch.float32), torch.empty_like(prev_bx, dtype=torch.float32),
           torch.empty_like(angle)]
    step_into(proj, A_log, D, dt_bias, B_norm_w, C_norm_w, B_bias, C_bias, mimo_x, mimo_z,
              mimo_down, dt_scale, h, prev_bx, angle, *out, nheads, headdim, d_state,
              mimo_rank, ngroups, trap, cplx, eps)
    return tuple(out)


step = torch.library.custom_op(f"{NS}::step", _step_eager, mutates_args=())


@step.register_fake
def _(proj, A_log, D, dt_bias, B_norm_w, C_norm_w, B_bias, C_bias, mimo_x, mimo_z, mimo_down,
      dt_scale, h, prev_bx, angle, nheads, headdim, d_state, mimo_rank, ngroups, trap, cplx, eps):
    return (proj.new_empty(proj.shape[0], nheads * headdim), h.new_empty(h.shape, dtype=torch.float32),
            prev_bx.new_empty(prev_bx.shape, dtype=torch.float32), angle.new_empty(angle.shape))


@torch.library.custom_op(f"{NS}::step_bwd", mutates_args=())
def step_bwd(proj: torch.Tensor, A_log: torch.Tensor, D: torch.Tensor, dt_bias: torch.Tensor,
             B_norm_w: torch.Tensor, C_norm_w: torch.Tensor, B_bias: torch.Tensor,
             C_bias: torch.Tensor, mimo_x: torch.Tensor, mimo_z: torch.Tensor,
             mimo_down: torch.Tensor, dt_scale: Optional[torch.Tensor], h: torch.Tensor,
             prev_bx: torch.Tensor, angle: torch.Tensor, g_y: torch.Tensor,
             g_h: Optional[torch.Tensor], g_prev: Optional[torch.Tensor],
             g_angle: Optional[torch.Tensor], nheads: int, headdim: int, d_state: int,
             mimo_rank: int, ngroups: int, trap: bool, cplx: bool,
             eps: float) -> list[torch.Tensor]:
    """m3_step_bwd: gradients of step's outputs with respect to proj, the ten parameters,
    dt_scale (zeros when None) and the incoming h, prev_BX and angle, all fp32."""
    proj32 = proj.detach().float().contiguous()
    desc = _desc(proj32.shape[0], 1, nheads, headdim, d_state, mimo_rank, ngroups, trap, cplx,
                 eps, torch.float32, proj32.stride(0))
    if not _native.step_bwd_supported(desc):
        raise _native.NativeError(
            f"KulaMamba.step backward: this shape (d_state={d_state}, headdim={headdim}, "
            f"mimo_rank={mimo_rank}) is not supported by m3_step_bwd")
    params = (A_log, D, dt_bias, B_norm_w, C_norm_w, B_bias, C_bias, mimo_x, mimo_z, mimo_down)
    pack, f32 = _f32_params(params)

    def f32c(t):
        return None if t is None else t.detach().float().contiguous()

    g_proj = torch.zeros_like(proj32)
    grads = [torch.empty_like(t) for t in f32]
    g_dts = torch.zeros(proj32.shape[0], nheads, device=proj.device, dtype=torch.float32)
    h32, prev32, ang32 = f32c(h), f32c(prev_bx), f32c(angle)
    g_h_in, g_prev_in, g_ang_in = (torch.empty_like(h32), torch.empty_like(prev32),
                                   torch.empty_like(ang32))
    _native.step_bwd(desc, pack, proj32, f32c(dt_scale), h32, prev32, ang32, f32c(g_y), f32c(g_h),
                     f32c(g_prev), f32c(g_angle), g_proj, g_h_in, g_prev_in, g_ang_in,
                     _native.LayerParamGrads(*[t.data_ptr() for t in grads],
                                             g_dts.data_ptr() if dt_scale is not None else None))
    return [g_proj, *grads, g_dts, g_h_in, g_prev_in, g_ang_in]


@step_bwd.register_fake
def _(proj, A_log, D, dt_bias, B_norm_w, C_norm_w, B_bias, C_bias, mimo_x, mimo_z, mimo_down,
      dt_scale, h, prev_bx, angle, g_y, g_h, g_prev, g_angle, nheads, headdim, d_state,
      mimo_rank, ngroups, trap, cplx, eps):
    params = (A_log, D, dt_bias, B_norm_w, C_norm_w, B_bias, C_bias, mimo_x, mimo_z, mimo_down)
    f = torch.float32
    return [proj.new_empty(proj.shape, dtype=f), *[t.new_empty(t.shape, dtype=f) for t in params],
            proj.new_empty(proj.shape[0], nheads, dtype=f), h.new_empty(h.shape, dtype=f),
            prev_bx.new_empty(prev_bx.shape, dtype=f), angle.new_empty(angle.shape, dtype=f)]


def _step_setup(ctx, inputs, output):
    ctx.cfg = inputs[15:]
    ctx.has_scale = inputs[11] is not None
    ctx.save_for_backward(*inputs[:15])
    ctx.set_materialize_grads(False)


def _step_backward(ctx, g_y, g_h, g_prev, g_angle):
    proj, *rest = ctx.saved_tensors
    params, dt_scale, h, prev_bx, angle = rest[:10], rest[10], rest[11], rest[12], rest[13]
    if g_y is None:
        g_y = proj.new_zeros(proj.shape[0], ctx.cfg[0] * ctx.cfg[1], dtype=torch.float32)
    out = step_bwd(proj, *params, dt_scale, h, prev_bx, angle, g_y, g_h, g_prev, g_angle,
                   *ctx.cfg)
    g_proj, g_params, g_dts, g_hin, g_pin, g_ain = out[0], out[1:11], out[11], out[12], out[13], out[14]
    grads = [g_proj.to(proj.dtype)] + [g.to(p.dtype) for g, p in zip(g_params, params)]
    grads.append(g_dts if ctx.has_scale else None)
    grads += [g_hin.to(h.dtype), g_pin.to(prev_bx.dtype), g_ain.to(angle.dtype)]
    return (*grads, None, None, None, None, None, None, None, None)


step.register_autograd(_step_backward, setup_context=_step_setup)


def step_into(proj, A_log, D, dt_bias, B_norm_w, C_norm_w, B_bias, C_bias, mimo_x, mimo_z,
              mimo_down, dt_scale, h, prev_bx, angle, y_out, h_out, prev_out, angle_out,
              nheads, headdim, d_state, mimo_rank, ngroups, trap, cplx, eps) -> None:
    """m3_step_fwd into caller-owned outputs (which must not alias the inputs); used by the
    captured decode loop, which alternates two state buffer sets."""
    _native.require_gpu(proj, h, prev_bx, angle)
    proj = proj.contiguous()
    h = h.float().contiguous()
    prev_bx = prev_bx.float().contiguous()
    if angle.dtype not in (torch.float32, torch.bfloat16):
        angle = angle.float()
    angle = angle.contiguous()
    if angle_out.dtype != angle.dtype:
        raise TypeError("angle_out must have the dtype of the input angle")
    desc = _desc(proj.shape[0], 1, nheads, headdim, d_state, mimo_rank, ngroups, trap, cplx, eps,
                 proj.dtype, proj.stride(0))
    pack, _ = _f32_params((A_log, D, dt_bias, B_norm_w, C_norm_w, B_bias, C_bias, mimo_x,
                           mimo_z, mimo_down))
    _native.step_fwd(desc, pack, proj, dt_scale, h, prev_bx, angle, y_out, h_out, prev_out,
                     angle_out)


# ---------------------------------------------------------------------------- scan
@torch.library.custom_op(f"{NS}::scan_fwd", mutates_args=())
def scan_fwd(decay: torch.Tensor, h_chunk: torch.Tensor,
             h_init: Optional[torch.Tensor]) -> torch.Tensor:
    """m3_scan_fwd on fp32 (B,K,H) decay, (B,K,H,PN) h_chunk, (B,H,PN) h_init -> fp32 states."""
    _native.require_gpu(decay, h_chunk, h_init)
    decay = decay.float().contiguous()
    h_chunk = h_chunk.float().contiguous()
    if h_init is not None:
        h_init = h_init.float().contiguous()
    out = torch.empty_like(h_chunk)
    _native.scan_fwd(decay, h_chunk, h_init, out)
    return out


@scan_fwd.register_fake
def _(decay, h_chunk, h_init):
    return h_chunk.new_empty(h_chunk.shape, dtype=torch.float32)


@torch.library.custom_op(f"{NS}::scan_bwd", mutates_args=())
def scan_bwd(decay: torch.Tensor, h_states: torch.Tensor, grad: torch.Tensor,
             with_init: bool) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """m3_scan_bwd -> (d_decay, d_chunk, d_h_init; the last empty without h_init)."""
    decay = decay.float().contiguous()
    grad = grad.float().contiguous()
    B, K, H, PN = h_states.shape
    d_decay = torch.empty_like(decay)
    d_chunk = torch.empty_like(h_states)
    d_init = torch.empty(B, H, PN, dtype=torch.float32, device=h_states.device) if with_init \
        else torch.empty(0, dtype=torch.float32, device=h_states.device)
    _native.scan_bwd(decay, h_states, grad, d_decay, d_chunk, d_init if with_init else None)
    return d_decay, d_chunk, d_init


@scan_bwd.register_fake
def _(decay, h_states, grad, with_init):
    B, K, H, PN = h_states.shape
    return (decay.new_empty(decay.shape, dtype=torch.float32),
            h_states.new_empty(h_states.shape, dtype=torch.float32),
            h_states.new_empty((B, H, PN) if with_init else (0,), dtype=torch.float32))


def _scan_setup(ctx, inputs, output):
    decay, h_chunk, h_init = inputs
    ctx.with_init = h_init is not None
    ctx.save_for_backward(decay, output)


def _scan_backward(ctx, grad):
    decay, states = ctx.saved_tensors
    d_decay, d_chunk, d_init = scan_bwd(decay, states, grad, ctx.with_init)
    return d_decay, d_chunk, (d_init if ctx.with_init else None)


scan_fwd.register_autograd(_scan_backward, setup_context=_scan_setup)


# ---------------------------------------------------------------------------- chunked SSD
@torch.library.custom_op(f"{NS}::chunked_fwd", mutates_args=())
def chunked_fwd(x_g: torch.Tensor, x_b: Optional[torch.Tensor], B_g: torch.Tensor,
                B_b: Optional[torch.Tensor], C: torch.Tensor, dt: torch.Tensor, A: torch.Tensor,
                D: torch.Tensor, x_raw: torch.Tensor,
                h_init: Optional[torch.Tensor]) -> tuple[torch.Tensor, torch.Tensor]:
    """m3_chunked_ssd_fwd: (y (B,T,H,P,R) in x_g.dtype, h_final (B,H,P,N) fp32). bf16 inputs
    of shapes the fp32-MFMA chunk kernels cover run on them in fp32 arithmetic."""
    Bat, T, H, P, R = x_g.shape
    N = B_g.shape[3]
    dtype = x_g.dtype
    calc = dtype
    if dtype != torch.float32 and _native.chunked_fwd_mfma_applies(Bat, T, H, P, N, R,
                                                                   x_b is not None):
        calc = torch.float32

    def prep(t):
        return None if t is None else t.to(calc).contiguous()

    xg, xb, Bg, Bb, Cc, dtc, xr = map(prep, (x_g, x_b, B_g, B_b, C, dt, x_raw))
    hi = None if h_init is None else h_init.reshape(Bat, H, P, N).float().contiguous()
    y = torch.empty(Bat, T, H, P, R, device=x_g.device, dtype=calc)
    h_final = torch.empty(Bat, H, P, N, device=x_g.device, dtype=torch.float32)
    _native.chunked_fwd(Bat, T, H, P, N, R, calc, xg, xb, Bg, Bb, Cc, dtc,
                        A.float().contiguous(), D.float().contiguous(), xr, hi, y, h_final, None)
    return y.to(dtype), h_final


@chunked_fwd.register_fake
def _(x_g, x_b, B_g, B_b, C, dt, A, D, x_raw, h_init):
    Bat, T, H, P, R = x_g.shape
    N = B_g.shape[3]
    return x_g.new_empty(x_g.shape), x_g.new_empty(Bat, H, P, N, dtype=torch.float32)


@torch.library.custom_op(f"{NS}::chunked_bwd", mutates_args=())
def chunked_bwd(x_g: torch.Tensor, x_b: Optional[torch.Tensor], B_g: torch.Tensor,
                B_b: Optional[torch.Tensor], C: torch.Tensor, dt: torch.Tensor, A: torch.Tensor,
                D: torch.Tensor, x_raw: torch.Tensor, h_init: Optional[torch.Tensor],
                dy: torch.Tensor, dh_final: Optional[torch.Tensor]) -> list[torch.Tensor]:
    """m3_chunked_ssd_bwd (fp32): [dx_g, dx_b, dB_g, dB_b, dC, ddt, dA, dD, dx_raw, dh_init];
    dx_b / dB_b / dh_init are empty when the input is None."""
    Bat, T, H, P, R = x_g.shape
    N = B_g.shape[3]
    dev = x_g.device

    def f32(t):
        return None if t is None else t.float().contiguous()

    def new(shape):
        return torch.empty(shape, device=dev, dtype=torch.float32)

    beta = x_b is not None
    g = [new(x_g.shape), new(x_b.shape) if beta else None, new(B_g.shape),
         new(B_b.shape) if beta else None, new(C.shape), new((Bat, T, H)), new((H,)), new((H,)),
         new(x_raw.shape), new((Bat, H, P, N)) if h_init is not None else None]
    hi = None if h_init is None else f32(h_init.reshape(Bat, H, P, N))
    _native.chunked_bwd(Bat, T, H, P, N, R, f32(x_g), f32(x_b), f32(B_g), f32(B_b), f32(C),
                        f32(dt), f32(A), f32(D), f32(x_raw), hi, f32(dy), f32(dh_final), *g)
    return [torch.empty(0, device=dev, dtype=torch.float32) if t is None else t for t in g]


@chunked_bwd.register_fake
def _(x_g, x_b, B_g, B_b, C, dt, A, D, x_raw, h_init, dy, dh_final):
    Bat, T, H, P, R = x_g.shape
    N = B_g.shape[3]

    def new(shape):
        return x_g.new_empty(shape, dtype=torch.float32)

    e = (0,)
    return [new(x_g.shape), new(x_b.shape if x_b is not None else e), new(B_g.shape),
            new(B_b.shape if B_b is not None else e), new(C.shape), new((Bat, T, H)), new((H,)),
            new((H,)), new(x_raw.shape), new((Bat, H, P, N) if h_init is not None else e)]


def _chunked_setup(ctx, inputs, output):
    ctx.save_for_backward(*inputs)
    ctx.set_materialize_grads(False)


def _chunked_backward(ctx, dy, dh_final):
    ins = ctx.saved_tensors
    x_g = ins[0]
    if dy is None:
        dy = torch.zeros(x_g.shape, device=x_g.device, dtype=torch.float32)
    g = chunked_bwd(*ins, dy, dh_final)
    out = []
    for grad, like in zip(g, ins):
        out.append(None if like is None else grad.to(like.dtype).reshape(like.shape))
    return tuple(out)


chunked_fwd.register_autograd(_chunked_backward, setup_context=_chunked_setup)


def layer_args(layer) -> tuple:
    """The integer / flag arguments of the layer ops for a KulaMamba module."""
    return (layer.nheads, layer.headdim, layer.d_state, layer.mimo_rank, layer.ngroups,
            bool(layer.use_trapezoidal), bool(layer.use_complex_ssm), float(layer.B_norm.eps))


# ---------------------------------------------------------------------------- RMSNorm
@torch.library.custom_op(f"{NS}::rmsnorm", mutates_args=())
def rmsnorm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> tuple[torch.Tensor, torch.Tensor]:
    """m3_rmsnorm_fwd over the last dimension of x: (y in the promotion of x's and the
    weight's dtypes, rstd (rows,) fp32)."""
    _native.require_gpu(x, weight)
    d = x.shape[-1]
    x2 = x.reshape(-1, d).contiguous()
    wc = weight.contiguous()
    y = torch.empty(x2.shape, device=x.device, dtype=torch.promote_types(x.dtype, weight.dtype))
    rstd = torch.empty(x2.shape[0], device=x.device, dtype=torch.float32)
    _native.rmsnorm_fwd(x2, wc, y, rstd, eps)
    return y.reshape(x.shape), rstd


@rmsnorm.register_fake
def _(x, weight, eps):
    rows = x.numel() // x.shape[-1]
    return (x.new_empty(x.shape, dtype=torch.promote_types(x.dtype, weight.dtype)),
            x.new_empty(rows, dtype=torch.float32))


@torch.library.custom_op(f"{NS}::rmsnorm_bwd", mutates_args=())
def rmsnorm_bwd(x: torch.Tensor, weight: torch.Tensor, rstd: torch.Tensor,
                grad: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """m3_rmsnorm_bwd: (dL/dx in x's dtype, dL/dweight in the weight's dtype)."""
    d = x.shape[-1]
    x2 = x.reshape(-1, d).contiguous()
    g2 = grad.reshape(-1, d).contiguous().to(torch.promote_types(x.dtype, weight.dtype))
    dx = torch.empty_like(x2)
    dw = torch.empty_like(weight.contiguous())
    _native.rmsnorm_bwd(x2, weight.contiguous(), rstd, g2, dx, dw)
    return dx.reshape(x.shape), dw


@rmsnorm_bwd.register_fake
def _(x, weight, rstd, grad):
    return x.new_empty(x.shape), weight.new_empty(weight.shape)


def _rmsnorm_setup(ctx, inputs, output):
    x, weight, eps = inputs
    ctx.save_for_backward(x, weight, output[1])


def _rmsnorm_backward(ctx, g_y, g_rstd):
    x, weight, rstd = ctx.saved_tensors
    dx, dw = rmsnorm_bwd(x, weight, rstd, g_y)
    return dx, dw, None


rmsnorm.register_autograd(_rmsnorm_backward, setup_context=_rmsnorm_setup)


# ---------------------------------------------------------------- small-batch projections
def small_proj_usable(x: torch.Tensor, *weights, norm: bool = False) -> bool:
    """True when m3_small_linear / m3_small_swiglu take x (m, k) with these weights (norm
    weight and projection weights): bf16, at most 8 rows, k a multiple of 64 that fits their
    LDS (with the norm weight when `norm`), contiguous 16-byte aligned rows, and no autograd
    to record (the kernels have no backward)."""
    if torch.compiler.is_compiling() or x.dim() != 2 or x.dtype != torch.bfloat16:
        return False
    if not _native.small_proj_ok(x.shape[0], x.shape[1], norm):
        return False
    grad = torch.is_grad_enabled()
    for t in (x, *weights):
        if t is None or t.dtype != torch.bfloat16 or not t.is_cuda or not t.is_contiguous():
            return False
        if t.data_ptr() % 16 != 0 or (grad and t.requires_grad):
            return False
    return True


def _small_linear_eager(x: torch.Tensor, norm_w: Optional[torch.Tensor], eps: float, weight: torch.Tensor,
                 residual: Optional[torch.Tensor], scale: float) -> torch.Tensor:
    """m3_small_linear: [residual +] scale * (n W^T), n = RMSNorm(x; norm_w) or x, for bf16
    x (m <= 8, k) (check with small_proj_usable); no backward."""
    _native.require_gpu(x, weight)
    out = torch.empty(x.shape[0], weight.shape[0], device=x.device, dtype=torch.bfloat16)
    res = None if residual is None else residual.contiguous()
    _native.small_linear(x, norm_w, eps, weight, res, scale, out)
    return out


small_linear = torch.library.custom_op(f"{NS}::small_linear", _small_linear_eager, mutates_args=())


@small_linear.register_fake
def _(x, norm_w, eps, weight, residual, scale):
    return x.new_empty(x.shape[0], weight.shape[0])


def _small_swiglu_eager(x: torch.Tensor, norm_w: Optional[torch.Tensor], eps: float,
                 w_gate: torch.Tensor, w_up: torch.Tensor) -> torch.Tensor:
    """m3_small_swiglu: silu(n W_gate^T) * (n W_up^T), n = RMSNorm(x; norm_w) or x, for bf16
    x (m <= 8, k); no backward."""
    _native.require_gpu(x, w_gate, w_up)
    out = torch.empty(x.shape[0], w_gate.shape[0], device=x.device, dtype=torch.bfloat16)
    _native.small_swiglu(x, norm_w, eps, w_gate, w_up, out)
    return out


small_swiglu = torch.library.custom_op(f"{NS}::small_swiglu", _small_swiglu_eager, mutates_args=())


@small_swiglu.register_fake
def _(x, norm_w, eps, w_gate, w_up):
    return x.new_empty(x.shape[0], w_gate.shape[0])


def _silu_mul_eager(gate_up: torch.Tensor, d_ff: int) -> torch.Tensor:
    """m3_silu_mul: silu(gate_up[..., :d_ff]) * gate_up[..., d_ff:2 d_ff] for bf16 rows (the
    output of one GEMM over [w_gate; w_up]); no backward."""
    _native.require_gpu(gate_up)
    g2 = gate_up.reshape(-1, gate_up.shape[-1])
    if g2.stride(-1) != 1:
        g2 = g2.contiguous()
    out = torch.empty(g2.shape[0], d_ff, device=gate_up.device, dtype=torch.bfloat16)
    _native.silu_mul(g2, d_ff, out)
    return out.view(*gate_up.shape[:-1], d_ff)


silu_mul = torch.library.custom_op(f"{NS}::silu_mul", _silu_mul_eager, mutates_args=())


@silu_mul.register_fake
def _(gate_up, d_ff):
    return gate_up.new_empty(*gate_up.shape[:-1], d_ff)


# ---------------------------------------------------------------- eager decode calls
def _direct() -> bool:
    """Eager calls with autograd off bypass the dispatcher: its per-call host time is what a
    per-token decode loop waits on. Traced calls and calls under autograd go through the
    registered ops and their autograd formulas."""
    return not torch.is_grad_enabled() and not torch.compiler.is_compiling()


def step_fast(*args):
    return (_step_eager if _direct() else step)(*args)


def small_linear_fast(*args):
    return (_small_linear_eager if _direct() else small_linear)(*args)


def small_swiglu_fast(*args):
    return (_small_swiglu_eager if _direct() else small_swiglu)(*args)


def silu_mul_fast(*args):
    return (_silu_mul_eager if _direct() else silu_mul)(*args)
