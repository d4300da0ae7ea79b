"""Chunked SSD op on pre-processed inputs: drop-in for mamba3.ssd.chunked_ssd
(mamba3/ssd.py:22-25, 118-244).

    h_t = exp(A dt_t) h_{t-1} + dt_t (B_g,t x_g,t^T + B_b,t x_b,t^T)   (rank-R factors)
    y_t[p,r] = C_t[:,r] . h_t[p,:] + D x_raw,t[p,r]

evaluated by the HIP kernel behind `m3_chunked_ssd_fwd`. `chunk_size` is accepted
for API compatibility; the kernel chooses its own chunking (results agree to rounding).
Under autograd the backward runs the HIP kernels behind `m3_chunked_ssd_bwd` (fp32), in
place of the reference's autograd through _IntraChunkFn (mamba3/ssd.py:67-115), the
scan backward (mamba3/scan.py:101-141) and ATen's bmm / cumsum backward.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from . import _native


@dataclass
class SSDOutput:
    y: torch.Tensor
    h_final: torch.Tensor | None = None


def chunked_ssd(
    x_g: torch.Tensor,
    x_b: torch.Tensor | None,
    B_g: torch.Tensor,
    B_b: torch.Tensor | None,
    C: torch.Tensor,
    dt: torch.Tensor,
    A: torch.Tensor,
    D: torch.Tensor,
    x_raw: torch.Tensor,
    chunk_size: int = 64,
    h_init: torch.Tensor | None = None,
    return_final_state: bool = False,
) -> SSDOutput:
    if (x_b is None) != (B_b is None):
        raise ValueError("x_b and B_b must both be given or both be None")
    Bat, T, H, P, R = x_g.shape
    N = B_g.shape[3]
    if tuple(B_g.shape) != (Bat, T, H, N, R) or tuple(C.shape) != (Bat, T, H, N, R):
        raise ValueError("B_g and C must be (B,T,H,N,R) matching x_g (B,T,H,P,R)")
    if tuple(dt.shape) != (Bat, T, H):
        raise ValueError(f"dt must be {(Bat, T, H)}, got {tuple(dt.shape)}")
    if tuple(x_raw.shape) != (Bat, T, H, P, R):
        raise ValueError("x_raw must match x_g")
    if x_b is not None and (tuple(x_b.shape) != tuple(x_g.shape) or
                            tuple(B_b.shape) != tuple(B_g.shape)):
        raise ValueError("x_b / B_b must match x_g / B_g")
    _native.require_gpu(x_g, x_b, B_g, B_b, C, dt, A, D, x_raw, h_init)
    _native.dtype_code(x_g.dtype)
    ins = (x_g, x_b, B_g, B_b, C, dt, A, D, x_raw, h_init)
    if torch.is_grad_enabled() and any(t is not None and t.requires_grad for t in ins):
        # Fails here, before the forward, when the backward kernels do not support the shape.
        _native.chunked_bwd_workspace_bytes(Bat, T, H, P, N, R, x_b is not None)
        y, h_final = _ChunkedFn.apply(*ins)
    else:
        y, h_final = _forward(*ins)
    return SSDOutput(y=y, h_final=h_final if return_final_state else None)


def _forward(x_g, x_b, B_g, B_b, C, dt, A, D, x_raw, h_init):
    Bat, T, H, P, R = x_g.shape
    N = B_g.shape[3]
    dtype = x_g.dtype
    if dtype != torch.float32 and _native.chunked_fwd_mfma_applies(Bat, T, H, P, N, R,
                                                                   x_b is not None):
        # bf16 inputs run on the fp32-MFMA chunk kernels (more accurate than the reference's
        # bf16 intermediates, and far faster than the generic kernel)
        f32 = [None if t is None else t.float() for t in (x_g, x_b, B_g, B_b, C, dt, x_raw)]
        y, h_final = _forward(f32[0], f32[1], f32[2], f32[3], f32[4], f32[5], A, D, f32[6],
                              h_init)
        return y.to(dtype), h_final

    def prep(t):
        return None if t is None else t.to(dtype).contiguous()

    xg, xb, Bg, Bb, Cc, dtc, xr = map(prep, (x_g, x_b, B_g, B_b, C, dt, x_raw))
    Af = A.float().contiguous()
    Df = D.float().contiguous()
    hi = None
    if h_init is not None:
        hi = h_init.reshape(Bat, H, P, N).float().contiguous()
    y = torch.empty(Bat, T, H, P, R, device=x_g.device, dtype=dtype)
    h_final = torch.empty(Bat, H, P, N, device=x_g.device, dtype=torch.float32)
    _native.chunked_fwd(Bat, T, H, P, N, R, dtype, xg, xb, Bg, Bb, Cc, dtc, Af, Df, xr, hi,
                        y, h_final, None)
    return y, h_final


class _ChunkedFn(torch.autograd.Function):
    """chunked_ssd with the HIP backward (m3_chunked_ssd_bwd, fp32 arithmetic). Gradients
    come back in each input's dtype and shape."""

    @staticmethod
    def forward(ctx, x_g, x_b, B_g, B_b, C, dt, A, D, x_raw, h_init):
        y, h_final = _forward(x_g, x_b, B_g, B_b, C, dt, A, D, x_raw, h_init)
        ctx.save_for_backward(x_g, x_b, B_g, B_b, C, dt, A, D, x_raw, h_init)
        ctx.set_materialize_grads(False)
        return y, h_final

    @staticmethod
    def backward(ctx, dy, dh_final):
        x_g, x_b, B_g, B_b, C, dt, A, D, x_raw, h_init = ctx.saved_tensors
        Bat, T, H, P, R = x_g.shape
        N = B_g.shape[3]

        def f32(t):
            return None if t is None else t.float().contiguous()

        if dy is None:
            dy = torch.zeros_like(x_g, dtype=torch.float32)
        hi = None if h_init is None else f32(h_init.reshape(Bat, H, P, N))
        dhf = None if dh_final is None else f32(dh_final)
        grads = dict(
            dx_g=torch.empty(x_g.shape, device=x_g.device, dtype=torch.float32),
            dx_b=None if x_b is None else torch.empty(x_b.shape, device=x_g.device,
                                                      dtype=torch.float32),
            dB_g=torch.empty(B_g.shape, device=x_g.device, dtype=torch.float32),
            dB_b=None if B_b is None else torch.empty(B_b.shape, device=x_g.device,
                                                      dtype=torch.float32),
            dC=torch.empty(C.shape, device=x_g.device, dtype=torch.float32),
            ddt=torch.empty(Bat, T, H, device=x_g.device, dtype=torch.float32),
            dA=torch.empty(H, device=x_g.device, dtype=torch.float32),
            dD=torch.empty(H, device=x_g.device, dtype=torch.float32),
            dx_raw=torch.empty(x_raw.shape, device=x_g.device, dtype=torch.float32),
            dh_init=None if h_init is None else torch.empty(Bat, H, P, N, device=x_g.device,
                                                            dtype=torch.float32),
        )
        _native.chunked_bwd(Bat, T, H, P, N, R, f32(x_g), f32(x_b), f32(B_g), f32(B_b), f32(C),
                            f32(dt), f32(A), f32(D), f32(x_raw), hi, f32(dy), dhf, *grads.values())

        def back(g, like):
            return None if g is None or like is None else g.to(like.dtype).reshape(like.shape)

        return (back(grads["dx_g"], x_g), back(grads["dx_b"], x_b), back(grads["dB_g"], B_g),
                back(grads["dB_b"], B_b), back(grads["dC"], C), back(grads["ddt"], dt),
                back(grads["dA"], A), back(grads["dD"], D), back(grads["dx_raw"], x_raw),
                back(grads["dh_init"], h_init))
