"""Chunked SSD op on pre-processed inputs: drop-in for mamba3.ssd.chunked_ssd
(mamba3/ssd.py:22-25, 118-244).

    h_t = exp(A dt_t) h_{t-1} + dt_t (B_g,t x_g,t^T + B_b,t x_b,t^T)   (rank-R factors)
    y_t[p,r] = C_t[:,r] . h_t[p,:] + D x_raw,t[p,r]

evaluated by the HIP kernel behind `m3_chunked_ssd_fwd` (the `mamba3_amd::chunked_fwd`
op). `chunk_size` is accepted for API compatibility; the kernel chooses its own chunking
(results agree to rounding). Under autograd the backward runs the HIP kernels behind
`m3_chunked_ssd_bwd` (fp32; `mamba3_amd::chunked_bwd`), in place of the reference's
autograd through _IntraChunkFn (mamba3/ssd.py:67-115), the scan backward
(mamba3/scan.py:101-141) and ATen's bmm / cumsum backward. Shapes the backward kernels do
not cover raise when the backward runs.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from . import _native, ops


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
    if (torch.is_grad_enabled() and not torch.compiler.is_compiling()
            and any(t is not None and t.requires_grad for t in ins)):
        # Fails here, before the forward, when the backward kernels do not cover the shape.
        _native.chunked_bwd_workspace_bytes(Bat, T, H, P, N, R, x_b is not None)
    y, h_final = ops.chunked_fwd(*ins)
    return SSDOutput(y=y, h_final=h_final if return_final_state else None)
