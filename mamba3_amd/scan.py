"""Inter-chunk state scan op: drop-in for mamba3.scan.ssd_scan (mamba3/scan.py:65-145).

    h[0] = h_init (or 0),   h[k+1] = decay[k] * h[k] + h_chunk[k]

Runs the HBM-bound HIP kernel `m3_scan_fwd` (mamba3_amd/csrc/m3_scan.hip) in fp32
and returns the states in h_chunk's dtype, like the reference (mamba3/scan.py:98). The
backward (mamba3/scan.py:101-141) runs `m3_scan_bwd` on the fp32 states saved by the
forward.
"""

from __future__ import annotations

import torch

from . import _native


class _ScanFn(torch.autograd.Function):
    """SSDScanFn (mamba3/scan.py:65-141) on the HIP kernels."""

    @staticmethod
    def forward(ctx, chunk_decay, h_chunk, h_init):
        states = _scan_fp32(chunk_decay, h_chunk, h_init)
        ctx.save_for_backward(chunk_decay, states)
        ctx.shape = h_chunk.shape
        ctx.init_shape = None if h_init is None else h_init.shape
        return states.reshape(h_chunk.shape).to(h_chunk.dtype)

    @staticmethod
    def backward(ctx, grad):
        chunk_decay, states = ctx.saved_tensors
        B, K, H, PN = states.shape
        g = grad.reshape(B, K, H, PN).float().contiguous()
        decay = chunk_decay.float().contiguous()
        d_decay = torch.empty_like(decay)
        d_chunk = torch.empty_like(states)
        d_init = None
        if ctx.init_shape is not None:
            d_init = torch.empty(B, H, PN, dtype=torch.float32, device=states.device)
        _native.scan_bwd(decay, states, g, d_decay, d_chunk, d_init)
        return (d_decay.to(chunk_decay.dtype), d_chunk.reshape(ctx.shape).to(grad.dtype),
                None if d_init is None else d_init.reshape(ctx.init_shape).to(grad.dtype))


def _scan_fp32(chunk_decay: torch.Tensor, h_chunk: torch.Tensor,
               h_init: torch.Tensor | None) -> torch.Tensor:
    """fp32 states (B, K, H, PN)."""
    if chunk_decay.dim() != 3 or h_chunk.dim() < 3:
        raise ValueError("ssd_scan expects chunk_decay (B,K,H) and h_chunk (B,K,H,...)")
    B, K, H = chunk_decay.shape
    if tuple(h_chunk.shape[:3]) != (B, K, H):
        raise ValueError(f"h_chunk leading dims {tuple(h_chunk.shape[:3])} != {(B, K, H)}")
    _native.require_gpu(chunk_decay, h_chunk, h_init)
    shape = h_chunk.shape
    flat = h_chunk.reshape(B, K, H, -1).float().contiguous()
    PN = flat.shape[-1]
    init = None
    if h_init is not None:
        if h_init.numel() != B * H * PN:
            raise ValueError(f"h_init has {h_init.numel()} elements, expected {B * H * PN}")
        init = h_init.reshape(B, H, PN).float().contiguous()
    decay = chunk_decay.float().contiguous()
    out = torch.empty_like(flat)
    _native.scan_fwd(decay, flat, init, out)
    return out


def ssd_scan(chunk_decay: torch.Tensor, h_chunk: torch.Tensor,
             h_init: torch.Tensor | None = None) -> torch.Tensor:
    """Exclusive chunk-state scan; returns h_states shaped like h_chunk."""
    if torch.is_grad_enabled() and any(
            t is not None and t.requires_grad for t in (chunk_decay, h_chunk, h_init)):
        return _ScanFn.apply(chunk_decay, h_chunk, h_init)
    return _scan_fp32(chunk_decay, h_chunk, h_init).reshape(h_chunk.shape).to(h_chunk.dtype)
