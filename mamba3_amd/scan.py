"""Inter-chunk state scan op: drop-in for mamba3.scan.ssd_scan (mamba3/scan.py:65-145).

    h[0] = h_init (or 0),   h[k+1] = decay[k] * h[k] + h_chunk[k]

Runs the HBM-bound HIP kernel `m3_scan_fwd` (mamba3_amd/csrc/m3_scan.hip) in fp32
and returns the states in h_chunk's dtype, like the reference (mamba3/scan.py:98).
Forward only: backward raises.
"""

from __future__ import annotations

import torch

from . import _native


class _ScanForwardOnly(torch.autograd.Function):
    @staticmethod
    def forward(ctx, chunk_decay, h_chunk, h_init):
        return _scan_impl(chunk_decay, h_chunk, h_init)

    @staticmethod
    def backward(ctx, grad):
        raise NotImplementedError("mamba3_amd.ssd_scan has no backward kernel")


def _scan_impl(chunk_decay: torch.Tensor, h_chunk: torch.Tensor,
               h_init: torch.Tensor | None) -> torch.Tensor:
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
    return out.reshape(shape).to(h_chunk.dtype)


def ssd_scan(chunk_decay: torch.Tensor, h_chunk: torch.Tensor,
             h_init: torch.Tensor | None = None) -> torch.Tensor:
    """Exclusive chunk-state scan; returns h_states shaped like h_chunk."""
    if torch.is_grad_enabled() and any(
            t is not None and t.requires_grad for t in (chunk_decay, h_chunk, h_init)):
        return _ScanForwardOnly.apply(chunk_decay, h_chunk, h_init)
    return _scan_impl(chunk_decay, h_chunk, h_init)
