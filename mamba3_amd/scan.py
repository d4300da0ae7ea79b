"""Inter-chunk state scan op: drop-in for mamba3.scan.ssd_scan (mamba3/scan.py:65-145).

    h[0] = h_init (or 0),   h[k+1] = decay[k] * h[k] + h_chunk[k]

Runs the HBM-bound HIP kernel `m3_scan_fwd` (mamba3_amd/csrc/m3_scan.hip; the
`mamba3_amd::scan_fwd` op) in fp32 and returns the states in h_chunk's dtype, like the
reference (mamba3/scan.py:98). The backward (mamba3/scan.py:101-141) runs `m3_scan_bwd`
on the fp32 states saved by the forward.
"""

from __future__ import annotations

import torch

from . import _native, ops


def ssd_scan(chunk_decay: torch.Tensor, h_chunk: torch.Tensor,
             h_init: torch.Tensor | None = None) -> torch.Tensor:
    """Exclusive chunk-state scan; returns h_states shaped like h_chunk, in its dtype."""
    if chunk_decay.dim() != 3 or h_chunk.dim() < 3:
        raise ValueError("ssd_scan expects chunk_decay (B,K,H) and h_chunk (B,K,H,...)")
    B, K, H = chunk_decay.shape
    if tuple(h_chunk.shape[:3]) != (B, K, H):
        raise ValueError(f"h_chunk leading dims {tuple(h_chunk.shape[:3])} != {(B, K, H)}")
    _native.require_gpu(chunk_decay, h_chunk, h_init)
    flat = h_chunk.reshape(B, K, H, -1)
    PN = flat.shape[-1]
    init = None
    if h_init is not None:
        if h_init.numel() != B * H * PN:
            raise ValueError(f"h_init has {h_init.numel()} elements, expected {B * H * PN}")
        init = h_init.reshape(B, H, PN)
    out = ops.scan_fwd(chunk_decay, flat, init)
    return out.reshape(h_chunk.shape).to(h_chunk.dtype)
