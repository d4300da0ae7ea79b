"""GPU parity of the residual blocks' RMSNorm (m3_rmsnorm_fwd / m3_rmsnorm_bwd,
mamba3/mamba3.py:19-35) and of the residual adds fused into the out_proj / w_down GEMMs
(mamba3/block.py:79-107): forward and gradients against the oracle's rmsnorm and
block_forward, in fp32 (1e-4 normwise max-relative, fp64 oracle) and bf16."""

from __future__ import annotations

import pytest
import torch

import mamba3_amd
from conftest import max_rel
from mamba3_amd import _native, ops
from mamba3_amd.layer import RMSNorm
from oracle import reference_path as ref

pytestmark = pytest.mark.gpu

FP32_TOL = 1e-4
BF16_TOL = 2e-2


@pytest.fixture(scope="module", autouse=True)
def _native_loaded(cuda_device):
    _native.lib()
    torch.backends.cuda.matmul.allow_tf32 = False


# (rows, d): a partial last block of 4 rows, d not a multiple of the 64-lane stride,
# several 256-row dw partials, the LM's 768 and a wide 2048.
NORM_SHAPES = [(1, 64), (7, 50), (1000, 768), (3, 2048), (4099, 96)]


@pytest.mark.parametrize("rows,d", NORM_SHAPES)
def test_rmsnorm_fp32_forward_and_gradients_match_oracle(rows, d, cuda_device):
    print(f"rmsnorm fp32 rows {rows} d {d}", flush=True)
    g = torch.Generator().manual_seed(rows * 7 + d)
    x = torch.randn(rows, d, generator=g) * 3
    w = torch.randn(d, generator=g)
    gy = torch.randn(rows, d, generator=g)
    xr = x.double().requires_grad_()
    wr = w.double().requires_grad_()
    y_ref = ref.rmsnorm(xr, wr, 1e-5)
    (y_ref * gy.double()).sum().backward()

    norm = RMSNorm(d).to(cuda_device)
    with torch.no_grad():
        norm.weight.copy_(w)
    xd = x.to(cuda_device).requires_grad_()
    y = norm(xd)
    (y * gy.to(cuda_device)).sum().backward()
    assert max_rel(y, y_ref) < 1e-5
    assert max_rel(xd.grad, xr.grad) < FP32_TOL
    assert max_rel(norm.weight.grad, wr.grad) < FP32_TOL
    _, rstd = ops.rmsnorm(x.to(cuda_device), w.to(cuda_device), 1e-5)
    want = torch.rsqrt(x.double().pow(2).mean(-1) + 1e-5)
    assert max_rel(rstd, want) < 1e-6


def test_rmsnorm_over_a_leading_dimension(cuda_device):
    """RMSNorm(d, dim=1) on (B, d, T) normalises over dim 1, as the reference's dim argument
    does (mamba3/mamba3.py:27-35)."""
    g = torch.Generator().manual_seed(4)
    x = torch.randn(3, 40, 17, generator=g)
    w = torch.randn(40, generator=g)
    norm = RMSNorm(40, dim=1).to(cuda_device)
    with torch.no_grad():
        norm.weight.copy_(w)
        y = norm(x.to(cuda_device))
    want = ref.rmsnorm(x.double().movedim(1, -1), w.double(), 1e-5).movedim(-1, 1)
    assert y.shape == x.shape
    assert max_rel(y, want) < 1e-5


@pytest.mark.parametrize("rows,d", [(7, 50), (4099, 768)])
def test_rmsnorm_bf16_rounds_like_the_reference(rows, d, cuda_device):
    """bf16 activations and weight: the scale and x * scale are rounded to bf16 before the
    weight multiplies (mamba3/mamba3.py:30-35). Against the oracle run in bf16 on the same
    inputs the results are bitwise equal except where the fp32 rsqrt's last bit moves the
    bf16 scale by one ulp (a row then moves by at most 2^-6 of its largest entry); against
    the fp64 oracle within 2e-2."""
    print(f"rmsnorm bf16 rows {rows} d {d}", flush=True)
    g = torch.Generator().manual_seed(rows + d)
    x = (torch.randn(rows, d, generator=g) * 2).to(torch.bfloat16)
    w = (torch.rand(d, generator=g) + 0.5).to(torch.bfloat16)
    gy = torch.randn(rows, d, generator=g).to(torch.bfloat16)
    norm = RMSNorm(d).to(cuda_device, torch.bfloat16)
    with torch.no_grad():
        norm.weight.copy_(w)
    xd = x.to(cuda_device).requires_grad_()
    y = norm(xd)
    assert y.dtype == torch.bfloat16
    (y.float() * gy.float().to(cuda_device)).sum().backward()
    y16 = ref.rmsnorm(x, w, 1e-5)
    xr = x.double().requires_grad_()
    wr = w.double().requires_grad_()
    y64 = ref.rmsnorm(xr, wr, 1e-5)
    (y64 * gy.double()).sum().backward()
    yc, y16 = y.float().cpu(), y16.float()
    diff = (yc - y16).abs() / y16.abs().amax(-1, keepdim=True)
    assert diff.max().item() <= 2.0 ** -6
    assert (yc == y16).float().mean().item() > 0.99
    assert max_rel(y, y64) < BF16_TOL
    assert max_rel(xd.grad, xr.grad) < BF16_TOL
    assert max_rel(norm.weight.grad, wr.grad) < BF16_TOL


def _block_params(block):
    return {k: v.detach().double().cpu().clone().requires_grad_()
            for k, v in block.state_dict().items()}


@pytest.mark.parametrize("use_mlp", [True, False])
def test_block_forward_and_gradients_match_oracle(use_mlp, cuda_device):
    """KulaMambaBlock in fp32 (norm kernel, layer kernels, residual adds as GEMM epilogues)
    against autograd through the oracle's block_forward in fp64: output, input gradient and
    every parameter's gradient (mamba3/block.py:29-92)."""
    print(f"block gradients use_mlp={use_mlp}", flush=True)
    kw = dict(d_model=64, d_state=16, headdim=16, mimo_rank=2, chunk_size=8)
    torch.manual_seed(0)
    block = mamba3_amd.KulaMambaBlock(use_mlp=use_mlp, residual_scale=0.7, **kw)
    block = block.to(cuda_device).train()
    cfg = ref.LayerCfg(d_model=64, d_state=16, headdim=16, mimo_rank=2, chunk_size=8)
    g = torch.Generator().manual_seed(9)
    x = torch.randn(2, 37, 64, generator=g)
    w = torch.randn(2, 37, 64, generator=g)
    p = _block_params(block)
    xr = x.double().requires_grad_()
    out_ref = ref.block_forward(cfg, p, "", xr, 0.7, use_mlp)
    (out_ref * w.double()).sum().backward()
    xd = x.to(cuda_device).requires_grad_()
    out = block(xd)
    (out * w.to(cuda_device)).sum().backward()
    assert max_rel(out, out_ref) < FP32_TOL
    assert max_rel(xd.grad, xr.grad) < FP32_TOL
    for name, prm in block.named_parameters():
        if prm.grad is None:
            assert p[name].grad is None or not p[name].grad.any(), name
            continue
        assert max_rel(prm.grad, p[name].grad) < FP32_TOL, name


def test_block_prefill_then_steps_match_oracle(cuda_device):
    """KulaMambaBlock.prefill then five steps (residual adds fused into the GEMMs) against
    the oracle's block_forward(return_state) and block_step chain (mamba3/block.py:94-107)."""
    kw = dict(d_model=64, d_state=16, headdim=16, mimo_rank=2, chunk_size=8)
    torch.manual_seed(1)
    block = mamba3_amd.KulaMambaBlock(residual_scale=0.5, **kw).to(cuda_device).eval()
    cfg = ref.LayerCfg(d_model=64, d_state=16, headdim=16, mimo_rank=2, chunk_size=8)
    p = {k: v.detach().double().cpu() for k, v in block.state_dict().items()}
    g = torch.Generator().manual_seed(3)
    x = torch.randn(3, 21, 64, generator=g)
    toks = torch.randn(5, 3, 64, generator=g)
    with torch.no_grad():
        y, st = block.prefill(x.to(cuda_device))
        y_ref, st_ref = ref.block_forward(cfg, p, "", x.double(), 0.5, True, return_state=True)
        assert max_rel(y, y_ref) < FP32_TOL
        for k in ("h", "prev_BX", "angle"):
            assert max_rel(st[k], st_ref[k]) < FP32_TOL, k
        for i in range(5):
            y, st = block.step(toks[i].to(cuda_device), st)
            y_ref, st_ref = ref.block_step(cfg, p, "", toks[i].double(), st_ref, 0.5, True)
            assert max_rel(y, y_ref) < FP32_TOL, i
            assert max_rel(st["h"], st_ref["h"]) < FP32_TOL, i
