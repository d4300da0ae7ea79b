"""torch.compile(fullgraph=True) through the custom ops (mamba3_amd/ops.py): the layer,
chunked_ssd and ssd_scan trace without graph breaks, forward and backward, and agree with
eager execution (mirrors the reference's tests/test_mamba3.py:584-616)."""

from __future__ import annotations

import pytest
import torch

import mamba3_amd
from conftest import max_rel
from mamba3_amd import _native

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _native_loaded(cuda_device):
    _native.lib()
    torch.backends.cuda.matmul.allow_tf32 = False
    torch._dynamo.reset()


def _layer(dev, train):
    torch.manual_seed(0)
    layer = mamba3_amd.KulaMamba(d_model=64, d_state=16, headdim=16, mimo_rank=2, expand=2,
                                 chunk_size=8).to(dev, torch.float32)
    return layer.train() if train else layer.eval()


def test_torch_compile_forward(cuda_device):
    print("compile: layer forward", flush=True)
    layer = _layer(cuda_device, train=False)
    compiled = torch.compile(layer, fullgraph=True)
    x = torch.randn(1, 16, 64, device=cuda_device)
    with torch.no_grad():
        y_eager = layer(x)
        y_compiled = compiled(x)
        y2, st = torch.compile(layer.prefill, fullgraph=True)(x)
    assert (y_eager - y_compiled).abs().max().item() < 1e-5
    assert (y_eager - y2).abs().max().item() < 1e-5
    assert st["h"].shape == (1, layer.nheads, 16, 16)


def test_torch_compile_backward(cuda_device):
    print("compile: layer backward", flush=True)
    layer = _layer(cuda_device, train=True)
    x = torch.randn(1, 16, 64, device=cuda_device)
    ds = torch.rand(1, 16, layer.nheads, device=cuda_device) + 0.5
    layer(x, dt_scale=ds).sum().backward()
    eager = {n: p.grad.clone() for n, p in layer.named_parameters()}
    layer.zero_grad(set_to_none=True)
    compiled = torch.compile(layer, fullgraph=True)
    compiled(x, dt_scale=ds).sum().backward()
    for name, p in layer.named_parameters():
        assert p.grad is not None, f"no gradient for {name} under compile"
        assert torch.isfinite(p.grad).all(), name
        assert max_rel(p.grad, eager[name]) < 1e-4, name


def test_torch_compile_chunked_ssd_and_scan(cuda_device):
    print("compile: chunked_ssd and ssd_scan", flush=True)
    g = torch.Generator(device=cuda_device).manual_seed(3)
    B, T, H, P, N, R = 1, 20, 2, 8, 8, 2

    def r(*s):
        return torch.randn(*s, device=cuda_device, generator=g).requires_grad_()

    ins = [r(B, T, H, P, R), r(B, T, H, P, R), r(B, T, H, N, R), r(B, T, H, N, R),
           r(B, T, H, N, R), (torch.rand(B, T, H, device=cuda_device, generator=g) * 0.3).requires_grad_(),
           (-torch.rand(H, device=cuda_device, generator=g) - 0.1).requires_grad_(), r(H),
           r(B, T, H, P, R)]

    def ssd(*a):
        out = mamba3_amd.chunked_ssd(*a, chunk_size=8, return_final_state=True)
        return out.y.square().sum() + out.h_final.sum()

    def run(fn):
        for t in ins:
            t.grad = None
        fn(*ins).backward()
        return [t.grad.clone() for t in ins]

    want = run(ssd)
    got = run(torch.compile(ssd, fullgraph=True))
    for a, b in zip(got, want):
        assert max_rel(a, b) < 1e-4

    d = (torch.rand(2, 5, 3, device=cuda_device, generator=g) * 0.9).requires_grad_()
    hc = torch.randn(2, 5, 3, 40, device=cuda_device, generator=g).requires_grad_()

    def scan(d, hc):
        return (mamba3_amd.ssd_scan(d, hc) ** 2).sum()

    scan(d, hc).backward()
    gd, gh = d.grad.clone(), hc.grad.clone()
    d.grad = hc.grad = None
    torch.compile(scan, fullgraph=True)(d, hc).backward()
    assert max_rel(d.grad, gd) < 1e-5 and max_rel(hc.grad, gh) < 1e-5
