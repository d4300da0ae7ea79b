"""m3_prefill_fwd_noalloc, the prefill entry point whose workspace is the library's static
per-device scratch, against m3_prefill_fwd with a caller workspace: the same kernels on
the same inputs, so every output must be bitwise equal. Two calls in a row, the second
smaller (the scratch keeps the first call's contents), on each dispatch path; a workload
beyond the scratch and the training forward are refused before any launch; and the entry
point under HIP graph capture, replayed with eager work in between."""

from __future__ import annotations

import ctypes

import pytest
import torch

import mamba3_amd
from mamba3_amd import _native

pytestmark = pytest.mark.gpu

# (layer kwargs, dtype, name of the path m3_prefill_fwd dispatches to)
PATHS = [
    (dict(d_model=768, d_state=128, headdim=64, mimo_rank=2), torch.bfloat16, "d768 MFMA"),
    (dict(d_model=128, d_state=64, headdim=32, mimo_rank=4), torch.bfloat16, "general MFMA"),
    (dict(d_model=128, d_state=32, headdim=32, mimo_rank=2), torch.float32, "fp32 layer"),
    (dict(d_model=64, d_state=16, headdim=16, mimo_rank=3), torch.float32, "fp32 layer rank 3"),
    (dict(d_model=64, d_state=16, headdim=16, mimo_rank=3), torch.bfloat16, "generic"),
]


def _layer(kw, dtype, dev):
    torch.manual_seed(0)
    return mamba3_amd.KulaMamba(**kw).to(dev, dtype).eval()


def _outputs(layer, B, T, dev, dtype):
    H, P, N = layer.nheads, layer.headdim, layer.d_state
    return (torch.empty(B, T, layer.d_inner, device=dev, dtype=dtype),
            torch.empty(B, H, P, N, device=dev), torch.empty(B, H, N // 2, device=dev),
            torch.empty(B, H, P, N, device=dev))


def _call(layer, proj, outs, noalloc):
    B, T, _ = proj.shape
    desc = layer._desc(B, T, proj)
    params = layer._param_pack()
    if noalloc:
        _native.prefill_fwd_noalloc(desc, params, proj, None, *outs)
    else:
        n = _native.prefill_workspace_bytes(desc)
        ws = torch.empty(max(n, 1), device=proj.device, dtype=torch.uint8)
        _native.prefill_fwd(desc, params, proj, None, *outs, ws, n)


@pytest.mark.parametrize("kw,dtype,path", PATHS, ids=[p[2] for p in PATHS])
def test_noalloc_equals_prefill_fwd_on_two_calls(kw, dtype, path, cuda_device):
    print(f"no-alloc prefill: {path} {kw}", flush=True)
    layer = _layer(kw, dtype, cuda_device)
    g = torch.Generator().manual_seed(1)
    for B, T in ((2, 300), (1, 70)):  # the second call is smaller
        x = torch.randn(B, T, kw["d_model"], generator=g).to(cuda_device, dtype)
        with torch.no_grad():
            proj = layer.in_proj(x).contiguous()
            got = _outputs(layer, B, T, cuda_device, dtype)
            want = _outputs(layer, B, T, cuda_device, dtype)
            _call(layer, proj, got, noalloc=True)
            _call(layer, proj, want, noalloc=False)
        torch.cuda.synchronize()
        for name, a, b in zip(("y", "h", "angle", "prev_BX"), got, want):
            assert torch.equal(a, b), (path, B, T, name)


def test_noalloc_refuses_a_workspace_beyond_its_scratch(cuda_device):
    """The (8, 8192) d768 prefill needs 64 MiB of normalised B/C rows plus 256 bytes: one
    more than the scratch holds, so the call returns M3_ERR_SCRATCH_LIMIT and launches
    nothing (the outputs keep their fill)."""
    layer = _layer(PATHS[0][0], torch.bfloat16, cuda_device)
    B, T = 8, 8192
    proj = torch.zeros(B, T, layer.in_proj.out_features, device=cuda_device, dtype=torch.bfloat16)
    desc = layer._desc(B, T, proj)
    assert _native.prefill_workspace_bytes(desc) > _native.NOALLOC_SCRATCH_BYTES
    outs = _outputs(layer, B, T, cuda_device, torch.bfloat16)
    outs[0].fill_(7.0)
    st = _native.lib().m3_prefill_fwd_noalloc(
        ctypes.byref(desc), ctypes.byref(layer._param_pack()), proj.data_ptr(), None,
        *[t.data_ptr() for t in outs], _native.stream_of(proj))
    assert st == _native.M3_ERR_SCRATCH_LIMIT
    assert "scratch" in _native.lib().m3_status_string(st).decode()
    torch.cuda.synchronize()
    assert bool((outs[0] == 7.0).all())


def test_noalloc_refuses_the_training_forward(cuda_device):
    """M3_FLAG_FOR_BACKWARD asks the forward to keep the backward's operands in its
    workspace; here that would be the shared scratch, which the next call overwrites, so the
    call returns M3_ERR_UNSUPPORTED and launches nothing (the outputs keep their fill)."""
    layer = _layer(PATHS[2][0], torch.float32, cuda_device)
    B, T = 1, 64
    proj = torch.zeros(B, T, layer.in_proj.out_features, device=cuda_device)
    desc = layer._desc(B, T, proj)
    desc.flags |= _native.M3_FLAG_FOR_BACKWARD
    outs = _outputs(layer, B, T, cuda_device, torch.float32)
    outs[0].fill_(7.0)
    st = _native.lib().m3_prefill_fwd_noalloc(
        ctypes.byref(desc), ctypes.byref(layer._param_pack()), proj.data_ptr(), None,
        *[t.data_ptr() for t in outs], _native.stream_of(proj))
    assert st == _native.M3_ERR_UNSUPPORTED
    torch.cuda.synchronize()
    assert bool((outs[0] == 7.0).all())


def test_noalloc_under_graph_capture_replays_equal_eager(cuda_device):
    """The entry point captured in a HIP graph (no allocation inside the capture), replayed
    three times with eager prefills on other inputs in between: every replay equals the
    eager m3_prefill_fwd result on the captured input."""
    kw, dtype, _ = PATHS[0]
    layer = _layer(kw, dtype, cuda_device)
    g = torch.Generator().manual_seed(2)
    B, T = 2, 200
    with torch.no_grad():
        proj = layer.in_proj(torch.randn(B, T, 768, generator=g).to(cuda_device, dtype)).contiguous()
        other = layer.in_proj(torch.randn(1, 130, 768, generator=g).to(cuda_device, dtype)).contiguous()
        want = _outputs(layer, B, T, cuda_device, dtype)
        _call(layer, proj, want, noalloc=False)
        got = _outputs(layer, B, T, cuda_device, dtype)
        _call(layer, proj, got, noalloc=True)  # warm-up: symbol lookup and parameter pack
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            _call(layer, proj, got, noalloc=True)
        for _ in range(3):
            for t in got:
                t.zero_()
            junk = _outputs(layer, 1, 130, cuda_device, dtype)
            _call(layer, other, junk, noalloc=True)  # eager use of the same scratch
            torch.cuda.synchronize()
            graph.replay()
            torch.cuda.synchronize()
            for a, b in zip(got, want):
                assert torch.equal(a, b)
