"""GPU parity of the backward path: chunked_ssd's HIP backward (m3_chunked_ssd_bwd) and the
layer's differentiable forward / prefill, against autograd through the float64 oracle
(whose gradients are pinned on the CPU against the per-token recurrence and finite
differences).

Tolerances (normwise max-relative error, max|g - g_ref| / max|g_ref|, per gradient):
  * fp32 kernels vs the oracle: 1e-4
  * bf16 layer vs the fp32 oracle on the bf16-rounded weights and inputs: 2e-2
"""

from __future__ import annotations

import pytest
import torch

import mamba3_amd
from conftest import max_rel, oracle_cfg
from oracle import reference_path as ref

pytestmark = pytest.mark.gpu

FP32_TOL = 1e-4
BF16_TOL = 2e-2

NAMES = ("x_g", "x_b", "B_g", "B_b", "C", "dt", "A", "D", "x_raw", "h_init")

# B, T, H, P, N, R, beta terms, h_init, dL/dh_final
CASES = [
    (2, 100, 3, 16, 32, 2, True, True, True),
    (1, 130, 2, 8, 16, 1, False, False, True),
    (1, 64, 2, 32, 64, 4, True, False, False),
    (2, 37, 1, 64, 128, 2, True, True, True),
    (1, 50, 2, 16, 16, 8, True, False, True),
    (1, 200, 1, 64, 128, 2, False, True, False),
    (1, 1, 2, 16, 32, 2, True, True, True),
    # two headdim and two d_state tiles, each second one partial (96 = 64 + 32, 160 = 128 + 32)
    (1, 70, 2, 96, 160, 2, True, True, True),
    (1, 45, 1, 96, 160, 1, False, False, True),
    # ranks 3, 5, 6, 7: rank-4 / rank-8 tiles with their extra slots read as zero
    (1, 90, 2, 16, 32, 3, True, True, True),
    (1, 70, 2, 16, 32, 3, False, False, True),
    (1, 45, 2, 16, 16, 5, False, True, False),
    (2, 33, 1, 32, 32, 6, True, True, True),
    (1, 20, 2, 8, 16, 7, True, False, True),
]


@pytest.fixture(scope="module", autouse=True)
def _no_tf32(cuda_device):
    torch.backends.cuda.matmul.allow_tf32 = False
    torch.backends.cudnn.allow_tf32 = False


def _inputs(case, seed=0):
    B, T, H, P, N, R, beta, with_init, _ = case
    g = torch.Generator().manual_seed(seed)
    r = lambda *s: torch.randn(*s, generator=g, dtype=torch.float64)
    return dict(x_g=r(B, T, H, P, R), x_b=r(B, T, H, P, R) if beta else None,
                B_g=r(B, T, H, N, R), B_b=r(B, T, H, N, R) if beta else None,
                C=r(B, T, H, N, R), dt=torch.rand(B, T, H, generator=g, dtype=torch.float64) * 0.5,
                A=-torch.rand(H, generator=g, dtype=torch.float64) - 0.2, D=r(H),
                x_raw=r(B, T, H, P, R), h_init=r(B, H, P, N) if with_init else None)


def _gpu_grads(ins, dy, dhf, dev):
    leaf = {k: (v.float().to(dev).requires_grad_() if v is not None else None) for k, v in ins.items()}
    out = mamba3_amd.chunked_ssd(*[leaf[k] for k in NAMES[:9]], chunk_size=64,
                                 h_init=leaf["h_init"], return_final_state=True)
    loss = (out.y * dy.float().to(dev)).sum()
    if dhf is not None:
        loss = loss + (out.h_final * dhf.float().to(dev)).sum()
    loss.backward()
    return out, {k: v.grad for k, v in leaf.items() if v is not None}


@pytest.mark.parametrize("case", CASES, ids=lambda c: "B{}T{}H{}P{}N{}R{}{}{}{}".format(
    *c[:6], "b" if c[6] else "", "i" if c[7] else "", "f" if c[8] else ""))
def test_chunked_ssd_backward_matches_oracle(case, cuda_device):
    B, T, H, P, N, R = case[:6]
    print(f"chunked_ssd backward case {case}", flush=True)
    ins = _inputs(case)
    g = torch.Generator().manual_seed(1)
    dy = torch.randn(B, T, H, P, R, generator=g, dtype=torch.float64)
    dhf = torch.randn(B, H, P, N, generator=g, dtype=torch.float64) if case[8] else None
    leaf = {k: (v.clone().requires_grad_() if v is not None else None) for k, v in ins.items()}
    y, hf = ref.chunked_ssd(*[leaf[k] for k in NAMES[:9]], chunk_size=64, h_init=leaf["h_init"],
                            return_final_state=True)
    loss = (y * dy).sum() + ((hf * dhf).sum() if dhf is not None else 0.0)
    loss.backward()
    out, grads = _gpu_grads(ins, dy, dhf, cuda_device)
    assert max_rel(out.y, y) < FP32_TOL
    for k, gk in grads.items():
        err = max_rel(gk, leaf[k].grad)
        assert err < FP32_TOL, (k, err)
        assert gk.dtype == torch.float32 and gk.shape == leaf[k].shape


def test_chunked_ssd_backward_bf16_inputs(cuda_device):
    """bf16 inputs (the backward upcasts them and runs in fp32; gradients come back in the
    inputs' dtype) against autograd through the fp64 oracle on the bf16-rounded inputs, at
    the bf16 tolerance; rank 3 with the beta terms (the padded tiles)."""
    case = (2, 77, 2, 16, 32, 3, True, True, True)
    B, T, H, P, N, R = case[:6]
    ins = {k: (v.to(torch.bfloat16).double() if v is not None and k not in ("A", "D", "h_init") else v)
           for k, v in _inputs(case, seed=31).items()}
    g = torch.Generator().manual_seed(32)
    dy = torch.randn(B, T, H, P, R, generator=g, dtype=torch.float64)
    dhf = torch.randn(B, H, P, N, generator=g, dtype=torch.float64)
    leaf = {k: (v.clone().requires_grad_() if v is not None else None) for k, v in ins.items()}
    y, hf = ref.chunked_ssd(*[leaf[k] for k in NAMES[:9]], chunk_size=64, h_init=leaf["h_init"],
                            return_final_state=True)
    ((y * dy).sum() + (hf * dhf).sum()).backward()
    dev = cuda_device
    bf = {"A", "D", "h_init"}
    gl = {k: (v.to(dev, torch.float32 if k in bf else torch.bfloat16).requires_grad_()
              if v is not None else None) for k, v in ins.items()}
    out = mamba3_amd.chunked_ssd(*[gl[k] for k in NAMES[:9]], h_init=gl["h_init"],
                                 return_final_state=True)
    ((out.y.float() * dy.float().to(dev)).sum() + (out.h_final * dhf.float().to(dev)).sum()).backward()
    assert out.y.dtype == torch.bfloat16
    for k, v in gl.items():
        if v is None:
            continue
        assert v.grad.dtype == v.dtype, k
        err = max_rel(v.grad.float(), leaf[k].grad)
        assert err < BF16_TOL, (k, err)


def test_chunked_ssd_backward_long_sequence(cuda_device):
    """2048 tokens (64 backward chunks): gradients carried through the state scans over many
    chunks, against the fp64 oracle at the fp32 tolerance."""
    case = (1, 2048, 2, 32, 64, 2, True, True, True)
    B, T, H, P, N, R = case[:6]
    ins = _inputs(case, seed=21)
    ins["dt"] = ins["dt"] * 0.2  # keep exp(sum A dt) from underflowing over the sequence
    g = torch.Generator().manual_seed(22)
    dy = torch.randn(B, T, H, P, R, generator=g, dtype=torch.float64)
    dhf = torch.randn(B, H, P, N, generator=g, dtype=torch.float64)
    leaf = {k: (v.clone().requires_grad_() if v is not None else None) for k, v in ins.items()}
    y, hf = ref.chunked_ssd(*[leaf[k] for k in NAMES[:9]], chunk_size=64, h_init=leaf["h_init"],
                            return_final_state=True)
    ((y * dy).sum() + (hf * dhf).sum()).backward()
    _, grads = _gpu_grads(ins, dy, dhf, cuda_device)
    for k, gk in grads.items():
        assert max_rel(gk, leaf[k].grad) < FP32_TOL, k


def test_chunked_ssd_backward_is_deterministic(cuda_device):
    case = (2, 150, 2, 32, 64, 2, True, True, True)
    B, T, H, P, N, R = case[:6]
    ins = _inputs(case, seed=3)
    g = torch.Generator().manual_seed(4)
    dy = torch.randn(B, T, H, P, R, generator=g, dtype=torch.float64)
    dhf = torch.randn(B, H, P, N, generator=g, dtype=torch.float64)
    _, g1 = _gpu_grads(ins, dy, dhf, cuda_device)
    _, g2 = _gpu_grads(ins, dy, dhf, cuda_device)
    for k in g1:
        assert torch.equal(g1[k], g2[k]), k


def test_chunked_ssd_unsupported_rank_fails_before_the_forward(cuda_device):
    x = torch.randn(1, 8, 1, 4, 9, device=cuda_device, requires_grad=True)
    Bm = torch.randn(1, 8, 1, 8, 9, device=cuda_device)
    with pytest.raises(RuntimeError, match="not supported"):
        mamba3_amd.chunked_ssd(x, None, Bm, None, Bm, torch.rand(1, 8, 1, device=cuda_device),
                               -torch.ones(1, device=cuda_device), torch.ones(1, device=cuda_device),
                               x.detach())


LAYER_KW = [
    dict(d_model=64, d_state=16, headdim=16, mimo_rank=2),
    dict(d_model=64, d_state=16, headdim=16, mimo_rank=2, use_trapezoidal=False),
    dict(d_model=64, d_state=16, headdim=16, mimo_rank=2, use_complex_ssm=False),
    dict(d_model=64, d_state=32, headdim=16, mimo_rank=4, ngroups=2),
    dict(d_model=64, d_state=16, headdim=16, mimo_rank=1, use_trapezoidal=False,
         use_complex_ssm=False),
    dict(d_model=128, d_state=64, headdim=32, mimo_rank=2),
    dict(d_model=128, d_state=32, headdim=128, mimo_rank=2),  # slots wider than a wave
    # ranks 3, 5, 6, 7 (the chunk kernels on rank-4 / rank-8 tiles)
    dict(d_model=64, d_state=16, headdim=16, mimo_rank=3),
    dict(d_model=64, d_state=16, headdim=16, mimo_rank=5, ngroups=2),
    dict(d_model=64, d_state=32, headdim=16, mimo_rank=6, use_trapezoidal=False),
    dict(d_model=64, d_state=16, headdim=16, mimo_rank=7, use_complex_ssm=False),
    # the B/C backward's LDS past 64 KB (83 KB: d_state 256, rank 8); one head per group
    dict(d_model=64, d_state=256, headdim=16, mimo_rank=8),
    dict(d_model=64, d_state=64, headdim=16, mimo_rank=4, ngroups=8),
]


def _oracle_layer_grads(kw, layer, x, w, wh, dt_scale=None):
    params = {k: v.detach().double().cpu().clone().requires_grad_()
              for k, v in layer.state_dict().items()}
    xr = x.detach().double().cpu().clone().requires_grad_()
    ds = None if dt_scale is None else dt_scale.double().cpu().clone().requires_grad_()
    out, st = ref.layer_forward(oracle_cfg(kw), params, xr, dt_scale=ds, return_state=True)
    ((out * w.double().cpu()).sum() + (st["h"] * wh.double().cpu()).sum()).backward()
    grads = {k: v.grad for k, v in params.items()}
    if ds is not None:
        grads["dt_scale"] = ds.grad
    return out, grads, xr.grad


@pytest.mark.parametrize("kw", LAYER_KW, ids=lambda k: "-".join(f"{a}{b}" for a, b in k.items()))
def test_layer_prefill_gradients_match_oracle(kw, cuda_device):
    """Autograd through KulaMamba.prefill (the fp32 layer path forward, m3_layer_bwd
    backward) against autograd through the fp64 oracle layer
    (mamba3/mamba3.py:192-258), for every parameter and the input; the loss also reads the
    returned state h."""
    print(f"layer backward {kw}", flush=True)
    torch.manual_seed(0)
    layer = mamba3_amd.KulaMamba(**kw).to(cuda_device).train()
    H, P, N = layer.nheads, layer.headdim, layer.d_state
    g = torch.Generator().manual_seed(2)
    x = torch.randn(2, 45, kw["d_model"], generator=g)
    w = torch.randn(2, 45, kw["d_model"], generator=g)
    wh = torch.randn(2, H, P, N, generator=g)
    out_ref, pg, xg_ref = _oracle_layer_grads(kw, layer, x, w, wh)
    xd = x.to(cuda_device).requires_grad_()
    out, st = layer.prefill(xd)
    ((out * w.to(cuda_device)).sum() + (st["h"] * wh.to(cuda_device)).sum()).backward()
    assert max_rel(out, out_ref) < FP32_TOL
    assert max_rel(xd.grad, xg_ref) < FP32_TOL
    for name, p in layer.named_parameters():
        err = max_rel(p.grad, pg[name])
        assert err < FP32_TOL, (name, err)


@pytest.mark.parametrize("rank,T", [(2, 1), (2, 32), (2, 33), (2, 64), (1, 65), (4, 17)])
def test_layer_gradients_at_chunk_edges(rank, T, cuda_device):
    """Sequence lengths at the chunk edges of the backward (chunks of 32 tokens at rank 2, 64
    at rank 1, 16 at rank 4 with the trapezoid): one token, exactly one chunk, one token past
    a chunk end (where the B gradient of the chunk's first token goes to the previous
    chunk's last token), against the fp64 oracle layer. A gradient that vanishes
    identically (A_log at one token: A only scales the zero initial state) is checked
    against the layer's gradient scale, since the oracle's value is fp64 rounding noise."""
    kw = dict(d_model=64, d_state=16, headdim=16, mimo_rank=rank)
    print(f"layer backward at chunk edges rank {rank} T {T}", flush=True)
    torch.manual_seed(0)
    layer = mamba3_amd.KulaMamba(**kw).to(cuda_device).train()
    H, P, N = layer.nheads, layer.headdim, layer.d_state
    g = torch.Generator().manual_seed(5)
    x = torch.randn(2, T, kw["d_model"], generator=g)
    w = torch.randn(2, T, kw["d_model"], generator=g)
    wh = torch.randn(2, H, P, N, generator=g)
    out_ref, pg, xg_ref = _oracle_layer_grads(kw, layer, x, w, wh)
    xd = x.to(cuda_device).requires_grad_()
    out, st = layer.prefill(xd)
    ((out * w.to(cuda_device)).sum() + (st["h"] * wh.to(cuda_device)).sum()).backward()
    assert max_rel(out, out_ref) < FP32_TOL
    assert max_rel(xd.grad, xg_ref) < FP32_TOL
    scale = max(v.abs().max().item() for v in pg.values())
    for name, p in layer.named_parameters():
        if pg[name].abs().max().item() < 1e-8 * scale:
            err = p.grad.detach().abs().max().item() / scale
        else:
            err = max_rel(p.grad, pg[name])
        assert err < FP32_TOL, (name, err)


def test_layer_d768_gradients_match_oracle(cuda_device):
    """The d_model 768 layer (24 heads, headdim 64, d_state 128, rank 2) over 160 tokens:
    every parameter's gradient and the input's against the fp64 oracle layer."""
    kw = dict(d_model=768, d_state=128, headdim=64, mimo_rank=2)
    torch.manual_seed(0)
    layer = mamba3_amd.KulaMamba(**kw).to(cuda_device).train()
    g = torch.Generator().manual_seed(23)
    x = torch.randn(1, 160, 768, generator=g)
    w = torch.randn(1, 160, 768, generator=g)
    wh = torch.randn(1, layer.nheads, 64, 128, generator=g)
    out_ref, pg, xg_ref = _oracle_layer_grads(kw, layer, x, w, wh)
    xd = x.to(cuda_device).requires_grad_()
    out, st = layer.prefill(xd)
    ((out * w.to(cuda_device)).sum() + (st["h"] * wh.to(cuda_device)).sum()).backward()
    assert max_rel(out, out_ref) < FP32_TOL
    assert max_rel(xd.grad, xg_ref) < FP32_TOL
    for name, p in layer.named_parameters():
        assert max_rel(p.grad, pg[name]) < FP32_TOL, name


def test_layer_d4096_gradients_match_oracle(cuda_device):
    """KulaMamba(d_model=4096) with the reference defaults (128 heads, headdim 64, d_state
    128, rank 2; mamba3/mamba3.py:50-64) over 40 tokens: the training forward keeps the
    sin / cos of the RoPE rotation for a tile of heads at a time, so a layer this wide
    trains like the reference's. Every parameter's gradient and the input's against the
    fp64 oracle layer."""
    kw = dict(d_model=4096)
    torch.manual_seed(0)
    layer = mamba3_amd.KulaMamba(**kw).to(cuda_device).train()
    assert layer.nheads == 128
    g = torch.Generator().manual_seed(31)
    x = torch.randn(1, 40, 4096, generator=g)
    w = torch.randn(1, 40, 4096, generator=g)
    wh = torch.randn(1, layer.nheads, 64, 128, generator=g)
    out_ref, pg, xg_ref = _oracle_layer_grads(kw, layer, x, w, wh)
    xd = x.to(cuda_device).requires_grad_()
    out, st = layer.prefill(xd)
    ((out * w.to(cuda_device)).sum() + (st["h"] * wh.to(cuda_device)).sum()).backward()
    assert max_rel(out, out_ref) < FP32_TOL
    assert max_rel(xd.grad, xg_ref) < FP32_TOL
    for name, p in layer.named_parameters():
        assert max_rel(p.grad, pg[name]) < FP32_TOL, name


@pytest.mark.parametrize("kw", [LAYER_KW[0], LAYER_KW[3], LAYER_KW[2]],
                         ids=["default", "rank4-groups2", "complex-off"])
def test_layer_state_gradients_match_oracle(kw, cuda_device):
    """A loss over every prefill state tensor (h, angle, prev_BX) as well as the output: the
    state-gradient paths of the backward against the fp64 oracle."""
    torch.manual_seed(0)
    layer = mamba3_amd.KulaMamba(**kw).to(cuda_device).train()
    H, P, N = layer.nheads, layer.headdim, layer.d_state
    g = torch.Generator().manual_seed(9)
    x = torch.randn(2, 37, kw["d_model"], generator=g)
    w = torch.randn(2, 37, kw["d_model"], generator=g)
    wst = {"h": torch.randn(2, H, P, N, generator=g), "angle": torch.randn(2, H, N // 2, generator=g),
           "prev_BX": torch.randn(2, H, P, N, generator=g)}
    params = {k: v.detach().double().cpu().clone().requires_grad_()
              for k, v in layer.state_dict().items()}
    xr = x.double().requires_grad_()
    out_ref, st_ref = ref.layer_forward(oracle_cfg(kw), params, xr, return_state=True)
    loss = (out_ref * w.double()).sum()
    for k, v in wst.items():
        loss = loss + (st_ref[k].double() * v.double()).sum()
    loss.backward()
    xd = x.to(cuda_device).requires_grad_()
    out, st = layer.prefill(xd)
    loss = (out * w.to(cuda_device)).sum()
    for k, v in wst.items():
        loss = loss + (st[k] * v.to(cuda_device)).sum()
    loss.backward()
    assert max_rel(xd.grad, xr.grad) < FP32_TOL
    for name, p in layer.named_parameters():
        assert max_rel(p.grad, params[name].grad) < FP32_TOL, name


D768_KW = dict(d_model=768, d_state=128, headdim=64, mimo_rank=2)


@pytest.mark.parametrize("extra", [{}, dict(use_trapezoidal=False), dict(use_complex_ssm=False),
                                   # 24 groups without the trapezoid: the forward's B^ / C^ rows
                                   # leave no room for the chunk-start states, which the
                                   # backward then recomputes
                                   dict(use_trapezoidal=False, ngroups=24)],
                         ids=["default", "trapezoid-off", "complex-off", "trapezoid-off-24-groups"])
def test_layer_d768_fused_training_forward_state_gradients(extra, cuda_device):
    """The d_model 768 shape (d_state 128, headdim 64, rank 2) trains on the fused fp32
    prefill kernel, which also writes the per-token operands m3_layer_bwd reads. Two
    sequences of 93 tokens (a partial last 32-token chunk) and a loss over the output and
    every state tensor (h, angle, prev_BX): the input's and every parameter's gradient
    against the fp64 oracle layer."""
    kw = dict(D768_KW, **extra)
    print(f"d768 fused training forward {kw}", flush=True)
    torch.manual_seed(0)
    layer = mamba3_amd.KulaMamba(**kw).to(cuda_device).train()
    H, P, N = layer.nheads, layer.headdim, layer.d_state
    g = torch.Generator().manual_seed(31)
    x = torch.randn(2, 93, 768, generator=g)
    w = torch.randn(2, 93, 768, generator=g)
    wst = {"h": torch.randn(2, H, P, N, generator=g), "angle": torch.randn(2, H, N // 2, generator=g),
           "prev_BX": torch.randn(2, H, P, N, generator=g)}
    params = {k: v.detach().double().cpu().clone().requires_grad_()
              for k, v in layer.state_dict().items()}
    xr = x.double().requires_grad_()
    out_ref, st_ref = ref.layer_forward(oracle_cfg(kw), params, xr, return_state=True)
    loss = (out_ref * w.double()).sum()
    for k, v in wst.items():
        loss = loss + (st_ref[k].double() * v.double()).sum()
    loss.backward()
    xd = x.to(cuda_device).requires_grad_()
    out, st = layer.prefill(xd)
    loss = (out * w.to(cuda_device)).sum()
    for k, v in wst.items():
        loss = loss + (st[k] * v.to(cuda_device)).sum()
    loss.backward()
    assert max_rel(out, out_ref) < FP32_TOL
    for k in wst:
        assert max_rel(st[k], st_ref[k]) < FP32_TOL, k
    assert max_rel(xd.grad, xr.grad) < FP32_TOL
    for name, p in layer.named_parameters():
        assert max_rel(p.grad, params[name].grad) < FP32_TOL, name


def test_layer_training_runs_on_the_native_backward(cuda_device):
    """The parity tests above go through m3_layer_bwd: it covers every configuration they use."""
    from mamba3_amd import _native
    for kw in LAYER_KW + [dict(d_model=768, d_state=128, headdim=64, mimo_rank=2)]:
        layer = mamba3_amd.KulaMamba(**kw).to(cuda_device)
        proj = torch.empty(1, 8, layer.in_proj.out_features, device=cuda_device)
        assert _native.layer_bwd_supported(layer._desc(1, 8, proj)), kw


def test_layer_training_outside_the_native_backward_raises(cuda_device):
    """A shape beyond the kernels (rank 9) raises a clear error when trained, before the
    forward runs, rather than falling back to another implementation."""
    from mamba3_amd import _native
    kw = dict(d_model=64, d_state=16, headdim=16, mimo_rank=9)
    torch.manual_seed(0)
    layer = mamba3_amd.KulaMamba(**kw).to(cuda_device).train()
    x = torch.randn(2, 40, 64, device=cuda_device)
    with pytest.raises(_native.NativeError, match="not supported by m3_layer_bwd"):
        layer(x.requires_grad_())


def test_layer_forward_gradients_with_dt_scale(cuda_device):
    kw = dict(d_model=64, d_state=16, headdim=16, mimo_rank=2)
    torch.manual_seed(0)
    layer = mamba3_amd.KulaMamba(**kw).to(cuda_device).train()
    g = torch.Generator().manual_seed(5)
    x = torch.randn(1, 30, 64, generator=g)
    w = torch.randn(1, 30, 64, generator=g)
    ds = torch.rand(1, 30, layer.nheads, generator=g) + 0.5
    wh = torch.zeros(1, layer.nheads, 16, 16)
    out_ref, pg, xg_ref = _oracle_layer_grads(kw, layer, x, w, wh, dt_scale=ds)
    xd = x.to(cuda_device).requires_grad_()
    dsd = ds.to(cuda_device).requires_grad_()
    out = layer(xd, dt_scale=dsd)
    (out * w.to(cuda_device)).sum().backward()
    assert max_rel(out, out_ref) < FP32_TOL
    assert max_rel(xd.grad, xg_ref) < FP32_TOL
    assert max_rel(dsd.grad, pg["dt_scale"]) < FP32_TOL
    for name, p in layer.named_parameters():
        assert max_rel(p.grad, pg[name]) < FP32_TOL, name


def test_layer_d768_fused_training_forward_with_dt_scale(cuda_device):
    """dt_scale through the fused fp32 training forward (d_model 768 shape): the output, the
    input's, dt_scale's and every parameter's gradient against the fp64 oracle."""
    torch.manual_seed(0)
    layer = mamba3_amd.KulaMamba(**D768_KW).to(cuda_device).train()
    g = torch.Generator().manual_seed(12)
    x = torch.randn(1, 70, 768, generator=g)
    w = torch.randn(1, 70, 768, generator=g)
    ds = torch.rand(1, 70, layer.nheads, generator=g) + 0.5
    wh = torch.randn(1, layer.nheads, 64, 128, generator=g)
    out_ref, pg, xg_ref = _oracle_layer_grads(D768_KW, layer, x, w, wh, dt_scale=ds)
    xd = x.to(cuda_device).requires_grad_()
    dsd = ds.to(cuda_device).requires_grad_()
    out, st = layer.prefill(xd, dt_scale=dsd)
    ((out * w.to(cuda_device)).sum() + (st["h"] * wh.to(cuda_device)).sum()).backward()
    assert max_rel(out, out_ref) < FP32_TOL
    assert max_rel(xd.grad, xg_ref) < FP32_TOL
    assert max_rel(dsd.grad, pg["dt_scale"]) < FP32_TOL
    for name, p in layer.named_parameters():
        assert max_rel(p.grad, pg[name]) < FP32_TOL, name


def test_layer_bf16_gradients_match_fp32_oracle(cuda_device):
    kw = dict(d_model=128, d_state=64, headdim=32, mimo_rank=2)
    torch.manual_seed(0)
    layer = mamba3_amd.KulaMamba(**kw).to(cuda_device, torch.bfloat16).train()
    g = torch.Generator().manual_seed(6)
    x = torch.randn(2, 70, 128, generator=g).bfloat16()
    w = torch.randn(2, 70, 128, generator=g)
    wh = torch.zeros(2, layer.nheads, 32, 64)
    out_ref, pg, xg_ref = _oracle_layer_grads(kw, layer, x.float(), w, wh)
    xd = x.to(cuda_device).requires_grad_()
    out = layer(xd)
    (out.float() * w.to(cuda_device)).sum().backward()
    assert max_rel(out, out_ref) < BF16_TOL
    assert max_rel(xd.grad, xg_ref) < BF16_TOL
    for name, p in layer.named_parameters():
        assert max_rel(p.grad, pg[name]) < BF16_TOL, name


def test_lm_training_steps_reduce_the_loss(cuda_device):
    """A few SGD steps of the LM through forward(ids, labels) (mamba3/block.py:168-178)
    lower the loss on a fixed batch, with finite gradients everywhere."""
    torch.manual_seed(0)
    lm = mamba3_amd.KulaMambaLM(vocab_size=64, d_model=64, n_layers=2, d_state=16, headdim=16,
                                mimo_rank=2).to(cuda_device).train()
    opt = torch.optim.SGD(lm.parameters(), lr=0.05)
    g = torch.Generator().manual_seed(7)
    ids = torch.randint(0, 64, (2, 33), generator=g).to(cuda_device)
    losses = []
    for _ in range(6):
        opt.zero_grad()
        loss = lm(ids, labels=ids)["loss"]
        loss.backward()
        for p in lm.parameters():
            assert p.grad is not None and torch.isfinite(p.grad).all()
        opt.step()
        losses.append(loss.item())
    assert losses[-1] < losses[0] - 1e-3, losses


def test_lm_gradient_checkpointing_gives_the_same_gradients(cuda_device):
    """KulaMambaLM(gradient_checkpointing=True) recomputes each block's forward during the
    backward (mamba3/block.py:79-92); the native kernels are deterministic, so the gradients
    equal the stored-activation run bit for bit."""
    def grads(ckpt):
        torch.manual_seed(0)
        lm = mamba3_amd.KulaMambaLM(vocab_size=64, d_model=64, n_layers=2, d_state=16, headdim=16,
                                    mimo_rank=2, gradient_checkpointing=ckpt).to(cuda_device).train()
        ids = torch.randint(0, 64, (2, 40), generator=torch.Generator().manual_seed(10)).to(cuda_device)
        lm(ids, labels=ids)["loss"].backward()
        return {n: p.grad.clone() for n, p in lm.named_parameters()}
    g0, g1 = grads(False), grads(True)
    for n in g0:
        assert torch.equal(g0[n], g1[n]), n


STEP_KW = LAYER_KW[:5] + [dict(d_model=768, d_state=128, headdim=64, mimo_rank=2),
                          dict(d_model=64, d_state=48, headdim=16, mimo_rank=8, ngroups=2),
                          # the head kernel's LDS past 64 KB (70 KB)
                          dict(d_model=64, d_state=512, headdim=16, mimo_rank=8)]


@pytest.mark.parametrize("kw", STEP_KW, ids=lambda k: "-".join(f"{a}{b}" for a, b in k.items()))
def test_step_gradients_match_oracle(kw, cuda_device):
    """Autograd through KulaMamba.step (m3_step_bwd between in_proj and out_proj) against
    autograd through the fp64 oracle step (mamba3/mamba3.py:267-322) from a random state: a
    loss over the output and every new-state tensor; the gradients of the input, of the
    incoming h, prev_BX and angle, of every parameter and of dt_scale at 1e-4."""
    print(f"step backward {kw}", flush=True)
    torch.manual_seed(0)
    layer = mamba3_amd.KulaMamba(**kw).to(cuda_device).train()
    H, P, N = layer.nheads, layer.headdim, layer.d_state
    g = torch.Generator().manual_seed(17)
    Bat = 3
    x = torch.randn(Bat, kw["d_model"], generator=g)
    st = {"h": torch.randn(Bat, H, P, N, generator=g), "prev_BX": torch.randn(Bat, H, P, N, generator=g),
          "angle": torch.randn(Bat, H, N // 2, generator=g)}
    ds = torch.rand(Bat, H, generator=g) + 0.5
    w = torch.randn(Bat, kw["d_model"], generator=g)
    wst = {k: torch.randn(v.shape, generator=g) for k, v in st.items()}

    params = {k: v.detach().double().cpu().clone().requires_grad_()
              for k, v in layer.state_dict().items()}
    xr = x.double().requires_grad_()
    st_r = {k: v.double().requires_grad_() for k, v in st.items()}
    ds_r = ds.double().requires_grad_()
    out_r, new_r = ref.layer_step(oracle_cfg(kw), params, xr, st_r, dt_scale=ds_r)
    loss = (out_r * w.double()).sum()
    for k in wst:
        loss = loss + (new_r[k] * wst[k].double()).sum()
    loss.backward()

    xd = x.to(cuda_device).requires_grad_()
    st_d = {k: v.to(cuda_device).requires_grad_() for k, v in st.items()}
    ds_d = ds.to(cuda_device).requires_grad_()
    out, new = layer.step(xd, st_d, dt_scale=ds_d)
    loss = (out * w.to(cuda_device)).sum()
    for k in wst:
        loss = loss + (new[k] * wst[k].to(cuda_device)).sum()
    loss.backward()
    assert max_rel(out, out_r) < FP32_TOL
    assert max_rel(xd.grad, xr.grad) < FP32_TOL
    assert max_rel(ds_d.grad, ds_r.grad) < FP32_TOL
    for k in st:
        assert max_rel(st_d[k].grad, st_r[k].grad) < FP32_TOL, k
    for name, p in layer.named_parameters():
        assert max_rel(p.grad, params[name].grad) < FP32_TOL, name


def test_step_gradients_of_the_output_alone(cuda_device):
    """A loss over the output only (the new state's gradients are None) and no dt_scale."""
    kw = dict(d_model=64, d_state=16, headdim=16, mimo_rank=2)
    torch.manual_seed(0)
    layer = mamba3_amd.KulaMamba(**kw).to(cuda_device).train()
    H, P, N = layer.nheads, layer.headdim, layer.d_state
    g = torch.Generator().manual_seed(18)
    x = torch.randn(2, 64, generator=g)
    st = {"h": torch.randn(2, H, P, N, generator=g), "prev_BX": torch.randn(2, H, P, N, generator=g),
          "angle": torch.randn(2, H, N // 2, generator=g)}
    params = {k: v.detach().double().cpu().clone().requires_grad_()
              for k, v in layer.state_dict().items()}
    xr = x.double().requires_grad_()
    out_r, _ = ref.layer_step(oracle_cfg(kw), params, xr, {k: v.double() for k, v in st.items()})
    out_r.square().sum().backward()
    xd = x.to(cuda_device).requires_grad_()
    out, _ = layer.step(xd, {k: v.to(cuda_device) for k, v in st.items()})
    out.square().sum().backward()
    assert max_rel(xd.grad, xr.grad) < FP32_TOL
    for name, p in layer.named_parameters():
        assert max_rel(p.grad, params[name].grad) < FP32_TOL, name


def test_lm_step_chain_backpropagates(cuda_device):
    """Gradients flow through a few chained decode steps of a two-layer LM (state carried from
    step to step) and are finite; bf16 parameters get bf16 gradients."""
    torch.manual_seed(0)
    lm = mamba3_amd.KulaMambaLM(vocab_size=64, d_model=64, n_layers=2, d_state=16, headdim=16,
                                mimo_rank=2).to(cuda_device, torch.bfloat16).train()
    states = [blk.ssm.allocate_inference_state(2) for blk in lm.layers]
    loss = 0.0
    tok = torch.tensor([3, 5], device=cuda_device)
    for _ in range(3):
        x = lm.embedding(tok)
        for i, blk in enumerate(lm.layers):
            x, states[i] = blk.step(x, states[i])
        logits = lm.lm_head(lm.norm(x))
        loss = loss + logits.float().logsumexp(-1).sum()
        tok = logits.argmax(-1)
    loss.backward()
    for name, p in lm.named_parameters():
        assert p.grad is not None and p.grad.dtype == p.dtype, name
        assert torch.isfinite(p.grad.float()).all(), name
