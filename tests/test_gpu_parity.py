"""GPU parity of the HIP path against the oracle and the reference's golden vectors.

Tolerances (normwise max-relative error, max|y - y_ref| / max|y_ref|):
  * fp32 kernels vs fp32 reference/oracle: 1e-4
  * bf16 kernels vs fp32 oracle on the bf16-rounded weights and inputs: 2e-2
Every test calls the kernels through the C-ABI library (mamba3_amd/lib).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import mamba3_amd
from conftest import (CHUNKED_CASES, LAYER_CASES, golden_config, golden_params, load_golden,
                      max_rel, oracle_cfg)
from mamba3_amd import _native
from oracle import recurrence as rec
from oracle import reference_path as ref

pytestmark = pytest.mark.gpu

FP32_TOL = 1e-4
BF16_TOL = 2e-2


@pytest.fixture(scope="module", autouse=True)
def _native_loaded(cuda_device):
    lib = _native.lib()  # raises if the library is missing
    assert lib.m3_version() >= 100
    torch.backends.cuda.matmul.allow_tf32 = False
    torch.backends.cudnn.allow_tf32 = False


def _layer_from_golden(g, dev, dtype=torch.float32):
    kw = golden_config(g)
    torch.manual_seed(0)
    layer = mamba3_amd.KulaMamba(**kw)
    layer.load_state_dict(golden_params(g))
    return layer.to(dev, dtype).eval(), kw


# ------------------------------------------------------------------ golden, fp32
@pytest.mark.parametrize("name", LAYER_CASES)
def test_forward_prefill_step_match_reference_golden(name, cuda_device):
    g = load_golden(name)
    layer, _ = _layer_from_golden(g, cuda_device)
    x = torch.from_numpy(g["x"]).to(cuda_device)
    with torch.no_grad():
        y = layer(x)
        assert max_rel(y, torch.from_numpy(g["y"])) < FP32_TOL
        y_pf, st = layer.prefill(x)
        assert max_rel(y_pf, torch.from_numpy(g["y_prefill"])) < FP32_TOL
        for k in ("h", "angle", "prev_BX"):
            assert max_rel(st[k], torch.from_numpy(g[f"prefill/{k}"])) < FP32_TOL, k
        xs = torch.from_numpy(g["x_steps"]).to(cuda_device)
        outs = []
        for t in range(xs.shape[1]):
            if t % 2 == 0:
                o, st = layer.step(xs[:, t], st)
            else:
                o, st = layer.step(xs[:, t:t + 1], st)
                assert o.dim() == 3
                o = o.squeeze(1)
            outs.append(o)
        assert max_rel(torch.stack(outs, 1), torch.from_numpy(g["y_steps"])) < FP32_TOL
        for k in ("h", "angle", "prev_BX"):
            assert max_rel(st[k], torch.from_numpy(g[f"steps/{k}"])) < FP32_TOL, k


def test_dt_scale_matches_reference_golden(cuda_device):
    g = load_golden("layer_tiny_dtscale")
    layer, _ = _layer_from_golden(g, cuda_device)
    x = torch.from_numpy(g["x"]).to(cuda_device)
    ds = torch.from_numpy(g["dt_scale"]).to(cuda_device)
    with torch.no_grad():
        y = layer(x, dt_scale=ds)
        y1 = layer(x)
    assert max_rel(y, torch.from_numpy(g["y"])) < FP32_TOL
    assert not torch.allclose(y, y1, atol=1e-5)


@pytest.mark.parametrize("name", CHUNKED_CASES)
def test_chunked_ssd_matches_reference_golden(name, cuda_device):
    g = load_golden(name)
    t = {k: torch.from_numpy(v).to(cuda_device) for k, v in g.items() if v.dtype != np.int64}
    res = mamba3_amd.chunked_ssd(t["x_g"], t.get("x_b"), t["B_g"], t.get("B_b"), t["C"],
                                 t["dt"], t["A"], t["D"], t["x_raw"], int(g["chunk_size"]),
                                 h_init=t.get("h_init"), return_final_state=True)
    assert max_rel(res.y, torch.from_numpy(g["y"])) < FP32_TOL
    assert max_rel(res.h_final, torch.from_numpy(g["h_final"])) < FP32_TOL


@pytest.mark.parametrize("beta,R", [(True, 2), (False, 1), (True, 4), (False, 3), (True, 3),
                                    (False, 5), (True, 6), (True, 7)])
def test_chunked_ssd_generic_and_mfma_paths_match_oracle(beta, R, cuda_device):
    """fp32 chunked_ssd on both native paths (the fp32-MFMA chunk kernels, used when a
    workspace is given -- ranks 3, 5, 6 and 7 on their rank-4 / rank-8 tiles -- and the
    generic kernel) and in bf16 against the fp32 oracle (mamba3/ssd.py:118-244)."""
    g = torch.Generator().manual_seed(13)
    Bt, T, H, P, N = 2, 150, 3, 16, 32
    r = lambda *s: torch.randn(*s, generator=g)
    x_g, x_raw = r(Bt, T, H, P, R), r(Bt, T, H, P, R)
    x_b = r(Bt, T, H, P, R) if beta else None
    B_g, C = r(Bt, T, H, N, R), r(Bt, T, H, N, R)
    B_b = r(Bt, T, H, N, R) if beta else None
    dt = torch.rand(Bt, T, H, generator=g) * 0.3
    A, D, h0 = -torch.rand(H, generator=g) - 0.1, r(H), r(Bt, H, P, N)
    y_ref, h_ref = ref.chunked_ssd(x_g.double(), None if x_b is None else x_b.double(),
                                   B_g.double(), None if B_b is None else B_b.double(),
                                   C.double(), dt.double(), A.double(), D.double(),
                                   x_raw.double(), 64, h_init=h0.double(), return_final_state=True)
    dev = cuda_device
    to = lambda t, dtype=torch.float32: None if t is None else t.to(dev, dtype).contiguous()
    for use_ws in (True, False):
        y = torch.empty(Bt, T, H, P, R, device=dev)
        hf = torch.empty(Bt, H, P, N, device=dev)
        _native.chunked_fwd(Bt, T, H, P, N, R, torch.float32, to(x_g), to(x_b), to(B_g), to(B_b),
                            to(C), to(dt), to(A), to(D), to(x_raw), to(h0), y, hf, None,
                            use_workspace=use_ws)
        assert max_rel(y, y_ref) < FP32_TOL, use_ws
        assert max_rel(hf, h_ref) < FP32_TOL, use_ws
    bf = lambda t: to(t, torch.bfloat16)
    out = mamba3_amd.chunked_ssd(bf(x_g), bf(x_b), bf(B_g), bf(B_b), bf(C), bf(dt), to(A), to(D),
                                 bf(x_raw), h_init=to(h0), return_final_state=True)
    assert out.y.dtype == torch.bfloat16
    y_ref_b, h_ref_b = ref.chunked_ssd(*[None if t is None else t.to(torch.bfloat16).double()
                                         for t in (x_g, x_b, B_g, B_b, C, dt)],
                                       A.double(), D.double(), x_raw.to(torch.bfloat16).double(),
                                       64, h_init=h0.double(), return_final_state=True)
    assert max_rel(out.y, y_ref_b) < BF16_TOL
    assert max_rel(out.h_final, h_ref_b) < BF16_TOL


def test_chunked_ssd_h_init_zero_equals_none(cuda_device):
    """Reference test_ssd_h_init (tests/test_mamba3.py:670-695)."""
    g = load_golden("chunked_beta_hinit")
    t = {k: torch.from_numpy(v).to(cuda_device) for k, v in g.items() if v.dtype != np.int64}
    args = (t["x_g"], t["x_b"], t["B_g"], t["B_b"], t["C"], t["dt"], t["A"], t["D"], t["x_raw"])
    out0 = mamba3_amd.chunked_ssd(*args, 8, return_final_state=True)
    out1 = mamba3_amd.chunked_ssd(*args, 8, h_init=torch.zeros_like(t["h_init"]),
                                  return_final_state=True)
    out2 = mamba3_amd.chunked_ssd(*args, 8, h_init=t["h_init"], return_final_state=True)
    assert (out0.y - out1.y).abs().max().item() < 1e-6
    assert (out0.y - out2.y).abs().max().item() > 1e-3


def test_d768_fp32_forward_matches_reference_golden(cuda_device):
    """d_model=768, N=128, P=64, R=2 layer, seed-0 weights, x (4,1024,768) from seed 1."""
    g = load_golden("layer_d768")
    torch.manual_seed(0)
    layer = mamba3_amd.KulaMamba(768, d_state=128, expand=2, headdim=64, mimo_rank=2)
    layer = layer.to(cuda_device).eval()
    torch.manual_seed(1)
    x = torch.randn(4, 1024, 768)
    assert float(x.double().sum()) == pytest.approx(float(g["x_sum"]), rel=1e-12)
    with torch.no_grad():
        y, st = layer.prefill(x.to(cuda_device))
    ys = torch.from_numpy(g["y_slice"])
    assert max_rel(y[:, ::64, ::16], ys) < FP32_TOL
    assert float(y.double().sum()) == pytest.approx(float(g["y_sum"]), rel=1e-3, abs=1e-2)
    assert max_rel(st["h"][:, :, ::8, ::16], torch.from_numpy(g["h_slice"])) < FP32_TOL
    assert max_rel(st["angle"][:, :, ::8], torch.from_numpy(g["angle_slice"])) < FP32_TOL
    assert max_rel(st["prev_BX"][:, :, ::8, ::16], torch.from_numpy(g["prev_slice"])) < FP32_TOL


def test_tiny_lm_logits_and_greedy_generation_match_reference(cuda_device):
    g = load_golden("lm_tiny")
    torch.manual_seed(0)
    lm = mamba3_amd.KulaMambaLM(vocab_size=256, d_model=64, n_layers=2, d_state=16, headdim=16,
                                mimo_rank=2, chunk_size=8)
    lm.load_state_dict(golden_params(g))
    lm = lm.to(cuda_device).eval()
    ids = torch.from_numpy(g["ids"]).to(cuda_device)
    with torch.no_grad():
        logits = lm(ids)["logits"]
        gen = lm.generate(ids[:, :5], max_new_tokens=6, temperature=0)
    assert max_rel(logits, torch.from_numpy(g["logits"])) < FP32_TOL
    assert torch.equal(gen.cpu(), torch.from_numpy(g["generated"]))


def test_lm_decode_graph_replays_equal_eager_steps(cuda_device):
    """The captured decode step (HIP graph) against the eager step loop, on a 3-layer
    d_model-768 LM in bf16: every replay's logits are bitwise the eager logits, with eager
    work and synchronisations between replays, and greedy generation agrees token for token."""
    from mamba3_amd.block import _DecodeGraph, _lm_logits
    torch.manual_seed(0)
    lm = mamba3_amd.KulaMambaLM(32000, 768, n_layers=3, d_state=128, headdim=64,
                                mimo_rank=2).to(cuda_device, torch.bfloat16).eval()
    torch.manual_seed(5)
    ids = torch.randint(0, 32000, (4, 64), device=cuda_device)
    with torch.no_grad():
        x = lm.embedding(ids)
        states = []
        for layer in lm.layers:
            x, st = layer.prefill(x)
            states.append(st)
        graph = _DecodeGraph(lm, states, 4)
        g = torch.Generator(device=cuda_device).manual_seed(1)
        for _ in range(8):
            tok = torch.randint(0, 32000, (4,), device=cuda_device, generator=g)
            xe = lm.embedding(tok)
            for i, layer in enumerate(lm.layers):
                xe, states[i] = layer.step(xe, states[i])
            ref_logits = _lm_logits(lm, xe)
            torch.cuda.synchronize()
            out = graph(tok)
            torch.cuda.synchronize()
            assert torch.equal(out, ref_logits)
        lm.decode_graph = False
        eager = lm.generate(ids, max_new_tokens=16, temperature=0)
        lm.decode_graph = True
        graphed = lm.generate(ids, max_new_tokens=16, temperature=0)
    assert torch.equal(eager, graphed)


# ------------------------------------------------------------------ scan
@pytest.mark.parametrize("shape", [(2, 4, 3, 8), (2, 7, 3, 10), (1, 33, 2, 32768), (8, 16, 24, 8192),
                                   (1, 3, 2, 1 << 20), (1, 1, 2, 1 << 20)])
@pytest.mark.parametrize("with_init", [True, False])
def test_scan_matches_closed_form(shape, with_init, cuda_device):
    B, K, H, PN = shape
    g = torch.Generator().manual_seed(K * 31 + PN)
    d = torch.rand(B, K, H, generator=g) * 0.9 + 0.05
    hc = torch.randn(B, K, H, PN, generator=g)
    h0 = torch.randn(B, H, PN, generator=g) if with_init else None
    out = mamba3_amd.ssd_scan(d.to(cuda_device), hc.to(cuda_device),
                              None if h0 is None else h0.to(cuda_device))
    if B * K * H * PN <= 1 << 20:
        expect = torch.from_numpy(rec.scan_closed_form(d.numpy(), hc.numpy(),
                                                       None if h0 is None else h0.numpy()))
    else:
        expect = ref.scan_forward(d, hc, h0)
    assert max_rel(out, expect) < 1e-5


@pytest.mark.parametrize("shape", [(2, 7, 3, 512), (2, 9, 3, 100), (1, 33, 2, 1024),
                                   (8, 16, 24, 8192), (1, 1, 2, 256), (1, 3, 2, 1 << 20),
                                   (1, 1, 2, 1 << 20)])
@pytest.mark.parametrize("with_init", [True, False])
def test_scan_backward_matches_oracle(shape, with_init, cuda_device):
    """ssd_scan's backward (m3_scan_bwd: eight float4 columns per lane for PN % 2048 == 0 and
    at least 262,144 float4 columns in all, one per lane for other PN % 256 == 0, the
    per-(b,h) block path otherwise) through autograd against the oracle's backward
    (mamba3/scan.py:47-62)."""
    B, K, H, PN = shape
    g = torch.Generator().manual_seed(K * 7 + PN)
    d = torch.rand(B, K, H, generator=g) * 0.5 + 0.5
    hc = torch.randn(B, K, H, PN, generator=g)
    h0 = torch.randn(B, H, PN, generator=g) if with_init else None
    gout = torch.randn(B, K, H, PN, generator=g)
    states = ref.scan_forward(d, hc, h0)
    dd_r, dc_r, dh_r = ref.scan_backward(d, states, gout, with_init)
    dg = d.to(cuda_device).requires_grad_()
    hg = hc.to(cuda_device).requires_grad_()
    ig = h0.to(cuda_device).requires_grad_() if with_init else None
    out = mamba3_amd.ssd_scan(dg, hg, ig)
    out.backward(gout.to(cuda_device))
    assert max_rel(out.detach(), states) < FP32_TOL
    assert max_rel(dg.grad, dd_r) < FP32_TOL
    assert max_rel(hg.grad, dc_r) < FP32_TOL
    if with_init:
        assert max_rel(ig.grad, dh_r) < FP32_TOL
    # deterministic: the same gradients twice, bit for bit
    dg2 = d.to(cuda_device).requires_grad_()
    mamba3_amd.ssd_scan(dg2, hc.to(cuda_device), ig.detach() if with_init else None).backward(
        gout.to(cuda_device))
    assert torch.equal(dg2.grad, dg.grad)


def test_scan_bf16_roundtrip_dtype(cuda_device):
    d = torch.rand(1, 5, 2, device=cuda_device)
    hc = torch.randn(1, 5, 2, 4, 6, device=cuda_device, dtype=torch.bfloat16)
    out = mamba3_amd.ssd_scan(d, hc)
    assert out.dtype == torch.bfloat16 and out.shape == hc.shape
    expect = ref.scan_forward(d.cpu(), hc.float().cpu().reshape(1, 5, 2, 24)).reshape(hc.shape)
    assert max_rel(out.float(), expect) < 1e-2


# ------------------------------------------------------------------ reference invariants
def _tiny(dev, **kw):
    d = dict(d_model=64, d_state=16, headdim=16, mimo_rank=2, expand=2, chunk_size=8)
    d.update(kw)
    torch.manual_seed(0)
    return mamba3_amd.KulaMamba(**d).to(dev).eval()


def _steps(layer, x):
    st = layer.allocate_inference_state(x.shape[0], device=x.device)
    outs = []
    for t in range(x.shape[1]):
        o, st = layer.step(x[:, t:t + 1], st)
        outs.append(o.squeeze(1))
    return torch.stack(outs, 1), st


@pytest.mark.parametrize("kw,T,tol", [
    ({}, 24, 1e-4), (dict(ngroups=2), 16, 1e-4), (dict(use_trapezoidal=False), 16, 1e-4),
    (dict(use_complex_ssm=False), 16, 1e-4),
    (dict(use_trapezoidal=False, use_complex_ssm=False, mimo_rank=1), 16, 1e-4),
    ({}, 512, 1e-3), ({}, 1, 1e-4)])
def test_forward_equals_sequential_steps(kw, T, tol, cuda_device):
    """Reference tests 35-52, 182-258, 355-374, 698-764: parallel == recurrent."""
    layer = _tiny(cuda_device, **kw)
    torch.manual_seed(1)
    x = torch.randn(1 if T > 1 else 2, T, 64, device=cuda_device)
    with torch.no_grad():
        y_par = layer(x)
        y_seq, st = _steps(layer, x)
        _, st_pf = layer.prefill(x)
    assert (y_par - y_seq).abs().max().item() < tol
    for k in ("h", "angle", "prev_BX"):
        assert (st[k] - st_pf[k]).abs().max().item() < tol, k


def test_prefill_then_step_equals_all_steps(cuda_device):
    layer = _tiny(cuda_device)
    torch.manual_seed(2)
    x = torch.randn(1, 24, 64, device=cuda_device)
    with torch.no_grad():
        y_gt, _ = _steps(layer, x)
        _, st = layer.prefill(x[:, :16])
        outs = []
        for t in range(16, 24):
            o, st = layer.step(x[:, t], st)
            outs.append(o)
    assert (torch.stack(outs, 1) - y_gt[:, 16:]).abs().max().item() < 1e-4


def test_extreme_decay(cuda_device):
    """Reference tests 410-447: A_log=0, dt_bias=3 finite; A_log=-0.5, dt_bias=2 within 5e-3."""
    layer = _tiny(cuda_device)
    with torch.no_grad():
        layer.A_log.fill_(0.0)
        layer.dt_bias.fill_(3.0)
        y = layer(torch.randn(1, 64, 64, device=cuda_device))
    assert torch.isfinite(y).all() and y.abs().max() > 0
    layer = _tiny(cuda_device)
    with torch.no_grad():
        layer.A_log.fill_(-0.5)
        layer.dt_bias.fill_(2.0)
        x = torch.randn(1, 24, 64, device=cuda_device)
        y_par = layer(x)
        y_seq, _ = _steps(layer, x)
    assert (y_par - y_seq).abs().max().item() < 5e-3


def test_mimo_cross_rank(cuda_device):
    layer = _tiny(cuda_device)
    x = torch.randn(1, 16, 64, device=cuda_device)
    with torch.no_grad():
        y_full = layer(x)
        layer.mimo_x.data[:, :, 1] = 0.0
        y_zero = layer(x)
    assert (y_full - y_zero).abs().max().item() > 1e-5


@pytest.mark.parametrize("PN,offset", [(20000, 0), (32768, 1)])
def test_scan_backward_many_columns_off_the_vector_path(PN, offset, cuda_device):
    """m3_scan_bwd with more than 16384 columns on the per-(b,h) kernel: PN not a multiple of
    256, or grad viewed at a 4-byte offset (not 16-byte aligned), so the vectorised path does
    not apply and the columns are walked in tiles. Called through the C-ABI against the
    oracle's backward (mamba3/scan.py:47-62)."""
    B, K, H = 1, 5, 2
    g = torch.Generator().manual_seed(PN + offset)
    d = torch.rand(B, K, H, generator=g) * 0.5 + 0.5
    hc = torch.randn(B, K, H, PN, generator=g)
    h0 = torch.randn(B, H, PN, generator=g)
    gout = torch.randn(B, K, H, PN, generator=g)
    states = ref.scan_forward(d, hc, h0)
    dd_r, dc_r, dh_r = ref.scan_backward(d, states, gout, True)
    gbuf = torch.zeros(B * K * H * PN + offset, device=cuda_device)
    grad = gbuf[offset:].view(B, K, H, PN)
    grad.copy_(gout.to(cuda_device))
    assert (grad.data_ptr() % 16 != 0) == (offset != 0)
    d_decay = torch.empty(B, K, H, device=cuda_device)
    d_chunk = torch.empty(B, K, H, PN, device=cuda_device)
    d_init = torch.empty(B, H, PN, device=cuda_device)
    _native.scan_bwd(d.to(cuda_device), states.to(cuda_device), grad, d_decay, d_chunk, d_init)
    torch.cuda.synchronize()
    assert max_rel(d_decay, dd_r) < FP32_TOL
    assert max_rel(d_chunk, dc_r) < FP32_TOL
    assert max_rel(d_init, dh_r) < FP32_TOL


# ------------------------------------------------------------------ bf16 vs fp32 oracle
def _bf16_pair(kw, dev, seed=0):
    torch.manual_seed(seed)
    layer = mamba3_amd.KulaMamba(**kw).to(dev, torch.bfloat16).eval()
    params = {k: v.detach().float().cpu() for k, v in layer.state_dict().items()}
    return layer, oracle_cfg(kw), params


@pytest.mark.parametrize("kw,shape", [
    (dict(d_model=64, d_state=16, headdim=16, mimo_rank=2, chunk_size=8), (2, 37, 64)),
    (dict(d_model=768, d_state=128, headdim=64, mimo_rank=2), (1, 1024, 768)),
    (dict(d_model=768, d_state=128, headdim=64, mimo_rank=2), (2, 333, 768)),
])
def test_bf16_prefill_matches_fp32_oracle(kw, shape, cuda_device):
    layer, cfg, p = _bf16_pair(kw, cuda_device)
    torch.manual_seed(2)
    x = torch.randn(*shape).to(torch.bfloat16)
    with torch.no_grad():
        y, st = layer.prefill(x.to(cuda_device))
        y_ref, st_ref = ref.layer_forward(cfg, p, x.float(), return_state=True)
    assert max_rel(y.float(), y_ref) < BF16_TOL
    for k in ("h", "prev_BX", "angle"):
        assert max_rel(st[k], st_ref[k]) < BF16_TOL, k


def test_bf16_generic_prefill_with_state_rows_beyond_the_lds(cuda_device):
    """d_state 512, headdim 256, rank 8 in bf16 (the generic kernel) at batch x heads = 130:
    a whole head's state rows would need 525 KB of LDS, so the launch narrows the headdim
    column blocks until they fit; output and state against the fp32 oracle (its chunk size
    of 4 keeps the oracle's per-chunk outer products small; the kernel ignores it)."""
    kw = dict(d_model=256, d_state=512, headdim=256, mimo_rank=8, chunk_size=4)
    layer, cfg, p = _bf16_pair(kw, cuda_device)
    torch.manual_seed(4)
    x = torch.randn(65, 5, 256).to(torch.bfloat16)
    with torch.no_grad():
        y, st = layer.prefill(x.to(cuda_device))
        y_ref, st_ref = ref.layer_forward(cfg, p, x.float(), return_state=True)
    assert max_rel(y.float(), y_ref) < BF16_TOL
    for k in ("h", "prev_BX", "angle"):
        assert max_rel(st[k], st_ref[k]) < BF16_TOL, k


def test_bf16_chunked_ssd_beyond_64kb_of_lds(cuda_device):
    """bf16 chunked_ssd (the generic kernel) at d_state 512, rank 8 with the beta terms, where
    one token per chunk needs 76 KB of LDS: the kernel's LDS limit is raised to 160 KB."""
    g = torch.Generator().manual_seed(19)
    Bt, T, H, P, N, R = 1, 10, 1, 256, 512, 8
    r = lambda *s: torch.randn(*s, generator=g)
    x_g, x_b, x_raw = r(Bt, T, H, P, R), r(Bt, T, H, P, R), r(Bt, T, H, P, R)
    B_g, B_b, C = r(Bt, T, H, N, R), r(Bt, T, H, N, R), r(Bt, T, H, N, R)
    dt = torch.rand(Bt, T, H, generator=g) * 0.3
    A, D = -torch.rand(H, generator=g) - 0.1, r(H)
    bf = lambda t: t.to(torch.bfloat16)
    y_ref, h_ref = ref.chunked_ssd(*[bf(t).double() for t in (x_g, x_b, B_g, B_b, C, dt)],
                                   A.double(), D.double(), bf(x_raw).double(), 64,
                                   return_final_state=True)
    dev = cuda_device
    out = mamba3_amd.chunked_ssd(*[bf(t).to(dev) for t in (x_g, x_b, B_g, B_b, C, dt)],
                                 A.to(dev), D.to(dev), bf(x_raw).to(dev), return_final_state=True)
    assert max_rel(out.y, y_ref) < BF16_TOL
    assert max_rel(out.h_final, h_ref) < BF16_TOL


@pytest.mark.parametrize("extra", [dict(ngroups=2), dict(use_trapezoidal=False),
                                   dict(use_complex_ssm=False), dict(ngroups=24)])
def test_bf16_d768_variants_match_fp32_oracle(extra, cuda_device):
    """The MFMA prefill kernel (d_state 128, headdim 64, rank 2) across its flags."""
    kw = dict(d_model=768, d_state=128, headdim=64, mimo_rank=2, **extra)
    layer, cfg, p = _bf16_pair(kw, cuda_device, seed=3)
    torch.manual_seed(4)
    x = torch.randn(2, 300, 768).to(torch.bfloat16)
    with torch.no_grad():
        y, st = layer.prefill(x.to(cuda_device))
        y_ref, st_ref = ref.layer_forward(cfg, p, x.float(), return_state=True)
    assert max_rel(y.float(), y_ref) < BF16_TOL
    for k in ("h", "prev_BX", "angle"):
        assert max_rel(st[k], st_ref[k]) < BF16_TOL, k


@pytest.mark.parametrize("scale", [4.0, 32.0, 256.0])
def test_bf16_d768_large_parameters_match_fp32_oracle(scale, cuda_device):
    """A checkpoint with large B/C norm weights and biases and mimo_x (all multiplied by
    `scale`): one rank's B^ row bound sqrt(N R) max|w| + sqrt(N) max|bias| reaches ~90 at
    x4, ~720 at x32 and ~5800 at x256, and |mimo_x| ~256 at x256. The MFMA kernel still
    runs (its f16 operands are held divided by powers of two derived from the parameters,
    mamba3/mamba3.py:147-168 has no such limit) and matches the fp32 oracle; so does the
    generic fp32 kernel that M3_FLAG_NO_F16_OPERANDS forces."""
    kw = dict(d_model=768, d_state=128, headdim=64, mimo_rank=2)
    layer, cfg, _ = _bf16_pair(kw, cuda_device, seed=9)
    with torch.no_grad():
        for name in ("B_norm.weight", "C_norm.weight", "B_bias", "C_bias", "mimo_x"):
            layer.get_parameter(name).mul_(scale)
    p = {k: v.detach().float().cpu() for k, v in layer.state_dict().items()}
    torch.manual_seed(10)
    x = torch.randn(1, 300, 768).to(torch.bfloat16)
    with torch.no_grad():
        proj = layer.in_proj(x.to(cuda_device)).contiguous()
        y_in = torch.empty(1, 300, layer.d_inner, device=cuda_device, dtype=torch.bfloat16)
        desc = layer._desc(1, 300, proj)
        assert _native.prefill_kernel_name(desc, proj, y_in) == "mfma_d128_p64_r2"
        y, st = layer.prefill(x.to(cuda_device))
        y_ref, st_ref = ref.layer_forward(cfg, p, x.float(), return_state=True)
    assert max_rel(y.float(), y_ref) < BF16_TOL
    for k in ("h", "prev_BX", "angle"):
        assert max_rel(st[k], st_ref[k]) < BF16_TOL, k
    if scale == 256.0:
        with torch.no_grad():
            desc.flags |= _native.M3_FLAG_NO_F16_OPERANDS
            assert _native.prefill_kernel_name(desc, proj, y_in) == "generic"
            n = _native.prefill_workspace_bytes(desc)
            ws = torch.empty(n, device=cuda_device, dtype=torch.uint8)
            _native.prefill_fwd(desc, layer._param_pack(), proj, None, y_in, None, None, None, ws, n)
            forced = layer.out_proj(y_in).float()
        assert max_rel(forced, y_ref) < BF16_TOL


@pytest.mark.parametrize("scale", [1.0, 64.0])
def test_bf16_general_kernel_large_parameters_match_fp32_oracle(scale, cuda_device):
    """The general MFMA kernel (d_state 256, rank 4, headdim 64, two groups) with B/C norm
    weights and biases and mimo_x multiplied by `scale` (x64: B^ row bound ~2000, |mimo_x|
    ~64): same kernel, every output against the fp32 oracle."""
    kw = dict(d_model=256, d_state=256, headdim=64, mimo_rank=4, ngroups=2)
    layer, cfg, _ = _bf16_pair(kw, cuda_device, seed=11)
    with torch.no_grad():
        for name in ("B_norm.weight", "C_norm.weight", "B_bias", "C_bias", "mimo_x"):
            layer.get_parameter(name).mul_(scale)
    p = {k: v.detach().float().cpu() for k, v in layer.state_dict().items()}
    torch.manual_seed(12)
    x = torch.randn(2, 150, 256).to(torch.bfloat16)
    with torch.no_grad():
        proj = layer.in_proj(x.to(cuda_device)).contiguous()
        h_out = torch.empty(2, layer.nheads, 64, 256, device=cuda_device)
        assert _native.prefill_kernel_name(layer._desc(2, 150, proj), proj, None, h_out) == "mfma_general"
        y, st = layer.prefill(x.to(cuda_device))
        y_ref, st_ref = ref.layer_forward(cfg, p, x.float(), return_state=True)
    assert max_rel(y.float(), y_ref) < BF16_TOL
    for k in ("h", "prev_BX", "angle"):
        assert max_rel(st[k], st_ref[k]) < BF16_TOL, k


def test_bf16_d768_dt_scale_matches_fp32_oracle(cuda_device):
    kw = dict(d_model=768, d_state=128, headdim=64, mimo_rank=2)
    layer, cfg, p = _bf16_pair(kw, cuda_device, seed=5)
    torch.manual_seed(6)
    x = torch.randn(1, 200, 768).to(torch.bfloat16)
    ds = torch.rand(1, 200, layer.nheads) * 1.5 + 0.5
    with torch.no_grad():
        y = layer(x.to(cuda_device), dt_scale=ds.to(cuda_device))
        y_ref, _ = ref.layer_forward(cfg, p, x.float(), dt_scale=ds)
    assert max_rel(y.float(), y_ref) < BF16_TOL


@pytest.mark.parametrize("T", [1, 63, 64, 65, 4096])
def test_bf16_d768_lengths_match_fp32_oracle(T, cuda_device):
    """Single token, chunk edges, and a long sequence split into many segments."""
    kw = dict(d_model=768, d_state=128, headdim=64, mimo_rank=2)
    layer, cfg, p = _bf16_pair(kw, cuda_device, seed=7)
    torch.manual_seed(T)
    x = torch.randn(1, T, 768).to(torch.bfloat16)
    with torch.no_grad():
        y, st = layer.prefill(x.to(cuda_device))
        y_ref, st_ref = ref.layer_forward(cfg, p, x.float(), return_state=True)
    assert max_rel(y.float(), y_ref) < BF16_TOL
    for k in ("h", "prev_BX", "angle"):
        assert max_rel(st[k], st_ref[k]) < BF16_TOL, k


def test_bf16_step_matches_fp32_oracle(cuda_device):
    """B=64 decode steps from a random state on the d768 layer, bf16 vs fp32."""
    kw = dict(d_model=768, d_state=128, headdim=64, mimo_rank=2)
    layer, cfg, p = _bf16_pair(kw, cuda_device)
    g = torch.Generator().manual_seed(4)
    B, H, P, N = 64, layer.nheads, 64, 128
    st = {"h": torch.randn(B, H, P, N, generator=g) * 0.5,
          "prev_BX": torch.randn(B, H, P, N, generator=g) * 0.5,
          "angle": torch.randn(B, H, N // 2, generator=g) * 3}
    st_dev = {k: v.to(cuda_device) for k, v in st.items()}
    for i in range(4):
        x = torch.randn(B, 768, generator=g).to(torch.bfloat16)
        with torch.no_grad():
            y, st_dev = layer.step(x.to(cuda_device), st_dev)
            y_ref, st = ref.layer_step(cfg, p, x.float(), st)
        assert max_rel(y.float(), y_ref) < BF16_TOL
        for k in ("h", "prev_BX", "angle"):
            assert max_rel(st_dev[k], st[k]) < BF16_TOL, (i, k)


def test_bf16_decode_1024_steps_match_fp32_oracle(cuda_device):
    """The decode workload: d768 layer in bf16, batch 64, the state filled by prefilling 512
    N(0,1) tokens, then 1024 sequential steps on (64, 768) N(0,1) tokens. The oracle steps
    in fp32 from the same prefilled state (copied to the host); every step's output and
    the final h, prev_BX and angle are compared, within the bf16 tolerance."""
    kw = dict(d_model=768, d_state=128, headdim=64, mimo_rank=2)
    layer, cfg, p = _bf16_pair(kw, cuda_device)
    g = torch.Generator().manual_seed(3)
    xp = torch.randn(64, 512, 768, generator=g).to(torch.bfloat16)
    with torch.no_grad():
        _, st_dev = layer.prefill(xp.to(cuda_device))
    st = {k: v.float().cpu() for k, v in st_dev.items()}
    worst = 0.0
    for i in range(1024):
        x = torch.randn(64, 768, generator=g).to(torch.bfloat16)
        with torch.no_grad():
            y, st_dev = layer.step(x.to(cuda_device), st_dev)
            y_ref, st = ref.layer_step(cfg, p, x.float(), st)
        e = max_rel(y.float(), y_ref)
        worst = max(worst, e)
        assert e < BF16_TOL, (i, e)
    for k in ("h", "prev_BX", "angle"):
        assert max_rel(st_dev[k], st[k]) < BF16_TOL, k
    assert worst > 0.0


STEP_SHAPES = [dict(d_state=48, mimo_rank=2), dict(d_state=96, mimo_rank=2),
               dict(d_state=128, mimo_rank=8), dict(d_state=16, mimo_rank=3),
               dict(d_state=6, mimo_rank=1), dict(d_state=130, mimo_rank=4),
               dict(d_state=258, mimo_rank=1), dict(d_state=300, mimo_rank=2),
               dict(d_state=4, mimo_rank=1), dict(d_state=64, mimo_rank=4),
               dict(d_state=512, mimo_rank=2), dict(d_state=510, mimo_rank=8),
               dict(d_state=2, mimo_rank=2)]


@pytest.mark.parametrize("shape", STEP_SHAPES, ids=lambda k: f"N{k['d_state']}-R{k['mimo_rank']}")
def test_step_any_even_d_state_and_rank_matches_oracle(shape, cuda_device):
    """The decode step for every even d_state up to 512 and every rank up to 8, as the
    reference's step (mamba3/mamba3.py:267-322): lanes past the row end (N/4 not a power of
    two), 2-wide column vectors (N % 4 == 2), several vectors per lane with a partial last
    lane (N > 256), ranks that run under a wider template, and the full layouts (power-of-two
    N >= 4, rank 1/2/4) with one to 64 lanes per row. fp32 prefill of 20 tokens,
    then 5 steps, each output and the final state against the oracle at 1e-4."""
    kw = dict(d_model=32, headdim=16, **shape)
    torch.manual_seed(0)
    layer = mamba3_amd.KulaMamba(**kw)
    p = {k: v.detach().clone() for k, v in layer.state_dict().items()}
    layer = layer.to(cuda_device).eval()
    cfg = oracle_cfg(kw)
    g = torch.Generator().manual_seed(shape["d_state"] * 10 + shape["mimo_rank"])
    x = torch.randn(2, 20, 32, generator=g)
    with torch.no_grad():
        _, st = layer.prefill(x.to(cuda_device))
        _, st_ref = ref.layer_forward(cfg, p, x, return_state=True)
        for i in range(5):
            xt = torch.randn(2, 32, generator=g)
            y, st = layer.step(xt.to(cuda_device), st)
            y_ref, st_ref = ref.layer_step(cfg, p, xt, st_ref)
            assert max_rel(y, y_ref) < FP32_TOL, i
    for k in ("h", "prev_BX", "angle"):
        assert max_rel(st[k], st_ref[k]) < FP32_TOL, k


def test_bf16_step_d_state_96_matches_fp32_oracle(cuda_device):
    """bf16 decode at d_state 96 (24 of 32 lanes per state row hold columns) and batch 16,
    steps from a random state against the fp32 oracle."""
    kw = dict(d_model=256, d_state=96, headdim=64, mimo_rank=2)
    layer, cfg, p = _bf16_pair(kw, cuda_device, seed=11)
    g = torch.Generator().manual_seed(12)
    B, H, P, N = 16, layer.nheads, 64, 96
    st = {"h": torch.randn(B, H, P, N, generator=g) * 0.5,
          "prev_BX": torch.randn(B, H, P, N, generator=g) * 0.5,
          "angle": torch.randn(B, H, N // 2, generator=g) * 3}
    st_dev = {k: v.to(cuda_device) for k, v in st.items()}
    for i in range(3):
        x = torch.randn(B, 256, generator=g).to(torch.bfloat16)
        with torch.no_grad():
            y, st_dev = layer.step(x.to(cuda_device), st_dev)
            y_ref, st = ref.layer_step(cfg, p, x.float(), st)
        assert max_rel(y.float(), y_ref) < BF16_TOL
        for k in ("h", "prev_BX", "angle"):
            assert max_rel(st_dev[k], st[k]) < BF16_TOL, (i, k)


def test_fp32_step_matches_oracle_from_random_state(cuda_device):
    kw = dict(d_model=768, d_state=128, headdim=64, mimo_rank=2)
    torch.manual_seed(0)
    layer = mamba3_amd.KulaMamba(**kw).to(cuda_device).eval()
    cfg = oracle_cfg(kw)
    p = {k: v.detach().cpu() for k, v in layer.state_dict().items()}
    g = torch.Generator().manual_seed(5)
    B, H, P, N = 16, layer.nheads, 64, 128
    st = {"h": torch.randn(B, H, P, N, generator=g), "prev_BX": torch.randn(B, H, P, N, generator=g),
          "angle": torch.randn(B, H, N // 2, generator=g)}
    x = torch.randn(B, 768, generator=g)
    with torch.no_grad():
        y, st2 = layer.step(x.to(cuda_device), {k: v.to(cuda_device) for k, v in st.items()})
        y_ref, st_ref = ref.layer_step(cfg, p, x, st)
    assert max_rel(y, y_ref) < FP32_TOL
    for k in ("h", "prev_BX", "angle"):
        assert max_rel(st2[k], st_ref[k]) < FP32_TOL, k


# ------------------------------------------------------------------ fused fp32 prefill
# fp32 layers with d_state 128 / headdim 64 / rank 2 run on the fused fp32 kernel
# (m3_ssd_f32.hip, 32-token chunks) when the forward keeps no intermediates for
# m3_layer_bwd; under autograd the staged fp32 layer path runs instead. Lengths of one token,
# one chunk plus one and ending mid-chunk, the layer variants and dt_scale: the fused path
# against the fp64 oracle at 1e-4, and the training forward against the fused one.
F32_FUSED_CASES = [
    (dict(), 1, False), (dict(), 33, False), (dict(), 300, True),
    (dict(use_trapezoidal=False), 100, False), (dict(use_complex_ssm=False), 100, False),
    (dict(ngroups=2), 77, True),
]


@pytest.mark.parametrize("extra,T,scaled", F32_FUSED_CASES)
def test_fp32_fused_prefill_matches_oracle(extra, T, scaled, cuda_device):
    kw = dict(d_model=768, d_state=128, headdim=64, mimo_rank=2, **extra)
    print(f"fused fp32 prefill {extra} T={T} dt_scale={scaled}", flush=True)
    torch.manual_seed(5)
    layer = mamba3_amd.KulaMamba(**kw).to(cuda_device).eval()
    p = {k: v.detach().double().cpu() for k, v in layer.state_dict().items()}
    g = torch.Generator().manual_seed(T)
    x = torch.randn(2, T, 768, generator=g)
    ds = torch.rand(2, T, layer.nheads, generator=g) + 0.5 if scaled else None
    dsd = ds.to(cuda_device) if scaled else None
    with torch.no_grad():
        y, st = layer.prefill(x.to(cuda_device), dt_scale=dsd)
    y_ref, st_ref = ref.layer_forward(oracle_cfg(kw), p, x.double(),
                                      dt_scale=ds.double() if scaled else None, return_state=True)
    assert max_rel(y, y_ref) < FP32_TOL
    for k in ("h", "prev_BX", "angle"):
        assert max_rel(st[k], st_ref[k]) < FP32_TOL, k
    xg = x.to(cuda_device).requires_grad_()
    y_train = layer(xg, dt_scale=dsd)
    assert max_rel(y_train.detach(), y) < FP32_TOL


# ------------------------------------------------------------------ general MFMA prefill kernel
# bf16 layers with d_state 64/128/256, rank 1/2/4 and headdim % 32 == 0 (other than
# d_state 128 / headdim 64 / rank 2) run on the general MFMA kernel: one case per
# (d_state, rank) instantiation, lengths that end mid-chunk, and the layer flags.
WIDE_CASES = [
    (dict(d_model=64, d_state=64, headdim=32, mimo_rank=1), 150),
    (dict(d_model=64, d_state=64, headdim=32, mimo_rank=2), 97),
    (dict(d_model=64, d_state=64, headdim=32, mimo_rank=4), 77),
    (dict(d_model=128, d_state=128, headdim=64, mimo_rank=1), 200),
    (dict(d_model=96, d_state=128, headdim=32, mimo_rank=2), 129),
    (dict(d_model=64, d_state=128, headdim=32, mimo_rank=4), 61),
    (dict(d_model=128, d_state=256, headdim=64, mimo_rank=1), 70),
    (dict(d_model=128, d_state=256, headdim=64, mimo_rank=2), 100),
    (dict(d_model=256, d_state=256, headdim=128, mimo_rank=4), 130),
    (dict(d_model=192, d_state=256, headdim=96, mimo_rank=4, ngroups=2), 45),
    (dict(d_model=256, d_state=256, headdim=128, mimo_rank=4, use_trapezoidal=False), 33),
    (dict(d_model=256, d_state=256, headdim=128, mimo_rank=4, use_complex_ssm=False), 17),
    (dict(d_model=128, d_state=128, headdim=32, mimo_rank=4, ngroups=8), 1),
]


@pytest.mark.parametrize("kw,T", WIDE_CASES)
def test_bf16_wide_prefill_matches_fp32_oracle(kw, T, cuda_device):
    layer, cfg, p = _bf16_pair(kw, cuda_device, seed=11)
    torch.manual_seed(T)
    x = torch.randn(2, T, kw["d_model"]).to(torch.bfloat16)
    with torch.no_grad():
        y, st = layer.prefill(x.to(cuda_device))
        y_ref, st_ref = ref.layer_forward(cfg, p, x.float(), return_state=True)
    assert max_rel(y.float(), y_ref) < BF16_TOL
    for k in ("h", "prev_BX", "angle"):
        assert max_rel(st[k], st_ref[k]) < BF16_TOL, k


@pytest.mark.parametrize("kw,expect", [
    (dict(d_model=256, d_state=256, headdim=128, mimo_rank=4, ngroups=2), "mfma_general"),
    (dict(d_model=256, d_state=128, headdim=32, mimo_rank=2), "mfma_general"),
    (dict(d_model=128, d_state=64, headdim=32, mimo_rank=1), "mfma_general"),
])
def test_general_kernel_odd_proj_row_stride_equals_contiguous(kw, expect, cuda_device):
    """proj handed over through the C-ABI with an odd row stride (a column slice of a wider
    buffer, as a caller's fused projection may give): the B / C normalisation reads each
    pair's raw values element by element instead of with one vector load, and every output
    equals, bit for bit, that of the same values at the contiguous stride."""
    dev = cuda_device
    layer, _, _ = _bf16_pair(kw, dev, seed=15)
    torch.manual_seed(16)
    Bat, T = 2, 77
    x = torch.randn(Bat, T, kw["d_model"]).to(torch.bfloat16).to(dev)
    outs = []
    with torch.no_grad():
        proj = layer.in_proj(x).contiguous()
        W = proj.shape[-1]
        wide = torch.zeros(Bat, T, W + 1, dtype=proj.dtype, device=dev)
        wide[..., :W] = proj
        for src in (proj, wide):
            desc = layer._desc(Bat, T, src)
            assert desc.proj_row_stride == src.stride(-2)
            y = torch.empty(Bat, T, layer.d_inner, device=dev, dtype=torch.bfloat16)
            h = torch.empty(Bat, layer.nheads, layer.headdim, layer.d_state, device=dev)
            angle = torch.empty(Bat, layer.nheads, layer.d_state // 2, device=dev)
            prev = torch.empty_like(h)
            assert _native.prefill_kernel_name(desc, src, y, h, prev) == expect
            n = _native.prefill_workspace_bytes(desc)
            ws = torch.empty(n, device=dev, dtype=torch.uint8)
            _native.prefill_fwd(desc, layer._param_pack(), src, None, y, h, angle, prev, ws, n)
            outs.append((y, h, angle, prev))
    assert outs[1][0].isfinite().all()
    for a, b in zip(*outs):
        assert torch.equal(a, b)


def test_bf16_d2048_prefill_matches_fp32_oracle(cuda_device):
    """The d_model 2048 layer (d_state 256, headdim 128, rank 4), with dt_scale."""
    kw = dict(d_model=2048, d_state=256, headdim=128, mimo_rank=4)
    layer, cfg, p = _bf16_pair(kw, cuda_device, seed=12)
    torch.manual_seed(13)
    x = torch.randn(1, 130, 2048).to(torch.bfloat16)
    ds = torch.rand(1, 130, layer.nheads) * 1.5 + 0.5
    with torch.no_grad():
        y, st = layer.prefill(x.to(cuda_device), dt_scale=ds.to(cuda_device))
        y_ref, st_ref = ref.layer_forward(cfg, p, x.float(), dt_scale=ds, return_state=True)
    assert max_rel(y.float(), y_ref) < BF16_TOL
    for k in ("h", "prev_BX", "angle"):
        assert max_rel(st[k], st_ref[k]) < BF16_TOL, k


# ------------------------------------------------------------------ full-size properties
def test_bf16_d768_long_prefill_properties(cuda_device):
    """x (8, 8192, 768) bf16 (the long-prefill workload): batch independence and causality
    of the kernel on the same in_proj output, and the prefill -> step hand-off through
    the full layer. The kernel splits each sequence into a number of segments that
    depends on batch*heads, so a sub-batch is evaluated in a different order and may
    round the bf16 output differently by one ulp (2^-7 of the largest |y| = 7.8e-3), and
    its RoPE angles are taken relative to different segment starts, so B~ and C~ round
    differently in bf16: the comparison allows 1e-2."""
    kw = dict(d_model=768, d_state=128, headdim=64, mimo_rank=2)
    torch.manual_seed(0)
    layer = mamba3_amd.KulaMamba(**kw).to(cuda_device, torch.bfloat16).eval()
    torch.manual_seed(2)
    x = torch.randn(8, 8192, 768, device=cuda_device).to(torch.bfloat16)
    with torch.no_grad():
        proj = layer.in_proj(x)
        y, st = layer.ssd_from_proj(proj, return_state=True)
        assert torch.isfinite(y.float()).all() and torch.isfinite(st["h"]).all()
        y3, st3 = layer.ssd_from_proj(proj[3:4].contiguous(), return_state=True)
        e1 = max_rel(y3.float(), y[3:4].float())
        e2 = max_rel(st3["h"], st["h"][3:4])
        yp, _ = layer.ssd_from_proj(proj[:2, :3000].contiguous())
        e3 = max_rel(yp.float(), y[:2, :3000].float())
        assert e1 < 1e-2 and e2 < 1e-2 and e3 < 1e-2, (e1, e2, e3)
        # hand-off: prefill 8176 tokens then 16 steps == prefill of all 8192
        _, sp = layer.prefill(x[:2, :8176])
        outs = []
        for t in range(8176, 8192):
            o, sp = layer.step(x[:2, t], sp)
            outs.append(o)
        y_full = layer.out_proj(y[:2, 8176:])
    ys = torch.stack(outs, 1).float()
    e4, e5 = max_rel(ys, y_full.float()), max_rel(sp["h"], st["h"][:2])
    assert e4 < BF16_TOL and e5 < BF16_TOL, (e4, e5)


def test_bf16_d2048_long_prefill_properties(cuda_device):
    """x (2, 16384, 2048) bf16 (the wide-layer workload): every (batch, head, column
    block) runs independently and chunks start at fixed positions, so a sub-batch and a
    prefix reproduce the full run bit for bit; the prefill -> step hand-off agrees with
    the full prefill."""
    kw = dict(d_model=2048, d_state=256, headdim=128, mimo_rank=4)
    torch.manual_seed(0)
    layer = mamba3_amd.KulaMamba(**kw).to(cuda_device, torch.bfloat16).eval()
    torch.manual_seed(6)
    x = torch.randn(2, 16384, 2048, device=cuda_device).to(torch.bfloat16)
    with torch.no_grad():
        proj = layer.in_proj(x)
        y, st = layer.ssd_from_proj(proj, return_state=True)
        assert torch.isfinite(y.float()).all() and torch.isfinite(st["h"]).all()
        y1, st1 = layer.ssd_from_proj(proj[1:2].contiguous(), return_state=True)
        assert torch.equal(y1, y[1:2]) and torch.equal(st1["h"], st["h"][1:2])
        yp, _ = layer.ssd_from_proj(proj[:, :3000].contiguous())
        assert torch.equal(yp, y[:, :3000])
        _, sp = layer.prefill(x[:, :16368])
        outs = []
        for t in range(16368, 16384):
            o, sp = layer.step(x[:, t], sp)
            outs.append(o)
        y_full = layer.out_proj(y[:, 16368:])
    ys = torch.stack(outs, 1).float()
    e4, e5 = max_rel(ys, y_full.float()), max_rel(sp["h"], st["h"])
    assert e4 < BF16_TOL and e5 < BF16_TOL, (e4, e5)


def test_prefill_of_a_strided_batch_view_equals_its_contiguous_copy(cuda_device):
    """A batch-sliced input view (rows not adjacent in memory) prefills exactly like its
    contiguous copy, through the width-padded in_proj of the d768 layer (3696 -> 3840
    columns): output and state bit for bit, all finite."""
    torch.manual_seed(0)
    layer = mamba3_amd.KulaMamba(768, d_state=128, headdim=64, mimo_rank=2)
    layer = layer.to(cuda_device, torch.bfloat16).eval()
    torch.manual_seed(7)
    x = torch.randn(4, 300, 768, device=cuda_device).to(torch.bfloat16)
    view = x[1:3, :250]
    assert not view.is_contiguous()
    with torch.no_grad():
        assert layer._in_proj_wide(view.contiguous()).shape[-1] == 3840
        y1, s1 = layer.prefill(view)
        y2, s2 = layer.prefill(view.contiguous())
    assert torch.isfinite(y1.float()).all()
    assert torch.equal(y1, y2)
    for k in ("h", "prev_BX", "angle"):
        assert torch.equal(s1[k], s2[k]), k
