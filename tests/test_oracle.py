"""Pin the CPU oracle (oracle/) before trusting it as the GPU parity checker.

Checks, each chosen so that a plausible slip (dropped term, wrong sign or index,
transposed operand) fails at least one of them:
  * golden vectors written from the reference (tests/golden/make_golden.py);
  * the fp64 token recurrence (the reference's own parallel == sequential invariant);
  * the textbook scalar-decay SSD as a dense masked L-matrix (reduced case);
  * closed forms of the chunk scan; dt=0 and A=0 special cases.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from conftest import (CHUNKED_CASES, LAYER_CASES, golden_config, golden_params, load_golden,
                      max_rel, oracle_cfg)
from oracle import recurrence as rec
from oracle import reference_path as ref

TOL = 2e-5  # fp32 oracle vs fp32 reference outputs (same algorithm, same op order)


def _run_layer_case(name):
    g = load_golden(name)
    kw = golden_config(g)
    cfg = oracle_cfg(kw)
    p = golden_params(g)
    x = torch.from_numpy(g["x"])
    return g, cfg, p, x


@pytest.mark.parametrize("name", LAYER_CASES)
def test_oracle_forward_matches_reference_golden(name):
    g, cfg, p, x = _run_layer_case(name)
    with torch.no_grad():
        y, _ = ref.layer_forward(cfg, p, x)
    assert max_rel(y, torch.from_numpy(g["y"])) < TOL


@pytest.mark.parametrize("name", LAYER_CASES)
def test_oracle_prefill_and_steps_match_reference_golden(name):
    g, cfg, p, x = _run_layer_case(name)
    with torch.no_grad():
        y, st = ref.layer_forward(cfg, p, x, return_state=True)
        assert max_rel(y, torch.from_numpy(g["y_prefill"])) < TOL
        for k in ("h", "angle", "prev_BX"):
            assert max_rel(st[k], torch.from_numpy(g[f"prefill/{k}"])) < TOL, k
        xs = torch.from_numpy(g["x_steps"])
        outs = []
        for t in range(xs.shape[1]):
            o, st = ref.layer_step(cfg, p, xs[:, t], st)
            outs.append(o)
        assert max_rel(torch.stack(outs, 1), torch.from_numpy(g["y_steps"])) < TOL
        for k in ("h", "angle", "prev_BX"):
            assert max_rel(st[k], torch.from_numpy(g[f"steps/{k}"])) < TOL, k


def test_oracle_dt_scale_matches_reference_golden():
    g, cfg, p, x = _run_layer_case("layer_tiny_dtscale")
    with torch.no_grad():
        y, _ = ref.layer_forward(cfg, p, x, dt_scale=torch.from_numpy(g["dt_scale"]))
    assert max_rel(y, torch.from_numpy(g["y"])) < TOL


@pytest.mark.parametrize("name", CHUNKED_CASES)
def test_oracle_chunked_ssd_matches_reference_golden(name):
    g = load_golden(name)
    t = {k: torch.from_numpy(v) for k, v in g.items()}
    y, hT = ref.chunked_ssd(t["x_g"], t.get("x_b"), t["B_g"], t.get("B_b"), t["C"], t["dt"],
                            t["A"], t["D"], t["x_raw"], int(g["chunk_size"]),
                            h_init=t.get("h_init"), return_final_state=True)
    assert max_rel(y, t["y"]) < TOL
    assert max_rel(hT, t["h_final"]) < TOL


@pytest.mark.parametrize("name", LAYER_CASES)
def test_oracle_prefill_equals_fp64_recurrence(name):
    """Parallel prefill == token recurrence (reference invariant, 1e-4 there)."""
    g, cfg, p, x = _run_layer_case(name)
    with torch.no_grad():
        proj = F.linear(x, p["in_proj.weight"])
        y, st = ref.layer_core(cfg, p, proj, return_state=True)
        y64, st64 = rec.layer_core_recurrent(cfg, p, proj)
    assert max_rel(y, y64) < 1e-5
    for k in ("h", "angle", "prev_BX"):
        assert max_rel(st[k], st64[k]) < 1e-5, k


def test_recurrence_continues_from_state():
    """Recurrence from a mid-sequence state == recurrence over the whole sequence."""
    g, cfg, p, x = _run_layer_case("layer_tiny")
    with torch.no_grad():
        proj = F.linear(x, p["in_proj.weight"]).double()
        y_all, st_all = rec.layer_core_recurrent(cfg, p, proj)
        y1, st1 = rec.layer_core_recurrent(cfg, p, proj[:, :20])
        y2, st2 = rec.layer_core_recurrent(cfg, p, proj[:, 20:], state=st1)
    assert torch.allclose(torch.cat([y1, y2], 1), y_all, rtol=0, atol=1e-12)
    assert torch.allclose(st2["h"], st_all["h"], rtol=0, atol=1e-12)


def test_chunked_reduces_to_textbook_scalar_ssd():
    """R=1, no beta: chunked factored-cumsum == dense masked L-matrix SSD. The reference
    keeps the decay cumsum in fp32 even for fp64 inputs (mamba3/ssd.py:153-159), which
    bounds the agreement at ~1e-6 relative."""
    g = torch.Generator().manual_seed(7)
    B, T, H, P, N = 2, 29, 3, 5, 6
    x = torch.randn(B, T, H, P, 1, generator=g, dtype=torch.float64)
    Bm = torch.randn(B, T, H, N, 1, generator=g, dtype=torch.float64)
    Cm = torch.randn(B, T, H, N, 1, generator=g, dtype=torch.float64)
    dt = torch.rand(B, T, H, generator=g, dtype=torch.float64) * 0.3 + 0.01
    A = -torch.rand(H, generator=g, dtype=torch.float64) * 2 - 0.1
    D = torch.randn(H, generator=g, dtype=torch.float64)
    h0 = torch.randn(B, H, P, N, generator=g, dtype=torch.float64)
    for CS in (4, 8, 64):
        y, hT = ref.chunked_ssd(x, None, Bm, None, Cm, dt, A, D, x, CS, h_init=h0,
                                return_final_state=True)
        y_q, hT_q = rec.ssd_quadratic(x[..., 0].numpy(), Bm[..., 0].numpy(), Cm[..., 0].numpy(),
                                      dt.numpy(), A.numpy(), D.numpy(), h0.numpy())
        np.testing.assert_allclose(y[..., 0].numpy(), y_q, rtol=1e-5, atol=1e-5)
        np.testing.assert_allclose(hT.numpy(), hT_q, rtol=1e-5, atol=1e-5)


def test_textbook_ssd_catches_planted_sign_error():
    """The L-matrix check is sensitive: a flipped decay sign breaks it."""
    g = torch.Generator().manual_seed(8)
    B, T, H, P, N = 1, 12, 2, 3, 4
    x = torch.randn(B, T, H, P, 1, generator=g, dtype=torch.float64)
    Bm = torch.randn(B, T, H, N, 1, generator=g, dtype=torch.float64)
    Cm = torch.randn(B, T, H, N, 1, generator=g, dtype=torch.float64)
    dt = torch.rand(B, T, H, generator=g, dtype=torch.float64) * 0.3 + 0.05
    A = -torch.rand(H, generator=g, dtype=torch.float64) - 0.5
    D = torch.zeros(H, dtype=torch.float64)
    y, _ = ref.chunked_ssd(x, None, Bm, None, Cm, dt, -A, D, x, 4)  # planted: wrong sign
    y_q, _ = rec.ssd_quadratic(x[..., 0].numpy(), Bm[..., 0].numpy(), Cm[..., 0].numpy(),
                               dt.numpy(), A.numpy(), D.numpy())
    assert np.abs(y[..., 0].numpy() - y_q).max() > 1e-3


def test_scan_matches_closed_form_and_reference_loop():
    g = torch.Generator().manual_seed(3)
    B, K, H, PN = 2, 6, 3, 10
    d = torch.rand(B, K, H, generator=g, dtype=torch.float64) * 0.9
    hc = torch.randn(B, K, H, PN, generator=g, dtype=torch.float64)
    h0 = torch.randn(B, H, PN, generator=g, dtype=torch.float64)
    # the reference scan computes in fp32 (mamba3/scan.py:37-39)
    out = ref.scan_forward(d, hc, h0)
    np.testing.assert_allclose(out.numpy(), rec.scan_closed_form(d, hc, h0), rtol=1e-5, atol=1e-6)
    out0 = ref.scan_forward(d, hc, None)
    np.testing.assert_allclose(out0.numpy(), rec.scan_closed_form(d, hc, None), rtol=1e-5,
                               atol=1e-6)
    assert torch.count_nonzero(out0[:, 0]) == 0


def test_scan_backward_equals_autograd_of_the_forward():
    """The oracle's scan backward (mamba3/scan.py:47-62) against torch autograd through the
    oracle's forward loop, with and without h_init; a backward that dropped the decay
    carry (G[k] = grad[k]) must fail."""
    g = torch.Generator().manual_seed(5)
    B, K, H, PN = 2, 6, 3, 5
    for with_init in (True, False):
        d = (torch.rand(B, K, H, generator=g, dtype=torch.float64) * 0.5 + 0.5).requires_grad_()
        hc = torch.randn(B, K, H, PN, generator=g, dtype=torch.float64, requires_grad=True)
        h0 = torch.randn(B, H, PN, generator=g, dtype=torch.float64, requires_grad=True) if with_init else None
        out = ref.scan_forward(d, hc, h0)
        gout = torch.randn(B, K, H, PN, generator=g, dtype=torch.float32)
        out.backward(gout)
        dd, dc, dh0 = ref.scan_backward(d.detach(), out.detach(), gout, with_init)
        np.testing.assert_allclose(dd.numpy(), d.grad.numpy(), rtol=1e-5, atol=1e-5)
        np.testing.assert_allclose(dc.numpy(), hc.grad.numpy(), rtol=1e-5, atol=1e-5)
        if with_init:
            np.testing.assert_allclose(dh0.numpy(), h0.grad.numpy(), rtol=1e-5, atol=1e-5)
        else:
            assert dh0 is None
        # planted mistake: no carry through the decay
        bad = gout.clone()
        bad[:, :-1] = gout[:, 1:]
        bad[:, -1] = 0
        assert np.abs(bad.numpy() - hc.grad.numpy()).max() > 1e-2


def test_zero_dt_leaves_only_skip_path():
    """dt=0: no state is injected, so y == D * x_raw exactly and h stays h_init."""
    g = torch.Generator().manual_seed(4)
    B, T, H, P, R, N = 1, 10, 2, 3, 2, 4
    r = lambda *s: torch.randn(*s, generator=g, dtype=torch.float64)
    x_raw = r(B, T, H, P, R)
    D = r(H)
    y, hT = ref.chunked_ssd(r(B, T, H, P, R), r(B, T, H, P, R), r(B, T, H, N, R),
                            r(B, T, H, N, R), torch.zeros(B, T, H, N, R, dtype=torch.float64),
                            torch.zeros(B, T, H, dtype=torch.float64), -torch.ones(H, dtype=torch.float64),
                            D, x_raw, 4, return_final_state=True)
    assert torch.allclose(y, D[None, None, :, None, None] * x_raw, atol=1e-14)
    assert torch.count_nonzero(hT) == 0


def test_no_decay_is_plain_prefix_sum():
    """A=0 (dA=1), C=e_n: y_t reads the running sum of dt_s x_s B_s[n]."""
    g = torch.Generator().manual_seed(5)
    B, T, H, P, N = 1, 9, 1, 2, 3
    x = torch.randn(B, T, H, P, 1, generator=g, dtype=torch.float64)
    Bm = torch.randn(B, T, H, N, 1, generator=g, dtype=torch.float64)
    dt = torch.rand(B, T, H, generator=g, dtype=torch.float64)
    C = torch.zeros(B, T, H, N, 1, dtype=torch.float64)
    C[..., 1, 0] = 1.0
    y, _ = ref.chunked_ssd(x, None, Bm, None, C, dt, torch.zeros(H, dtype=torch.float64),
                           torch.zeros(H, dtype=torch.float64), x, 4)
    expect = torch.cumsum(dt[..., None] * x[..., 0] * Bm[..., 1:2, 0], dim=1)
    assert torch.allclose(y[..., 0], expect, atol=1e-13)


def test_rope_is_rotation_and_pairs_adjacent_columns():
    """Rotation preserves pair norms, composes additively, and pairs (2i, 2i+1)."""
    g = torch.Generator().manual_seed(6)
    t = torch.randn(3, 8, 2, generator=g, dtype=torch.float64)
    a1 = torch.rand(3, 4, 1, generator=g, dtype=torch.float64)
    a2 = torch.rand(3, 4, 1, generator=g, dtype=torch.float64)
    r1 = ref.rope_pairs(t, a1.cos(), a1.sin())
    r12 = ref.rope_pairs(r1, a2.cos(), a2.sin())
    r_sum = ref.rope_pairs(t, (a1 + a2).cos(), (a1 + a2).sin())
    assert torch.allclose(r12, r_sum, atol=1e-13)
    n0 = t.reshape(3, 4, 2, 2).pow(2).sum(2)
    n1 = r1.reshape(3, 4, 2, 2).pow(2).sum(2)
    assert torch.allclose(n0, n1, atol=1e-13)
    # quarter turn maps (e, o) -> (-o, e) on each adjacent pair
    q = torch.full((3, 4, 1), np.pi / 2, dtype=torch.float64)
    rq = ref.rope_pairs(t, q.cos(), q.sin()).reshape(3, 4, 2, 2)
    tp = t.reshape(3, 4, 2, 2)
    assert torch.allclose(rq[:, :, 0], -tp[:, :, 1], atol=1e-12)
    assert torch.allclose(rq[:, :, 1], tp[:, :, 0], atol=1e-12)


def test_trapezoid_collapse_identity():
    """The fused kernels fold the trapezoid's beta term into per-token coefficients
    a_u = lam_u dt_u and b_u = (1-lam_{u+1}) dt_{u+1}; check that this L-matrix form
    equals the reference's rank-2R two-term form on random data (float64)."""
    g = torch.Generator().manual_seed(9)
    B, T, H, P, R, N = 1, 21, 2, 3, 2, 4
    r = lambda *s: torch.randn(*s, generator=g, dtype=torch.float64)
    x = r(B, T, H, P, R)
    Bt = r(B, T, H, N, R)
    Ct = r(B, T, H, N, R)
    dt = torch.rand(B, T, H, generator=g, dtype=torch.float64) * 0.2 + 0.01
    lam = torch.rand(B, T, H, generator=g, dtype=torch.float64)
    A = -torch.rand(H, generator=g, dtype=torch.float64) - 0.2
    D = torch.zeros(H, dtype=torch.float64)
    dA = torch.exp(A * dt)
    x_g = x * lam[..., None, None]
    x_b = F.pad(x[:, :-1], (0, 0, 0, 0, 0, 0, 1, 0)) * ((1 - lam) * dA)[..., None, None]
    B_prev = F.pad(Bt[:, :-1], (0, 0, 0, 0, 0, 0, 1, 0))
    y_ref, h_ref = ref.chunked_ssd(x_g, x_b, Bt, B_prev, Ct, dt, A, D, x, 8,
                                   return_final_state=True)
    # collapsed L-matrix evaluation
    c = torch.cumsum(A * dt, dim=1)
    a = lam * dt
    bco = torch.zeros_like(a)
    bco[:, :-1] = (1 - lam[:, 1:]) * dt[:, 1:]
    y = torch.zeros_like(y_ref)
    for t in range(T):
        for u in range(t + 1):
            m = torch.exp(c[:, t] - c[:, u]) * (a[:, u] + (bco[:, u] if u < t else 0))
            score = torch.einsum("bhnr,bhns->bhrs", Ct[:, t], Bt[:, u])
            y[:, t] += m[:, :, None, None] * torch.einsum("bhrs,bhps->bhpr", score, x[:, u])
    w = torch.exp(c[:, -1:] - c) * (a + bco)
    h = torch.einsum("bth,bthpr,bthnr->bhpn", w, x, Bt)
    # agreement is bounded by the reference's fp32 decay cumsum
    assert torch.allclose(y, y_ref, atol=1e-6)
    assert torch.allclose(h, h_ref.double(), atol=1e-6)


def _chunked_inputs(g, B, T, H, P, N, R, beta, with_init):
    r = lambda *s: torch.randn(*s, generator=g, dtype=torch.float64)
    ins = dict(x_g=r(B, T, H, P, R), x_b=r(B, T, H, P, R) if beta else None,
               B_g=r(B, T, H, N, R), B_b=r(B, T, H, N, R) if beta else None,
               C=r(B, T, H, N, R), dt=torch.rand(B, T, H, generator=g, dtype=torch.float64) * 0.5,
               A=-torch.rand(H, generator=g, dtype=torch.float64) - 0.2, D=r(H),
               x_raw=r(B, T, H, P, R), h_init=r(B, H, P, N) if with_init else None)
    return {k: (v.requires_grad_() if v is not None else None) for k, v in ins.items()}


def _grads(fn, ins, dy, dhf):
    for v in ins.values():
        if v is not None:
            v.grad = None
    y, hf = fn(ins)
    ((y * dy).sum() + (hf * dhf).sum()).backward()
    return {k: v.grad.clone() for k, v in ins.items() if v is not None and v.grad is not None}


def test_chunked_gradients_of_the_oracle_equal_the_recurrence():
    """Autograd through the oracle's chunked_ssd (factored cumsum, chunk states, scan;
    mamba3/ssd.py:118-244) equals autograd through the independent per-token recurrence
    for every input, including h_init and a dL/dh_final; chunks of 4 over a ragged T. A
    recurrence that dropped the beta term must disagree."""
    g = torch.Generator().manual_seed(11)
    for (B, T, H, P, N, R, beta, with_init) in [(2, 11, 2, 3, 4, 2, True, True),
                                                (1, 9, 1, 2, 6, 1, False, False),
                                                (1, 7, 2, 3, 2, 4, True, False)]:
        ins = _chunked_inputs(g, B, T, H, P, N, R, beta, with_init)
        dy = torch.randn(B, T, H, P, R, generator=g, dtype=torch.float64)
        dhf = torch.randn(B, H, P, N, generator=g, dtype=torch.float64)
        chunk = lambda d: ref.chunked_ssd(*[d[k] for k in ("x_g", "x_b", "B_g", "B_b", "C", "dt", "A",
                                                            "D", "x_raw")], chunk_size=4,
                                          h_init=d["h_init"], return_final_state=True)
        recur = lambda d: rec.chunked_recurrent(**d)
        ga = _grads(chunk, ins, dy, dhf)
        gb = _grads(recur, ins, dy, dhf)
        for k in ga:
            # the oracle, like the reference, takes the within-chunk cumsum in fp32
            assert (ga[k] - gb[k]).abs().max() <= 1e-5 * gb[k].abs().max(), k
        if beta:
            nob = lambda d: rec.chunked_recurrent(**{**d, "x_b": None, "B_b": None})
            gc = _grads(nob, ins, dy, dhf)
            assert (gc["dt"] - gb["dt"]).abs().max() > 1e-3 * gb["dt"].abs().max()


def test_chunked_recurrent_gradcheck():
    """Finite differences pin the recurrence's gradients (torch.autograd.gradcheck)."""
    g = torch.Generator().manual_seed(12)
    ins = _chunked_inputs(g, 1, 5, 2, 2, 3, 2, True, True)
    keys = [k for k, v in ins.items() if v is not None]
    fn = lambda *vs: rec.chunked_recurrent(**dict(zip(keys, vs)))
    assert torch.autograd.gradcheck(fn, tuple(ins[k] for k in keys), eps=1e-6, atol=1e-6)


def _lm_tiny():
    g = load_golden("lm_tiny")
    cfg = ref.LayerCfg(d_model=64, d_state=16, headdim=16, mimo_rank=2, chunk_size=8)
    return g, cfg, golden_params(g), 1.0 / math.sqrt(2 * 2)


def test_oracle_lm_matches_reference_golden():
    """Teacher-forced logits of the tiny LM (two blocks, final norm, tied head;
    mamba3/block.py:79-92, 178-184) and its greedy generation (mamba3/block.py:195-231)
    against the reference's fixture. Leaving out the depth residual scale, or the MLP
    branch, must break the logits."""
    g, cfg, p, scale = _lm_tiny()
    ids = torch.from_numpy(g["ids"])
    want = torch.from_numpy(g["logits"])
    with torch.no_grad():
        assert max_rel(ref.lm_forward(cfg, p, ids, 2, scale), want) < TOL
        gen = ref.lm_generate_greedy(cfg, p, ids[:, :5], 2, scale, 6)
        assert torch.equal(gen, torch.from_numpy(g["generated"]))
        assert max_rel(ref.lm_forward(cfg, p, ids, 2, 1.0), want) > 1e-2
        assert max_rel(ref.lm_forward(cfg, p, ids, 2, scale, use_mlp=False), want) > 1e-2


def test_oracle_lm_steps_equal_parallel_logits():
    """Prefill of a prompt, then one lm_step per remaining token (mamba3/block.py:94-107,
    199-229), gives the teacher-forced logits of the parallel forward at every position."""
    g, cfg, p, scale = _lm_tiny()
    ids = torch.from_numpy(g["ids"])
    with torch.no_grad():
        full = ref.lm_forward(cfg, p, ids, 2, scale)
        logits, states = ref.lm_prefill(cfg, p, ids[:, :5], 2, scale)
        assert max_rel(logits, full[:, 4]) < TOL
        for t in range(5, ids.shape[1]):
            logits, states = ref.lm_step(cfg, p, ids[:, t], states, scale)
            assert max_rel(logits, full[:, t]) < TOL, t


def test_oracle_step_dt_scale_equals_reference_forward():
    """The step's dt_scale branch (mamba3/mamba3.py:278-282): one layer_step per token with
    that token's dt_scale, from a zero state, reproduces the reference-written forward
    output under the same per-token dt_scale, and the fp64 recurrence's final state.
    Applying dt_scale to the decay dA alone (the angle and the trapezoid weights left
    unscaled) must break the outputs; that slip is emulated exactly by the oracle step
    without dt_scale on a layer whose A_log is shifted by log(dt_scale) for each token."""
    g, cfg, p, x = _run_layer_case("layer_tiny_dtscale")
    s = torch.from_numpy(g["dt_scale"])
    want = torch.from_numpy(g["y"])
    T = x.shape[1]
    with torch.no_grad():
        st = ref.zero_state(cfg, x.shape[0])
        outs = []
        for t in range(T):
            o, st = ref.layer_step(cfg, p, x[:, t], st, dt_scale=s[:, t])
            outs.append(o)
        got = torch.stack(outs, 1)
        assert max_rel(got, want) < 1e-4
        proj = F.linear(x, p["in_proj.weight"])
        _, st64 = rec.layer_core_recurrent(cfg, p, proj, dt_scale=s)
        for k in ("h", "angle", "prev_BX"):
            assert max_rel(st[k], st64[k]) < 1e-5, k
        # planted slip: dt_scale on dA only (batch row 0; the shift is per head)
        st = ref.zero_state(cfg, 1)
        bad = []
        for t in range(T):
            pt = dict(p)
            pt["A_log"] = p["A_log"] + torch.log(s[0, t])
            o, st = ref.layer_step(cfg, pt, x[0:1, t], st)
            bad.append(o)
        assert max_rel(torch.stack(bad, 1), want[0:1]) > 1e-2
        # and dt_scale dropped altogether
        st = ref.zero_state(cfg, x.shape[0])
        drop = []
        for t in range(T):
            o, st = ref.layer_step(cfg, p, x[:, t], st)
            drop.append(o)
        assert max_rel(torch.stack(drop, 1), want) > 1e-2
