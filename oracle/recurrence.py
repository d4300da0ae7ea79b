"""Float64 ground truth for the Mamba-3 SSD (TEST INFRASTRUCTURE).

* `layer_core_recurrent` runs the per-token decode equations (mamba3/mamba3.py:267-316,
  Appendix A.1 of the equations restated there) token by token in float64, from an
  optional initial state. Parallel prefill must equal it (the reference's own central
  invariant, tests/test_mamba3.py:35-52, 294-314).
* `ssd_quadratic` is the textbook scalar-decay SSD evaluated as a dense masked
  L-matrix product (no chunking, no factored cumsum), used to pin the chunked algorithm
  on the reduced case trapezoid-off / complex-off / rank-1.
* `scan_closed_form` evaluates the chunk recurrence as explicit sums of products.
* `chunked_recurrent` runs chunked_ssd's inputs (mamba3/ssd.py:118-244) through the
  per-token recurrence in float64, as differentiable torch ops: autograd through it is an
  independent formulation of chunked_ssd's gradients.
"""

from __future__ import annotations

import numpy as np
import torch
import torch.nn.functional as F

from .reference_path import LayerCfg, split_proj


def _f64(p: dict) -> dict:
    return {k: (v.double() if torch.is_tensor(v) else v) for k, v in p.items()}


def layer_core_recurrent(cfg: LayerCfg, p: dict, proj: torch.Tensor, state: dict | None = None,
                         dt_scale=None):
    """proj (B,T,W) -> (y (B,T,d_inner) float64, final state dict float64).

    Equations (per token, head h, group g = h // (H/G)):
      dt = softplus(dt_raw + dt_bias) [* dt_scale];  dA = exp(-exp(A_log) dt)
      B~ = rot(phi, RMSNorm(B) w + b);  C~ likewise;  phi -= dt * theta
      x[p,r] = x_in[h,p] mimo_x[h,p,r];  gamma = lam dt;  beta = (1-lam) dt dA
      h = dA h + gamma B~ x^T + beta prev;  prev = B~ x^T
      y[p,r] = C~[:,r] . h[p,:] + D x[p,r];  out[p] = sum_r down y silu(z mimo_z)
    """
    p = _f64(p)
    proj = proj.double()
    Bat, T, _ = proj.shape
    H, P, N, R, G = cfg.H, cfg.headdim, cfg.d_state, cfg.mimo_rank, cfg.ngroups
    hpg = H // G
    z, xf, Bf, Cf, dt_raw, lam_raw, theta = split_proj(cfg, proj)
    if state is None:
        h = torch.zeros(Bat, H, P, N, dtype=torch.float64)
        prev = torch.zeros(Bat, H, P, N, dtype=torch.float64)
        phi = torch.zeros(Bat, H, N // 2, dtype=torch.float64)
    else:
        h, prev, phi = (state[k].double().clone() for k in ("h", "prev_BX", "angle"))
    A = -torch.exp(p["A_log"])
    ys = []
    for t in range(T):
        dt = F.softplus(dt_raw[:, t] + p["dt_bias"])
        if dt_scale is not None:
            dt = dt * dt_scale[:, t].double()
        dA = torch.exp(A * dt)

        def norm(v, w, bias):
            v = v.reshape(Bat, G, N * R)
            v = v * torch.rsqrt(v.pow(2).mean(-1, keepdim=True) + cfg.eps) * w
            v = v.reshape(Bat, G, N, R) + bias
            return v.repeat_interleave(hpg, dim=1)  # (B,H,N,R)

        Bt = norm(Bf[:, t], p["B_norm.weight"], p["B_bias"])
        Ct = norm(Cf[:, t], p["C_norm.weight"], p["C_bias"])
        if cfg.use_complex_ssm:
            phi = phi - dt[:, :, None] * theta[:, t][:, None, :]
            c, s = torch.cos(phi)[..., None], torch.sin(phi)[..., None]

            def rot(v):
                v = v.reshape(Bat, H, N // 2, 2, R)
                e, o = v[..., 0, :], v[..., 1, :]
                return torch.stack((e * c - o * s, e * s + o * c), dim=-2).reshape(Bat, H, N, R)

            Bt, Ct = rot(Bt), rot(Ct)
        x = xf[:, t].reshape(Bat, H, P, 1) * p["mimo_x"]
        if cfg.use_trapezoidal:
            lam = torch.sigmoid(lam_raw[:, t])
            gamma, beta = lam * dt, (1 - lam) * dt * dA
        else:
            gamma, beta = dt, torch.zeros_like(dt)
        cur = torch.einsum("bhnr,bhpr->bhpn", Bt, x)
        h = dA[..., None, None] * h + gamma[..., None, None] * cur + beta[..., None, None] * prev
        prev = cur
        y = torch.einsum("bhnr,bhpn->bhpr", Ct, h) + p["D"][None, :, None, None] * x
        zr = z[:, t].reshape(Bat, H, P, 1) * p["mimo_z"]
        ys.append((y * F.silu(zr) * p["mimo_down"]).sum(-1).reshape(Bat, H * P))
    return torch.stack(ys, dim=1), {"h": h, "angle": phi, "prev_BX": prev}


def ssd_quadratic(x: np.ndarray, Bm: np.ndarray, Cm: np.ndarray, dt: np.ndarray,
                  A: np.ndarray, D: np.ndarray, h_init: np.ndarray | None = None):
    """Scalar-decay, rank-1 SSD as one dense masked product, float64.

    x (B,T,H,P), Bm/Cm (B,T,H,N), dt (B,T,H), A/D (H,), h_init (B,H,P,N) or None:
      L[t,s]   = exp(sum_{s<j<=t} A dt_j) for s <= t else 0
      y[t,p]   = sum_s L[t,s] (C_t . B_s) dt_s x_s[p] + exp(sum_{j<=t} A dt_j) C_t . h0[p,:]
                 + D x_t[p]
      h_T[p,n] = sum_s L[T-1,s] dt_s x_s[p] B_s[n] + exp(sum_j A dt_j) h0[p,n]
    """
    x, Bm, Cm, dt = (np.asarray(a, np.float64) for a in (x, Bm, Cm, dt))
    Bat, T, H, P = x.shape
    a = dt * np.asarray(A, np.float64)[None, None, :]
    cs = np.cumsum(a, axis=1)  # (B,T,H) inclusive
    diff = cs[:, :, None, :] - cs[:, None, :, :]  # [t,s] = c_t - c_s
    mask = np.tril(np.ones((T, T), bool))[None, :, :, None]
    L = np.where(mask, np.exp(np.where(mask, diff, 0.0)), 0.0)  # (B,T,T,H)
    G = np.einsum("bthn,bshn->btsh", Cm, Bm)
    y = np.einsum("btsh,bsh,bshp->bthp", L * G, dt, x)
    y += np.asarray(D, np.float64)[None, None, :, None] * x
    hT = np.einsum("bsh,bsh,bshp,bshn->bhpn", L[:, T - 1], dt, x, Bm)
    if h_init is not None:
        h0 = np.asarray(h_init, np.float64)
        y += np.exp(cs)[..., None] * np.einsum("bthn,bhpn->bthp", Cm, h0)
        hT += np.exp(cs[:, T - 1])[:, :, None, None] * h0
    return y, hT


def scan_closed_form(decay: np.ndarray, h_chunk: np.ndarray, h_init: np.ndarray | None = None):
    """h_states[:,k] = (prod_{j<k} d_j) h_init + sum_{i<k} (prod_{i<j<k} d_j) h_chunk[:,i]."""
    d = np.asarray(decay, np.float64)
    hc = np.asarray(h_chunk, np.float64)
    B, K, H = d.shape
    out = np.zeros_like(hc)
    for k in range(K):
        acc = np.zeros_like(hc[:, 0])
        if h_init is not None:
            acc += np.prod(d[:, :k], axis=1)[..., None] * np.asarray(h_init, np.float64)
        for i in range(k):
            acc += np.prod(d[:, i + 1:k], axis=1)[..., None] * hc[:, i]
        out[:, k] = acc
    return out


def chunked_recurrent(x_g, x_b, B_g, B_b, C, dt, A, D, x_raw, h_init=None):
    """chunked_ssd's contract (mamba3/ssd.py:118-244) token by token, float64, autograd-able:
        h_t = exp(A dt_t) h_{t-1} + dt_t (sum_r x_g[t,:,r] B_g[t,:,r]^T + x_b B_b likewise)
        y_t[p,r] = sum_n C[t,n,r] h_t[p,n] + D x_raw[t,p,r]
    (the per-token update of mamba3/mamba3.py:298-310 with the chunked inputs). Returns
    (y (B,T,H,P,R), h_final (B,H,P,N))."""
    Bat, T, H, P, R = x_g.shape
    N = B_g.shape[3]
    f = lambda t: None if t is None else t.double()
    x_g, x_b, B_g, B_b, C, dt, A, D, x_raw, h_init = map(f, (x_g, x_b, B_g, B_b, C, dt, A, D,
                                                            x_raw, h_init))
    h = h_init.reshape(Bat, H, P, N) if h_init is not None else x_g.new_zeros(Bat, H, P, N)
    ys = []
    for t in range(T):
        bx = torch.einsum("bhpr,bhnr->bhpn", x_g[:, t], B_g[:, t])
        if x_b is not None:
            bx = bx + torch.einsum("bhpr,bhnr->bhpn", x_b[:, t], B_b[:, t])
        h = torch.exp(A * dt[:, t])[..., None, None] * h + dt[:, t][..., None, None] * bx
        ys.append(torch.einsum("bhnr,bhpn->bhpr", C[:, t], h) + D[None, :, None, None] * x_raw[:, t])
    return torch.stack(ys, dim=1), h
