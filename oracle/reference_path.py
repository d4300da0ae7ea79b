"""PyTorch-CPU restatement of the reference Mamba-3 forward path (TEST INFRASTRUCTURE).

Follows the reference's own algorithm and op order so it can serve both as the parity
oracle and as the timed "reference CPU path":
  * layer prep         mamba3/mamba3.py:19-45, 125-168, 192-258
  * chunked SSD        mamba3/ssd.py:118-244 (factored cumsum, ssd.py:30-65)
  * inter-chunk scan   mamba3/scan.py:34-44
  * decode step        mamba3/mamba3.py:170-190, 267-322
  * block / LM glue    mamba3/block.py:16-26, 79-107, 178-231 (forward, prefill, step,
                       greedy generate)
Parameters are passed as a plain dict keyed by the reference's state_dict names, so the
oracle never touches the product modules.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch
import torch.nn.functional as F


@dataclass(frozen=True)
class LayerCfg:
    d_model: int
    d_state: int = 128
    expand: int = 2
    headdim: int = 64
    ngroups: int = 1
    mimo_rank: int = 2
    chunk_size: int = 64
    use_trapezoidal: bool = True
    use_complex_ssm: bool = True
    eps: float = 1e-5

    @property
    def d_inner(self) -> int:
        return self.expand * self.d_model

    @property
    def H(self) -> int:
        return self.d_inner // self.headdim

    @property
    def split_sizes(self) -> list:
        # [z | x | B | C | dt | lambda | theta]  (mamba3/mamba3.py:125-140)
        N, R, G, H = self.d_state, self.mimo_rank, self.ngroups, self.H
        sizes = [self.d_inner, self.d_inner, G * N * R, G * N * R, H]
        if self.use_trapezoidal:
            sizes.append(H)
        if self.use_complex_ssm:
            sizes.append(N // 2)
        return sizes


def rmsnorm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """mamba3/mamba3.py:28-35: x * rsqrt(mean(x^2)+eps) (fp32 stats, cast back) * w."""
    rms = torch.rsqrt(x.float().pow(2).mean(-1, keepdim=True) + eps).to(x.dtype)
    return x * rms * weight


def rope_pairs(t: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """mamba3/mamba3.py:38-45: rotate pairs (2i, 2i+1) of the N axis of (..., N, R) by the
    angle whose cos/sin have shape (..., N/2, 1)."""
    *lead, N, R = t.shape
    pairs = t.reshape(*lead, N // 2, 2, R)
    even, odd = pairs[..., 0, :], pairs[..., 1, :]
    out = torch.stack((even * cos - odd * sin, even * sin + odd * cos), dim=-2)
    return out.reshape(*lead, N, R)


def split_proj(cfg: LayerCfg, proj: torch.Tensor):
    """mamba3/mamba3.py:125-140."""
    parts = list(proj.split(cfg.split_sizes, dim=-1))
    z, x, Bf, Cf, dt_raw = parts[:5]
    rest = parts[5:]
    lam_raw = rest.pop(0) if cfg.use_trapezoidal else None
    theta = rest.pop(0) if cfg.use_complex_ssm else None
    return z, x, Bf, Cf, dt_raw, lam_raw, theta


def expand_groups(cfg: LayerCfg, t: torch.Tensor) -> torch.Tensor:
    """Group -> head repeat_interleave on dim -3 (mamba3/mamba3.py:142-145)."""
    hpg = cfg.H // cfg.ngroups
    return t if hpg == 1 else t.repeat_interleave(hpg, dim=-3)


def scan_forward(decay: torch.Tensor, h_chunk: torch.Tensor,
                 h_init: torch.Tensor | None = None) -> torch.Tensor:
    """mamba3/scan.py:34-44: h[0]=h_init or 0; h[k+1] = d[k] h[k] + h_chunk[k] (fp32)."""
    B, K, H = decay.shape
    d = decay.float()
    hc = h_chunk.float()
    h = h_init.float() if h_init is not None else hc.new_zeros(B, H, hc.shape[-1])
    states = [h]
    for k in range(K - 1):
        h = h * d[:, k, :, None] + hc[:, k]
        states.append(h)
    return torch.stack(states, dim=1)


def scan_backward(decay: torch.Tensor, h_states: torch.Tensor, grad: torch.Tensor,
                  has_h_init: bool = False):
    """mamba3/scan.py:47-62: walk k down; G[k] = grad[k] + d[k] G[k+1]; d_chunk[k] = G[k+1],
    d_decay[k] = sum_j G[k+1] h[k] (both 0 at k = K-1); d_h_init = G[0]."""
    B, K, H, PN = h_states.shape
    d = decay.float()
    hs = h_states.float()
    dh = grad.float().clone()
    d_decay = torch.zeros_like(d)
    d_chunk = torch.zeros_like(hs)
    for k in range(K - 2, -1, -1):
        g = dh[:, k + 1]
        d_chunk[:, k] = g
        d_decay[:, k] = (g * hs[:, k]).sum(dim=-1)
        dh[:, k] = dh[:, k] + d[:, k, :, None] * g
    return d_decay, d_chunk, (dh[:, 0] if has_h_init else None)


def _intra_chunk(BX: torch.Tensor, cum: torch.Tensor, Cw: torch.Tensor):
    """mamba3/ssd.py:30-65 forward: factored cumsum.
    BX (B,K,H,Q,P,N), cum (B,K,H,Q) fp32, Cw (B,K,H,R,Q,N)."""
    B, K, H, Q, P, N = BX.shape
    R = Cw.shape[3]
    wdt = BX.dtype
    acc = torch.float32 if wdt in (torch.float16, torch.bfloat16) else wdt
    e_neg = (-cum).exp()[..., None, None]
    e_pos = cum.exp()[..., None, None]
    scaled = BX.to(acc) * e_neg
    mid = (e_pos * scaled.cumsum(dim=3)).to(wdt)
    lhs = Cw.permute(0, 1, 2, 4, 3, 5).reshape(B * K * H * Q, R, N)
    rhs = mid.reshape(B * K * H * Q, P, N).transpose(-2, -1)
    y = torch.bmm(lhs, rhs).reshape(B * K * H, Q, R, P).permute(0, 2, 1, 3)
    return y.reshape(B, K, H, R, Q, P), scaled.sum(dim=3)


def chunked_ssd(x_g, x_b, B_g, B_b, C, dt, A, D, x_raw, chunk_size=64, h_init=None,
                return_final_state=False):
    """mamba3/ssd.py:118-244. Returns (y (B,T,H,P,R), h_final (B,H,P,N) fp32 or None)."""
    Bat, T, H, P, R = x_g.shape
    N = B_g.shape[3]
    Q = chunk_size
    K = (T + Q - 1) // Q
    pad = K * Q - T
    if pad:
        p5 = (0, 0, 0, 0, 0, 0, 0, pad)
        x_g, B_g, C, x_raw = (F.pad(t, p5) for t in (x_g, B_g, C, x_raw))
        dt = F.pad(dt, (0, 0, 0, pad))
        if x_b is not None:
            x_b, B_b = F.pad(x_b, p5), F.pad(B_b, p5)

    cum = (A[None, None, :] * dt).reshape(Bat, K, Q, H).float().cumsum(dim=2).permute(0, 1, 3, 2)
    e_cum = cum.exp()
    chunk_decay = e_cum[..., -1]

    def chunk(t):  # (B,T,H,X,R) -> (B,K,H,R,Q,X)
        return t.reshape(Bat, K, Q, H, t.shape[3], R).permute(0, 1, 3, 5, 2, 4).contiguous()

    wdt = x_g.dtype
    dt_w = dt.reshape(Bat, K, Q, H).permute(0, 1, 3, 2).to(wdt)[:, :, :, None, :, None]
    BKH = Bat * K * H
    dtx = dt_w * chunk(x_g)
    Bc = chunk(B_g)
    if x_b is not None:
        dtx = torch.cat([dtx, dt_w * chunk(x_b)], dim=3)
        Bc = torch.cat([Bc, chunk(B_b)], dim=3)
    R2 = dtx.shape[3]
    lhs = dtx.reshape(BKH, R2, Q, P).permute(0, 2, 3, 1).reshape(BKH * Q, P, R2)
    rhs = Bc.reshape(BKH, R2, Q, N).permute(0, 2, 1, 3).reshape(BKH * Q, R2, N)
    BX = torch.bmm(lhs, rhs).reshape(Bat, K, H, Q, P, N)

    Cw = chunk(C).to(wdt)
    y_intra, s_sum = _intra_chunk(BX, cum, Cw)
    h_chunk = (chunk_decay[..., None, None] * s_sum).to(wdt)
    h0 = h_init.reshape(Bat, H, P * N) if h_init is not None else None
    h_states = scan_forward(chunk_decay, h_chunk.reshape(Bat, K, H, P * N), h0)
    h_states = h_states.to(h_chunk.dtype).reshape(Bat, K, H, P, N)

    hm = h_states.to(wdt).reshape(BKH, P, N).transpose(-2, -1)
    y_inter = (torch.bmm(Cw.reshape(BKH, R * Q, N), hm).reshape(Bat, K, H, R, Q, P).float()
               * e_cum[:, :, :, None, :, None]).to(wdt)
    y_d = D[None, None, :, None, None, None] * chunk(x_raw).to(wdt)
    y = (y_intra + y_inter + y_d).permute(0, 1, 4, 2, 5, 3).reshape(Bat, K * Q, H, P, R)[:, :T]

    h_final = None
    if return_final_state:
        h_final = (chunk_decay[:, K - 1, :, None, None] * h_states[:, K - 1].float()
                   + h_chunk[:, K - 1].float())
    return y.to(x_g.dtype), h_final


def _prep_bc(cfg: LayerCfg, p: dict, Bf, Cf, lead):
    """RMSNorm over N*R, bias, group expand (mamba3/mamba3.py:151-157, 174-180).
    `lead` is the leading shape ((B,T) or (B,))."""
    G, N, R = cfg.ngroups, cfg.d_state, cfg.mimo_rank
    Bn = rmsnorm(Bf.reshape(*lead, G, N * R), p["B_norm.weight"], cfg.eps).reshape(*lead, G, N, R)
    Cn = rmsnorm(Cf.reshape(*lead, G, N * R), p["C_norm.weight"], cfg.eps).reshape(*lead, G, N, R)
    Bn = expand_groups(cfg, Bn + p["B_bias"])
    Cn = expand_groups(cfg, Cn + p["C_bias"])
    return Bn, Cn


def layer_core(cfg: LayerCfg, p: dict, proj: torch.Tensor, dt_scale=None,
               return_state: bool = False):
    """The region between in_proj and out_proj (mamba3/mamba3.py:199-256): in_proj output
    (B,T,W) -> gated, rank-reduced activation (B,T,d_inner) that feeds out_proj, and the
    prefill state (or None)."""
    Bat, T, _ = proj.shape
    H, P, N, R = cfg.H, cfg.headdim, cfg.d_state, cfg.mimo_rank
    z, xf, Bf, Cf, dt_raw, lam_raw, theta = split_proj(cfg, proj)
    dt = F.softplus(dt_raw + p["dt_bias"])
    if dt_scale is not None:
        dt = dt * dt_scale
    A = -torch.exp(p["A_log"])
    dA = torch.exp(A[None, None, :] * dt)

    Bt, Ct = _prep_bc(cfg, p, Bf, Cf, (Bat, T))
    angles = None
    if cfg.use_complex_ssm:
        angles = -(dt.unsqueeze(-1) * theta.unsqueeze(-2)).cumsum(dim=1)
        c = torch.cos(angles).unsqueeze(-1)
        s = torch.sin(angles).unsqueeze(-1)
        Bt, Ct = rope_pairs(Bt, c, s), rope_pairs(Ct, c, s)

    x_r = xf.reshape(Bat, T, H, P, 1) * p["mimo_x"][None, None]
    if cfg.use_trapezoidal:
        lam = torch.sigmoid(lam_raw)
        x_g = x_r * lam[..., None, None]
        x_prev = F.pad(x_r[:, :-1], (0, 0, 0, 0, 0, 0, 1, 0))
        B_prev = F.pad(Bt[:, :-1], (0, 0, 0, 0, 0, 0, 1, 0))
        x_b = x_prev * ((1.0 - lam) * dA)[..., None, None]
    else:
        x_g, x_b, B_prev = x_r, None, None

    y_ssd, h_final = chunked_ssd(x_g, x_b, Bt, B_prev, Ct, dt, A, p["D"], x_r, cfg.chunk_size,
                                 return_final_state=return_state)
    z_r = z.reshape(Bat, T, H, P).unsqueeze(-1) * p["mimo_z"][None, None]
    y = ((y_ssd * F.silu(z_r)) * p["mimo_down"][None, None]).sum(dim=-1)
    y = y.reshape(Bat, T, cfg.d_inner)

    state = None
    if return_state:
        angle = angles[:, T - 1] if angles is not None else \
            torch.zeros(Bat, H, N // 2, dtype=proj.dtype)
        prev_bx = torch.einsum("bhnr,bhpr->bhpn", Bt[:, T - 1], x_r[:, T - 1])
        state = {"h": h_final.float(), "angle": angle, "prev_BX": prev_bx.float()}
    return y, state


def layer_forward(cfg: LayerCfg, p: dict, x: torch.Tensor, dt_scale=None,
                  return_state: bool = False):
    """mamba3/mamba3.py:192-258: in_proj -> layer_core -> out_proj. Returns (out, state)."""
    proj = F.linear(x, p["in_proj.weight"], p.get("in_proj.bias"))
    y, state = layer_core(cfg, p, proj, dt_scale, return_state)
    out = F.linear(y, p["out_proj.weight"], p.get("out_proj.bias"))
    return out, state


def zero_state(cfg: LayerCfg, batch: int, dtype=torch.float32) -> dict:
    """mamba3/mamba3.py:324-332."""
    H, P, N = cfg.H, cfg.headdim, cfg.d_state
    return {"h": torch.zeros(batch, H, P, N), "angle": torch.zeros(batch, H, N // 2, dtype=dtype),
            "prev_BX": torch.zeros(batch, H, P, N)}


def layer_step(cfg: LayerCfg, p: dict, x_tok: torch.Tensor, state: dict, dt_scale=None):
    """mamba3/mamba3.py:267-322 for x_tok (B, d_model). Returns (out (B,d_model), state)."""
    proj = F.linear(x_tok, p["in_proj.weight"], p.get("in_proj.bias"))
    y, new_state = layer_step_core(cfg, p, proj, state, dt_scale)
    out = F.linear(y, p["out_proj.weight"], p.get("out_proj.bias"))
    return out, new_state


def layer_step_core(cfg: LayerCfg, p: dict, proj: torch.Tensor, state: dict, dt_scale=None):
    """The step between in_proj and out_proj (mamba3/mamba3.py:275-317): in_proj output
    proj (B, W) -> (gated activation (B, d_inner) that feeds out_proj, new state)."""
    H, P, N, R = cfg.H, cfg.headdim, cfg.d_state, cfg.mimo_rank
    Bat = proj.shape[0]
    z, xf, Bf, Cf, dt_raw, lam_raw, theta = split_proj(cfg, proj)
    dt = F.softplus(dt_raw + p["dt_bias"])
    if dt_scale is not None:
        dt = dt * dt_scale
    A = -torch.exp(p["A_log"])
    dA = torch.exp(A * dt)

    Bt, Ct = _prep_bc(cfg, p, Bf, Cf, (Bat,))
    angle = state["angle"]
    if cfg.use_complex_ssm:
        angle = angle - dt.unsqueeze(-1) * theta.unsqueeze(-2)
        # cos / sin in the activation dtype: the reference's angle is in that dtype
        # (mamba3/mamba3.py:330), so this is its arithmetic; an fp32 angle state (kept by
        # mamba3_amd) then rotates bf16 activations in bf16 as well
        c = torch.cos(angle).to(Bt.dtype).unsqueeze(-1)
        s = torch.sin(angle).to(Bt.dtype).unsqueeze(-1)
        Bt, Ct = rope_pairs(Bt, c, s), rope_pairs(Ct, c, s)

    x_r = xf.reshape(Bat, H, P, 1) * p["mimo_x"][None]
    if cfg.use_trapezoidal:
        lam = torch.sigmoid(lam_raw)
        gamma, beta = lam * dt, (1.0 - lam) * dt * dA
    else:
        gamma, beta = dt, torch.zeros_like(dt)
    cur = torch.einsum("bhnr,bhpr->bhpn", Bt, x_r)
    h = (dA[:, :, None, None].float() * state["h"].float()
         + gamma[:, :, None, None].float() * cur.float()
         + beta[:, :, None, None].float() * state["prev_BX"].float())
    y_r = torch.einsum("bhnr,bhpn->bhpr", Ct.float(), h).to(proj.dtype) + p["D"][None, :, None, None] * x_r
    z_r = z.reshape(Bat, H, P).unsqueeze(-1) * p["mimo_z"][None]
    y = ((y_r * F.silu(z_r)) * p["mimo_down"][None]).sum(dim=-1).reshape(Bat, cfg.d_inner)
    return y, {"h": h, "angle": angle, "prev_BX": cur.float()}


def _block_sub(p: dict, prefix: str) -> dict:
    """Parameters of block `prefix`'s KulaMamba, under the layer's own names."""
    return {k[len(prefix) + 4:]: v for k, v in p.items() if k.startswith(prefix + "ssm.")}


def _swiglu(p: dict, prefix: str, xn: torch.Tensor) -> torch.Tensor:
    """mamba3/block.py:16-26: w_down(silu(w_gate x) * w_up x)."""
    g = F.linear(xn, p[prefix + "mlp.w_gate.weight"], p.get(prefix + "mlp.w_gate.bias"))
    u = F.linear(xn, p[prefix + "mlp.w_up.weight"], p.get(prefix + "mlp.w_up.bias"))
    return F.linear(F.silu(g) * u, p[prefix + "mlp.w_down.weight"], p.get(prefix + "mlp.w_down.bias"))


def block_forward(cfg: LayerCfg, p: dict, prefix: str, x: torch.Tensor, scale: float,
                  use_mlp: bool, norm_eps: float = 1e-5, return_state: bool = False):
    """mamba3/block.py:79-92 (no checkpointing) with parameters under `prefix`; with
    return_state, mamba3/block.py:102-107 (prefill) and returns (x, state)."""
    h, state = layer_forward(cfg, _block_sub(p, prefix),
                             rmsnorm(x, p[prefix + "ssm_norm.weight"], norm_eps),
                             return_state=return_state)
    x = x + h * scale
    if use_mlp:
        x = x + _swiglu(p, prefix, rmsnorm(x, p[prefix + "mlp_norm.weight"], norm_eps)) * scale
    return (x, state) if return_state else x


def block_step(cfg: LayerCfg, p: dict, prefix: str, x: torch.Tensor, state: dict, scale: float,
               use_mlp: bool, norm_eps: float = 1e-5):
    """mamba3/block.py:94-100: one decode token (B, d_model) through block `prefix`."""
    h, state = layer_step(cfg, _block_sub(p, prefix),
                          rmsnorm(x, p[prefix + "ssm_norm.weight"], norm_eps), state)
    x = x + h * scale
    if use_mlp:
        x = x + _swiglu(p, prefix, rmsnorm(x, p[prefix + "mlp_norm.weight"], norm_eps)) * scale
    return x, state


def lm_head(p: dict, x: torch.Tensor, norm_eps: float = 1e-5) -> torch.Tensor:
    """mamba3/block.py:182-183: final RMSNorm, then the (tied) lm_head."""
    return F.linear(rmsnorm(x, p["norm.weight"], norm_eps), p["lm_head.weight"])


def lm_forward(cfg: LayerCfg, p: dict, ids: torch.Tensor, n_layers: int, scale: float,
               use_mlp: bool = True, norm_eps: float = 1e-5) -> torch.Tensor:
    """mamba3/block.py:178-184: embedding, n_layers blocks, norm, lm_head -> logits."""
    x = F.embedding(ids, p["embedding.weight"])
    for i in range(n_layers):
        x = block_forward(cfg, p, f"layers.{i}.", x, scale, use_mlp, norm_eps)
    return lm_head(p, x, norm_eps)


def lm_prefill(cfg: LayerCfg, p: dict, ids: torch.Tensor, n_layers: int, scale: float,
               use_mlp: bool = True, norm_eps: float = 1e-5):
    """mamba3/block.py:199-206: prefill every block; returns (last-token logits, states)."""
    x = F.embedding(ids, p["embedding.weight"])
    states = []
    for i in range(n_layers):
        x, st = block_forward(cfg, p, f"layers.{i}.", x, scale, use_mlp, norm_eps,
                              return_state=True)
        states.append(st)
    return lm_head(p, x[:, -1], norm_eps), states


def lm_step(cfg: LayerCfg, p: dict, tok: torch.Tensor, states: list, scale: float,
            use_mlp: bool = True, norm_eps: float = 1e-5):
    """mamba3/block.py:226-229: one token id per row through every block's step; returns
    (logits, new states)."""
    x = F.embedding(tok, p["embedding.weight"])
    new = []
    for i, st in enumerate(states):
        x, st = block_step(cfg, p, f"layers.{i}.", x, st, scale, use_mlp, norm_eps)
        new.append(st)
    return lm_head(p, x, norm_eps), new


def lm_generate_greedy(cfg: LayerCfg, p: dict, ids: torch.Tensor, n_layers: int, scale: float,
                       max_new_tokens: int, use_mlp: bool = True, norm_eps: float = 1e-5):
    """mamba3/block.py:195-231 at temperature 0 (argmax, no top-k)."""
    logits, states = lm_prefill(cfg, p, ids, n_layers, scale, use_mlp, norm_eps)
    out = [ids]
    for _ in range(max_new_tokens):
        nxt = logits.argmax(dim=-1, keepdim=True)
        out.append(nxt)
        logits, states = lm_step(cfg, p, nxt.squeeze(1), states, scale, use_mlp, norm_eps)
    return torch.cat(out, dim=1)
