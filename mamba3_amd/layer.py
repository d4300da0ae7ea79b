"""KulaMamba layer: drop-in for mamba3.mamba3 (mamba3/mamba3.py:19-332).

The projections stay PyTorch GEMMs (hipBLASLt); everything between in_proj and
out_proj — dt/decay, B/C RMSNorm + bias + data-dependent RoPE, MIMO expansion, the
trapezoidal two-term update, the chunked SSD with its inter-chunk recurrence, the SiLU
gate and the MIMO-down sum — runs as hand-written gfx950 HIP kernels through the C-ABI
in include/mamba3_amd.h. There is no CPU path: the module must live on the GPU.

State dict compatibility: parameter names, shapes and registration order equal the
reference's (mamba3/mamba3.py:95-111), and the initialisation consumes the RNG in the
same order (mamba3/mamba3.py:95, 111-123), so seeded modules hold identical weights.
"""

from __future__ import annotations

import math

import torch
import torch.nn as nn

from . import _native


class RMSNorm(nn.Module):
    """Root-mean-square norm with learned scale (mamba3/mamba3.py:19-35).

    Used as a PyTorch op by the block/LM glue; inside KulaMamba only its weight is read
    (the B/C normalisation itself runs in the HIP kernels).
    """

    def __init__(self, d: int, eps: float = 1e-5, dim: int = -1):
        super().__init__()
        self.weight = nn.Parameter(torch.ones(d))
        self.eps = eps
        self.dim = dim

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        scale = torch.rsqrt(x.float().square().mean(self.dim, keepdim=True) + self.eps)
        shape = [1] * x.ndim
        shape[self.dim] = -1
        return x * scale.to(x.dtype) * self.weight.view(*shape)


class _ForwardOnly(torch.autograd.Function):
    """Ties a decode-step output to its input so that backward raises instead of silently
    producing wrong gradients (the step kernel has no backward)."""

    @staticmethod
    def forward(ctx, anchor, out):
        return out

    @staticmethod
    def backward(ctx, grad):
        raise NotImplementedError(
            "KulaMamba.step has no backward in mamba3_amd; train through forward / prefill")


class _LayerTrainFn(torch.autograd.Function):
    """Differentiable ssd_from_proj on HIP kernels in both directions: the forward is the fp32
    layer prefill (m3_prefill_fwd on an fp32 desc), whose workspace keeps its intermediates
    for the backward, m3_layer_bwd (gate, chunked SSD and preparation backward). bf16
    inputs and parameters are computed in fp32; gradients come back in their dtypes."""

    @staticmethod
    def forward(ctx, layer, proj, dt_scale, return_state, *params):
        Bat, T, _ = proj.shape
        H, P, N = layer.nheads, layer.headdim, layer.d_state
        dev = proj.device
        proj32 = proj.detach().float().contiguous()
        p32 = [t.detach().float().contiguous() for t in params]
        desc = layer._desc(Bat, T, proj32)
        pack = _native.LayerParams(*[t.data_ptr() for t in p32])
        scale = layer._dt_scale(dt_scale, (Bat, T, H), dev)
        ws_bytes = _native.prefill_workspace_bytes(desc)
        ws = torch.empty(max(ws_bytes, 1), device=dev, dtype=torch.uint8)
        y = torch.empty(Bat, T, layer.d_inner, device=dev, dtype=torch.float32)
        h_final = angle = prev_bx = None
        if return_state:
            h_final = torch.empty(Bat, H, P, N, device=dev, dtype=torch.float32)
            angle = torch.empty(Bat, H, N // 2, device=dev, dtype=torch.float32)
            prev_bx = torch.empty(Bat, H, P, N, device=dev, dtype=torch.float32)
        _native.prefill_fwd(desc, pack, proj32, scale, y, h_final, angle, prev_bx, ws, ws_bytes)
        ctx.save_for_backward(proj32, ws, scale, *p32)
        ctx.desc = desc
        ctx.proj_dtype = proj.dtype
        ctx.param_dtypes = [t.dtype for t in params]
        ctx.set_materialize_grads(False)
        return y.to(proj.dtype), h_final, angle, prev_bx

    @staticmethod
    def backward(ctx, g_y, g_h, g_angle, g_prev):
        proj32, ws, scale, *p32 = ctx.saved_tensors
        if g_y is None:
            g_y = torch.zeros(proj32.shape[0], proj32.shape[1], ctx.desc.nheads * ctx.desc.headdim,
                              device=proj32.device)

        def f32(t):
            return None if t is None else t.float().contiguous()

        g_proj = torch.empty_like(proj32)
        grads = [torch.empty_like(t) for t in p32]
        _native.layer_bwd(ctx.desc, _native.LayerParams(*[t.data_ptr() for t in p32]), proj32,
                          scale, ws, f32(g_y), f32(g_h), f32(g_angle), f32(g_prev), g_proj,
                          _native.LayerParamGrads(*[t.data_ptr() for t in grads]))
        return (None, g_proj.to(ctx.proj_dtype), None, None,
                *[g.to(dt) for g, dt in zip(grads, ctx.param_dtypes)])


class KulaMamba(nn.Module):
    """Mamba-3 SSD layer (mamba3/mamba3.py:48-332) on MI355X HIP kernels."""

    def __init__(
        self,
        d_model: int,
        d_state: int = 128,
        expand: int = 2,
        headdim: int = 64,
        ngroups: int | None = None,
        mimo_rank: int = 2,
        chunk_size: int = 64,
        bias: bool = False,
        dt_min: float = 0.001,
        dt_max: float = 0.1,
        use_trapezoidal: bool = True,
        use_complex_ssm: bool = True,
    ):
        super().__init__()
        self.d_model = d_model
        self.d_state = d_state
        self.expand = expand
        self.headdim = headdim
        self.mimo_rank = max(mimo_rank, 1)
        # The kernels pick their own internal chunking; chunk_size is kept for API
        # compatibility (results do not depend on it beyond rounding).
        self.chunk_size = chunk_size
        self.use_trapezoidal = use_trapezoidal
        self.use_complex_ssm = use_complex_ssm

        self.d_inner = expand * d_model
        if self.d_inner % headdim != 0:
            raise ValueError(f"d_inner={self.d_inner} is not a multiple of headdim={headdim}")
        self.nheads = self.d_inner // headdim
        if d_state % 2 != 0:
            raise ValueError("d_state must be even (RoPE acts on pairs)")
        self.ngroups = 1 if ngroups is None else ngroups
        if self.nheads % self.ngroups != 0:
            raise ValueError(f"nheads={self.nheads} is not a multiple of ngroups={self.ngroups}")
        self.heads_per_group = self.nheads // self.ngroups

        H, P, N, R, G = self.nheads, headdim, d_state, self.mimo_rank, self.ngroups
        self._d_bc = G * N * R
        self._d_x = self.d_inner
        width = 2 * self.d_inner + 2 * self._d_bc + H
        width += H if use_trapezoidal else 0
        width += N // 2 if use_complex_ssm else 0
        self.in_proj = nn.Linear(d_model, width, bias=bias)

        self.A_log = nn.Parameter(torch.zeros(H))
        self.D = nn.Parameter(torch.ones(H))
        self.dt_bias = nn.Parameter(torch.zeros(H))
        self.B_norm = RMSNorm(N * R)
        self.C_norm = RMSNorm(N * R)
        self.B_bias = nn.Parameter(torch.ones(G, N, R))
        self.C_bias = nn.Parameter(torch.ones(G, N, R))
        self.mimo_x = nn.Parameter(torch.ones(H, P, R))
        self.mimo_z = nn.Parameter(torch.ones(H, P, R))
        self.mimo_down = nn.Parameter(torch.full((H, P, R), 1.0 / R))
        self.out_proj = nn.Linear(self.d_inner, d_model, bias=bias)
        self._init_weights(dt_min, dt_max)
        self._pack_key = None
        self._pack = None

    def _init_weights(self, dt_min: float, dt_max: float) -> None:
        """Reference initialisation (mamba3/mamba3.py:114-123): kaiming in_proj, dt_bias
        as the inverse softplus of a log-uniform dt in [dt_min, dt_max], A_log ~ U(-4,-1)."""
        nn.init.kaiming_uniform_(self.in_proj.weight, a=math.sqrt(5))
        with torch.no_grad():
            lo, hi = math.log(dt_min), math.log(dt_max)
            dt = torch.exp(torch.rand(self.nheads) * (hi - lo) + lo)
            self.dt_bias.copy_(dt + torch.log(-torch.expm1(-dt)))
            nn.init.uniform_(self.A_log, -4.0, -1.0)

    # ------------------------------------------------------------------ native glue
    def _small_params(self):
        return (self.A_log, self.D, self.dt_bias, self.B_norm.weight, self.C_norm.weight,
                self.B_bias, self.C_bias, self.mimo_x, self.mimo_z, self.mimo_down)

    def _param_pack(self) -> _native.LayerParams:
        """fp32 contiguous copies of the small parameters, rebuilt when any changes."""
        tensors = self._small_params()
        key = tuple((t.data_ptr(), t._version, t.dtype, t.device) for t in tensors)
        if key != self._pack_key:
            with torch.no_grad():
                f32 = [t.detach().float().contiguous() for t in tensors]
            pack = _native.LayerParams(*[t.data_ptr() for t in f32])
            self._pack = (pack, f32)
            self._pack_key = key
        return self._pack[0]

    def _desc(self, batch: int, seqlen: int, proj: torch.Tensor) -> _native.LayerDesc:
        return _native.LayerDesc(
            batch=batch, seqlen=seqlen, nheads=self.nheads, headdim=self.headdim,
            d_state=self.d_state, mimo_rank=self.mimo_rank, ngroups=self.ngroups,
            use_trapezoidal=int(self.use_trapezoidal), use_complex=int(self.use_complex_ssm),
            dtype=_native.dtype_code(proj.dtype), proj_row_stride=proj.stride(-2),
            rms_eps=float(self.B_norm.eps))

    def _check_norm_eps(self) -> None:
        if self.B_norm.eps != self.C_norm.eps:
            raise ValueError("B_norm and C_norm must share eps")

    @staticmethod
    def _dt_scale(dt_scale, shape, device):
        if dt_scale is None:
            return None
        if not torch.is_tensor(dt_scale):
            dt_scale = torch.tensor(float(dt_scale), device=device)
        return dt_scale.to(device=device, dtype=torch.float32).expand(shape).contiguous()

    # ------------------------------------------------------------------ forward paths
    def _forward_impl(self, x: torch.Tensor, dt_scale=None, return_state: bool = False):
        if x.dim() != 3:
            raise ValueError(f"expected (batch, seqlen, d_model), got {tuple(x.shape)}")
        if x.shape[1] <= 0:
            raise ValueError(f"Sequence length must be positive, got {x.shape[1]}")
        _native.require_gpu(x)
        proj = self.in_proj(x)
        y, state = self.ssd_from_proj(proj, dt_scale, return_state)
        return self.out_proj(y), state

    def ssd_from_proj(self, proj: torch.Tensor, dt_scale=None, return_state: bool = False):
        """Everything between in_proj and out_proj (mamba3/mamba3.py:199-256) on the HIP
        kernels: proj (B,T,d_in_proj) -> (y (B,T,d_inner) in proj.dtype, state or None)."""
        _native.require_gpu(proj)
        self._check_norm_eps()
        if torch.is_grad_enabled() and (proj.requires_grad or
                                        any(p.requires_grad for p in self._small_params())):
            Bat, T, _ = proj.shape
            desc32 = self._desc(Bat, T, proj.detach().float())
            if _native.layer_bwd_supported(desc32):
                y, h, angle, prev = _LayerTrainFn.apply(self, proj, dt_scale, return_state,
                                                        *self._small_params())
                state = {"h": h, "angle": angle, "prev_BX": prev} if return_state else None
                return y, state
            return self._ssd_train(proj, dt_scale, return_state)
        proj = proj.contiguous()
        Bat, T, _ = proj.shape
        H, P, N = self.nheads, self.headdim, self.d_state
        desc = self._desc(Bat, T, proj)
        params = self._param_pack()
        scale = self._dt_scale(dt_scale, (Bat, T, H), proj.device)

        dev = proj.device
        y = torch.empty(Bat, T, self.d_inner, device=dev, dtype=proj.dtype)
        h_final = angle = prev_bx = None
        if return_state:
            h_final = torch.empty(Bat, H, P, N, device=dev, dtype=torch.float32)
            angle = torch.empty(Bat, H, N // 2, device=dev, dtype=torch.float32)
            prev_bx = torch.empty(Bat, H, P, N, device=dev, dtype=torch.float32)
        ws_bytes = _native.prefill_workspace_bytes(desc)
        workspace = torch.empty(max(ws_bytes, 1), device=dev, dtype=torch.uint8)
        _native.prefill_fwd(desc, params, proj, scale, y, h_final, angle, prev_bx, workspace,
                            ws_bytes)
        state = None
        if return_state:
            state = {"h": h_final, "angle": angle, "prev_BX": prev_bx}
        return y, state

    def _ssd_train(self, proj: torch.Tensor, dt_scale=None, return_state: bool = False):
        """Differentiable form of ssd_from_proj for the shapes m3_layer_bwd does not cover
        (its per-token LDS would exceed 64 KB): the reference's element-wise preparation and
        gate (mamba3/mamba3.py:142-166, 197-239) as PyTorch ops in fp32 around chunked_ssd,
        whose forward and backward run on the HIP kernels (m3_chunked_ssd_fwd /
        m3_chunked_ssd_bwd). The state it returns matches the fused path's (fp32 h, angle
        and prev_BX; mamba3/mamba3.py:241-256)."""
        from .ssd import chunked_ssd

        Bat, T, _ = proj.shape
        H, P, N, R, G = self.nheads, self.headdim, self.d_state, self.mimo_rank, self.ngroups
        sizes = [self.d_inner, self._d_x, self._d_bc, self._d_bc, H]
        sizes += [H] if self.use_trapezoidal else []
        sizes += [N // 2] if self.use_complex_ssm else []
        parts = list(proj.float().split(sizes, dim=-1))
        z, x_flat, B_flat, C_flat, dt_raw = parts[:5]
        lam_raw = parts[5] if self.use_trapezoidal else None
        theta_raw = parts[-1] if self.use_complex_ssm else None

        dt = nn.functional.softplus(dt_raw + self.dt_bias.float())
        if dt_scale is not None:
            dt = dt * self._dt_scale(dt_scale, (Bat, T, H), proj.device)
        A = -torch.exp(self.A_log.float())
        dA = torch.exp(A * dt)

        def norm_bias(flat, norm, bias):
            v = norm(flat.reshape(Bat, T, G, N * R)).float().reshape(Bat, T, G, N, R)
            v = v + bias.float()
            return v.repeat_interleave(H // G, dim=2) if G != H else v

        B_r = norm_bias(B_flat, self.B_norm, self.B_bias)
        C_r = norm_bias(C_flat, self.C_norm, self.C_bias)
        angles = None
        if self.use_complex_ssm:
            angles = -(dt.unsqueeze(-1) * theta_raw.unsqueeze(-2)).cumsum(dim=1)  # (B,T,H,N/2)
            cos = torch.cos(angles)[..., None, None]
            sin = torch.sin(angles)[..., None, None]

            def rope(v):
                v = v.reshape(Bat, T, H, N // 2, 2, R)
                ev, od = v[..., 0:1, :], v[..., 1:2, :]
                return torch.cat([ev * cos - od * sin, ev * sin + od * cos], dim=-2).reshape(
                    Bat, T, H, N, R)

            B_r, C_r = rope(B_r), rope(C_r)

        x_r = x_flat.reshape(Bat, T, H, P, 1) * self.mimo_x.float()
        if self.use_trapezoidal:
            lam = torch.sigmoid(lam_raw)
            x_g = x_r * lam[..., None, None]
            x_b = nn.functional.pad(x_r[:, :-1], (0, 0, 0, 0, 0, 0, 1, 0)) * \
                ((1.0 - lam) * dA)[..., None, None]
            B_b = nn.functional.pad(B_r[:, :-1], (0, 0, 0, 0, 0, 0, 1, 0))
        else:
            x_g, x_b, B_b = x_r, None, None
        out = chunked_ssd(x_g, x_b, B_r, B_b, C_r, dt, A, self.D.float(), x_r,
                          self.chunk_size, return_final_state=return_state)
        z_r = z.reshape(Bat, T, H, P, 1) * self.mimo_z.float()
        y = (out.y * nn.functional.silu(z_r) * self.mimo_down.float()).sum(dim=-1)
        y = y.reshape(Bat, T, self.d_inner).to(proj.dtype)
        state = None
        if return_state:
            angle = angles[:, T - 1] if angles is not None else \
                torch.zeros(Bat, H, N // 2, device=proj.device, dtype=torch.float32)
            prev_bx = torch.einsum("bhnr,bhpr->bhpn", B_r[:, T - 1], x_r[:, T - 1])
            state = {"h": out.h_final, "angle": angle, "prev_BX": prev_bx}
        return y, state

    def forward(self, x: torch.Tensor, dt_scale=None) -> torch.Tensor:
        output, _ = self._forward_impl(x, dt_scale, return_state=False)
        return output

    def prefill(self, x: torch.Tensor, dt_scale=None):
        """Parallel prefill returning (output, state) for subsequent `step` calls."""
        return self._forward_impl(x, dt_scale, return_state=True)

    def step(self, hidden_states: torch.Tensor, ssm_state: dict, dt_scale=None):
        """One decode step (mamba3/mamba3.py:267-322). `hidden_states` is (B, d_model)
        or (B, 1, d_model); the output has the same rank. Returns a new state dict."""
        squeeze = hidden_states.dim() == 2
        x_in = hidden_states if squeeze else hidden_states.squeeze(1)
        if x_in.dim() != 2:
            raise ValueError(f"expected (B, d_model) or (B, 1, d_model), got {tuple(hidden_states.shape)}")
        _native.require_gpu(x_in)
        self._check_norm_eps()
        Bat = x_in.shape[0]
        H, P, N = self.nheads, self.headdim, self.d_state

        proj = self.in_proj(x_in).contiguous()
        desc = self._desc(Bat, 1, proj)
        params = self._param_pack()
        scale = self._dt_scale(dt_scale, (Bat, H), x_in.device)

        h_in = ssm_state["h"]
        prev_in = ssm_state["prev_BX"]
        angle_in = ssm_state["angle"]
        for name, t, shape in (("h", h_in, (Bat, H, P, N)), ("prev_BX", prev_in, (Bat, H, P, N)),
                               ("angle", angle_in, (Bat, H, N // 2))):
            if tuple(t.shape) != shape:
                raise ValueError(f"state['{name}'] has shape {tuple(t.shape)}, expected {shape}")
        _native.require_gpu(h_in, prev_in, angle_in)
        h_in = h_in.float().contiguous()
        prev_in = prev_in.float().contiguous()
        if angle_in.dtype not in (torch.float32, torch.bfloat16):
            angle_in = angle_in.float()
        angle_in = angle_in.contiguous()

        dev = x_in.device
        y = torch.empty(Bat, self.d_inner, device=dev, dtype=proj.dtype)
        h_out = torch.empty_like(h_in)
        prev_out = torch.empty_like(prev_in)
        angle_out = torch.empty_like(angle_in)
        _native.step_fwd(desc, params, proj, scale, h_in, prev_in, angle_in, y, h_out,
                         prev_out, angle_out)
        if torch.is_grad_enabled() and (proj.requires_grad or
                                        any(p.requires_grad for p in self._small_params())):
            y = _ForwardOnly.apply(proj, y)
        out = self.out_proj(y)
        if not squeeze:
            out = out.unsqueeze(1)
        return out, {"h": h_out, "angle": angle_out, "prev_BX": prev_out}

    def allocate_inference_state(self, batch_size: int, dtype=None, device=None) -> dict:
        """Zero decode state (mamba3/mamba3.py:324-332). 'h' and 'prev_BX' are fp32 as in
        the reference; 'angle' is kept in fp32 whatever `dtype` says (a bf16 running angle
        loses whole radians after a few thousand tokens). `dtype` is accepted for API
        compatibility."""
        device = device or self.in_proj.weight.device
        H, P, N = self.nheads, self.headdim, self.d_state
        return {
            "h": torch.zeros(batch_size, H, P, N, dtype=torch.float32, device=device),
            "angle": torch.zeros(batch_size, H, N // 2, dtype=torch.float32, device=device),
            "prev_BX": torch.zeros(batch_size, H, P, N, dtype=torch.float32, device=device),
        }
