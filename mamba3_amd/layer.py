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

from . import _native, ops


class RMSNorm(nn.Module):
    """Root-mean-square norm with learned scale (mamba3/mamba3.py:19-35).

    The block / LM norms run as one HIP kernel pass (m3_rmsnorm_fwd, backward
    m3_rmsnorm_bwd) with the reference's arithmetic: fp32 statistics, the scale and x*scale
    rounded to x's dtype. Inside KulaMamba only B_norm / C_norm's weights are read (that
    normalisation is fused into the SSD kernels). GPU tensors only, like the rest of the
    package."""

    def __init__(self, d: int, eps: float = 1e-5, dim: int = -1):
        super().__init__()
        self.weight = nn.Parameter(torch.ones(d))
        self.eps = eps
        self.dim = dim

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        _native.require_gpu(x)
        d = self.dim % x.ndim
        if d != x.ndim - 1:
            y, _ = ops.rmsnorm(x.movedim(d, -1), self.weight, float(self.eps))
            return y.movedim(-1, d)
        y, _ = ops.rmsnorm(x, self.weight, float(self.eps))
        return y


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
        """fp32 copies of the small parameters as the C-ABI struct (cached per version)."""
        return ops._f32_params(self._small_params())[0]

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
    def _pre_out(self, x: torch.Tensor, dt_scale=None, return_state: bool = False):
        """in_proj and the SSD core: x (B,T,d_model) -> (out_proj's input (B,T,d_inner),
        state or None)."""
        if x.dim() != 3:
            raise ValueError(f"expected (batch, seqlen, d_model), got {tuple(x.shape)}")
        if x.shape[1] <= 0:
            raise ValueError(f"Sequence length must be positive, got {x.shape[1]}")
        _native.require_gpu(x)
        # A 3-D input whose batch rows are not adjacent would send the projection down
        # torch's batched bf16 GEMM with a transposed weight view, which returned wrong rows
        # on this GPU; a contiguous input folds to one 2-D GEMM.
        return self.ssd_from_proj(self._in_proj_wide(x.contiguous()), dt_scale, return_state)

    def _in_proj_wide(self, x: torch.Tensor) -> torch.Tensor:
        """in_proj(x) for the prefill. Without autograd the output width is padded to a
        multiple of 256 columns when that adds at most 1/16 (zero weight rows): hipBLASLt's
        256-wide output tiles then cover each row exactly (d_model 768: 3696 -> 3840 columns,
        the (65536, 768) x (768, N) GEMM measured 443 -> 331 us), and the kernels read proj
        through its row stride, never the padding. With autograd the plain projection runs
        (the layer backward leaves the padding columns of its proj gradient unwritten)."""
        w = self.in_proj.weight
        n = w.shape[0]
        npad = -(-n // 256) * 256
        if (torch.is_grad_enabled() or npad == n or (npad - n) * 16 > n
                or torch.compiler.is_compiling()):
            return self.in_proj(x)
        b = self.in_proj.bias
        key = (w.data_ptr(), w._version, w.dtype, w.device,
               None if b is None else (b.data_ptr(), b._version))
        cache = self.__dict__.get("_wide_in_proj")
        if cache is None or cache[0] != key:
            wp = torch.zeros(npad, w.shape[1], dtype=w.dtype, device=w.device)
            wp[:n] = w
            bp = None
            if b is not None:
                bp = torch.zeros(npad, dtype=b.dtype, device=b.device)
                bp[:n] = b
            cache = (key, wp, bp)
            self.__dict__["_wide_in_proj"] = cache
        return nn.functional.linear(x, cache[1], cache[2])

    def _forward_impl(self, x: torch.Tensor, dt_scale=None, return_state: bool = False):
        y, state = self._pre_out(x, dt_scale, return_state)
        return self.out_proj(y), state

    def ssd_from_proj(self, proj: torch.Tensor, dt_scale=None, return_state: bool = False):
        """Everything between in_proj and out_proj (mamba3/mamba3.py:199-256) on the HIP
        kernels: proj (B,T,d_in_proj) -> (y (B,T,d_inner) in proj.dtype, state or None).

        With autograd recording (proj, a parameter or dt_scale requires grad) this is the
        differentiable `prefill_train` op: fp32 arithmetic on the fp32 layer path, whose
        backward is m3_layer_bwd. Shapes m3_layer_bwd does not cover raise there."""
        _native.require_gpu(proj)
        self._check_norm_eps()
        Bat, T, _ = proj.shape
        scale = self._dt_scale(dt_scale, (Bat, T, self.nheads), proj.device)
        params = self._small_params()
        args = ops.layer_args(self)
        if torch.is_grad_enabled() and (proj.requires_grad or
                                        (scale is not None and scale.requires_grad) or
                                        any(p.requires_grad for p in params)):
            y, h, angle, prev, _ = ops.prefill_train(proj, *params, scale, *args)
        else:
            y, h, angle, prev = ops.prefill(proj, *params, scale, *args, return_state)
        state = {"h": h, "angle": angle, "prev_BX": prev} if return_state else None
        return y, state

    def forward(self, x: torch.Tensor, dt_scale=None) -> torch.Tensor:
        output, _ = self._forward_impl(x, dt_scale, return_state=False)
        return output

    def prefill(self, x: torch.Tensor, dt_scale=None):
        """Parallel prefill returning (output, state) for subsequent `step` calls."""
        return self._forward_impl(x, dt_scale, return_state=True)

    def step(self, hidden_states: torch.Tensor, ssm_state: dict, dt_scale=None):
        """One decode step (mamba3/mamba3.py:267-322). `hidden_states` is (B, d_model)
        or (B, 1, d_model); the output has the same rank. Returns a new state dict. Under
        autograd the step is differentiable (m3_step_bwd) with respect to the input, the
        incoming state, the parameters and dt_scale, as the reference's is."""
        squeeze = hidden_states.dim() == 2
        y, state = self._step_pre_out(hidden_states, ssm_state, dt_scale)
        w = self.out_proj.weight
        if self.out_proj.bias is None and ops.small_proj_usable(y, w):
            out = ops.small_linear_fast(y, None, 0.0, w, None, 1.0)
        else:
            out = self.out_proj(y)
        if not squeeze:
            out = out.unsqueeze(1)
        return out, state

    def _step_pre_out(self, hidden_states: torch.Tensor, ssm_state: dict, dt_scale=None):
        """in_proj and the step kernel: (out_proj's input (B, d_inner), new state)."""
        x_in = hidden_states if hidden_states.dim() == 2 else hidden_states.squeeze(1)
        if x_in.dim() != 2:
            raise ValueError(f"expected (B, d_model) or (B, 1, d_model), got {tuple(hidden_states.shape)}")
        _native.require_gpu(x_in)
        w = self.in_proj.weight
        if self.in_proj.bias is None and ops.small_proj_usable(x_in, w):
            proj = ops.small_linear_fast(x_in, None, 0.0, w, None, 1.0)
        else:
            proj = self.in_proj(x_in)
        return self._step_from_proj(proj, ssm_state, dt_scale)

    def _step_from_proj(self, proj: torch.Tensor, ssm_state: dict, dt_scale=None):
        """The step kernel on the in_proj output proj (B, d_in_proj): (out_proj's input
        (B, d_inner), new state)."""
        self._check_norm_eps()
        h_in, prev_in, angle_in = self._check_state(ssm_state, proj.shape[0])
        scale = self._dt_scale(dt_scale, (proj.shape[0], self.nheads), proj.device)
        y, h_out, prev_out, angle_out = ops.step_fast(proj, *self._small_params(), scale, h_in,
                                                 prev_in, angle_in, *ops.layer_args(self))
        return y, {"h": h_out, "angle": angle_out, "prev_BX": prev_out}

    def _check_state(self, ssm_state: dict, batch: int):
        H, P, N = self.nheads, self.headdim, self.d_state
        h_in, prev_in, angle_in = ssm_state["h"], ssm_state["prev_BX"], ssm_state["angle"]
        for name, t, shape in (("h", h_in, (batch, H, P, N)), ("prev_BX", prev_in, (batch, H, P, N)),
                               ("angle", angle_in, (batch, H, N // 2))):
            if tuple(t.shape) != shape:
                raise ValueError(f"state['{name}'] has shape {tuple(t.shape)}, expected {shape}")
        _native.require_gpu(h_in, prev_in, angle_in)
        return h_in, prev_in, angle_in

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
