"""Residual block and language model around KulaMamba: drop-in for mamba3.block
(mamba3/block.py:16-231).

These are the callers of the SSD path (norms, SwiGLU MLP, embedding, tied lm_head,
greedy/sampled decode loop) and run as PyTorch ops; the SSD itself runs in the HIP
kernels through KulaMamba. Module names, registration order and initialisation order
equal the reference's so seeded models hold identical weights.
"""

from __future__ import annotations

import math

import torch
import torch.nn as nn
import torch.nn.functional as F
from torch.utils.checkpoint import checkpoint as grad_checkpoint

from . import _native, ops
from .layer import KulaMamba, RMSNorm


def add_scaled_linear(x: torch.Tensor, lin: nn.Linear, inp: torch.Tensor, scale: float,
                      inplace: bool = False) -> torch.Tensor:
    """x + scale * lin(inp) as one GEMM: the residual x enters hipBLASLt as C with beta = 1
    and the scale as alpha, so the projection's output is neither rounded nor stored before
    the add (the reference runs the projection, the scale and the add as three ops,
    mamba3/block.py:84-91). torch.addmm first copies x into its new output; with inplace
    (x is the caller's own intermediate and no autograd graph needs it) the GEMM accumulates
    into x itself and that copy is saved."""
    inp2 = inp.reshape(-1, inp.shape[-1])
    if inplace and x.is_contiguous():
        x2 = x.view(-1, x.shape[-1])
        x2.addmm_(inp2, lin.weight.t(), beta=1.0, alpha=scale)
        if lin.bias is not None:
            x2.add_(lin.bias, alpha=scale)
        return x
    out = torch.addmm(x.reshape(-1, x.shape[-1]), inp2, lin.weight.t(), beta=1.0, alpha=scale)
    if lin.bias is not None:
        out = out + lin.bias * scale
    return out.view(x.shape)


class SwiGLU(nn.Module):
    """w_down(silu(w_gate x) * w_up x) (mamba3/block.py:16-26)."""

    def __init__(self, d_model: int, d_ff: int | None = None, bias: bool = False):
        super().__init__()
        if d_ff is None:
            d_ff = int(d_model * 8 / 3 / 64 + 1) * 64
        self.w_gate = nn.Linear(d_model, d_ff, bias=bias)
        self.w_up = nn.Linear(d_model, d_ff, bias=bias)
        self.w_down = nn.Linear(d_ff, d_model, bias=bias)

    def hidden(self, x: torch.Tensor) -> torch.Tensor:
        """silu(w_gate x) * w_up x: w_down's input. For bf16 without autograd this is one GEMM
        over the concatenated [w_gate; w_up] weight (zero rows pad it to whole 256-column
        tiles; cached per weight version) and one silu * mul pass (m3_silu_mul) instead of
        two GEMMs and two element-wise passes."""
        wg, wu = self.w_gate.weight, self.w_up.weight
        if (torch.is_grad_enabled() or torch.compiler.is_compiling() or x.dtype != torch.bfloat16
                or wg.dtype != torch.bfloat16 or self.w_gate.bias is not None
                or self.w_up.bias is not None or not x.is_cuda):
            return F.silu(self.w_gate(x)) * self.w_up(x)
        d_ff = wg.shape[0]
        key = (wg.data_ptr(), wg._version, wu.data_ptr(), wu._version, wg.device)
        cache = self.__dict__.get("_gate_up")
        if cache is None or cache[0] != key:
            n = 2 * d_ff
            npad = -(-n // 256) * 256 if (-(-n // 256) * 256 - n) * 16 <= n else n
            w = torch.zeros(npad, wg.shape[1], dtype=wg.dtype, device=wg.device)
            w[:d_ff] = wg
            w[d_ff:n] = wu
            cache = (key, w)
            self.__dict__["_gate_up"] = cache
        gu = F.linear(x.reshape(-1, x.shape[-1]), cache[1])
        return ops.silu_mul_fast(gu, d_ff).view(*x.shape[:-1], d_ff)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return self.w_down(self.hidden(x))


class KulaMambaBlock(nn.Module):
    """Pre-norm residual block: x + s*ssm(norm(x)), then x + s*mlp(norm(x))
    (mamba3/block.py:29-107)."""

    def __init__(
        self,
        d_model: int,
        d_state: int = 128,
        expand: int = 2,
        headdim: int = 64,
        ngroups: int | None = None,
        mimo_rank: int = 2,
        chunk_size: int = 64,
        use_mlp: bool = True,
        mlp_expand: float = 2.667,
        norm_eps: float = 1e-5,
        bias: bool = False,
        residual_scale: float = 1.0,
        gradient_checkpointing: bool = False,
        use_trapezoidal: bool = True,
        use_complex_ssm: bool = True,
    ):
        super().__init__()
        self.residual_scale = residual_scale
        self.gradient_checkpointing = gradient_checkpointing
        self.ssm_norm = RMSNorm(d_model, eps=norm_eps)
        self.ssm = KulaMamba(
            d_model=d_model, d_state=d_state, expand=expand, headdim=headdim,
            ngroups=ngroups, mimo_rank=mimo_rank, chunk_size=chunk_size, bias=bias,
            use_trapezoidal=use_trapezoidal, use_complex_ssm=use_complex_ssm,
        )
        self.use_mlp = use_mlp
        if use_mlp:
            d_ff = int(d_model * mlp_expand / 64 + 1) * 64
            self.mlp_norm = RMSNorm(d_model, eps=norm_eps)
            self.mlp = SwiGLU(d_model, d_ff, bias=bias)

    def _ssm_forward(self, x_normed):
        return self.ssm(x_normed)

    def _mlp_forward(self, x_normed):
        return self.mlp(x_normed)

    # The residual adds run as the beta = 1 input of the out_proj / w_down GEMMs
    # (add_scaled_linear); with gradient checkpointing the branches are recomputed whole.
    def forward(self, x: torch.Tensor, _own_input: bool = False) -> torch.Tensor:
        """_own_input (internal): x is an intermediate of the caller's forward
        (KulaMambaLM), so without autograd the first residual add may overwrite it. The
        second add overwrites the first one's output whenever no autograd graph needs it."""
        ckpt = self.gradient_checkpointing and self.training
        nograd = not torch.is_grad_enabled()
        if ckpt:
            h = grad_checkpoint(self._ssm_forward, self.ssm_norm(x), use_reentrant=False)
            x = x + h * self.residual_scale
        else:
            y, _ = self.ssm._pre_out(self.ssm_norm(x))
            x = add_scaled_linear(x, self.ssm.out_proj, y, self.residual_scale,
                                  inplace=_own_input and nograd)
        if self.use_mlp:
            if ckpt:
                m = grad_checkpoint(self._mlp_forward, self.mlp_norm(x), use_reentrant=False)
                x = x + m * self.residual_scale
            else:
                x = self._mlp_residual(x, inplace=nograd)
        return x

    def _mlp_residual(self, x: torch.Tensor, inplace: bool = False) -> torch.Tensor:
        return add_scaled_linear(x, self.mlp.w_down, self.mlp.hidden(self.mlp_norm(x)),
                                 self.residual_scale, inplace=inplace)

    def _small_step_usable(self, x: torch.Tensor) -> bool:
        """The decode step runs on the small-batch projection kernels (norm + in_proj,
        out_proj + residual, norm + SwiGLU, w_down + residual): bf16, at most 8 rows, no
        biases, last-dimension norms, nothing to differentiate."""
        ssm = self.ssm
        ws = [self.ssm_norm.weight, ssm.in_proj.weight, ssm.out_proj.weight]
        lins = [ssm.in_proj, ssm.out_proj]
        if self.use_mlp:
            ws += [self.mlp_norm.weight, self.mlp.w_gate.weight, self.mlp.w_up.weight,
                   self.mlp.w_down.weight]
            lins += [self.mlp.w_gate, self.mlp.w_up, self.mlp.w_down]
        norms = [self.ssm_norm] + ([self.mlp_norm] if self.use_mlp else [])
        m = x.shape[0]
        # every projection's K: d_model (with a norm), d_inner, d_ff
        ks_ok = _native.small_proj_ok(m, ssm.out_proj.in_features) and (
            not self.use_mlp or _native.small_proj_ok(m, self.mlp.w_down.in_features))
        return (ks_ok and all(l.bias is None for l in lins) and all(n.dim in (-1, 1) for n in norms)
                and ops.small_proj_usable(x, *ws, norm=True))

    def _small_step_tail(self, x: torch.Tensor, y: torch.Tensor) -> torch.Tensor:
        """x + s out_proj(y), then the MLP residual, on the small-batch kernels."""
        s = self.residual_scale
        x = ops.small_linear_fast(y, None, 0.0, self.ssm.out_proj.weight, x, s)
        if self.use_mlp:
            mlp = self.mlp
            h = ops.small_swiglu_fast(x, self.mlp_norm.weight, float(self.mlp_norm.eps),
                                 mlp.w_gate.weight, mlp.w_up.weight)
            x = ops.small_linear_fast(h, None, 0.0, mlp.w_down.weight, x, s)
        return x

    def step(self, x: torch.Tensor, ssm_state: dict):
        if self._small_step_usable(x):
            proj = ops.small_linear_fast(x, self.ssm_norm.weight, float(self.ssm_norm.eps),
                                    self.ssm.in_proj.weight, None, 1.0)
            y, new_state = self.ssm._step_from_proj(proj, ssm_state)
            return self._small_step_tail(x, y), new_state
        y, new_state = self.ssm._step_pre_out(self.ssm_norm(x), ssm_state)
        x = add_scaled_linear(x, self.ssm.out_proj, y.view(*x.shape[:-1], -1), self.residual_scale)
        if self.use_mlp:
            x = self._mlp_residual(x, inplace=not torch.is_grad_enabled())
        return x, new_state

    def prefill(self, x: torch.Tensor, _own_input: bool = False):
        """_own_input as in forward."""
        nograd = not torch.is_grad_enabled()
        y, state = self.ssm._pre_out(self.ssm_norm(x), return_state=True)
        x = add_scaled_linear(x, self.ssm.out_proj, y, self.residual_scale,
                              inplace=_own_input and nograd)
        if self.use_mlp:
            x = self._mlp_residual(x, inplace=nograd)
        return x, state


class KulaMambaLM(nn.Module):
    """Embedding -> n_layers KulaMambaBlock -> RMSNorm -> (tied) lm_head
    (mamba3/block.py:110-231)."""

    def __init__(
        self,
        vocab_size: int,
        d_model: int = 768,
        n_layers: int = 12,
        d_state: int = 128,
        expand: int = 2,
        headdim: int = 64,
        ngroups: int | None = None,
        mimo_rank: int = 2,
        chunk_size: int = 64,
        use_mlp: bool = True,
        tie_weights: bool = True,
        norm_eps: float = 1e-5,
        bias: bool = False,
        residual_scale: str = "depth",
        gradient_checkpointing: bool = False,
        use_trapezoidal: bool = True,
        use_complex_ssm: bool = True,
    ):
        super().__init__()
        self.d_model = d_model
        self.n_layers = n_layers
        scale = 1.0 / math.sqrt(2 * n_layers) if residual_scale == "depth" else 1.0
        self.embedding = nn.Embedding(vocab_size, d_model)
        self.layers = nn.ModuleList([
            KulaMambaBlock(
                d_model=d_model, d_state=d_state, expand=expand, headdim=headdim,
                ngroups=ngroups, mimo_rank=mimo_rank, chunk_size=chunk_size, use_mlp=use_mlp,
                norm_eps=norm_eps, bias=bias, residual_scale=scale,
                gradient_checkpointing=gradient_checkpointing,
                use_trapezoidal=use_trapezoidal, use_complex_ssm=use_complex_ssm,
            )
            for _ in range(n_layers)
        ])
        self.norm = RMSNorm(d_model, eps=norm_eps)
        self.lm_head = nn.Linear(d_model, vocab_size, bias=False)
        if tie_weights:
            self.lm_head.weight = self.embedding.weight
        self._init_weights()

    def _init_weights(self) -> None:
        """N(0, 0.02) for the embedding and every Linear except the (tied) head, then the
        KulaMamba-specific re-initialisation (mamba3/block.py:166-176)."""
        nn.init.normal_(self.embedding.weight, std=0.02)
        for m in self.modules():
            if isinstance(m, nn.Linear) and m is not self.lm_head:
                nn.init.normal_(m.weight, std=0.02)
                if m.bias is not None:
                    nn.init.zeros_(m.bias)
        for m in self.modules():
            if isinstance(m, KulaMamba):
                m._init_weights(dt_min=0.001, dt_max=0.1)

    def forward(self, input_ids: torch.Tensor, labels: torch.Tensor | None = None) -> dict:
        x = self.embedding(input_ids)
        for layer in self.layers:
            x = layer(x, _own_input=True)
        logits = self.lm_head(self.norm(x))
        result = {"logits": logits}
        if labels is not None:
            pred = logits[:, :-1].contiguous()
            tgt = labels[:, 1:].contiguous()
            result["loss"] = F.cross_entropy(pred.view(-1, pred.size(-1)), tgt.view(-1))
        return result

    # Replay the per-token decode step (embedding, every block's step, norm, lm_head) as one
    # captured HIP graph instead of launching each op from Python. Sampling stays eager.
    decode_graph: bool = True

    @torch.no_grad()
    def generate(self, input_ids: torch.Tensor, max_new_tokens: int = 100,
                 temperature: float = 1.0, top_k: int | None = None) -> torch.Tensor:
        """Parallel prefill of the prompt, then one `step` per new token
        (mamba3/block.py:195-231). temperature=0 is greedy argmax."""
        x = self.embedding(input_ids)
        states = []
        for layer in self.layers:
            x, st = layer.prefill(x, _own_input=True)
            states.append(st)
        logits = self.lm_head(self.norm(x)[:, -1])
        out = [input_ids]
        graph = None
        if self.decode_graph and max_new_tokens > 1 and input_ids.is_cuda:
            graph = _DecodeGraph(self, states, input_ids.shape[0])
        for _ in range(max_new_tokens):
            scores = logits / temperature if temperature > 0 else logits
            if top_k is not None:
                kth = torch.topk(scores, min(top_k, scores.size(-1))).values[:, -1:]
                scores = scores.masked_fill(scores < kth, float("-inf"))
            if temperature > 0:
                nxt = torch.multinomial(F.softmax(scores, dim=-1), num_samples=1)
            else:
                nxt = scores.argmax(dim=-1, keepdim=True)
            out.append(nxt)
            if graph is not None:
                logits = graph(nxt.squeeze(1))
                continue
            x = self.embedding(nxt.squeeze(1))
            for i, layer in enumerate(self.layers):
                x, states[i] = layer.step(x, states[i])
            logits = _lm_logits(self, x)
        return torch.cat(out, dim=1)


def _block_step_into(block: KulaMambaBlock, x: torch.Tensor, st_in: dict, st_out: dict):
    """KulaMambaBlock.step (mamba3/block.py:94-100) with the SSM step written into the
    caller's state buffers `st_out` (which must not alias `st_in`)."""
    ssm = block.ssm
    small = block._small_step_usable(x)
    if small:
        proj = ops.small_linear_fast(x, block.ssm_norm.weight, float(block.ssm_norm.eps),
                                ssm.in_proj.weight, None, 1.0)
    else:
        proj = ssm.in_proj(block.ssm_norm(x))
    y = torch.empty(x.shape[0], ssm.d_inner, device=x.device, dtype=proj.dtype)
    ops.step_into(proj, *ssm._small_params(), None, st_in["h"], st_in["prev_BX"],
                  st_in["angle"], y, st_out["h"], st_out["prev_BX"], st_out["angle"],
                  *ops.layer_args(ssm))
    if small:
        return block._small_step_tail(x, y)
    x = add_scaled_linear(x, ssm.out_proj, y, block.residual_scale)
    if block.use_mlp:
        x = block._mlp_residual(x)
    return x


def _lm_logits(lm: "KulaMambaLM", x: torch.Tensor) -> torch.Tensor:
    """lm_head(norm(x)) for decode rows x (B, d_model): one small-batch kernel (norm in its
    prologue) when it applies (mamba3/block.py:182-183)."""
    w = lm.lm_head.weight
    if (lm.lm_head.bias is None and lm.norm.dim in (-1, 1)
            and ops.small_proj_usable(x, lm.norm.weight, w, norm=True)):
        return ops.small_linear_fast(x, lm.norm.weight, float(lm.norm.eps), w, None, 1.0)
    return lm.lm_head(lm.norm(x))


class _DecodeGraph:
    """One decode step of a KulaMambaLM captured as HIP graphs (torch.cuda.CUDAGraph):
    token ids -> embedding -> every block's step -> norm -> lm_head logits. The decode
    state lives in two static buffer sets; graph 0 reads set 0 and writes set 1, graph 1
    the reverse, and replays alternate between them, so no state is copied. Outputs are
    bitwise those of the eager step (same kernels, same order)."""

    def __init__(self, lm: KulaMambaLM, states: list, batch: int):
        dev = lm.embedding.weight.device
        self.tok = torch.zeros(batch, dtype=torch.long, device=dev)
        self.bufs = [[{k: v.clone() for k, v in st.items()} for st in states],
                     [{k: torch.empty_like(v) for k, v in st.items()} for st in states]]

        def step(src: int):
            x = lm.embedding(self.tok)
            for i, block in enumerate(lm.layers):
                x = _block_step_into(block, x, self.bufs[src][i], self.bufs[1 - src][i])
            return _lm_logits(lm, x)

        # Warm up outside the capture on a side stream (allocator and library handles);
        # it reads set 0 and writes set 1, which the first replay rewrites.
        side = torch.cuda.Stream(device=dev)
        side.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(side):
            step(0)
        torch.cuda.current_stream(dev).wait_stream(side)
        self.graphs, self.logits = [], []
        for src in (0, 1):
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                self.logits.append(step(src))
            self.graphs.append(g)
        torch.cuda.synchronize(dev)
        self.phase = 0

    def __call__(self, tok: torch.Tensor) -> torch.Tensor:
        self.tok.copy_(tok)
        self.graphs[self.phase].replay()
        out = self.logits[self.phase]
        self.phase ^= 1
        return out
