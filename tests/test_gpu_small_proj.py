"""GPU parity of the small-batch decode projections (m3_small_linear, m3_small_swiglu): the
block step's norm + in_proj, out_proj + residual, norm + SwiGLU and w_down + residual, and
the LM's norm + lm_head (mamba3/block.py:16-26, 94-100, 182-183; mamba3/mamba3.py:19-35).

Reference: the oracle's RMSNorm in bf16 (the reference's roundings) on the same bf16 inputs,
then the products and the residual in fp32 on the host. The kernels accumulate in fp32 and
round once to bf16, so the bound is a few bf16 ulps of the largest output (8e-3 normwise)."""

from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

import mamba3_amd
from conftest import max_rel
from mamba3_amd import _native, ops
from oracle import reference_path as ref

pytestmark = pytest.mark.gpu

TOL = 8e-3
BF16_TOL = 2e-2


@pytest.fixture(scope="module", autouse=True)
def _native_loaded(cuda_device):
    _native.lib()


def _inputs(m, n, k, seed):
    g = torch.Generator().manual_seed(seed)
    x = (torch.randn(m, k, generator=g) * 1.5).to(torch.bfloat16)
    w = (torch.randn(n, k, generator=g) * k ** -0.5).to(torch.bfloat16)
    nw = (torch.rand(k, generator=g) + 0.5).to(torch.bfloat16)
    res = torch.randn(m, n, generator=g).to(torch.bfloat16)
    return x, w, nw, res


# (n, k): a block of one row, the d768 layer's in_proj (3696 x 768), out_proj (768 x 1536),
# w_down (768 x 2112, 33 steps of 64: a partial last group), w_gate (2112 x 768).
SHAPES = [(17, 64), (3696, 768), (768, 1536), (768, 2112), (2112, 768)]


@pytest.mark.parametrize("m", [1, 3, 4, 8])
@pytest.mark.parametrize("n,k", SHAPES)
@pytest.mark.parametrize("norm,residual", [(False, False), (True, False), (False, True)])
def test_small_linear_matches_host_reference(m, n, k, norm, residual, cuda_device):
    x, w, nw, res = _inputs(m, n, k, seed=m * 1000 + n + k)
    xn = ref.rmsnorm(x, nw, 1e-5) if norm else x
    want = xn.float() @ w.float().t()
    if residual:
        want = res.float() + 0.37 * want
    d = lambda t: t.to(cuda_device)
    with torch.no_grad():
        got = ops.small_linear(d(x), d(nw) if norm else None, 1e-5, d(w),
                               d(res) if residual else None, 0.37)
    assert got.dtype == torch.bfloat16 and got.shape == (m, n)
    assert max_rel(got, want) < TOL


@pytest.mark.parametrize("m", [1, 4, 8])
@pytest.mark.parametrize("n,k", [(2112, 768), (40, 128)])
def test_small_swiglu_matches_host_reference(m, n, k, cuda_device):
    x, wg, nw, _ = _inputs(m, n, k, seed=7 + m)
    g = torch.Generator().manual_seed(8 + m)
    wu = (torch.randn(n, k, generator=g) * k ** -0.5).to(torch.bfloat16)
    xn = ref.rmsnorm(x, nw, 1e-5).float()
    want = F.silu(xn @ wg.float().t()) * (xn @ wu.float().t())
    d = lambda t: t.to(cuda_device)
    with torch.no_grad():
        got = ops.small_swiglu(d(x), d(nw), 1e-5, d(wg), d(wu))
        plain = ops.small_swiglu(d(x), None, 0.0, d(wg), d(wu))
    assert max_rel(got, want) < TOL
    want_plain = F.silu(x.float() @ wg.float().t()) * (x.float() @ wu.float().t())
    assert max_rel(plain, want_plain) < TOL


def test_small_linear_residual_in_place(cuda_device):
    """out may alias the residual: each element is read and written by one thread."""
    x, w, _, res = _inputs(4, 768, 1536, seed=3)
    xd, wd = x.to(cuda_device), w.to(cuda_device)
    fresh = torch.empty(4, 768, device=cuda_device, dtype=torch.bfloat16)
    acc = res.to(cuda_device).clone()
    with torch.no_grad():
        _native.small_linear(xd, None, 0.0, wd, res.to(cuda_device), 0.5, fresh)
        _native.small_linear(xd, None, 0.0, wd, acc, 0.5, acc)
    assert torch.equal(fresh, acc)


def test_block_step_on_small_kernels_matches_unfused_step(cuda_device):
    """A bf16 d_model-768 block's decode step at batch 4 on the small-batch kernels against
    the same step on the library GEMMs and the standalone norm kernel (2e-2: the two differ
    in where bf16 rounding happens), then against the fp32 oracle's block_step on the
    bf16-rounded weights."""
    torch.manual_seed(0)
    block = mamba3_amd.KulaMambaBlock(768, d_state=128, headdim=64, mimo_rank=2,
                                      residual_scale=0.2).to(cuda_device, torch.bfloat16).eval()
    p = {k: v.detach().float().cpu() for k, v in block.state_dict().items()}
    cfg = ref.LayerCfg(d_model=768, d_state=128, headdim=64, mimo_rank=2)
    g = torch.Generator().manual_seed(4)
    x0 = torch.randn(4, 64, 768, generator=g).to(torch.bfloat16)
    tok = torch.randn(4, 768, generator=g).to(torch.bfloat16).to(cuda_device)
    with torch.no_grad():
        _, st = block.prefill(x0.to(cuda_device))
        assert block._small_step_usable(tok)
        y_small, st_small = block.step(tok, st)
        block._small_step_usable = lambda x: False
        y_lib, st_lib = block.step(tok, st)
        del block._small_step_usable
    assert max_rel(y_small, y_lib) < BF16_TOL
    for k in ("h", "prev_BX", "angle"):
        assert max_rel(st_small[k], st_lib[k]) < BF16_TOL, k
    st_ref = {k: v.float().cpu() for k, v in st.items()}
    y_ref, _ = ref.block_step(cfg, p, "", tok.float().cpu(), st_ref, 0.2, True)
    assert max_rel(y_small, y_ref) < BF16_TOL


def test_lm_logits_on_small_kernel(cuda_device):
    """The LM's final norm + tied lm_head (32000 x 768) for decode rows in one kernel."""
    from mamba3_amd.block import _lm_logits
    torch.manual_seed(0)
    lm = mamba3_amd.KulaMambaLM(32000, 768, n_layers=1, d_state=128, headdim=64,
                                mimo_rank=2).to(cuda_device, torch.bfloat16).eval()
    g = torch.Generator().manual_seed(9)
    x = torch.randn(4, 768, generator=g).to(torch.bfloat16)
    with torch.no_grad():
        got = _lm_logits(lm, x.to(cuda_device))
    want = ref.rmsnorm(x, lm.norm.weight.detach().cpu(), 1e-5).float() @ lm.lm_head.weight.detach().float().cpu().t()
    assert got.shape == (4, 32000)
    assert max_rel(got, want) < TOL


@pytest.mark.parametrize("rows,d_ff,stride", [(8192, 2112, 4352), (7, 100, 256), (33, 64, 128)])
def test_silu_mul_matches_host_reference(rows, d_ff, stride, cuda_device):
    """m3_silu_mul on a concatenated gate / up projection: 16-byte pieces (d_ff and the row
    stride multiples of 8) and the element path (d_ff = 100)."""
    g = torch.Generator().manual_seed(rows + d_ff)
    gu = (torch.randn(rows, stride, generator=g) * 2).to(torch.bfloat16)
    want = F.silu(gu[:, :d_ff].float()) * gu[:, d_ff:2 * d_ff].float()
    with torch.no_grad():
        got = ops.silu_mul(gu.to(cuda_device), d_ff)
    assert got.shape == (rows, d_ff) and got.dtype == torch.bfloat16
    assert max_rel(got, want) < TOL


def test_swiglu_hidden_one_gemm_matches_two(cuda_device):
    """SwiGLU.hidden in bf16 without autograd (one GEMM over [w_gate; w_up], padded to whole
    256-column tiles, then m3_silu_mul) against the two-GEMM form with autograd on."""
    from mamba3_amd.block import SwiGLU
    torch.manual_seed(0)
    mlp = SwiGLU(768, 2112).to(cuda_device, torch.bfloat16)
    x = torch.randn(3, 100, 768, device=cuda_device).to(torch.bfloat16)
    with torch.no_grad():
        fused = mlp.hidden(x)
        assert mlp.__dict__["_gate_up"][1].shape == (4352, 768)
    two = mlp.hidden(x)  # autograd on: the two-GEMM form
    assert fused.shape == two.shape == (3, 100, 2112)
    assert max_rel(fused, two.detach()) < BF16_TOL


def test_d2048_block_step_on_small_kernels_matches_unfused_step(cuda_device):
    """The d_model-2048 block (d_state 256, headdim 128, rank 4; in_proj K 2048 with its
    norm, out_proj K 4096, w_down K 5504) at batch 4 on the small-batch kernels against the
    library path."""
    torch.manual_seed(0)
    block = mamba3_amd.KulaMambaBlock(2048, d_state=256, headdim=128, mimo_rank=4,
                                      residual_scale=0.125).to(cuda_device, torch.bfloat16).eval()
    g = torch.Generator().manual_seed(5)
    x0 = torch.randn(4, 32, 2048, generator=g).to(torch.bfloat16).to(cuda_device)
    tok = torch.randn(4, 2048, generator=g).to(torch.bfloat16).to(cuda_device)
    with torch.no_grad():
        _, st = block.prefill(x0)
        assert block._small_step_usable(tok)
        y_small, st_small = block.step(tok, st)
        block._small_step_usable = lambda x: False
        y_lib, st_lib = block.step(tok, st)
        del block._small_step_usable
        # 8 rows: w_down's 5504-wide rows no longer fit the staged LDS, so the library runs
        assert not block._small_step_usable(torch.cat([tok, tok]))
    assert max_rel(y_small, y_lib) < BF16_TOL
    for k in ("h", "prev_BX", "angle"):
        assert max_rel(st_small[k], st_lib[k]) < BF16_TOL, k
