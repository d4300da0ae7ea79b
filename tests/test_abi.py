"""The C-ABI library: loads, exports every symbol include/mamba3_amd.h declares, and
rejects bad arguments on the host before any launch (no GPU needed for these paths)."""

from __future__ import annotations

import ctypes
import re

import pytest

from conftest import ROOT
from mamba3_amd import _native

HEADER = ROOT / "include" / "mamba3_amd.h"


@pytest.fixture(scope="module")
def lib():
    if not _native.LIB_PATH.exists():
        from mamba3_amd import build
        build.build(verbose=False)
    return _native.lib()


def declared_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(m3_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_binding_list():
    assert declared_functions() == sorted(_native.EXPORTED_SYMBOLS)


def test_library_exports_every_declared_symbol(lib):
    for name in declared_functions():
        assert hasattr(lib, name), name


def test_status_strings(lib):
    assert lib.m3_status_string(0) == b"ok"
    for code in range(1, 8):
        assert lib.m3_status_string(code) != b"unknown status"
    assert lib.m3_status_string(99) == b"unknown status"
    # 0.2.0: m3_layer_param_grads has its dt_scale field, m3_prefill_kernel_name exists
    assert lib.m3_version() == 200


def test_scan_rejects_bad_arguments(lib):
    assert lib.m3_scan_fwd(None, None, None, None, 1, 1, 1, 1, None) == 1
    fake = 256  # never dereferenced: validation fails before any launch
    assert lib.m3_scan_fwd(fake, fake, None, fake, 0, 1, 1, 1, None) == 2
    assert lib.m3_scan_fwd(fake, fake, None, fake, 1, -1, 1, 1, None) == 2
    n = ctypes.c_size_t(7)
    assert lib.m3_scan_bwd_workspace_size(2, 16, 24, 8192, ctypes.byref(n)) == 0
    assert n.value == 2 * 16 * 24 * (8192 // 256) * 4  # one partial per wave and chunk
    assert lib.m3_scan_bwd_workspace_size(2, 16, 24, 100, ctypes.byref(n)) == 0 and n.value == 0
    # any PN: beyond 16384 and not a multiple of 256 the per-(b,h) kernel tiles the columns
    assert lib.m3_scan_bwd_workspace_size(2, 16, 24, 20000, ctypes.byref(n)) == 0 and n.value == 0
    assert lib.m3_scan_bwd(None, fake, fake, fake, fake, None, None, 0, 1, 2, 1, 256, None) == 1
    assert lib.m3_scan_bwd(fake, fake, fake, fake, fake, None, None, 0, 1, 0, 1, 256, None) == 2
    # the per-wave partials need a workspace
    assert lib.m3_scan_bwd(fake, fake, fake, fake, fake, None, None, 0, 1, 2, 1, 256, None) == 4


def test_chunked_bwd_workspace_and_validation(lib):
    n = ctypes.c_size_t(0)
    # d_model 768 shapes: B=4, T=1024, H=24, P=64, N=128, R=2 with beta terms -> chunks of 32
    assert lib.m3_chunked_ssd_bwd_workspace_size(4, 1024, 24, 64, 128, 2, 1, ctypes.byref(n)) == 0
    K = 1024 // 32
    states = 4 * (K + 1) * 24 * 64 * 128 * 4
    scores = 4 * K * 24 * 64 * 128 * 4
    # chunk-local, scanned and adjoint states (the reverse scan runs in place); with the beta
    # terms the masked scores stay in LDS (one fused kernel per chunk)
    assert 3 * states <= n.value < 3 * states + scores
    assert lib.m3_chunked_ssd_bwd_workspace_size(4, 1024, 24, 64, 128, 2, 0, ctypes.byref(n)) == 0
    K0 = 1024 // 64  # without the beta terms: chunks of 64 tokens, 128 x 128 score tiles in scratch
    states0 = 4 * (K0 + 1) * 24 * 64 * 128 * 4
    assert n.value >= 3 * states0 + 2 * 4 * K0 * 24 * 128 * 128 * 4
    # rank 3 on rank-4 tiles; rank 9 is beyond every kernel
    assert lib.m3_chunked_ssd_bwd_workspace_size(4, 1024, 24, 64, 128, 3, 1, ctypes.byref(n)) == 0
    assert n.value > 0
    assert lib.m3_chunked_ssd_bwd_workspace_size(4, 1024, 24, 64, 128, 9, 1, ctypes.byref(n)) == 3
    assert lib.m3_chunked_ssd_bwd_workspace_size(4, 1024, 24, 64, 128, 2, 2, ctypes.byref(n)) == 2
    assert lib.m3_chunked_ssd_bwd_workspace_size(0, 1024, 24, 64, 128, 2, 1, ctypes.byref(n)) == 2
    assert lib.m3_chunked_ssd_bwd_workspace_size(1, 8, 1, 8, 128, 2, 1, None) == 1
    fake = ctypes.c_void_p(256)
    ins = [fake] * 10  # x_g x_b B_g B_b C dt A D x_raw h_init
    outs = [fake] * 10  # dx_g dx_b dB_g dB_b dC ddt dA dD dx_raw dh_init
    args = lambda i, o: [1, 8, 1, 16, 16, 2, *i, fake, None, *o]
    # missing dy
    a = args(ins, outs)
    a[6 + 10] = None
    assert lib.m3_chunked_ssd_bwd(*a, fake, 1 << 30, None) == 1
    # x_b given but dx_b missing
    o = list(outs)
    o[1] = None
    assert lib.m3_chunked_ssd_bwd(*args(ins, o), fake, 1 << 30, None) == 1
    # rank 9 is beyond every kernel
    a = args(ins, outs)
    a[5] = 9
    assert lib.m3_chunked_ssd_bwd(*a, fake, 1 << 30, None) == 3
    # no workspace
    assert lib.m3_chunked_ssd_bwd(*args(ins, outs), None, 0, None) == 4


def _desc(**kw):
    d = dict(batch=1, seqlen=4, nheads=8, headdim=16, d_state=16, mimo_rank=2, ngroups=1,
             use_trapezoidal=1, use_complex=1, dtype=0, proj_row_stride=0, rms_eps=1e-5)
    d.update(kw)
    if d["proj_row_stride"] == 0:
        H, P, N, R, G = d["nheads"], d["headdim"], d["d_state"], d["mimo_rank"], d["ngroups"]
        d["proj_row_stride"] = (2 * H * P + 2 * G * N * R + H + d["use_trapezoidal"] * H
                                + d["use_complex"] * (N // 2))
    return _native.LayerDesc(**d)


def test_workspace_query_and_desc_validation(lib):
    n = ctypes.c_size_t(0)
    # fp32 layers run on the fp32-MFMA chunk kernels: chunked_ssd's inputs and the chunk
    # workspace (B=1, T=4, H=8, P=16, N=16, R=2 with beta terms: chunks of 32 tokens)
    assert lib.m3_prefill_workspace_size(ctypes.byref(_desc()), ctypes.byref(n)) == 0
    assert n.value >= 4 * 8 * (3 * 16 * 2 + 3 * 16 * 2 + 16 * 2) * 4
    # rank 3 runs there too, on the chunk kernels' rank-4 tiles
    assert lib.m3_prefill_workspace_size(ctypes.byref(_desc(mimo_rank=3)), ctypes.byref(n)) == 0
    assert n.value > 0
    # wide layers run there too: the per-token preparation holds the sin / cos of a tile of
    # heads at a time (64 heads x d_state 256 needed 64 KB of them at once)
    assert lib.m3_prefill_workspace_size(ctypes.byref(_desc(nheads=64, d_state=256)),
                                         ctypes.byref(n)) == 0
    assert n.value > 0
    # and so do many groups: the preparation normalises one group at a time (32 groups x
    # d_state 256 x rank 2 needed 128 KB of LDS at once)
    assert lib.m3_prefill_workspace_size(ctypes.byref(_desc(nheads=32, ngroups=32, d_state=256)),
                                         ctypes.byref(n)) == 0
    assert n.value > 0
    # bf16 d_state 128 / headdim 64 / rank 2: normalised B^ and C^ in f16, per token
    d768 = _desc(dtype=1, seqlen=64, nheads=24, headdim=64, d_state=128)
    assert lib.m3_prefill_workspace_size(ctypes.byref(d768), ctypes.byref(n)) == 0
    assert n.value >= 2 * 64 * 128 * 2 * 2
    bad = [dict(batch=0), dict(d_state=15), dict(nheads=8, ngroups=3), dict(dtype=7),
           dict(proj_row_stride=10), dict(use_complex=2), dict(rms_eps=float("nan"))]
    for kw in bad:
        st = lib.m3_prefill_workspace_size(ctypes.byref(_desc(**kw)), ctypes.byref(n))
        assert st in (2, 3), (kw, st)
    assert lib.m3_prefill_workspace_size(None, ctypes.byref(n)) == 1


def test_prefill_and_step_reject_missing_pointers(lib):
    params = _native.LayerParams()
    d = _desc()
    assert lib.m3_prefill_fwd(ctypes.byref(d), ctypes.byref(params), 256, None, 256, None,
                              None, None, None, 0, None) == 1
    full = _native.LayerParams(*([256] * 10))
    # a bf16 MFMA-path layer without its workspace
    d768 = _desc(dtype=1, seqlen=64, nheads=24, headdim=64, d_state=128)
    assert lib.m3_prefill_fwd(ctypes.byref(d768), ctypes.byref(full), 256, None, 256, None,
                              None, None, None, 0, None) == 4
    assert lib.m3_step_fwd(ctypes.byref(d), ctypes.byref(full), 256, None, None, 256, 256, 0,
                           256, 256, 256, 256, None) == 1
    # d_state beyond the kernels' 512 is refused on the host, before any launch (every
    # even d_state up to 512 is supported)
    d600 = _desc(d_state=600)
    assert lib.m3_step_fwd(ctypes.byref(d600), ctypes.byref(full), 256, None, 256, 512, 256, 0,
                           256, 768, 1024, 256, None) == 3
    # aliasing in/out state is refused
    assert lib.m3_step_fwd(ctypes.byref(d), ctypes.byref(full), 256, None, 256, 512, 256, 0,
                           256, 256, 1024, 256, None) == 2


def test_chunked_rejects_bad_arguments(lib):
    assert lib.m3_chunked_ssd_fwd(1, 4, 2, 4, 8, 2, 0, 256, 256, 256, None, 256, 256, 256, 256,
                                  256, None, 256, 256, None, None, 0, None) == 1
    assert lib.m3_chunked_ssd_fwd(1, 0, 2, 4, 8, 2, 0, 256, None, 256, None, 256, 256, 256, 256,
                                  256, None, 256, 256, None, None, 0, None) == 2
    assert lib.m3_chunked_ssd_fwd(1, 4, 2, 4, 8, 2, 5, 256, None, 256, None, 256, 256, 256, 256,
                                  256, None, 256, 256, None, None, 0, None) == 3
    # the generic path needs h_final or state_ws when no (or too small a) workspace is given
    assert lib.m3_chunked_ssd_fwd(1, 4, 2, 4, 8, 2, 0, 256, None, 256, None, 256, 256, 256, 256,
                                  256, None, 256, None, None, None, 0, None) == 4
    # a misaligned workspace for the fp32-MFMA path
    assert lib.m3_chunked_ssd_fwd(1, 4, 2, 4, 8, 2, 0, 256, None, 256, None, 256, 256, 256, 256,
                                  256, None, 256, 256, None, 260, 1 << 30, None) == 5


def test_layer_bwd_workspace_and_validation(lib):
    n = ctypes.c_size_t(0)
    d32 = _desc(seqlen=64)
    assert lib.m3_layer_bwd_workspace_size(ctypes.byref(d32), ctypes.byref(n)) == 0 and n.value > 0
    # every rank up to 8 is covered (3, 5, 6 and 7 on the chunk kernels' rank-4 / rank-8 tiles)
    for r in (3, 5, 6, 7):
        assert lib.m3_layer_bwd_workspace_size(ctypes.byref(_desc(seqlen=64, mimo_rank=r)),
                                               ctypes.byref(n)) == 0 and n.value > 0
    # so is every d_state / group count: the B/C kernel works one group at a time, in up to
    # 160 KB of LDS (d_state 512, rank 8: 132 KB)
    for kw in (dict(d_state=256, mimo_rank=8), dict(d_state=512, mimo_rank=8),
               dict(nheads=32, ngroups=32, d_state=256)):
        assert lib.m3_layer_bwd_workspace_size(ctypes.byref(_desc(seqlen=64, **kw)),
                                               ctypes.byref(n)) == 0 and n.value > 0, kw
    # bf16 layers are not covered (the autograd path runs bf16 layers in fp32), nor ranks
    # beyond 8
    assert lib.m3_layer_bwd_workspace_size(ctypes.byref(_desc(dtype=1)), ctypes.byref(n)) == 3
    assert lib.m3_layer_bwd_workspace_size(ctypes.byref(_desc(mimo_rank=9)), ctypes.byref(n)) == 3
    assert lib.m3_layer_bwd_workspace_size(ctypes.byref(_desc(batch=0)), ctypes.byref(n)) == 2
    fake = ctypes.c_void_p(256)
    params = _native.LayerParams(*([256] * 10))
    grads = _native.LayerParamGrads(*([256] * 10))
    args = lambda **kw: dict(dict(proj=fake, fws=fake, fbytes=1 << 40, gout=fake, gproj=fake,
                                  grads=ctypes.byref(grads), ws=fake, wbytes=1 << 40), **kw)
    def call(**kw):
        a = args(**kw)
        return lib.m3_layer_bwd(ctypes.byref(d32), ctypes.byref(params), a["proj"], None, a["fws"],
                                a["fbytes"], a["gout"], None, None, None, a["gproj"], a["grads"],
                                a["ws"], a["wbytes"], None)
    assert call(gout=None) == 1
    assert call(gproj=None) == 1
    bad = _native.LayerParamGrads(*([256] * 9 + [0]))
    assert call(grads=ctypes.byref(bad)) == 1
    assert call(fbytes=16) == 4   # the forward's workspace must be the whole fp32-layer one
    assert call(ws=None) == 4
    assert call(ws=ctypes.c_void_p(260)) == 5


def test_chunked_fwd_workspace_query(lib):
    n = ctypes.c_size_t(7)
    # fp32 d_model 768 shapes: c, decays, two (B, K+1, H, P*N) state arrays and W o G
    assert lib.m3_chunked_ssd_fwd_workspace_size(4, 1024, 24, 64, 128, 2, 0, 1, ctypes.byref(n)) == 0
    K = 1024 // 32
    assert n.value >= 2 * 4 * (K + 1) * 24 * 64 * 128 * 4 + 4 * K * 24 * 64 * 128 * 4
    # bf16 takes the generic kernel: no workspace
    assert lib.m3_chunked_ssd_fwd_workspace_size(4, 1024, 24, 64, 128, 2, 1, 1, ctypes.byref(n)) == 0
    assert n.value == 0
    # rank 3 with beta terms runs on rank-4 tiles: 16-token chunks, W o G of 64 x 128 per chunk
    assert lib.m3_chunked_ssd_fwd_workspace_size(4, 1024, 24, 64, 128, 3, 0, 1, ctypes.byref(n)) == 0
    K = 1024 // 16
    assert n.value >= 2 * 4 * (K + 1) * 24 * 64 * 128 * 4 + 4 * K * 24 * 64 * 128 * 4
    assert lib.m3_chunked_ssd_fwd_workspace_size(4, 1024, 24, 64, 128, 2, 0, 2, ctypes.byref(n)) == 2
    assert lib.m3_chunked_ssd_fwd_workspace_size(4, 1024, 24, 64, 128, 2, 7, 1, ctypes.byref(n)) == 3


def test_custom_op_fake_kernels_give_output_shapes():
    """The ops' fake kernels (used by torch.compile) on meta tensors, no GPU needed."""
    import torch
    import mamba3_amd  # noqa: F401  (registers the ops)
    from mamba3_amd import ops
    from torch._subclasses.fake_tensor import FakeTensorMode
    torch.manual_seed(0)
    layer = mamba3_amd.KulaMamba(d_model=64, d_state=16, headdim=16, mimo_rank=2)
    real = [p.detach() for p in layer._small_params()]
    proj_real = torch.empty(2, 9, layer.in_proj.out_features)
    with FakeTensorMode() as mode:
        proj = mode.from_tensor(proj_real)
        params = [mode.from_tensor(p) for p in real]
        y, h, a, pb = torch.ops.mamba3_amd.prefill(proj, *params, None, *ops.layer_args(layer), True)
        assert y.shape == (2, 9, layer.d_inner) and h.shape == (2, layer.nheads, 16, 16)
        assert a.shape == (2, layer.nheads, 8) and pb.shape == h.shape
        y, h, a, pb, ws = torch.ops.mamba3_amd.prefill_train(proj, *params, None,
                                                            *ops.layer_args(layer))
        assert ws.dtype == torch.uint8 and ws.numel() > 1
        st = torch.ops.mamba3_amd.step(proj[:, 0], *params, None, h, pb, a, *ops.layer_args(layer))
        assert st[0].shape == (2, layer.d_inner) and st[1].shape == h.shape
        out = torch.ops.mamba3_amd.scan_fwd(mode.from_tensor(torch.empty(2, 3, 4)),
                                            mode.from_tensor(torch.empty(2, 3, 4, 10)), None)
        assert out.shape == (2, 3, 4, 10)


def test_noalloc_prefill_refuses_workspace_beyond_scratch_before_any_launch():
    """m3_prefill_fwd_noalloc rejects a workload whose workspace exceeds the static scratch
    on the host, before touching the device (so this runs without a GPU); the pointers
    are never dereferenced."""
    lib = _native.lib()
    d = _desc(dtype=1, batch=8, seqlen=8192, nheads=24, headdim=64, d_state=128)
    n = ctypes.c_size_t(0)
    assert lib.m3_prefill_workspace_size(ctypes.byref(d), ctypes.byref(n)) == 0
    assert n.value > _native.NOALLOC_SCRATCH_BYTES
    fake = ctypes.c_void_p(1 << 20)
    params = _native.LayerParams(*([fake.value] * 10))
    st = lib.m3_prefill_fwd_noalloc(ctypes.byref(d), ctypes.byref(params), fake, None, fake,
                                    None, None, None, None)
    assert st == _native.M3_ERR_SCRATCH_LIMIT
    assert b"scratch" in lib.m3_status_string(st)


def test_rmsnorm_rejects_bad_arguments(lib):
    fake = 256  # never dereferenced: validation fails before any launch
    F32, BF16 = 0, 1
    assert lib.m3_rmsnorm_fwd(None, F32, fake, F32, fake, F32, None, 4, 8, 1e-5, None) == 1
    assert lib.m3_rmsnorm_fwd(fake, F32, fake, F32, fake, F32, None, 0, 8, 1e-5, None) == 2
    assert lib.m3_rmsnorm_fwd(fake, F32, fake, F32, fake, F32, None, 4, (1 << 24) + 1, 1e-5, None) == 2
    assert lib.m3_rmsnorm_fwd(fake, F32, fake, F32, fake, F32, None, 1 << 33, 8, 1e-5, None) == 2
    assert lib.m3_rmsnorm_fwd(fake, F32, fake, F32, fake, F32, None, 4, 8, -1.0, None) == 2
    assert lib.m3_rmsnorm_fwd(fake, F32, fake, F32, fake, F32, None, 4, 8, float("nan"), None) == 2
    # y must be the promotion of x's and the weight's dtypes
    assert lib.m3_rmsnorm_fwd(fake, BF16, fake, BF16, fake, F32, None, 4, 8, 1e-5, None) == 3
    assert lib.m3_rmsnorm_fwd(fake, BF16, fake, F32, fake, BF16, None, 4, 8, 1e-5, None) == 3
    assert lib.m3_rmsnorm_fwd(fake, 7, fake, F32, fake, F32, None, 4, 8, 1e-5, None) == 3
    n = ctypes.c_size_t(0)
    assert lib.m3_rmsnorm_bwd_workspace_size(1000, 768, ctypes.byref(n)) == 0
    assert n.value == 4 * 768 * 4  # one fp32 partial row per 256 rows
    assert lib.m3_rmsnorm_bwd_workspace_size(0, 768, ctypes.byref(n)) == 2
    args = [fake, F32, fake, F32, fake, fake, F32, fake, fake]
    assert lib.m3_rmsnorm_bwd(*args, None, 0, 1000, 768, None) == 4
    assert lib.m3_rmsnorm_bwd(*args, fake, 4 * 768 * 4 - 1, 1000, 768, None) == 4
    assert lib.m3_rmsnorm_bwd(*args, fake + 4, 4 * 768 * 4, 1000, 768, None) == 5
    assert lib.m3_rmsnorm_bwd(fake, F32, fake, F32, None, fake, F32, fake, fake, fake, 1 << 20,
                              1000, 768, None) == 1


def test_small_projections_reject_bad_arguments(lib):
    fake = 256  # 16-byte aligned, never dereferenced: validation fails before any launch
    args = lambda m, n, k: (m, n, k, None)
    assert lib.m3_small_linear(None, None, 0.0, fake, None, 1.0, fake, *args(4, 8, 64)) == 1
    assert lib.m3_small_linear(fake, None, 0.0, fake, None, 1.0, None, *args(4, 8, 64)) == 1
    assert lib.m3_small_linear(fake, None, 0.0, fake, None, 1.0, fake, *args(0, 8, 64)) == 2
    assert lib.m3_small_linear(fake, None, 0.0, fake, None, 1.0, fake, *args(9, 8, 64)) == 2
    assert lib.m3_small_linear(fake, None, 0.0, fake, None, 1.0, fake, *args(4, 0, 64)) == 2
    assert lib.m3_small_linear(fake, None, 0.0, fake, None, 1.0, fake, *args(4, 8, 96)) == 2
    # staged rows beyond 64 KB of LDS: 8 rows x 4160 bf16
    assert lib.m3_small_linear(fake, None, 0.0, fake, None, 1.0, fake, *args(8, 8, 4160)) == 3
    assert lib.m3_small_linear(fake + 8, None, 0.0, fake, None, 1.0, fake, *args(4, 8, 64)) == 5
    assert lib.m3_small_linear(fake, fake, -1.0, fake, None, 1.0, fake, *args(4, 8, 64)) == 2
    assert lib.m3_small_swiglu(fake, None, 0.0, fake, None, fake, *args(4, 8, 64)) == 1
    assert lib.m3_small_swiglu(fake, None, 0.0, fake, fake + 2, fake, *args(4, 8, 64)) == 5
    # (8 rows x k + one 8-element zero piece [+ the k-element norm weight]) x 2 bytes <= 65536
    assert _native.small_proj_ok(8, 4032) and not _native.small_proj_ok(8, 4096)
    assert _native.small_proj_ok(4, 8128) and not _native.small_proj_ok(9, 64)
    assert _native.small_proj_ok(8, 3584, norm=True) and not _native.small_proj_ok(8, 3648, norm=True)
    # the norm weight counts toward the limit on the C side too (8 x 3648 + 8 + 3648 > 32768)
    assert lib.m3_small_linear(fake, fake, 1e-5, fake, None, 1.0, fake, *args(8, 8, 3648)) == 3
    assert lib.m3_small_linear(fake, fake + 8, 1e-5, fake, None, 1.0, fake, *args(4, 8, 64)) == 5


def test_silu_mul_rejects_bad_arguments(lib):
    fake = 256
    assert lib.m3_silu_mul(None, 4, 8, 16, fake, None) == 1
    assert lib.m3_silu_mul(fake, 4, 8, 16, None, None) == 1
    assert lib.m3_silu_mul(fake, 0, 8, 16, fake, None) == 2
    assert lib.m3_silu_mul(fake, 4, 8, 15, fake, None) == 2  # the row must hold gate and up
    assert lib.m3_silu_mul(fake, 1 << 30, 1 << 10, 1 << 11, fake, None) == 2  # 32-bit grid


def test_ctypes_structs_match_the_header(tmp_path):
    """sizeof and every field offset of the ctypes mirrors of m3_layer_desc,
    m3_layer_params and m3_layer_param_grads equal the C header's, compiled with gcc."""
    import shutil
    import subprocess
    cc = shutil.which("gcc") or shutil.which("cc")
    if cc is None:
        pytest.skip("no C compiler")
    structs = {"m3_layer_desc": _native.LayerDesc, "m3_layer_params": _native.LayerParams,
               "m3_layer_param_grads": _native.LayerParamGrads}
    lines = ['#include <stdio.h>', '#include <stddef.h>', '#include "mamba3_amd.h"',
             'int main(void) {']
    for cname, cls in structs.items():
        lines.append(f'printf("{cname} size %zu\\n", sizeof({cname}));')
        for field, _ in cls._fields_:
            lines.append(f'printf("{cname} {field} %zu\\n", offsetof({cname}, {field}));')
    lines += ["return 0;", "}"]
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines) + "\n")
    exe = tmp_path / "layout"
    subprocess.run([cc, f"-I{ROOT / 'include'}", str(src), "-o", str(exe)], check=True)
    got = {}
    for line in subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.splitlines():
        cname, field, val = line.split()
        got[(cname, field)] = int(val)
    for cname, cls in structs.items():
        assert got[(cname, "size")] == ctypes.sizeof(cls), cname
        for field, _ in cls._fields_:
            assert got[(cname, field)] == getattr(cls, field).offset, (cname, field)


def test_prefill_kernel_name_and_noalloc_refusal(lib):
    """The dispatch query names the kernel from the descriptor alone (null pointers are
    aligned); the no-allocation entry refuses M3_FLAG_FOR_BACKWARD before any launch."""
    def desc(**kw):
        d = dict(batch=2, seqlen=64, nheads=24, headdim=64, d_state=128, mimo_rank=2, ngroups=1,
                 use_trapezoidal=1, use_complex=1, dtype=1, proj_row_stride=3696, rms_eps=1e-5,
                 flags=0)
        d.update(kw)
        return _native.LayerDesc(**d)
    name = lambda d: lib.m3_prefill_kernel_name(ctypes.byref(d), None, None, None, None)
    assert name(desc()) == b"mfma_d128_p64_r2"
    assert name(desc(flags=_native.M3_FLAG_NO_F16_OPERANDS)) == b"generic"
    assert name(desc(headdim=32, nheads=48, d_state=256, mimo_rank=4, proj_row_stride=
                     2 * 1536 + 2 * 256 * 4 + 3 * 48 + 128)) == b"mfma_general"
    assert name(desc(dtype=0)) == b"fp32_fused"
    assert name(desc(dtype=0, mimo_rank=4, proj_row_stride=3072 + 2 * 512 + 3 * 24 + 64)) == b"fp32_layer"
    assert name(desc(batch=0)) is None
    fake = ctypes.c_void_p(256)
    params = _native.LayerParams(*([256] * 10))
    d = desc(dtype=0, flags=_native.M3_FLAG_FOR_BACKWARD)
    assert lib.m3_prefill_fwd_noalloc(ctypes.byref(d), ctypes.byref(params), fake, None, fake,
                                      None, None, None, None) == 3
