"""Host-side behaviour of the drop-in modules (no GPU needed).

* seeded construction reproduces the reference's weights exactly (RNG order);
* state-dict names/shapes/order match the reference;
* the SSD path refuses CPU tensors (no CPU fallback);
* inference-state layout.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import mamba3_amd
from conftest import LAYER_CASES, golden_config, load_golden


def _make(kw):
    torch.manual_seed(0)
    return mamba3_amd.KulaMamba(**kw)


@pytest.mark.parametrize("name", LAYER_CASES + ["layer_tiny_dtscale"])
def test_seeded_layer_weights_equal_reference(name):
    g = load_golden(name)
    layer = _make(golden_config(g))
    sd = layer.state_dict()
    ref_keys = [k[len("param/"):] for k in g if k.startswith("param/")]
    assert list(sd.keys()) == ref_keys
    for k in ref_keys:
        assert torch.equal(sd[k], torch.from_numpy(g["param/" + k])), k


def test_seeded_d768_layer_checksums_equal_reference():
    g = load_golden("layer_d768")
    layer = _make(dict(d_model=768, d_state=128, expand=2, headdim=64, mimo_rank=2))
    sd = layer.state_dict()
    assert list(sd.keys()) == list(g["names"])
    for k, s, a in zip(g["names"], g["sums"], g["abs_sums"]):
        assert float(sd[k].double().sum()) == pytest.approx(float(s), rel=1e-12, abs=1e-9), k
        assert float(sd[k].double().abs().sum()) == pytest.approx(float(a), rel=1e-12), k
    np.testing.assert_array_equal(layer.in_proj.weight[::97, ::13].detach().numpy(),
                                  g["in_proj_slice"])


def test_seeded_tiny_lm_weights_equal_reference():
    g = load_golden("lm_tiny")
    torch.manual_seed(0)
    lm = mamba3_amd.KulaMambaLM(vocab_size=256, d_model=64, n_layers=2, d_state=16,
                                headdim=16, mimo_rank=2, chunk_size=8)
    sd = lm.state_dict()
    ref_keys = [k[len("param/"):] for k in g if k.startswith("param/")]
    assert list(sd.keys()) == ref_keys
    for k in ref_keys:
        assert torch.equal(sd[k], torch.from_numpy(g["param/" + k])), k
    assert lm.lm_head.weight is lm.embedding.weight


def test_seeded_d768_lm_checksums_equal_reference():
    g = load_golden("lm_d768_checksums")
    torch.manual_seed(0)
    lm = mamba3_amd.KulaMambaLM(32000, d_model=768, n_layers=24, d_state=128, headdim=64,
                                mimo_rank=2, residual_scale="depth")
    sd = lm.state_dict()
    assert list(sd.keys()) == list(g["names"])
    for k, s in zip(g["names"], g["sums"]):
        assert float(sd[k].double().sum()) == pytest.approx(float(s), rel=1e-10, abs=1e-8), k
    assert lm.layers[0].residual_scale == pytest.approx(1 / np.sqrt(48))


def test_public_api_names():
    assert set(mamba3_amd.__all__) == {"KulaMamba", "KulaMambaBlock", "KulaMambaLM", "RMSNorm",
                                       "SwiGLU", "SSDOutput", "chunked_ssd", "ssd_scan"}


def test_state_shapes_and_dtypes():
    layer = mamba3_amd.KulaMamba(64, d_state=16, headdim=16, mimo_rank=2, chunk_size=8)
    st = layer.allocate_inference_state(2, dtype=torch.bfloat16)
    H, P, N = layer.nheads, layer.headdim, layer.d_state
    assert st["h"].shape == (2, H, P, N) and st["h"].dtype == torch.float32
    assert st["prev_BX"].shape == (2, H, P, N) and st["prev_BX"].dtype == torch.float32
    assert st["angle"].shape == (2, H, N // 2) and st["angle"].dtype == torch.float32


def test_default_ngroups_and_param_count():
    g1 = mamba3_amd.KulaMamba(64, d_state=16, headdim=16, chunk_size=8)
    gh = mamba3_amd.KulaMamba(64, d_state=16, headdim=16, chunk_size=8, ngroups=g1.nheads)
    assert g1.ngroups == 1
    assert sum(p.numel() for p in g1.parameters()) < sum(p.numel() for p in gh.parameters())


def test_cpu_tensors_are_refused_loudly():
    layer = mamba3_amd.KulaMamba(64, d_state=16, headdim=16, chunk_size=8)
    x = torch.randn(1, 8, 64)
    with pytest.raises(RuntimeError, match="GPU"):
        layer(x)
    with pytest.raises(RuntimeError, match="GPU"):
        layer.step(x[:, 0], layer.allocate_inference_state(1))
    with pytest.raises(RuntimeError, match="GPU"):
        mamba3_amd.ssd_scan(torch.rand(1, 2, 3), torch.randn(1, 2, 3, 4))


def test_constructor_validation():
    with pytest.raises(ValueError):
        mamba3_amd.KulaMamba(64, d_state=15, headdim=16)
    with pytest.raises(ValueError):
        mamba3_amd.KulaMamba(64, d_state=16, headdim=24)
    with pytest.raises(ValueError):
        mamba3_amd.KulaMamba(64, d_state=16, headdim=16, ngroups=3)
