"""Shared pytest configuration: the `gpu` marker and fixture helpers."""

from __future__ import annotations

import ast
import sys
from pathlib import Path

import numpy as np
import pytest
import torch

ROOT = Path(__file__).resolve().parents[1]
GOLDEN = ROOT / "tests" / "golden"
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD GPU (MI355X) and the built HIP library")


def load_golden(name: str) -> dict:
    with np.load(GOLDEN / f"{name}.npz", allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def golden_params(g: dict) -> dict:
    return {k[len("param/"):]: torch.from_numpy(v) for k, v in g.items() if k.startswith("param/")}


def golden_config(g: dict) -> dict:
    return ast.literal_eval(str(g["config"]))


def max_rel(a: torch.Tensor, b: torch.Tensor) -> float:
    """Normwise max-relative error max|a-b| / max|b|."""
    a = a.detach().double().cpu()
    b = b.detach().double().cpu()
    den = b.abs().max().item()
    return (a - b).abs().max().item() / (den if den > 0 else 1.0)


LAYER_CASES = ["layer_tiny", "layer_trap_off", "layer_complex_off", "layer_rank1",
               "layer_groups2", "layer_all_off", "layer_rank4_n32"]
CHUNKED_CASES = ["chunked_beta_hinit", "chunked_ragged", "chunked_nobeta"]


def oracle_cfg(kw: dict):
    from oracle.reference_path import LayerCfg
    return LayerCfg(d_model=kw["d_model"], d_state=kw.get("d_state", 128),
                    expand=kw.get("expand", 2), headdim=kw.get("headdim", 64),
                    ngroups=kw.get("ngroups") or 1, mimo_rank=kw.get("mimo_rank", 2),
                    chunk_size=kw.get("chunk_size", 64),
                    use_trapezoidal=bool(kw.get("use_trapezoidal", True)),
                    use_complex_ssm=bool(kw.get("use_complex_ssm", True)))


@pytest.fixture(scope="session")
def cuda_device():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")
