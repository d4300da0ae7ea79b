"""Write the golden fixtures under tests/golden/ from the reference implementation.

Run in the development container only (the reference is not available elsewhere):

    python tests/golden/make_golden.py [/path/to/reference]

What the fixtures pin that the mathematics alone does not: the exact seeded weights
(RNG consumption order of the reference constructors) and the layer-level semantics
(projection split, RMSNorm over N*R with rank fastest, RoPE pairing and sign, trapezoid
shift, MIMO gate) of the reference's forward, prefill and step. Everything is fp32 on
the CPU. Fixtures are data only: inputs, parameters and outputs as .npz arrays.
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
REF = Path(sys.argv[1]) if len(sys.argv) > 1 else Path("/root/reference")


def _np(t):
    return t.detach().cpu().float().numpy().copy()


def _state(prefix, st, out):
    for k in ("h", "angle", "prev_BX"):
        out[f"{prefix}/{k}"] = _np(st[k])


def layer_case(KulaMamba, name, kw, x_shape, n_steps, dt_scale=False):
    torch.manual_seed(0)
    layer = KulaMamba(**kw).eval()
    out = {f"param/{k}": _np(v) for k, v in layer.state_dict().items()}
    torch.manual_seed(1)
    x = torch.randn(*x_shape)
    out["x"] = _np(x)
    with torch.no_grad():
        if dt_scale:
            torch.manual_seed(3)
            ds = torch.rand(x_shape[0], x_shape[1], layer.nheads) * 1.5 + 0.5
            out["dt_scale"] = _np(ds)
            out["y"] = _np(layer(x, dt_scale=ds))
        else:
            out["y"] = _np(layer(x))
            y_pf, st = layer.prefill(x)
            out["y_prefill"] = _np(y_pf)
            _state("prefill", st, out)
            torch.manual_seed(2)
            xs = torch.randn(x_shape[0], n_steps, x_shape[2])
            out["x_steps"] = _np(xs)
            outs = []
            for t in range(n_steps):
                # alternate (B,D) and (B,1,D) inputs to pin both ranks
                if t % 2 == 0:
                    o, st = layer.step(xs[:, t], st)
                else:
                    o, st = layer.step(xs[:, t:t + 1], st)
                    o = o.squeeze(1)
                outs.append(o)
            out["y_steps"] = _np(torch.stack(outs, 1))
            _state("steps", st, out)
    cfg = {k: (int(v) if isinstance(v, (bool, int)) else v) for k, v in kw.items()}
    out["config"] = np.array(repr(cfg))
    np.savez_compressed(HERE / f"{name}.npz", **out)
    print("wrote", name)


def chunked_case(chunked_ssd, name, B, T, H, P, R, N, CS, beta, h_init):
    g = torch.Generator().manual_seed(11)
    r = lambda *s: torch.randn(*s, generator=g)
    x_g, B_g, C = r(B, T, H, P, R), r(B, T, H, N, R), r(B, T, H, N, R)
    x_b = r(B, T, H, P, R) if beta else None
    B_b = r(B, T, H, N, R) if beta else None
    dt = torch.rand(B, T, H, generator=g) * 0.1 + 0.01
    A = -torch.exp(r(H).clamp(-4, -1))
    D = r(H)
    x_raw = r(B, T, H, P, R)
    h0 = r(B, H, P, N) if h_init else None
    res = chunked_ssd(x_g, x_b, B_g, B_b, C, dt, A, D, x_raw, CS, h_init=h0,
                      return_final_state=True)
    out = dict(x_g=_np(x_g), B_g=_np(B_g), C=_np(C), dt=_np(dt), A=_np(A), D=_np(D),
               x_raw=_np(x_raw), y=_np(res.y), h_final=_np(res.h_final),
               chunk_size=np.array(CS))
    if beta:
        out.update(x_b=_np(x_b), B_b=_np(B_b))
    if h_init:
        out["h_init"] = _np(h0)
    np.savez_compressed(HERE / f"{name}.npz", **out)
    print("wrote", name)


def checksums(module):
    names, sums, abs_sums = [], [], []
    for k, v in module.state_dict().items():
        names.append(k)
        sums.append(float(v.double().sum()))
        abs_sums.append(float(v.double().abs().sum()))
    return np.array(names), np.array(sums), np.array(abs_sums)


def main():
    sys.path.insert(0, str(REF))
    from mamba3 import KulaMamba, KulaMambaLM, chunked_ssd  # noqa: E402

    torch.set_num_threads(8)
    tiny = dict(d_model=64, d_state=16, headdim=16, mimo_rank=2, expand=2, chunk_size=8)
    layer_case(KulaMamba, "layer_tiny", tiny, (2, 37, 64), 8)
    layer_case(KulaMamba, "layer_tiny_dtscale", tiny, (1, 19, 64), 0, dt_scale=True)
    for name, extra in (("layer_trap_off", dict(use_trapezoidal=False)),
                        ("layer_complex_off", dict(use_complex_ssm=False)),
                        ("layer_rank1", dict(mimo_rank=1)),
                        ("layer_groups2", dict(ngroups=2)),
                        ("layer_all_off", dict(use_trapezoidal=False, use_complex_ssm=False,
                                               mimo_rank=1)),
                        ("layer_rank4_n32", dict(mimo_rank=4, d_state=32, headdim=32))):
        layer_case(KulaMamba, name, {**tiny, **extra}, (1, 19, 64), 3)

    chunked_case(chunked_ssd, "chunked_beta_hinit", 1, 16, 2, 4, 2, 8, 8, True, True)
    chunked_case(chunked_ssd, "chunked_ragged", 2, 13, 3, 4, 2, 8, 4, True, False)
    chunked_case(chunked_ssd, "chunked_nobeta", 1, 20, 2, 8, 1, 16, 8, False, True)

    # d_model=768 layer (d_state 128, headdim 64, rank 2), seed 0 weights, seed 1 input.
    torch.manual_seed(0)
    big = KulaMamba(768, d_state=128, expand=2, headdim=64, mimo_rank=2).eval()
    names, sums, abs_sums = checksums(big)
    torch.manual_seed(1)
    x = torch.randn(4, 1024, 768)
    with torch.no_grad():
        y, st = big.prefill(x)
    np.savez_compressed(
        HERE / "layer_d768.npz", names=names, sums=sums, abs_sums=abs_sums,
        in_proj_slice=_np(big.in_proj.weight[::97, ::13]), x_sum=np.array(float(x.double().sum())),
        y_slice=_np(y[:, ::64, ::16]), y_sum=np.array(float(y.double().sum())),
        y_abs_sum=np.array(float(y.double().abs().sum())),
        h_slice=_np(st["h"][:, :, ::8, ::16]), angle_slice=_np(st["angle"][:, :, ::8]),
        prev_slice=_np(st["prev_BX"][:, :, ::8, ::16]))
    print("wrote layer_d768")

    # Tiny LM: full weights, logits and greedy generation.
    torch.manual_seed(0)
    lm = KulaMambaLM(vocab_size=256, d_model=64, n_layers=2, d_state=16, headdim=16,
                     mimo_rank=2, chunk_size=8).eval()
    g = torch.Generator().manual_seed(5)
    ids = torch.randint(0, 256, (2, 12), generator=g)
    with torch.no_grad():
        logits = lm(ids)["logits"]
        gen = lm.generate(ids[:, :5], max_new_tokens=6, temperature=0)
    out = {f"param/{k}": _np(v) for k, v in lm.state_dict().items()}
    out.update(ids=ids.numpy(), logits=_np(logits), generated=gen.numpy())
    np.savez_compressed(HERE / "lm_tiny.npz", **out)
    print("wrote lm_tiny")

    # Full-size LM parameter checksums (vocab 32000, d768, 24 layers).
    torch.manual_seed(0)
    lm_big = KulaMambaLM(32000, d_model=768, n_layers=24, d_state=128, headdim=64, mimo_rank=2,
                         residual_scale="depth")
    names, sums, abs_sums = checksums(lm_big)
    np.savez_compressed(HERE / "lm_d768_checksums.npz", names=names, sums=sums,
                        abs_sums=abs_sums)
    print("wrote lm_d768_checksums")


if __name__ == "__main__":
    main()
