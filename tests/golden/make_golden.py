"""Write the golden fixtures of tests/golden/ (run: python tests/golden/make_golden.py).

The reference ships no golden vectors; its checks compare against
torch.optim at run time (adam_benchmark.py:113-115, muon_benchmark.py:104-106,
muon_adamw_benchmark.py:130-134).  These fixtures freeze what that library
routine -- fused torch.optim.AdamW + torch.optim.Muon, as wrapped by
PyTorchMuonAdamW (optimizer.py:178-260) -- returns on the CPU for seeded
inputs (torch 2.10.0), so later runs are checked against stored data:

c1_toy_mlp.npz   config 1: Linear(512,2048) -> LayerNorm(2048) -> Linear(2048,512),
                 every parameter N(0,0.02), grads N(0,1e-3), torch.Generator seed 0
                 (parameters, then gradients, in named_parameters order); one
                 step.  Full AdamW outputs; for the two Muon weights a strided
                 sample of 4096 updated values and of the orthogonalised update,
                 with the update's Frobenius norm.  Input fingerprints
                 (sum, sum of squares, 64 strided values) detect generator drift.
adamw_c2_head.npz  six tensors with config 2 distributions at the 10th step
                 (state step 9), fused AdamW output.
ns_small.npz     torch.optim._muon._zeropower_via_newtonschulz on small bf16
                 inputs (wide, tall, square, ns_steps 5 and 2), output bits.
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import torch
from torch.optim._muon import _zeropower_via_newtonschulz

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1] / "triton-muonadamw_amd"))
COEFFS = (3.4445, -4.7750, 2.0315)


def fingerprint(t: torch.Tensor) -> np.ndarray:
    a = t.detach().double().flatten()
    idx = torch.linspace(0, a.numel() - 1, 64).long()
    return np.concatenate([[a.sum().item(), (a * a).sum().item()], a[idx].numpy()])


def c1_inputs():
    """Config 1 model, parameters and gradients (deterministic)."""
    model = torch.nn.Sequential(torch.nn.Linear(512, 2048), torch.nn.LayerNorm(2048), torch.nn.Linear(2048, 512))
    gen = torch.Generator().manual_seed(0)
    with torch.no_grad():
        for p in model.parameters():
            p.copy_(torch.randn(p.shape, generator=gen) * 0.02)
        for p in model.parameters():
            p.grad = torch.randn(p.shape, generator=gen) * 1e-3
    return model


def c1_configs():
    from triton_muon_adamw import AdamConfig, MuonConfig

    mc = MuonConfig(lr=1e-3, beta=0.95, eps=1e-7, weight_decay=0.1, coeffs=COEFFS, nesterov=True, ns_steps=5,
                    adjust_lr_fn="original")
    ac = AdamConfig(lr=3e-4, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1)
    return mc, ac


def make_c1():
    from triton_muon_adamw import PyTorchMuonAdamW

    model = c1_inputs()
    names = [n for n, _ in model.named_parameters()]
    params = list(model.parameters())
    out = {"names": np.array(names)}
    for n, p in zip(names, params):
        out[f"fp_param/{n}"] = fingerprint(p)
        out[f"fp_grad/{n}"] = fingerprint(p.grad)
    p0 = [p.detach().clone() for p in params]
    mc, ac = c1_configs()
    split = {"adam": [p for p in params if p.ndim != 2], "muon": [p for p in params if p.ndim == 2]}
    opt = PyTorchMuonAdamW(split, muon_config=mc, adam_config=ac, parameter_split="explicit")
    opt.step()
    for n, p, q in zip(names, params, p0):
        if p.ndim != 2:
            out[f"adam/{n}"] = p.detach().numpy().copy()
        else:
            R, C = p.shape
            adj = mc.lr * max(1.0, R / C) ** 0.5
            upd = (q.double() * float(np.float32(1 - mc.lr * mc.weight_decay)) - p.detach().double()) / adj
            idx = torch.linspace(0, p.numel() - 1, 4096).long()
            out[f"muon_idx/{n}"] = idx.numpy()
            out[f"muon_param/{n}"] = p.detach().flatten()[idx].numpy().copy()
            out[f"muon_update/{n}"] = upd.flatten()[idx].numpy().astype(np.float32)
            out[f"muon_update_fro/{n}"] = np.array([upd.norm().item()])
    np.savez_compressed(HERE / "c1_toy_mlp.npz", **out)


ADAMW_HEAD_SIZES = [1000, 1500, 4096, 4097, 7000, 12345]


def adamw_head_inputs():
    gen = torch.Generator().manual_seed(2)
    ps = [torch.randn(s, generator=gen) * 0.02 for s in ADAMW_HEAD_SIZES]
    gs = [torch.randn(s, generator=gen) * 1e-3 for s in ADAMW_HEAD_SIZES]
    ms = [torch.randn(s, generator=gen) * 1e-4 for s in ADAMW_HEAD_SIZES]
    vs = [(torch.randn(s, generator=gen) * 1e-6).abs() for s in ADAMW_HEAD_SIZES]
    return ps, gs, ms, vs


def make_adamw_head():
    ps, gs, ms, vs = adamw_head_inputs()
    out = {"sizes": np.array(ADAMW_HEAD_SIZES)}
    params = [torch.nn.Parameter(p.clone()) for p in ps]
    opt = torch.optim.AdamW(params, lr=3e-4, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1, fused=True)
    for i, p in enumerate(params):
        p.grad = gs[i].clone()
        opt.state[p] = {"step": torch.tensor(9.0), "exp_avg": ms[i].clone(), "exp_avg_sq": vs[i].clone()}
        out[f"fp_in/{i}"] = np.concatenate([fingerprint(t) for t in (ps[i], gs[i], ms[i], vs[i])])
    opt.step()
    for i, p in enumerate(params):
        out[f"param/{i}"] = p.detach().numpy().copy()
        out[f"exp_avg/{i}"] = opt.state[p]["exp_avg"].numpy().copy()
        out[f"exp_avg_sq/{i}"] = opt.state[p]["exp_avg_sq"].numpy().copy()
    np.savez_compressed(HERE / "adamw_c2_head.npz", **out)


NS_CASES = [((40, 64), 5), ((64, 40), 5), ((96, 96), 5), ((48, 160), 2)]


def ns_input(i, shape):
    gen = torch.Generator().manual_seed(100 + i)
    return torch.randn(shape, generator=gen)


def make_ns():
    out = {}
    for i, (shape, steps) in enumerate(NS_CASES):
        g = ns_input(i, shape)
        o = _zeropower_via_newtonschulz(g, COEFFS, steps, 1e-7)
        out[f"fp/{i}"] = fingerprint(g)
        out[f"out_bits/{i}"] = o.contiguous().view(torch.int16).numpy().astype(np.uint16)
    np.savez_compressed(HERE / "ns_small.npz", **out)


if __name__ == "__main__":
    torch.set_num_threads(min(8, torch.get_num_threads()))
    make_c1()
    make_adamw_head()
    make_ns()
    for f in sorted(HERE.glob("*.npz")):
        print(f.name, f.stat().st_size)
