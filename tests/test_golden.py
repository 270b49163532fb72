"""Golden fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py
from torch.optim on the CPU) against the oracle (CPU) and the HIP path (GPU).

Inputs are regenerated from their seeds and their fingerprints checked first,
so a change of torch's generator shows up as a fingerprint failure rather
than a parity failure.
"""

import importlib.util
from pathlib import Path

import numpy as np
import pytest
import torch

import oracle
from oracle.bf16 import from_bits

GOLDEN = Path(__file__).resolve().parent / "golden"
_spec = importlib.util.spec_from_file_location("make_golden", GOLDEN / "make_golden.py")
mg = importlib.util.module_from_spec(_spec)
_spec.loader.exec_module(mg)


def _fixture(name):
    return np.load(GOLDEN / name, allow_pickle=False)


def _c1():
    d = _fixture("c1_toy_mlp.npz")
    model = mg.c1_inputs()
    for n, p in model.named_parameters():
        np.testing.assert_allclose(mg.fingerprint(p), d[f"fp_param/{n}"], rtol=1e-12, atol=0)
        np.testing.assert_allclose(mg.fingerprint(p.grad), d[f"fp_grad/{n}"], rtol=1e-12, atol=0)
    return d, model


def _check_c1(d, model, p_after, upd_after):
    """p_after / upd_after: name -> numpy array (full tensors) of the result under test."""
    mc, _ = mg.c1_configs()
    for n, p in model.named_parameters():
        if p.ndim != 2:
            np.testing.assert_allclose(p_after[n], d[f"adam/{n}"], rtol=0, atol=1e-7, err_msg=n)
        else:
            idx = d[f"muon_idx/{n}"]
            R, C = p.shape
            adj = mc.lr * max(1.0, R / C) ** 0.5
            got_u = upd_after[n].flatten()
            fro = np.linalg.norm(got_u.astype(np.float64))
            assert abs(fro - d[f"muon_update_fro/{n}"][0]) / fro < 1e-2, n
            su, eu = got_u[idx], d[f"muon_update/{n}"]
            assert np.linalg.norm(su - eu) / np.linalg.norm(eu) < 1e-2, n
            np.testing.assert_allclose(p_after[n].flatten()[idx], d[f"muon_param/{n}"], rtol=0, atol=adj * 1e-2,
                                       err_msg=n)


def test_c1_oracle_vs_golden():
    d, model = _c1()
    mc, ac = mg.c1_configs()
    p_after, upd = {}, {}
    step = 1
    b1, b2 = oracle.adamw.bias_corrections(*ac.betas, step)
    for n, p in model.named_parameters():
        p0, g = p.detach().numpy(), p.grad.numpy()
        if p.ndim != 2:
            p_after[n], _, _ = oracle.adamw.adamw_update(p0, g, np.zeros_like(p0), np.zeros_like(p0), lr=ac.lr,
                                                         bias1=b1, bias2=b2, beta1=ac.betas[0], beta2=ac.betas[1],
                                                         weight_decay=ac.weight_decay, eps=ac.eps)
        else:
            p_after[n], _, upd[n] = oracle.muon.muon_update(p0, g, np.zeros_like(p0), lr=mc.lr,
                                                            weight_decay=mc.weight_decay, beta=mc.beta,
                                                            nesterov=mc.nesterov, coeffs=mc.coeffs,
                                                            ns_steps=mc.ns_steps, eps=mc.eps)
    _check_c1(d, model, p_after, upd)


def test_adamw_head_oracle_vs_golden():
    d = _fixture("adamw_c2_head.npz")
    ps, gs, ms, vs = mg.adamw_head_inputs()
    b1, b2 = oracle.adamw.bias_corrections(0.9, 0.95, 10)
    for i in range(len(ps)):
        fp = np.concatenate([mg.fingerprint(t) for t in (ps[i], gs[i], ms[i], vs[i])])
        np.testing.assert_allclose(fp, d[f"fp_in/{i}"], rtol=1e-12, atol=0)
        p, m, v = oracle.adamw.adamw_update(ps[i].numpy(), gs[i].numpy(), ms[i].numpy(), vs[i].numpy(), lr=3e-4,
                                            bias1=b1, bias2=b2, beta1=0.9, beta2=0.95, weight_decay=0.1, eps=1e-8)
        np.testing.assert_allclose(p, d[f"param/{i}"], rtol=0, atol=1e-8)
        np.testing.assert_allclose(m, d[f"exp_avg/{i}"], rtol=1e-6, atol=5e-10)  # lerp vs mul-add rounding
        np.testing.assert_allclose(v, d[f"exp_avg_sq/{i}"], rtol=1e-6, atol=0)


def test_ns_small_oracle_vs_golden():
    d = _fixture("ns_small.npz")
    for i, (shape, steps) in enumerate(mg.NS_CASES):
        g = mg.ns_input(i, shape)
        np.testing.assert_allclose(mg.fingerprint(g), d[f"fp/{i}"], rtol=1e-12, atol=0)
        exp = from_bits(d[f"out_bits/{i}"])
        got = oracle.muon.zeropower_ns(g.numpy(), mg.COEFFS, steps, 1e-7)
        assert got.shape == exp.shape
        assert np.linalg.norm(got - exp) / np.linalg.norm(exp) < 1e-2, i


# ---- GPU: the HIP path against the same fixtures ----------------------------------

@pytest.mark.gpu
def test_c1_hip_vs_golden(gpu):
    from triton_muon_adamw import MuonAdamW

    d, model = _c1()
    names = [n for n, _ in model.named_parameters()]
    model = model.to(gpu)  # grads move with the parameters
    params = dict(model.named_parameters())
    mc, ac = mg.c1_configs()
    split = {"adam": [p for p in params.values() if p.ndim != 2], "muon": [p for p in params.values() if p.ndim == 2]}
    p0 = {n: params[n].detach().clone() for n in names}
    opt = MuonAdamW(split, muon_config=mc, adam_config=ac, parameter_split="explicit")
    opt.step()
    torch.cuda.synchronize()
    keep = np.float32(1 - mc.lr * mc.weight_decay)
    p_after, upd = {}, {}
    for n in names:
        p = params[n]
        p_after[n] = p.detach().cpu().numpy()
        if p.ndim == 2:
            R, C = p.shape
            adj = mc.lr * max(1.0, R / C) ** 0.5
            upd[n] = ((p0[n].cpu().double().numpy() * keep - p_after[n]) / adj).astype(np.float32)
    _check_c1(d, model, p_after, upd)


@pytest.mark.gpu
def test_adamw_head_hip_vs_golden(gpu):
    from triton_muon_adamw.adamw import HipAdamW

    d = _fixture("adamw_c2_head.npz")
    ps, gs, ms, vs = mg.adamw_head_inputs()
    params = [torch.nn.Parameter(p.to(gpu)) for p in ps]
    opt = HipAdamW(params, lr=3e-4, betas=(0.9, 0.95), weight_decay=0.1, eps=1e-8)
    for i, p in enumerate(params):
        p.grad = gs[i].to(gpu)
        opt.m[p].copy_(ms[i])
        opt.v[p].copy_(vs[i])
    opt.step_num = 9
    opt.step()
    torch.cuda.synchronize()
    for i, p in enumerate(params):
        np.testing.assert_allclose(p.detach().cpu().numpy(), d[f"param/{i}"], rtol=0, atol=1e-8)
        np.testing.assert_allclose(opt.m[p].cpu().numpy(), d[f"exp_avg/{i}"], rtol=1e-6, atol=5e-10)
        np.testing.assert_allclose(opt.v[p].cpu().numpy(), d[f"exp_avg_sq/{i}"], rtol=1e-6, atol=0)


@pytest.mark.gpu
def test_ns_small_hip_vs_golden(gpu):
    from triton_muon_adamw.muon import muon_step

    d = _fixture("ns_small.npz")
    for i, (shape, steps) in enumerate(mg.NS_CASES):
        g = mg.ns_input(i, shape).to(gpu)
        # beta = 0, no Nesterov: momentum = grad, so the update is NS(grad) exactly
        w = torch.zeros(shape, device=gpu)
        mom = torch.zeros(shape, device=gpu)
        out = torch.empty(shape, device=gpu)
        muon_step(w, g, mom, 0.0, *mg.COEFFS, 1.0, 1.0, 0.0, steps, 1e-7, False, out=out)
        torch.cuda.synchronize()
        exp = from_bits(d[f"out_bits/{i}"])
        got = out.cpu().numpy()
        assert np.linalg.norm(got - exp) / np.linalg.norm(exp) < 1e-2, i
        assert np.array_equal(-w.cpu().numpy(), got)  # param = 0 - 1.0 * update
