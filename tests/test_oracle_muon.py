"""Pins the Muon oracle (oracle/muon.py, oracle/bf16.py) before it is trusted.

* bf16 rounding and lerp: bit-exact against torch on the CPU;
* Newton-Schulz in float64: the closed form on singular values (for
  X = U diag(s) V^T, each iteration maps s -> a s + b s^3 + c s^5 after
  normalising by ||s||_2 = ||X||_F);
* Newton-Schulz in bf16: against torch.optim._muon._zeropower_via_newtonschulz,
  the routine PyTorchMuonAdamW reaches (optimizer.py:228-241), at bf16 noise;
* invariants: transpose symmetry, singular values of the result in the
  band the quintic maps [3e-3, 1] into, ns_steps = 0;
* one full step against torch.optim.Muon on the CPU;
* the learning-rate scaling closed forms;
* planted mistakes (dropped term, wrong sign, transposed operand) must fail.
"""

import math

import numpy as np
import pytest
import torch
from torch.optim._muon import _zeropower_via_newtonschulz

from oracle import bf16, muon as om

COEFFS = (3.4445, -4.7750, 2.0315)


def test_bf16_round_matches_torch_bitexact():
    rng = np.random.default_rng(0)
    x = np.concatenate([
        (rng.standard_normal(200000) * 10).astype(np.float32),
        (rng.standard_normal(1000) * 1e-39).astype(np.float32),  # subnormals
        np.array([0.0, -0.0, np.inf, -np.inf, 3.0e38, -3.4e38, 1.0 + 2**-8, 1.0 + 3 * 2**-8], np.float32),
    ])
    # exact ties: mantissa low half 0x8000 with both parities of bit 16
    ties = (rng.integers(0, 2**31, 1000, dtype=np.uint64).astype(np.uint32) & 0xFFFF0000) | 0x8000
    x = np.concatenate([x, ties.view(np.float32)])
    x = x[np.isfinite(x) | np.isinf(x)]
    t = torch.from_numpy(x.copy()).bfloat16().float().numpy()
    o = bf16.round_bf16(x)
    same = (t == o) | (np.isnan(t) & np.isnan(o))
    assert same.all()
    assert np.array_equal(bf16.from_bits(bf16.to_bits(o)), o)
    assert np.isnan(bf16.round_bf16(np.array([np.nan], np.float32)))[0]


@pytest.mark.parametrize("w", [1 - 0.95, 0.95, 0.5, 0.3, 0.7, 0.0, 1.0])
def test_lerp_matches_torch_bitexact(w):
    rng = np.random.default_rng(1)
    s = (rng.standard_normal(300000) * 1e-3).astype(np.float32)
    e = rng.standard_normal(300000).astype(np.float32)
    t = torch.from_numpy(s).lerp(torch.from_numpy(e), w).numpy()
    assert np.array_equal(om.lerp(s, e, w), t)


def _known_svd(m, n, sig, seed):
    rng = np.random.default_rng(seed)
    U, _ = np.linalg.qr(rng.standard_normal((m, m)))
    V, _ = np.linalg.qr(rng.standard_normal((n, n)))
    k = min(m, n)
    return U[:, :k], V[:, :k], np.asarray(sig, np.float64)


@pytest.mark.parametrize("m,n,steps", [(16, 40, 5), (40, 16, 5), (32, 32, 3), (8, 100, 1), (20, 30, 0)])
def test_ns_exact_closed_form(m, n, steps):
    k = min(m, n)
    sig = np.geomspace(1.0, 1e-3, k)
    U, V, s = _known_svd(m, n, sig, seed=m * n)
    G = (U * s) @ V.T
    got = om.zeropower_ns(G, COEFFS, steps, eps=1e-7, exact=True)
    a, b, c = COEFFS
    t = s / np.linalg.norm(s)
    for _ in range(steps):
        t = a * t + b * t**3 + c * t**5
    np.testing.assert_allclose(got, (U * t) @ V.T, rtol=0, atol=1e-12)


@pytest.mark.parametrize("shape", [(64, 128), (128, 64), (96, 200), (256, 512), (1, 40), (40, 1)])
def test_ns_bf16_vs_torch(shape):
    G = np.random.default_rng(2).standard_normal(shape).astype(np.float32)
    t = _zeropower_via_newtonschulz(torch.from_numpy(G), COEFFS, 5, 1e-7).float().numpy()
    o = om.zeropower_ns(G, COEFFS, 5, 1e-7)
    err = np.linalg.norm(o - t) / np.linalg.norm(t)
    assert err < 1e-2, err
    ex = om.zeropower_ns(G, COEFFS, 5, 1e-7, exact=True)
    assert np.linalg.norm(o - ex) / np.linalg.norm(ex) < 3e-2


def test_ns_transpose_symmetry():
    G = np.random.default_rng(3).standard_normal((48, 112)).astype(np.float32)
    assert np.array_equal(om.zeropower_ns(G.T, COEFFS), om.zeropower_ns(G, COEFFS).T)


def test_ns_steps_zero_is_normalised_input():
    G = np.random.default_rng(4).standard_normal((20, 30)).astype(np.float32)
    X = bf16.round_bf16(G)
    nrm = om.frobenius_norm_bf16(X)
    assert np.array_equal(om.zeropower_ns(G, COEFFS, 0), bf16.round_bf16(X / nrm))


def test_ns_singular_value_band():
    # Five quintic steps map normalised singular values in [3e-3, 1] into [0.68, 1.21].
    a, b, c = COEFFS
    t = np.geomspace(3e-3, 1.0, 4000)
    for _ in range(5):
        t = a * t + b * t**3 + c * t**5
    assert t.min() > 0.68 and t.max() < 1.21
    k = 24
    sig = np.geomspace(1.0, 3e-3, k)
    U, V, s = _known_svd(k, 60, sig / np.linalg.norm(sig), seed=5)
    out = om.zeropower_ns((U * s) @ V.T, COEFFS, 5, exact=True)
    sv = np.linalg.svd(out, compute_uv=False)
    assert sv.min() > 0.68 and sv.max() < 1.21


def test_adjust_lr_closed_forms():
    lr = 0.02
    assert om.adjust_lr(lr, "original", (2048, 512)) == lr * 2.0
    assert om.adjust_lr(lr, "original", (512, 2048)) == lr
    assert om.adjust_lr(lr, "original", (14336, 4096)) == lr * math.sqrt(3.5)
    assert om.adjust_lr(lr, "match_rms_adamw", (512, 2048)) == lr * (0.2 * math.sqrt(2048))
    assert om.adjust_lr(lr, "spectral_unclamped", (512, 2048)) == lr * 0.5
    with pytest.raises(AssertionError):
        om.adjust_lr(lr, "nope", (2, 2))


@pytest.mark.parametrize("adjust", ["original", "match_rms_adamw"])
@pytest.mark.parametrize("shape,nesterov", [((64, 96), True), ((96, 64), True), ((80, 80), False)])
def test_full_step_vs_torch_optim_muon(shape, nesterov, adjust):
    rng = np.random.default_rng(6)
    p0 = (rng.standard_normal(shape) * 0.02).astype(np.float32)
    g = rng.standard_normal(shape).astype(np.float32)
    m0 = (rng.standard_normal(shape) * 1e-3).astype(np.float32)
    tp = torch.nn.Parameter(torch.from_numpy(p0.copy()))
    opt = torch.optim.Muon([tp], lr=0.02, weight_decay=0.1, momentum=0.95, nesterov=nesterov,
                           ns_coefficients=COEFFS, eps=1e-7, ns_steps=5, adjust_lr_fn=adjust)
    opt.state[tp]["momentum_buffer"] = torch.from_numpy(m0.copy())
    tp.grad = torch.from_numpy(g.copy())
    opt.step()
    op, om_, _ = om.muon_update(p0, g, m0, lr=0.02, weight_decay=0.1, beta=0.95, nesterov=nesterov,
                                coeffs=COEFFS, ns_steps=5, eps=1e-7, adjust_lr_fn=adjust)
    assert np.array_equal(om_, opt.state[tp]["momentum_buffer"].numpy())
    adj = om.adjust_lr(0.02, adjust, shape)
    # torch's own scale for this shape (torch/optim/_muon.py:73-84) is the oracle's
    assert adj == torch.optim._muon._adjust_lr(0.02, adjust, torch.Size(shape))
    # parameter differences are adj * (bf16 noise of the update)
    np.testing.assert_allclose(op, tp.detach().numpy(), rtol=0, atol=adj * 8e-3)
    upd_t = (p0 * np.float32(1 - 0.02 * 0.1) - tp.detach().numpy()) / adj
    upd_o = (p0 * np.float32(1 - 0.02 * 0.1) - op) / adj
    assert np.linalg.norm(upd_o - upd_t) / np.linalg.norm(upd_t) < 1e-2


@pytest.mark.parametrize("shape", [(64, 96), (96, 64)])
def test_spectral_unclamped_step_vs_torch_direction(shape):
    """``spectral_unclamped`` exists only in the reference (triton_muon.py:430-431):
    torch pins the update direction (its "original" step on the same inputs,
    divided by its own scale) and the reference's closed form sqrt(R/C) the
    scale; for a tall matrix the two scales coincide."""
    rng = np.random.default_rng(16)
    p0 = (rng.standard_normal(shape) * 0.02).astype(np.float32)
    g = rng.standard_normal(shape).astype(np.float32)
    tp = torch.nn.Parameter(torch.from_numpy(p0.copy()))
    opt = torch.optim.Muon([tp], lr=0.02, weight_decay=0.1, momentum=0.95, nesterov=True,
                           ns_coefficients=COEFFS, eps=1e-7, ns_steps=5, adjust_lr_fn="original")
    tp.grad = torch.from_numpy(g.copy())
    opt.step()
    keep = np.float32(1 - 0.02 * 0.1)
    adj_t = torch.optim._muon._adjust_lr(0.02, "original", torch.Size(shape))
    upd_t = (p0 * keep - tp.detach().numpy()) / adj_t
    op, _, _ = om.muon_update(p0, g, np.zeros_like(p0), lr=0.02, weight_decay=0.1, beta=0.95, nesterov=True,
                              coeffs=COEFFS, ns_steps=5, eps=1e-7, adjust_lr_fn="spectral_unclamped")
    adj_o = om.adjust_lr(0.02, "spectral_unclamped", shape)
    assert adj_o == pytest.approx(0.02 * math.sqrt(shape[0] / shape[1]), rel=1e-15)
    if shape[0] > shape[1]:
        assert adj_o == pytest.approx(adj_t, rel=1e-15)
    upd_o = (p0 * keep - op) / adj_o
    assert np.linalg.norm(upd_o - upd_t) / np.linalg.norm(upd_t) < 1e-2


# --- planted mistakes --------------------------------------------------------

def _ns_mutant(G, kind, steps=5):
    a, b, c = COEFFS
    r = bf16.round_bf16
    tall = G.shape[0] > G.shape[1]
    X = r(G.T if tall else G)
    X = r(X / om.frobenius_norm_bf16(X))
    for _ in range(steps):
        A = r(X @ X.T)
        if kind == "drop_bA":
            B = r(c * (A @ A))
        elif kind == "sign_c":
            B = r(-c * (A @ A) + b * A)
        else:
            B = r(c * (A @ A) + b * A)
        if kind == "transposed_operand":
            X = r(a * X + (B @ X.T[: X.shape[0]].T if X.shape[0] == X.shape[1] else B.T @ X) + 0.01 * X)
        else:
            X = r(a * X + B @ X)
    return X.T if tall else X


@pytest.mark.parametrize("kind", ["drop_bA", "sign_c", "transposed_operand"])
def test_planted_ns_mistakes_are_caught(kind):
    G = np.random.default_rng(7).standard_normal((64, 128)).astype(np.float32)
    t = _zeropower_via_newtonschulz(torch.from_numpy(G), COEFFS, 5, 1e-7).float().numpy()
    with np.errstate(all="ignore"):
        bad = _ns_mutant(G, kind)
    err = np.linalg.norm(bad - t) / np.linalg.norm(t)
    assert not err < 1e-2, f"{kind} not caught (err {err})"


def test_planted_momentum_mistake_is_caught():
    rng = np.random.default_rng(8)
    s = (rng.standard_normal(10000) * 1e-3).astype(np.float32)
    e = rng.standard_normal(10000).astype(np.float32)
    t = torch.from_numpy(s).lerp(torch.from_numpy(e), 0.05).numpy()
    wrong = om.lerp(e, s, 0.05)  # start and end swapped
    assert not np.allclose(wrong, t, rtol=1e-3, atol=0)


def test_bf16_param_step_matches_torch_fp32_rounded():
    """bf16 parameter and gradient with an fp32 momentum: torch.optim.Muon in fp32
    on the bf16 values, the parameter rounded to bf16 after the step."""
    rng = np.random.default_rng(9)
    shape = (64, 96)
    p0 = bf16.round_bf16((rng.standard_normal(shape) * 0.02).astype(np.float32))
    g = bf16.round_bf16(rng.standard_normal(shape).astype(np.float32))
    m0 = (rng.standard_normal(shape) * 1e-3).astype(np.float32)
    tp = torch.nn.Parameter(torch.from_numpy(p0.copy()))
    opt = torch.optim.Muon([tp], lr=0.02, weight_decay=0.1, momentum=0.95, nesterov=True,
                           ns_coefficients=COEFFS, eps=1e-7, ns_steps=5, adjust_lr_fn="original")
    opt.state[tp]["momentum_buffer"] = torch.from_numpy(m0.copy())
    tp.grad = torch.from_numpy(g.copy())
    opt.step()
    t = tp.detach().bfloat16().float().numpy()
    op, om_, _ = om.muon_update(p0, g, m0, lr=0.02, weight_decay=0.1, beta=0.95, nesterov=True,
                                coeffs=COEFFS, ns_steps=5, eps=1e-7, param_bf16=True)
    assert np.array_equal(om_, opt.state[tp]["momentum_buffer"].numpy())
    assert np.array_equal(bf16.round_bf16(op), op)
    adj = om.adjust_lr(0.02, "original", shape)
    ulp = np.exp2(np.floor(np.log2(np.maximum(np.abs(t), 1e-30))) - 7)
    assert (np.abs(op - t) <= ulp + adj * 8e-3).all()
