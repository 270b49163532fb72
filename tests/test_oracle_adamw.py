"""Pins the AdamW oracle (oracle/adamw.py) before it is trusted as a checker.

The reference holds no golden vectors for this path (its only checks are
runtime comparisons with torch.optim in the benchmark scripts), so the oracle
is pinned by:
* known answers: the first step from zero state, and a zero gradient;
* the library routine the reference compares against: fused torch.optim.AdamW
  (adam_benchmark.py:35-42, optimizer.py:220-227) over several steps;
* a float64 evaluation of the same formula;
* planted mistakes in a copy of the oracle, each of which must fail the pins.
"""

import numpy as np
import pytest
import torch

from oracle import adamw as oa

HP = dict(lr=3e-4, beta1=0.9, beta2=0.95, weight_decay=0.1, eps=1e-8)


def _rand(n, std, seed):
    return (np.random.default_rng(seed).standard_normal(n) * std).astype(np.float32)


def test_first_step_known_answer():
    # t = 1 from zero state: m_hat = g, v_hat = g^2, so p1 = p0 (1 - lr wd) - lr g / (|g| + eps).
    p, g = _rand(10000, 0.02, 0), _rand(10000, 1e-3, 1)
    b1, b2 = oa.bias_corrections(0.9, 0.95, 1)
    p1, m1, v1 = oa.adamw_update(p, g, np.zeros_like(p), np.zeros_like(p), bias1=b1, bias2=b2, **HP)
    pd = p.astype(np.float64) * (1 - 3e-4 * 0.1)
    expect = pd - 3e-4 * g / (np.abs(g.astype(np.float64)) + 1e-8)
    np.testing.assert_allclose(p1, expect, rtol=0, atol=2e-8)  # a few fp32 ulps of |p| ~ 0.02-0.1
    np.testing.assert_allclose(m1, 0.1 * g, rtol=1e-6)
    np.testing.assert_allclose(v1, 0.05 * g.astype(np.float64) ** 2, rtol=1e-6)


def test_zero_gradient_is_pure_decay():
    p = _rand(5000, 0.02, 2)
    z = np.zeros_like(p)
    b1, b2 = oa.bias_corrections(0.9, 0.95, 1)
    p1, m1, v1 = oa.adamw_update(p, z, z, z, bias1=b1, bias2=b2, **HP)
    assert np.array_equal(p1, (np.float32(1) - np.float32(3e-4) * np.float32(0.1)) * p)
    assert not m1.any() and not v1.any()


def _torch_fused_run(p0, grads, steps):
    tp = torch.nn.Parameter(torch.from_numpy(p0.copy()))
    opt = torch.optim.AdamW([tp], lr=3e-4, betas=(0.9, 0.95), weight_decay=0.1, eps=1e-8, fused=True)
    for g in grads[:steps]:
        tp.grad = torch.from_numpy(g.copy())
        opt.step()
    st = opt.state[tp]
    return tp.detach().numpy(), st["exp_avg"].numpy(), st["exp_avg_sq"].numpy()


def _oracle_run(p0, grads, steps, update=oa.adamw_update):
    p, m, v = p0.copy(), np.zeros_like(p0), np.zeros_like(p0)
    for t in range(1, steps + 1):
        b1, b2 = oa.bias_corrections(0.9, 0.95, t)
        p, m, v = update(p, grads[t - 1], m, v, bias1=b1, bias2=b2, **HP)
    return p, m, v


def test_matches_fused_torch_adamw_over_steps():
    p0 = _rand(200000, 0.02, 3)
    grads = [_rand(200000, 1e-3, 10 + i) for i in range(12)]
    tp, tm, tv = _torch_fused_run(p0, grads, 12)
    op, om, ov = _oracle_run(p0, grads, 12)
    np.testing.assert_allclose(op, tp, rtol=0, atol=1e-7)
    # torch forms m with a lerp, the reference as beta1*m + (1-beta1)*g: rounding-level differences
    np.testing.assert_allclose(om, tm, rtol=0, atol=1e-9)
    np.testing.assert_allclose(ov, tv, rtol=1e-6, atol=1e-16)


def test_matches_float64_formula():
    p, g = _rand(50000, 0.02, 4), _rand(50000, 1e-3, 5)
    m, v = _rand(50000, 1e-4, 6), np.abs(_rand(50000, 1e-6, 7))
    b1, b2 = oa.bias_corrections(0.9, 0.95, 10)
    p1, m1, v1 = oa.adamw_update(p, g, m, v, bias1=b1, bias2=b2, **HP)
    d = lambda x: np.asarray(x, np.float64)  # noqa: E731
    mt = 0.9 * d(m) + 0.1 * d(g)
    vt = 0.95 * d(v) + 0.05 * d(g) ** 2
    pe = (1 - 3e-5) * d(p) - 3e-4 * ((mt / d(b1)) / (np.sqrt(vt / d(b2)) + 1e-8))
    np.testing.assert_allclose(p1, pe, rtol=0, atol=2e-8)  # a few fp32 ulps


def test_step_counter_semantics():
    # One global step counter (triton_adam.py:137): a parameter whose grad was
    # None at step 1 uses the step-2 bias correction when it first updates.
    pa, pb = _rand(100, 0.02, 8), _rand(100, 0.02, 9)
    ga = _rand(100, 1e-3, 10)
    o = oa.AdamWOracle([pa.copy(), pb.copy()], lr=3e-4, betas=(0.9, 0.95), weight_decay=0.1, eps=1e-8)
    o.step([ga, None])
    assert np.array_equal(o.params[1], pb)
    o.step([ga, ga])
    b1, b2 = oa.bias_corrections(0.9, 0.95, 2)
    expect, _, _ = oa.adamw_update(pb, ga, np.zeros_like(pb), np.zeros_like(pb), bias1=b1, bias2=b2, **HP)
    assert np.array_equal(o.params[1], expect)


# --- planted mistakes: each must be caught by the torch comparison -----------

def _mutant(kind):
    def update(p, g, m, v, *, lr, bias1, bias2, beta1, beta2, weight_decay, eps):
        f = np.float32
        if kind == "no_decay":
            weight_decay = 0.0
        if kind == "swap_bias":
            bias1, bias2 = bias2, bias1
        if kind == "eps_inside_sqrt":
            m_t = f(beta1) * m + (f(1) - f(beta1)) * g
            v_t = f(beta2) * v + (f(1) - f(beta2)) * (g * g)
            p_new = (f(1) - f(lr) * f(weight_decay)) * p - f(lr) * ((m_t / f(bias1)) / np.sqrt(v_t / f(bias2) + f(eps)))
            return p_new, m_t, v_t
        p_new, m_t, v_t = oa.adamw_update(p, g, m, v, lr=lr, bias1=bias1, bias2=bias2, beta1=beta1,
                                          beta2=beta2, weight_decay=weight_decay, eps=eps)
        if kind == "sign":
            p_new = 2 * ((np.float32(1) - np.float32(lr) * np.float32(weight_decay)) * p) - p_new
        return p_new, m_t, v_t

    return update


@pytest.mark.parametrize("kind", ["no_decay", "swap_bias", "eps_inside_sqrt", "sign"])
def test_planted_mistakes_are_caught(kind):
    p0 = _rand(20000, 0.02, 11)
    grads = [_rand(20000, 1e-3, 20 + i) for i in range(5)]
    tp, _, _ = _torch_fused_run(p0, grads, 5)
    mp, _, _ = _oracle_run(p0, grads, 5, update=_mutant(kind))
    with pytest.raises(AssertionError):
        np.testing.assert_allclose(mp, tp, rtol=0, atol=1e-7)


# --- bf16 parameters / gradients (fp32 moments) --------------------------------

def _bf16(x):
    return torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).bfloat16().float().numpy()


def test_bf16_param_matches_torch_fp32_rounded_each_step():
    """The bf16 semantics (fp32 update and moments, parameter rounded to bf16 after
    every step) equal torch's fp32 AdamW with the parameter rounded each step."""
    p0 = _bf16(_rand(100000, 0.02, 21))
    grads = [_bf16(_rand(100000, 1e-3, 30 + i)) for i in range(6)]
    tp = torch.nn.Parameter(torch.from_numpy(p0.copy()))
    opt = torch.optim.AdamW([tp], lr=3e-4, betas=(0.9, 0.95), weight_decay=0.1, eps=1e-8, fused=True)
    o = oa.AdamWOracle([p0.copy()], lr=3e-4, betas=(0.9, 0.95), weight_decay=0.1, eps=1e-8, param_bf16=True)
    for g in grads:
        tp.grad = torch.from_numpy(g.copy())
        opt.step()
        with torch.no_grad():
            tp.copy_(tp.bfloat16().float())
        o.step([g])
    t = tp.detach().numpy()
    got = o.params[0]
    assert np.array_equal(_bf16(got), got)  # every value is a bf16
    ulp = np.exp2(np.floor(np.log2(np.maximum(np.abs(t), 1e-30))) - 7)
    assert (np.abs(got - t) <= ulp).all()
    assert (got == t).mean() > 0.999  # torch's fp32 rounding differs by ~1e-7: rare boundary flips only
    np.testing.assert_allclose(o.m[0], opt.state[tp]["exp_avg"].numpy(), rtol=0, atol=1e-9)


def test_bf16_planted_missing_rounding_is_caught():
    p0 = _bf16(_rand(20000, 0.02, 22))
    g = _bf16(_rand(20000, 1e-3, 23))
    b1, b2 = oa.bias_corrections(0.9, 0.95, 1)
    z = np.zeros_like(p0)
    good, _, _ = oa.adamw_update(p0, g, z, z, bias1=b1, bias2=b2, param_bf16=True, **HP)
    bad, _, _ = oa.adamw_update(p0, g, z, z, bias1=b1, bias2=b2, param_bf16=False, **HP)
    assert np.array_equal(_bf16(good), good)
    assert not np.array_equal(_bf16(bad), bad)  # an unrounded parameter is not a bf16 tensor
