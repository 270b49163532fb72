"""GPU parity of the AdamW kernels (gfx950) through the C ABI.

* bit-exact against the CPU oracle (oracle/adamw.py, an IEEE fp32 restatement
  of triton_adam.py:53-59) over ragged sizes, unaligned views and
  several steps;
* within the reference tolerance (atol 1e-4, rtol 1e-3; adam_benchmark.py:114)
  of fused torch.optim.AdamW on the config 2 workload;
* the reference's own end check (adam_benchmark.py:14-43,57-62,75-114): its
  LayerNorm MLP, gradients from one MSE backward pass, 10 x (100 + 500)
  static-gradient steps against torch.optim.AdamW (its default, foreach),
  every parameter within that tolerance.
"""

import numpy as np
import pytest
import torch

import oracle
from helpers import adamw_state, c2_sizes
from triton_muon_adamw.adamw import HipAdamW, solve_adamw_step

pytestmark = pytest.mark.gpu

HP = dict(lr=3e-4, betas=(0.9, 0.95), weight_decay=0.1, eps=1e-8)
RAGGED = [1, 3, 4, 5, 1000, 4095, 4096, 4097, 8191, 12288, 100003]


def _params(sizes, dev, seed=0):
    ps, gs, ms, vs = adamw_state(sizes, seed)
    return ps, gs, ms, vs


def test_adamw_multi_tensor_bitexact_vs_oracle(gpu):
    ps, gs, ms, vs = _params(RAGGED, gpu)
    # one parameter is a view 1 element into a buffer: not 16-byte aligned
    base = torch.zeros(5001)
    base[1:] = torch.randn(5000, generator=torch.Generator().manual_seed(7)) * 0.02
    params = [torch.nn.Parameter(p.to(gpu)) for p in ps]
    buf = base.to(gpu)
    params.append(torch.nn.Parameter(buf[1:]))
    opt = HipAdamW(params, **HP)
    ref = oracle.adamw.AdamWOracle([p.detach().cpu().numpy().copy() for p in params], **HP)
    gen = torch.Generator().manual_seed(3)
    for step in range(3):
        grads = [torch.randn(p.shape, generator=gen) * 1e-3 for p in params]
        for p, g in zip(params, grads):
            p.grad = g.to(gpu)
        opt.step()
        ref.step([g.numpy() for g in grads])
    torch.cuda.synchronize()
    for i, p in enumerate(params):
        got = p.detach().cpu().numpy()
        assert np.array_equal(got, ref.params[i]), f"tensor {i} (numel {p.numel()}) differs from oracle"
        assert np.array_equal(opt.m[p].cpu().numpy(), ref.m[i])
        assert np.array_equal(opt.v[p].cpu().numpy(), ref.v[i])


def test_adamw_tensor_beyond_2pow31_elements(gpu):
    """One tensor of 2^31 + 4097 elements (element offsets past 32 bits, a
    ragged tail): one step, bit-exact against the oracle on three slices of
    2^20 elements (the start, across element 2^31, and the end); the update
    is elementwise, so each slice is checked on its own."""
    n = (1 << 31) + 4097
    gen = torch.Generator(device=gpu).manual_seed(13)
    p = torch.nn.Parameter(torch.empty(n, device=gpu).normal_(0.0, 0.02, generator=gen))
    p.grad = torch.empty(n, device=gpu).normal_(0.0, 1e-3, generator=gen)
    opt = HipAdamW([p], **HP)
    opt.m[p].normal_(0.0, 1e-4, generator=gen)
    opt.v[p].normal_(0.0, 1e-6, generator=gen).abs_()
    w = 1 << 20
    cuts = [0, (1 << 31) - w // 2, n - w]
    before = [[t[c:c + w].cpu().numpy() for t in (p.detach(), p.grad, opt.m[p], opt.v[p])] for c in cuts]
    opt.step()
    torch.cuda.synchronize()
    b1, b2 = oracle.adamw.bias_corrections(*HP["betas"], 1)
    for c, (p0, g0, m0, v0) in zip(cuts, before):
        exp = oracle.adamw.adamw_update(p0, g0, m0, v0, lr=HP["lr"], bias1=b1, bias2=b2, beta1=HP["betas"][0],
                                        beta2=HP["betas"][1], weight_decay=HP["weight_decay"], eps=HP["eps"])
        for name, got, e in zip("pmv", (p.detach(), opt.m[p], opt.v[p]), exp):
            assert np.array_equal(got[c:c + w].cpu().numpy(), e), f"{name}[{c}:{c + w}] differs from the oracle"
    del p, opt
    torch.cuda.empty_cache()


def test_adamw_skips_none_grad_but_counts_step(gpu):
    p1 = torch.nn.Parameter(torch.randn(1000, device=gpu))
    p2 = torch.nn.Parameter(torch.randn(1000, device=gpu))
    before = p2.detach().clone()
    opt = HipAdamW([p1, p2], **HP)
    p1.grad = torch.randn(1000, device=gpu)
    opt.step()
    assert opt.step_num == 1
    assert torch.equal(p2.detach(), before)
    p2.grad = torch.randn(1000, device=gpu)
    opt.step()  # step 2 for both (one global counter, triton_adam.py:137)
    assert opt.step_num == 2


def test_adamw_parameter_listed_twice_updates_in_sequence(gpu):
    """A parameter listed k times is updated k times in sequence, each with the
    step's one bias correction, as the reference's per-parameter loop does
    (triton_adam.py:137-153; its state is keyed by the parameter): launch pass
    i takes every parameter's i-th occurrence.  Bit-exact against the oracle's
    update applied that many times, for a plain step and for a gradient-scaler
    step (its device counter advances once per step, not once per pass; a
    skipped step leaves everything and the counter as they were)."""
    ps, gs, ms, vs = _params([1000, 4097, 333], gpu, seed=9)
    a, b, c = (torch.nn.Parameter(p.to(gpu)) for p in ps)
    opt = HipAdamW([a, b, a, c, a], **HP)
    times = {0: 3, 1: 1, 2: 1}
    ref = [[p.numpy().copy(), np.zeros_like(p.numpy()), np.zeros_like(p.numpy())] for p in ps]
    for step in (1, 2, 3):
        for p, g in zip((a, b, c), gs):
            p.grad = (g * 4.0).to(gpu) if step > 1 else g.to(gpu)
        if step == 1:
            opt.step()
        else:
            found = torch.tensor(1.0 if step == 3 else 0.0, device=gpu)
            opt._step_amp(torch.tensor(4.0, device=gpu), found)
        if step == 3:
            continue
        b1, b2 = oracle.adamw.bias_corrections(0.9, 0.95, step)
        for i, r in enumerate(ref):
            for _ in range(times[i]):
                r[:] = oracle.adamw.adamw_update(*r[:1], gs[i].numpy(), *r[1:], lr=HP["lr"], bias1=b1, bias2=b2,
                                                 beta1=0.9, beta2=0.95, weight_decay=HP["weight_decay"],
                                                 eps=HP["eps"])
    torch.cuda.synchronize()
    assert opt.step_num == 2
    for p, r in zip((a, b, c), ref):
        assert np.array_equal(p.detach().cpu().numpy(), r[0])
        assert np.array_equal(opt.m[p].cpu().numpy(), r[1])
        assert np.array_equal(opt.v[p].cpu().numpy(), r[2])


def test_solve_adamw_step_bitexact(gpu):
    ps, gs, ms, vs = _params([4097 * 3], gpu, seed=5)
    p, g, m, v = (t[0].to(gpu) for t in (ps, gs, ms, vs))
    b1, b2 = oracle.adamw.bias_corrections(0.9, 0.95, 10)
    exp = oracle.adamw.adamw_update(ps[0].numpy(), gs[0].numpy(), ms[0].numpy(), vs[0].numpy(), lr=3e-4,
                                    bias1=b1, bias2=b2, beta1=0.9, beta2=0.95, weight_decay=0.1, eps=1e-8)
    solve_adamw_step(p, g, m, v, 3e-4, float(b1), float(b2), 0.9, 0.95, 0.1, 1e-8)
    torch.cuda.synchronize()
    for got, e in zip((p, m, v), exp):
        assert np.array_equal(got.cpu().numpy(), e)


def test_adamw_config2_vs_torch_fused(gpu):
    """Config 2: 256 tensors (2**26 elements), the 10th step, vs fused torch AdamW."""
    sizes = c2_sizes()
    assert sum(sizes) == 1 << 26
    ps, gs, ms, vs = adamw_state(sizes, seed=0)
    mine = [torch.nn.Parameter(p.to(gpu)) for p in ps]
    theirs = [torch.nn.Parameter(p.to(gpu)) for p in ps]
    opt = HipAdamW(mine, **HP)
    topt = torch.optim.AdamW(theirs, fused=True, **HP)
    for i in range(len(sizes)):
        g = gs[i].to(gpu)
        mine[i].grad = g
        theirs[i].grad = g.clone()
        opt.m[mine[i]].copy_(ms[i])
        opt.v[mine[i]].copy_(vs[i])
        topt.state[theirs[i]] = {"step": torch.tensor(9.0, device=gpu), "exp_avg": ms[i].to(gpu),
                                 "exp_avg_sq": vs[i].to(gpu)}
    opt.step_num = 9
    opt.step()
    topt.step()
    torch.cuda.synchronize()
    worst = 0.0
    for a, b in zip(mine, theirs):
        torch.testing.assert_close(a.detach(), b.detach(), atol=1e-4, rtol=1e-3)
        worst = max(worst, (a.detach() - b.detach()).abs().max().item())
    # the two formulas differ only in rounding: far inside the reference tolerance
    assert worst < 1e-7, worst


def test_adamw_mlp_long_horizon_against_torch(gpu):
    """The reference's AdamW benchmark model and end check: 6000 steps of this
    build's AdamW and of torch.optim.AdamW (foreach, as the reference runs it
    by default) on the same static gradients, then every parameter within
    atol = 1e-4, rtol = 1e-3 of torch's, and every parameter moved."""
    import copy

    import torch.nn as nn

    torch.manual_seed(6)
    model = nn.Sequential(nn.Linear(1024, 4096), nn.LayerNorm(4096), nn.ReLU(), nn.Linear(4096, 4096),
                          nn.LayerNorm(4096), nn.ReLU(), nn.Linear(4096, 4096), nn.LayerNorm(4096), nn.ReLU(),
                          nn.Linear(4096, 1024)).to(gpu)
    twin = copy.deepcopy(model)
    x = torch.randn(1000, 1024, device=gpu)
    y = torch.randn(1000, 1024, device=gpu)
    for m in (model, twin):
        torch.nn.functional.mse_loss(m(x), y).backward()
    start = [p.detach().clone() for p in model.parameters()]
    mine = HipAdamW(model.parameters(), betas=(0.9, 0.999), lr=1e-3, weight_decay=1e-4, eps=1e-8)
    ref = torch.optim.AdamW(twin.parameters(), lr=1e-3, betas=(0.9, 0.999), weight_decay=1e-4, eps=1e-8)
    for _ in range(10 * (100 + 500)):
        mine.step()
        ref.step()
    torch.cuda.synchronize()
    for (name, p), q, p0 in zip(model.named_parameters(), twin.parameters(), start):
        torch.testing.assert_close(p.detach(), q.detach(), atol=1e-4, rtol=1e-3, msg=name)
        assert not torch.equal(p.detach(), p0), name
