"""Checkpoint/resume and the torch.optim surface on the GPU.

* Resume: k steps, ``state_dict()`` saved (deep copy, with the parameters);
  a fresh optimizer over fresh copies of those parameters, loaded, takes the
  next step bit for bit like the original.
* Cross-load: ``PyTorchMuonAdamW`` (the reference's torch wrapper,
  optimizer.py:178-260) runs k steps, its ``state_dict()`` goes into
  ``MuonAdamW``, and both take the next step: AdamW within 1e-6 absolute (the
  kernels match fused torch AdamW to that), the Muon update within the
  reference tolerance (relative Frobenius error 1e-2 on the update).
* An LR schedule attached to ``MuonAdamW`` gives the same parameters bit for
  bit as the same learning rates set by hand each step, and ``step(closure)``
  returns the closure's loss.
"""

import copy
import math

import pytest
import torch

from helpers import gpt2_layout
from triton_muon_adamw import AdamConfig, MuonAdamW, MuonConfig, PyTorchMuonAdamW

pytestmark = pytest.mark.gpu

MC = MuonConfig(lr=1e-3, beta=0.95, eps=1e-7, weight_decay=0.1, coeffs=(3.4445, -4.7750, 2.0315), nesterov=True,
                ns_steps=5)
AC = AdamConfig(lr=3e-4, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1)
LAYOUT = [(n, s, b) for n, s, b in gpt2_layout(n_layer=2) if not n.startswith("wte")]


def _params(dev, seed=0):
    gen = torch.Generator(device=dev).manual_seed(seed)
    return [(n, torch.nn.Parameter(torch.empty(s, device=dev).normal_(0.0, 0.02, generator=gen)), b)
            for n, s, b in LAYOUT]


def _split(named):
    return {"adam": [p for _, p, b in named if b == "adam"], "muon": [p for _, p, b in named if b == "muon"]}


def _grads(named, dev, gen):
    return [torch.empty(p.shape, device=dev).normal_(0.0, 1e-3, generator=gen) for _, p, _ in named]


def _set(named, grads):
    for (_, p, _), g in zip(named, grads):
        p.grad = g.clone()


def test_resume_is_bit_exact(gpu):
    named = _params(gpu)
    opt = MuonAdamW(_split(named), muon_config=MC, adam_config=AC, parameter_split="explicit")
    gen = torch.Generator(device=gpu).manual_seed(1)
    for _ in range(2):
        _set(named, _grads(named, gpu, gen))
        opt.step()
    torch.cuda.synchronize()
    saved_params = [p.detach().clone() for _, p, _ in named]
    saved = copy.deepcopy(opt.state_dict())
    last = _grads(named, gpu, gen)
    _set(named, last)
    opt.step()
    torch.cuda.synchronize()

    fresh = [(n, torch.nn.Parameter(w.clone()), b) for (n, _, b), w in zip(named, saved_params)]
    opt2 = MuonAdamW(_split(fresh), muon_config=MuonConfig(lr=0.5), adam_config=AdamConfig(lr=0.5),
                     parameter_split="explicit")
    opt2.load_state_dict(saved)
    _set(fresh, last)
    opt2.step()
    torch.cuda.synchronize()
    for (n, p, _), (_, q, _) in zip(named, fresh):
        assert torch.equal(p.detach(), q.detach()), n
    assert opt2.adamw.step_num == 3


def test_torch_wrapper_state_loads_into_muonadamw(gpu):
    theirs = _params(gpu)
    ref = PyTorchMuonAdamW(_split(theirs), muon_config=MC, adam_config=AC, parameter_split="explicit")
    gen = torch.Generator(device=gpu).manual_seed(2)
    for _ in range(2):
        _set(theirs, _grads(theirs, gpu, gen))
        ref.step()
    torch.cuda.synchronize()
    mine = [(n, torch.nn.Parameter(p.detach().clone()), b) for n, p, b in theirs]
    opt = MuonAdamW(_split(mine), muon_config=MuonConfig(lr=0.5), adam_config=AdamConfig(lr=0.5),
                    parameter_split="explicit")
    opt.load_state_dict(ref.state_dict())
    before = [p.detach().clone() for _, p, _ in mine]
    g = _grads(mine, gpu, gen)
    _set(mine, g)
    _set(theirs, g)
    opt.step()
    ref.step()
    torch.cuda.synchronize()
    keep = 1 - MC.lr * MC.weight_decay
    for (n, p, b), (_, q, _), p0 in zip(mine, theirs, before):
        if b == "adam":
            torch.testing.assert_close(p.detach(), q.detach(), atol=1e-6, rtol=0)
        else:
            adj = MC.lr * math.sqrt(max(1.0, p.shape[0] / p.shape[1]))
            u_mine = (p0.double() * keep - p.detach().double()) / adj
            u_ref = (p0.double() * keep - q.detach().double()) / adj
            assert ((u_mine - u_ref).norm() / u_ref.norm()).item() <= 1e-2, n


@pytest.mark.filterwarnings("ignore:Detected call of")
def test_lr_schedule_matches_manual_rates(gpu):
    a, b = _params(gpu), _params(gpu)
    opt_a = MuonAdamW(_split(a), muon_config=MC, adam_config=AC, parameter_split="explicit")
    opt_b = MuonAdamW(_split(b), muon_config=MC, adam_config=AC, parameter_split="explicit")
    sched = torch.optim.lr_scheduler.LambdaLR(opt_a, lambda s: 0.5 ** s)
    gen = torch.Generator(device=gpu).manual_seed(3)
    for k in range(3):
        g = _grads(a, gpu, gen)
        _set(a, g)
        _set(b, g)
        opt_a.step()
        sched.step()
        opt_b.adamw.lr, opt_b.muon.lr = AC.lr * 0.5 ** k, MC.lr * 0.5 ** k
        opt_b.param_groups[0]["lr"], opt_b.param_groups[1]["lr"] = opt_b.adamw.lr, opt_b.muon.lr
        opt_b.step()
    torch.cuda.synchronize()
    for (n, p, _), (_, q, _) in zip(a, b):
        assert torch.equal(p.detach(), q.detach()), n


def test_step_closure_returns_loss(gpu):
    named = _params(gpu)
    opt = MuonAdamW(_split(named), muon_config=MC, adam_config=AC, parameter_split="explicit")
    w = next(p for _, p, b in named if b == "muon")

    def closure():
        opt.zero_grad(set_to_none=True)
        loss = (w.float() ** 2).sum()
        loss.backward()
        return loss

    before = w.detach().clone()
    loss = opt.step(closure)
    torch.cuda.synchronize()
    assert torch.is_tensor(loss) and loss.item() > 0
    assert not torch.equal(before, w.detach())  # only w has a gradient; it moved


def _state(opt):
    return ([opt.adamw.m[p] for p in opt.adamw.model_params] + [opt.adamw.v[p] for p in opt.adamw.model_params]
            + [opt.muon.momentum[p] for p in opt.muon.model_params])


def test_grad_scaler_unscales_and_skips_inf_steps(gpu):
    """torch.amp.GradScaler drives MuonAdamW through its device-side path
    (grad_scale / found_inf handed to step()): gradients are divided by the
    scale in the kernels (power-of-two scale: exact); a step with a non-finite
    gradient is skipped entirely on the device (parameters, moments, momentum
    and the AdamW step counter untouched), as torch's fused AdamW does; the
    next step's bias corrections come from the device counter."""
    a, b = _params(gpu), _params(gpu)
    opt_a = MuonAdamW(_split(a), muon_config=MC, adam_config=AC, parameter_split="explicit")
    opt_b = MuonAdamW(_split(b), muon_config=MC, adam_config=AC, parameter_split="explicit")
    scaler = torch.amp.GradScaler("cuda", init_scale=1024.0, growth_interval=1000)
    scaler.scale(torch.ones((), device=gpu))  # initialise the scale on the device
    gen = torch.Generator(device=gpu).manual_seed(4)
    g = _grads(a, gpu, gen)
    for (_, p, _), gi in zip(a, g):
        p.grad = gi * 1024.0
    _set(b, g)
    scaler.step(opt_a)
    scaler.update()
    opt_b.step()
    torch.cuda.synchronize()
    assert opt_a.adamw._dev_steps, "the scaler did not take the device-side path"
    for (n, p, _), (_, q, _) in zip(a, b):
        assert torch.equal(p.detach(), q.detach()), n
    before = [p.detach().clone() for _, p, _ in a]
    g = _grads(a, gpu, gen)
    g[0][0] = float("inf")
    for (_, p, _), gi in zip(a, g):
        p.grad = gi * scaler.get_scale()
    state_before = [t.clone() for t in _state(opt_a)]
    scaler.step(opt_a)
    scaler.update()
    torch.cuda.synchronize()
    assert all(torch.equal(p.detach(), q) for (_, p, _), q in zip(a, before))
    assert all(torch.equal(t, u) for t, u in zip(_state(opt_a), state_before))
    assert opt_a.adamw.step_num == 1 and scaler.get_scale() == 512.0
    # a finite step after the skipped one: step 2 on both sides
    g = _grads(a, gpu, gen)
    for (_, p, _), gi in zip(a, g):
        p.grad = gi * 512.0
    _set(b, g)
    scaler.step(opt_a)
    scaler.update()
    opt_b.step()
    torch.cuda.synchronize()
    for (n, p, _), (_, q, _) in zip(a, b):
        assert torch.equal(p.detach(), q.detach()), n
    assert all(torch.equal(t, u) for t, u in zip(_state(opt_a), _state(opt_b)))
    assert opt_a.adamw.step_num == 2 and opt_b.adamw.step_num == 2


def test_grad_scaler_after_explicit_unscale(gpu):
    """scaler.unscale_(opt) before scaler.step(opt) (e.g. to clip gradients):
    the scaler then hands over found_inf only; the result equals a plain step
    on the unscaled gradients, and a non-finite step is still skipped."""
    a, b = _params(gpu), _params(gpu)
    opt_a = MuonAdamW(_split(a), muon_config=MC, adam_config=AC, parameter_split="explicit")
    opt_b = MuonAdamW(_split(b), muon_config=MC, adam_config=AC, parameter_split="explicit")
    scaler = torch.amp.GradScaler("cuda", init_scale=256.0, growth_interval=1000)
    scaler.scale(torch.ones((), device=gpu))  # initialise the scale on the device
    gen = torch.Generator(device=gpu).manual_seed(6)
    for it in range(3):
        g = _grads(a, gpu, gen)
        if it == 1:
            g[-1][0] = float("nan")
        scale = scaler.get_scale()
        for (_, p, _), gi in zip(a, g):
            p.grad = gi * scale
        scaler.unscale_(opt_a)
        scaler.step(opt_a)
        scaler.update()
        if it != 1:
            _set(b, g)
            opt_b.step()
    torch.cuda.synchronize()
    for (n, p, _), (_, q, _) in zip(a, b):
        assert torch.equal(p.detach(), q.detach()), n
    assert all(torch.equal(t, u) for t, u in zip(_state(opt_a), _state(opt_b)))
    assert opt_a.adamw.step_num == 2


@pytest.mark.filterwarnings("ignore:Synchronization debug mode is a prototype")
def test_steps_do_not_synchronise(gpu):
    """The device-side GradScaler path reads nothing back to the host: with
    torch's sync debug mode set to "error", scaler.step / scaler.update raise
    on a synchronising call (after a warm-up step that builds the plans).  The
    gradients are new tensors every step, so the AdamW table is rebuilt and
    uploaded each time, as under zero_grad(set_to_none=True).  (torch documents
    the mode as a prototype that does not catch every synchronising call.)"""
    a = _params(gpu)
    opt = MuonAdamW(_split(a), muon_config=MC, adam_config=AC, parameter_split="explicit")
    scaler = torch.amp.GradScaler("cuda", init_scale=1024.0, growth_interval=1000)
    scaler.scale(torch.ones((), device=gpu))
    gen = torch.Generator(device=gpu).manual_seed(8)

    def one_step():
        for (_, p, _), gi in zip(a, _grads(a, gpu, gen)):
            p.grad = gi * 1024.0
        scaler.step(opt)
        scaler.update()

    def plain_step():
        for (_, p, _), gi in zip(a, _grads(a, gpu, gen)):
            p.grad = gi
        opt.step()

    one_step()
    torch.cuda.synchronize()
    torch.cuda.set_sync_debug_mode("error")
    try:
        for _ in range(2):
            one_step()
    finally:
        torch.cuda.set_sync_debug_mode("default")
    torch.cuda.synchronize()
    assert opt.adamw.step_num == 3
    # the plain step (no scaler) does not synchronise either
    plain_step()
    torch.cuda.synchronize()
    torch.cuda.set_sync_debug_mode("error")
    try:
        for _ in range(2):
            plain_step()
    finally:
        torch.cuda.set_sync_debug_mode("default")
    torch.cuda.synchronize()
    assert opt.adamw.step_num == 6


@pytest.mark.parametrize("in_order", [True, False])
def test_steps_under_a_side_stream(gpu, in_order):
    """Steps taken with a side stream current (every other step), with new
    gradient tensors each step so that the AdamW table is re-packed and the
    launch groups rebuilt while earlier launches may still be queued, give the
    same parameters bit for bit as steps on the default stream.  ``in_order``
    runs the Muon shape classes in order on the caller's stream (the path of
    large steps) instead of on forked side streams."""
    a, b = _params(gpu), _params(gpu)
    opt_a = MuonAdamW(_split(a), muon_config=MC, adam_config=AC, parameter_split="explicit")
    opt_b = MuonAdamW(_split(b), muon_config=MC, adam_config=AC, parameter_split="explicit")
    if in_order:
        opt_a.muon.concurrent_flops_limit = opt_b.muon.concurrent_flops_limit = 0.0
    gen = torch.Generator(device=gpu).manual_seed(12)
    side = torch.cuda.Stream(device=gpu)
    main = torch.cuda.current_stream(gpu)
    for k in range(4):
        grads = _grads(a, gpu, gen)
        _set(a, grads)
        _set(b, grads)
        opt_a.step()
        if k % 2:
            side.wait_stream(main)
            with torch.cuda.stream(side):
                opt_b.step()
            main.wait_stream(side)
        else:
            opt_b.step()
        del grads
    torch.cuda.synchronize()
    assert opt_b.muon._concurrent is not in_order
    for (n, p, _), (_, q, _) in zip(a, b):
        assert torch.equal(p, q), n


@pytest.mark.parametrize("in_order", [True, False])
def test_graph_captured_step_replays_like_eager_steps(gpu, in_order):
    """``capturable=True``: one eager step, then a step captured with
    ``torch.cuda.graph`` and replayed three times (new gradients copied into the
    static ``.grad`` tensors before each replay, eager steps of a twin
    optimizer and a synchronisation between replays) gives the parameters,
    moments and momentum of four eager steps bit for bit, each replay checked;
    the device step counter reads 4.  ``in_order``: Muon shape classes in
    order on the capture stream, else forked onto side streams inside the
    graph."""
    a, b = _params(gpu), _params(gpu)
    opt_a = MuonAdamW(_split(a), muon_config=MC, adam_config=AC, parameter_split="explicit", capturable=True)
    opt_b = MuonAdamW(_split(b), muon_config=MC, adam_config=AC, parameter_split="explicit")
    if in_order:
        opt_a.muon.concurrent_flops_limit = opt_b.muon.concurrent_flops_limit = 0.0
    gen = torch.Generator(device=gpu).manual_seed(13)
    grads = _grads(a, gpu, gen)
    _set(a, grads)
    _set(b, grads)
    opt_a.step()
    opt_b.step()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        opt_a.step()
    assert opt_a.param_groups[0]["params"][0].grad is not None
    for k in range(3):
        grads = _grads(a, gpu, gen)
        for (_, p, _), g in zip(a, grads):
            p.grad.copy_(g)
        graph.replay()
        _set(b, grads)
        opt_b.step()
        torch.cuda.synchronize()
        for (n, p, _), (_, q, _) in zip(a, b):
            assert torch.equal(p, q), (k, n)
    assert opt_b.muon._concurrent is not in_order
    for (n, p, br), (_, q, _) in zip(a, b):
        if br == "adam":
            assert torch.equal(opt_a.adamw.m[p], opt_b.adamw.m[q]) and torch.equal(opt_a.adamw.v[p], opt_b.adamw.v[q]), n
        else:
            assert torch.equal(opt_a.muon.momentum[p], opt_b.muon.momentum[q]), n
    assert opt_a.adamw.step_num == 4 and opt_b.adamw.step_num == 4
    assert opt_a.adamw.state_dict()["param_groups"][0]["capturable"] is True


@pytest.mark.filterwarnings("ignore:The CUDA Graph is empty")
def test_capture_refuses_a_plan_change(gpu):
    """A step whose launch plan would be built during capture (no eager step
    yet) raises instead of recording pointers that a replay could not keep."""
    a = _params(gpu)
    opt = MuonAdamW(_split(a), muon_config=MC, adam_config=AC, parameter_split="explicit", capturable=True)
    _set(a, _grads(a, gpu, torch.Generator(device=gpu).manual_seed(14)))
    graph = torch.cuda.CUDAGraph()
    with pytest.raises(RuntimeError, match="during graph capture"):
        with torch.cuda.graph(graph):
            opt.step()
    torch.cuda.synchronize()
    opt.step()  # eager steps still work after the failed capture
    torch.cuda.synchronize()
    assert opt.adamw.step_num == 1


def test_launch_plan_follows_the_parameters_layout(gpu):
    """The cached launch plan is keyed by each parameter's and gradient's
    address, type, shape and strides: a parameter whose ``.data`` becomes a
    view starting at the same address (fewer rows, or every other row) is
    checked again at the next step and rejected (its optimizer state no longer
    matches; a strided view is not contiguous) before anything launches, with
    the AdamW step counter unchanged.  Restoring the original tensor steps
    again."""
    p = torch.nn.Parameter(torch.randn(512, 256, device=gpu) * 0.02)
    w = torch.nn.Parameter(torch.randn(512, 256, device=gpu) * 0.02)
    opt = MuonAdamW({"adam": [p], "muon": [w]}, muon_config=MC, adam_config=AC, parameter_split="explicit")
    full_p, full_w = p.data, w.data
    for q in (p, w):
        q.grad = torch.randn_like(q) * 1e-3
    opt.step()
    torch.cuda.synchronize()
    for view, err in ((lambda t: t[:256], "shape"), (lambda t: t[::2], "contiguous")):
        for q, full in ((p, full_p), (w, full_w)):
            q.data = view(full)
            q.grad = torch.randn_like(q) * 1e-3
            assert q.data_ptr() == full.data_ptr()
            with pytest.raises(ValueError, match=err):
                opt.step()
            assert opt.adamw.step_num == 1
            q.data = full
            q.grad = torch.randn_like(q) * 1e-3
    opt.step()
    torch.cuda.synchronize()
    assert opt.adamw.step_num == 2


def test_parameter_appended_to_a_branch_steps_from_zero_state(gpu):
    """A parameter appended to a branch's list after some steps takes part from
    the next step on, from zero state: the Muon matrix equals a fresh
    single-matrix optimizer's first step bit for bit; the AdamW vector gets
    the global step counter's bias corrections (step 2, triton_adam.py:137),
    bit-exact against the oracle from zero moments."""
    import numpy as np

    import oracle
    from triton_muon_adamw.muon import HipMuon

    p = torch.nn.Parameter(torch.randn(300, device=gpu) * 0.02)
    w = torch.nn.Parameter(torch.randn(256, 512, device=gpu) * 0.02)
    opt = MuonAdamW({"adam": [p], "muon": [w]}, muon_config=MC, adam_config=AC, parameter_split="explicit")
    p.grad, w.grad = torch.randn_like(p) * 1e-3, torch.randn_like(w) * 1e-3
    opt.step()
    q = torch.nn.Parameter(torch.randn(1000, device=gpu) * 0.02)
    u = torch.nn.Parameter(torch.randn(512, 384, device=gpu) * 0.02)
    q0, u0 = q.detach().clone(), u.detach().clone()
    opt.param_group["adam"].append(q)
    opt.param_group["muon"].append(u)
    for t in (p, w, q, u):
        t.grad = torch.randn_like(t) * 1e-3
    opt.step()
    torch.cuda.synchronize()
    v = torch.nn.Parameter(u0.clone())
    v.grad = u.grad.clone()
    twin = HipMuon([v], lr=MC.lr, weight_decay=MC.weight_decay, coeffs=MC.coeffs, nesterov=MC.nesterov,
                   beta=MC.beta, ns_steps=MC.ns_steps, eps=MC.eps)
    twin.step()
    torch.cuda.synchronize()
    assert torch.equal(u.detach(), v.detach())
    b1, b2 = oracle.adamw.bias_corrections(AC.betas[0], AC.betas[1], 2)
    zero = np.zeros(1000, np.float32)
    exp = oracle.adamw.adamw_update(q0.cpu().numpy(), q.grad.cpu().numpy(), zero, zero, lr=AC.lr, bias1=b1,
                                    bias2=b2, beta1=AC.betas[0], beta2=AC.betas[1],
                                    weight_decay=AC.weight_decay, eps=AC.eps)
    assert np.array_equal(q.detach().cpu().numpy(), exp[0])
    assert opt.adamw.step_num == 2


def test_load_state_dict_keeps_the_captured_step_counter(gpu):
    """``capturable=True``: loading a checkpoint after a step was captured
    writes the loaded step into the device counter the graph advances (the
    tensor is kept, not replaced), so replays after the load follow the loaded
    step: bit for bit equal to an eager twin loaded from the same checkpoint,
    and ``step_num`` reads the loaded step plus the replays."""
    a, b = _params(gpu), _params(gpu)
    opt_a = MuonAdamW(_split(a), muon_config=MC, adam_config=AC, parameter_split="explicit", capturable=True)
    opt_b = MuonAdamW(_split(b), muon_config=MC, adam_config=AC, parameter_split="explicit")
    opt_a.muon.concurrent_flops_limit = opt_b.muon.concurrent_flops_limit = 0.0
    gen = torch.Generator(device=gpu).manual_seed(21)
    grads = _grads(a, gpu, gen)
    _set(a, grads)
    _set(b, grads)
    opt_a.step()
    opt_b.step()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        opt_a.step()

    def replay_both(grads):
        for (_, p, _), g in zip(a, grads):
            p.grad.copy_(g)
        graph.replay()
        _set(b, grads)
        opt_b.step()
        torch.cuda.synchronize()

    replay_both(_grads(a, gpu, gen))  # step 2 on both
    saved = copy.deepcopy(opt_b.state_dict())
    saved_params = [p.detach().clone() for _, p, _ in b]
    for _ in range(2):  # steps 3 and 4
        replay_both(_grads(a, gpu, gen))
    assert opt_a.adamw.step_num == 4
    with torch.no_grad():
        for named in (a, b):
            for (_, p, _), s in zip(named, saved_params):
                p.copy_(s)
    opt_a.load_state_dict(copy.deepcopy(saved))
    opt_b.load_state_dict(copy.deepcopy(saved))
    assert opt_a.adamw.step_num == 2
    for k in range(2):  # steps 3 and 4 again, from the checkpoint
        replay_both(_grads(a, gpu, gen))
        for (n, p, _), (_, q, _) in zip(a, b):
            assert torch.equal(p, q), (k, n)
    assert opt_a.adamw.step_num == 4 and opt_b.adamw.step_num == 4
