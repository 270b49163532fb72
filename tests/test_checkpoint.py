"""Optimizer-state checkpoints and the torch.optim surface, on the CPU.

The reference's ``MuonAdamW.state_dict`` returns only the parameter lists
(optimizer.py:166-175) while its torch wrapper returns real state
(optimizer.py:248-260).  Here ``MuonAdamW.state_dict()`` carries the moments,
step and momentum in the wrapper's format (torch.optim.AdamW / torch.optim.Muon
state dicts), so checkpoints move between the two; ``param_groups`` make it a
``torch.optim.Optimizer`` that LR schedulers attach to.  No kernel runs here:
state is planted directly.  The GPU resume and cross-load tests are in
test_gpu_checkpoint.py.
"""

import copy

import pytest
import torch
import torch.nn as nn

from triton_muon_adamw import AdamConfig, MuonAdamW, MuonConfig, PyTorchMuonAdamW
from test_api import TinyLM


def _planted(seed=0, step=3):
    torch.manual_seed(seed)
    model = TinyLM()
    opt = MuonAdamW(model, MuonConfig(lr=0.02, weight_decay=0.05), AdamConfig(lr=3e-4, betas=(0.9, 0.95), eps=1e-8),
                    "auto")
    g = torch.Generator().manual_seed(seed + 1)
    for p in opt.adamw.model_params:
        opt.adamw.m[p].copy_(torch.randn(p.shape, generator=g) * 1e-3)
        opt.adamw.v[p].copy_(torch.rand(p.shape, generator=g) * 1e-6)
    for p in opt.muon.model_params:
        opt.muon.momentum[p].copy_(torch.randn(p.shape, generator=g) * 1e-3)
    opt.adamw.step_num = step
    return model, opt


def test_state_dict_layout_matches_torch_optim():
    model, opt = _planted()
    sd = opt.state_dict()
    a, m = sd["adam"], sd["muon"]
    ref = PyTorchMuonAdamW(model, MuonConfig(lr=0.02), AdamConfig(lr=3e-4)).state_dict()
    assert set(a["param_groups"][0]) == set(ref["adam"]["param_groups"][0])
    assert set(m["param_groups"][0]) == set(ref["muon"]["param_groups"][0])
    assert a["param_groups"][0]["params"] == list(range(len(opt.adamw.model_params)))
    for i, p in enumerate(opt.adamw.model_params):
        st = a["state"][i]
        assert float(st["step"]) == 3.0
        assert st["exp_avg"] is opt.adamw.m[p] and st["exp_avg_sq"] is opt.adamw.v[p]
    for i, p in enumerate(opt.muon.model_params):
        assert m["state"][i]["momentum_buffer"] is opt.muon.momentum[p]
    g = m["param_groups"][0]
    assert (g["lr"], g["momentum"], g["weight_decay"], g["nesterov"]) == (0.02, 0.95, 0.05, True)
    assert g["adjust_lr_fn"] is None  # "original", written as torch writes its default


def test_no_adamw_state_before_the_first_step():
    _, opt = _planted(step=0)
    assert opt.state_dict()["adam"]["state"] == {}


def test_roundtrip_through_the_torch_wrapper():
    model, opt = _planted()
    sd = copy.deepcopy(opt.state_dict())
    ref = PyTorchMuonAdamW(model, MuonConfig(lr=0.5), AdamConfig(lr=0.5))
    ref.load_state_dict(sd)
    # torch.optim holds the same state (and took the hyperparameters)
    for i, p in enumerate(opt.adamw.model_params):
        st = ref.adamw.state[p]
        assert torch.equal(st["exp_avg"], opt.adamw.m[p]) and torch.equal(st["exp_avg_sq"], opt.adamw.v[p])
        assert float(st["step"]) == 3.0
    for p in opt.muon.model_params:
        assert torch.equal(ref.muon.state[p]["momentum_buffer"], opt.muon.momentum[p])
    assert ref.adamw.param_groups[0]["lr"] == 3e-4 and ref.muon.param_groups[0]["lr"] == 0.02
    # and back into a fresh MuonAdamW
    fresh = MuonAdamW(model, MuonConfig(lr=1.0), AdamConfig(lr=1.0), "auto")
    fresh.load_state_dict(ref.state_dict())
    for p in opt.adamw.model_params:
        assert torch.equal(fresh.adamw.m[p], opt.adamw.m[p]) and torch.equal(fresh.adamw.v[p], opt.adamw.v[p])
    for p in opt.muon.model_params:
        assert torch.equal(fresh.muon.momentum[p], opt.muon.momentum[p])
    assert fresh.adamw.step_num == 3
    assert (fresh.adamw.lr, fresh.adamw.beta2, fresh.adamw.eps) == (3e-4, 0.95, 1e-8)
    assert (fresh.muon.lr, fresh.muon.weight_decay, fresh.muon.adjust_lr_fn) == (0.02, 0.05, "original")
    assert fresh.param_groups[0]["lr"] == 3e-4 and fresh.param_groups[1]["lr"] == 0.02


def test_load_copies_into_the_branch_buffers():
    model, opt = _planted()
    sd = copy.deepcopy(opt.state_dict())
    fresh = MuonAdamW(model, parameter_split="auto")
    bufs = {id(p): fresh.adamw.m[p] for p in fresh.adamw.model_params}
    fresh.load_state_dict(sd)
    assert all(fresh.adamw.m[p] is bufs[id(p)] for p in fresh.adamw.model_params)  # launch plans stay valid


def test_load_rejects_mismatches():
    model, opt = _planted()
    sd = copy.deepcopy(opt.state_dict())
    sd["adam"]["param_groups"][0]["params"] = sd["adam"]["param_groups"][0]["params"][:-1]
    with pytest.raises(ValueError, match="doesn't match the size"):
        opt.load_state_dict(sd)
    sd = copy.deepcopy(opt.state_dict())
    sd["adam"]["state"][0]["step"] = torch.tensor(7.0)
    with pytest.raises(ValueError, match="steps differ"):
        opt.load_state_dict(sd)
    sd = copy.deepcopy(opt.state_dict())
    sd["muon"]["param_groups"][0]["adjust_lr_fn"] = "nope"
    with pytest.raises(AssertionError, match="Invalid adjust_lr_fn"):
        opt.load_state_dict(sd)


def test_is_a_torch_optimizer_with_branch_groups():
    model, opt = _planted()
    assert isinstance(opt, torch.optim.Optimizer)
    ga, gm = opt.param_groups
    assert ga["name"] == "adam" and gm["name"] == "muon"
    assert ga["params"] is opt.adamw.model_params and gm["params"] is opt.muon.model_params
    assert ga["betas"] == (0.9, 0.95) and gm["ns_coefficients"] == (3.445, -4.775, 2.0315)


@pytest.mark.filterwarnings("ignore:Detected call of")
def test_lr_scheduler_drives_both_branches():
    model, opt = _planted()
    sched = torch.optim.lr_scheduler.LambdaLR(opt, lambda s: 0.5 ** s)
    for _ in range(3):
        sched.step()
    assert opt.param_groups[0]["lr"] == pytest.approx(3e-4 / 8) and opt.param_groups[1]["lr"] == pytest.approx(0.02 / 8)
    sd = opt.state_dict()  # pulls the scheduled values into the branches
    assert opt.adamw.lr == pytest.approx(3e-4 / 8) and opt.muon.lr == pytest.approx(0.02 / 8)
    assert sd["muon"]["param_groups"][0]["lr"] == pytest.approx(0.02 / 8)
    opt.param_groups[1]["weight_decay"] = 0.3
    opt.state_dict()
    assert opt.muon.weight_decay == 0.3


def test_zero_grad_modes():
    model, opt = _planted()
    for p in model.parameters():
        p.grad = torch.ones_like(p)
    opt.zero_grad()  # reference behaviour: zero-fill
    assert all(p.grad is not None and not p.grad.any() for p in model.parameters() if p.requires_grad)
    opt.zero_grad(set_to_none=True)
    assert all(p.grad is None for p in opt.adamw.model_params + opt.muon.model_params)
