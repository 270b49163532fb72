"""GPU parity under the reference's own protocols and its non-default options.

* Long horizon (muon_adamw_benchmark.py:99-134): the reference steps its
  hybrid optimizer and the torch wrapper many times on static gradients and
  then compares every parameter at atol = rtol = 1e-2.  Here: the
  GPT-2-124M-shaped set (config 4), 750 static-gradient steps (that script's
  five 50 + 100 loops), this build against ``PyTorchMuonAdamW`` on the GPU.
* The reference's hybrid benchmark end check on its own model and configs
  (muon_adamw_benchmark.py:9-65,128-134), 750 static-gradient steps.
* The reference's Muon benchmark end check (muon_benchmark.py:95-101): its
  five-layer model, 750 static-gradient steps of this build's Muon against
  ``torch.optim.Muon``, every parameter at atol = rtol = 1e-2.
* ``parameter_split="auto"`` (optimizer.py:117-130, the reference's default)
  on an HF-style module: ``get_input_embeddings`` / ``get_output_embeddings``,
  a head tied to the embedding (deduplicated by ``data_ptr``), a frozen
  weight (skipped), a 2-D position embedding that goes to Muon; real
  backward passes; three steps against ``PyTorchMuonAdamW(..., "auto")``.
* ``adjust_lr_fn`` (triton_muon.py:424-431): ``"match_rms_adamw"`` against
  ``torch.optim.Muon`` with the same option; ``"spectral_unclamped"`` (which
  torch does not have) against the CPU oracle.
* Mixed precision and LR schedules against torch: ``torch.amp.GradScaler``
  driving this build (its device-side path) and, beside it, fused torch
  AdamW + torch Muon (the scaler's unscale/skip path), with a non-finite step
  that both skip; a ``LambdaLR`` schedule on this build and the same schedule
  on the two torch optimizers.  AdamW parameters within 1e-6, every Muon
  update within the reference tolerance of torch's (relative Frobenius error
  <= 1e-2), step counters equal.
"""

import copy
import math

import numpy as np
import pytest
import torch
import torch.nn as nn

import oracle
from helpers import gpt2_layout, rel_fro
from triton_muon_adamw import AdamConfig, MuonAdamW, MuonConfig, PyTorchMuonAdamW
from triton_muon_adamw.muon import HipMuon

pytestmark = pytest.mark.gpu

COEFFS = (3.4445, -4.7750, 2.0315)
AC = AdamConfig(lr=3e-4, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1)


def _mc(**kw):
    base = dict(lr=1e-3, beta=0.95, eps=1e-7, weight_decay=0.1, coeffs=COEFFS, nesterov=True, ns_steps=5)
    base.update(kw)
    return MuonConfig(**base)


def _split(named):
    return {"adam": [p for _, p, b in named if b == "adam"], "muon": [p for _, p, b in named if b == "muon"]}


def test_gpt2_long_horizon_static_gradients(gpu):
    """750 steps on one fixed set of gradients (the reference's five rounds of
    50 warm-up + 100 timed steps, muon_adamw_benchmark.py:99-124), then every
    parameter within atol = rtol = 1e-2 of the torch wrapper's (its end check,
    :128-134), AdamW parameters within 1e-5."""
    mc = _mc()
    gen = torch.Generator(device=gpu).manual_seed(3)
    mine, theirs = [], []
    for name, shape, branch in gpt2_layout():
        w = torch.empty(shape, device=gpu).normal_(0.0, 0.02, generator=gen)
        g = torch.empty(shape, device=gpu).normal_(0.0, 1e-3, generator=gen)
        p, q = nn.Parameter(w.clone()), nn.Parameter(w.clone())
        p.grad, q.grad = g.clone(), g.clone()
        mine.append((name, p, branch))
        theirs.append((name, q, branch))
    start = [p.detach().clone() for _, p, _ in mine]
    opt = MuonAdamW(_split(mine), muon_config=mc, adam_config=AC, parameter_split="explicit")
    ref = PyTorchMuonAdamW(_split(theirs), muon_config=mc, adam_config=AC, parameter_split="explicit")
    for _ in range(5 * (50 + 100)):
        opt.step()
        ref.step()
    torch.cuda.synchronize()
    for (name, p, b), (_, q, _), p0 in zip(mine, theirs, start):
        assert torch.isfinite(p).all(), name
        torch.testing.assert_close(p.detach(), q.detach(), atol=1e-2, rtol=1e-2, msg=name)
        if b == "adam":
            torch.testing.assert_close(p.detach(), q.detach(), atol=1e-5, rtol=0, msg=name)
        else:
            # not vacuous: each matrix moved (relative Frobenius) at least 20x more
            # than it differs from the torch wrapper's
            moved = ((p.detach() - p0).norm() / p0.norm()).item()
            diff = ((p.detach() - q.detach()).norm() / p0.norm()).item()
            assert moved > 20 * diff, (name, moved, diff)


def test_hybrid_mlp_long_horizon_against_torch_wrapper(gpu):
    """The reference's hybrid benchmark itself (muon_adamw_benchmark.py:9-65,
    84-134): its LayerNorm MLP and configs, 2-D weights to Muon and the rest to
    AdamW, gradients from one MSE backward pass, 5 x (50 + 100) steps of this
    build and of PyTorchMuonAdamW; every parameter within atol = rtol = 1e-2,
    the AdamW ones within the AdamW tolerance (atol 1e-4, rtol 1e-3,
    adam_benchmark.py:114), and each Muon matrix moved at least 20x more than
    it differs from the wrapper's."""
    torch.manual_seed(4)
    model = nn.Sequential(nn.Linear(1024, 2048), nn.LayerNorm(2048), nn.ReLU(), nn.Linear(2048, 4096),
                          nn.LayerNorm(4096), nn.ReLU(), nn.Linear(4096, 4096), nn.LayerNorm(4096), nn.ReLU(),
                          nn.Linear(4096, 1024)).to(gpu)
    twin = copy.deepcopy(model)
    x = torch.randn(1000, 1024, device=gpu)
    y = torch.randn(1000, 1024, device=gpu)
    for m in (model, twin):
        torch.nn.functional.mse_loss(m(x), y).backward()
    ac = AdamConfig(lr=1e-3, betas=(0.9, 0.999), eps=1e-7, weight_decay=0.01)
    mc = MuonConfig(lr=1e-3, beta=0.95, eps=1e-7, weight_decay=0.1, coeffs=(3.445, -4.775, 2.0315), nesterov=True,
                    ns_steps=5, adjust_lr_fn="original")

    def split(m):
        ps = [p for p in m.parameters() if p.requires_grad]
        return {"adam": [p for p in ps if p.ndim != 2], "muon": [p for p in ps if p.ndim == 2]}

    start = [p.detach().clone() for p in model.parameters()]
    mine = MuonAdamW(split(model), muon_config=mc, adam_config=ac, parameter_split="explicit")
    ref = PyTorchMuonAdamW(split(twin), muon_config=mc, adam_config=ac, parameter_split="explicit")
    for _ in range(5 * (50 + 100)):
        mine.step()
        ref.step()
    torch.cuda.synchronize()
    for (name, p), q, p0 in zip(model.named_parameters(), twin.parameters(), start):
        torch.testing.assert_close(p.detach(), q.detach(), atol=1e-2, rtol=1e-2, msg=name)
        if p.ndim != 2:
            torch.testing.assert_close(p.detach(), q.detach(), atol=1e-4, rtol=1e-3, msg=name)
        else:
            moved = ((p.detach() - p0).norm() / p0.norm()).item()
            diff = ((p.detach() - q.detach()).norm() / p0.norm()).item()
            assert moved > 20 * diff, (name, moved, diff)


def test_muon_mlp_long_horizon_against_torch_muon(gpu):
    """The reference's Muon benchmark end check (muon_benchmark.py:14-35,
    50-60, 95-101): five bias-free linear layers, gradients from one MSE
    backward pass on random data, then 5 x (50 + 100) steps of this build's
    Muon and of torch.optim.Muon with the reference's settings; every
    parameter within atol = rtol = 1e-2, and each matrix moved at least 20x
    more than it differs from torch's."""
    torch.manual_seed(5)
    model = nn.Sequential(nn.Linear(1024, 2048, bias=False), nn.ReLU(), nn.Linear(2048, 4096, bias=False),
                          nn.ReLU(), nn.Linear(4096, 4096, bias=False), nn.ReLU(),
                          nn.Linear(4096, 4096, bias=False), nn.ReLU(), nn.Linear(4096, 1024, bias=False)).to(gpu)
    twin = copy.deepcopy(model)
    x = torch.randn(1000, 1024, device=gpu)
    y = torch.randn(1000, 1024, device=gpu)
    for m in (model, twin):
        torch.nn.functional.mse_loss(m(x), y).backward()
    start = [p.detach().clone() for p in model.parameters()]
    mine = HipMuon(model.parameters(), coeffs=(3.4445, -4.775, 2.0315), beta=0.95, lr=1e-3, weight_decay=0.1,
                   ns_steps=5)
    ref = torch.optim.Muon(twin.parameters(), lr=1e-3, momentum=0.95, nesterov=True, ns_steps=5)
    for _ in range(5 * (50 + 100)):
        mine.step()
        ref.step()
    torch.cuda.synchronize()
    for (name, p), q, p0 in zip(model.named_parameters(), twin.parameters(), start):
        torch.testing.assert_close(p.detach(), q.detach(), atol=1e-2, rtol=1e-2, msg=name)
        moved = ((p.detach() - p0).norm() / p0.norm()).item()
        diff = ((p.detach() - q.detach()).norm() / p0.norm()).item()
        assert moved > 20 * diff, (name, moved, diff)


class _TinyLM(nn.Module):
    """A GPT-style module with the HF accessors ``auto`` routing uses."""

    def __init__(self, vocab=1000, d=256, n_ctx=128, n_layer=2):
        super().__init__()
        self.wte = nn.Embedding(vocab, d)
        self.wpe = nn.Embedding(n_ctx, d)
        self.blocks = nn.ModuleList()
        for _ in range(n_layer):
            self.blocks.append(nn.ModuleDict({
                "ln": nn.LayerNorm(d), "fc": nn.Linear(d, 4 * d), "proj": nn.Linear(4 * d, d),
                "attn": nn.Linear(d, 3 * d), "out": nn.Linear(d, d)}))
        self.frozen = nn.Linear(d, d)
        self.frozen.weight.requires_grad_(False)
        self.ln_f = nn.LayerNorm(d)
        self.lm_head = nn.Linear(d, vocab, bias=False)
        self.lm_head.weight = self.wte.weight  # tied

    def get_input_embeddings(self):
        return self.wte

    def get_output_embeddings(self):
        return self.lm_head

    def forward(self, idx):
        pos = torch.arange(idx.shape[1], device=idx.device)
        h = self.wte(idx) + self.wpe(pos)[None]
        for blk in self.blocks:
            a = blk["attn"](blk["ln"](h))
            h = h + blk["out"](a[..., : h.shape[-1]] * torch.sigmoid(a[..., h.shape[-1]:2 * h.shape[-1]]))
            h = h + blk["proj"](torch.relu(blk["fc"](h)))
        h = h + self.frozen(h)
        return self.lm_head(self.ln_f(h))


def test_auto_split_on_an_hf_style_module(gpu):
    torch.manual_seed(0)
    model_a = _TinyLM().to(gpu)
    model_b = copy.deepcopy(model_a)
    mc = _mc(lr=2e-2)
    opt = MuonAdamW(model_a, muon_config=mc, adam_config=AC, parameter_split="auto")
    ref = PyTorchMuonAdamW(model_b, muon_config=mc, adam_config=AC, parameter_split="auto")
    names_a = {id(p): n for n, p in model_a.named_parameters()}
    muon_names = [names_a[id(p)] for p in opt.param_group["muon"]]
    adam_names = [names_a[id(p)] for p in opt.param_group["adam"]]
    # the reference's rules (optimizer.py:117-130): wpe is 2-D and not the input embedding -> Muon;
    # the tied head is the embedding's storage -> seen once, as the embedding; the frozen weight is skipped
    assert "wpe.weight" in muon_names and "wte.weight" in adam_names
    assert "frozen.weight" not in muon_names + adam_names and "frozen.bias" in adam_names
    assert len(muon_names + adam_names) == len(set(muon_names + adam_names))
    names_b = {id(p): n for n, p in model_b.named_parameters()}
    assert [names_b[id(p)] for p in ref.muon.param_groups[0]["params"]] == muon_names
    assert [names_b[id(p)] for p in ref.adamw.param_groups[0]["params"]] == adam_names

    gen = torch.Generator(device=gpu).manual_seed(1)
    keep = 1 - mc.lr * mc.weight_decay
    for _ in range(3):
        idx = torch.randint(0, 1000, (4, 64), device=gpu, generator=gen)
        tgt = torch.randint(0, 1000, (4, 64), device=gpu, generator=gen)
        for m, o in ((model_a, opt), (model_b, ref)):
            o.zero_grad()
            loss = nn.functional.cross_entropy(m(idx).flatten(0, 1), tgt.flatten())
            loss.backward()
        before = {n: p.detach().clone() for n, p in model_b.named_parameters()}
        opt.step()
        ref.step()
        torch.cuda.synchronize()
        pb = dict(model_b.named_parameters())
        for n, p in model_a.named_parameters():
            q = pb[n]
            torch.testing.assert_close(p.detach(), q.detach(), atol=1e-2, rtol=1e-2, msg=n)
            if n in adam_names or n == "lm_head.weight":
                torch.testing.assert_close(p.detach(), q.detach(), atol=1e-6, rtol=0, msg=n)
            elif n in muon_names:
                adj = mc.lr * math.sqrt(max(1.0, p.shape[0] / p.shape[1]))
                u_mine = (before[n].double() * keep - p.detach().double()) / adj
                u_ref = (before[n].double() * keep - q.detach().double()) / adj
                err = ((u_mine - u_ref).norm() / u_ref.norm()).item()
                assert err <= 1e-2, f"{n}: update rel err {err}"
            else:  # frozen weight: untouched by both
                assert n == "frozen.weight" and torch.equal(p, before[n])
        # both sides keep the model's parameters synchronised for the next step
        with torch.no_grad():
            for n, p in model_a.named_parameters():
                p.copy_(pb[n])


SHAPES = [(256, 768), (768, 256), (384, 384), (1024, 300)]


@pytest.mark.parametrize("adjust", ["match_rms_adamw", "original"])
def test_adjust_lr_fn_against_torch_muon(gpu, adjust):
    """Two steps of HipMuon and torch.optim.Muon (same adjust_lr_fn) on the
    same parameters and gradients: updates within 1e-2 relative Frobenius,
    parameters within the reference tolerance."""
    gen = torch.Generator(device=gpu).manual_seed(7)
    ps = [torch.empty(s, device=gpu).normal_(0.0, 0.02, generator=gen) for s in SHAPES]
    mine = [nn.Parameter(p.clone()) for p in ps]
    theirs = [nn.Parameter(p.clone()) for p in ps]
    opt = HipMuon(mine, lr=2e-2, weight_decay=0.1, coeffs=COEFFS, nesterov=True, beta=0.95, ns_steps=5, eps=1e-7,
                  adjust_lr_fn=adjust)
    ref = torch.optim.Muon(theirs, lr=2e-2, weight_decay=0.1, momentum=0.95, nesterov=True, ns_coefficients=COEFFS,
                           eps=1e-7, ns_steps=5, adjust_lr_fn=adjust)
    keep = 1 - 2e-2 * 0.1
    for _ in range(2):
        for p, q in zip(mine, theirs):
            g = torch.empty(p.shape, device=gpu).normal_(0.0, 1.0, generator=gen)
            p.grad, q.grad = g.clone(), g.clone()
        before = [q.detach().clone() for q in theirs]
        opt.step()
        ref.step()
        torch.cuda.synchronize()
        for p, q, b0 in zip(mine, theirs, before):
            adj = torch.optim._muon._adjust_lr(2e-2, adjust, p.shape)
            u_mine = (b0.double() * keep - p.detach().double()) / adj
            u_ref = (b0.double() * keep - q.detach().double()) / adj
            assert ((u_mine - u_ref).norm() / u_ref.norm()).item() <= 1e-2, p.shape
            torch.testing.assert_close(p.detach(), q.detach(), atol=1e-2, rtol=1e-2)


def test_adjust_lr_spectral_unclamped_against_oracle(gpu):
    """``spectral_unclamped`` (reference only, triton_muon.py:430-431): the HIP
    step against the CPU oracle on the same inputs; momentum bit-exact, the
    update within 1e-2 relative Frobenius, parameters within the scale's
    multiple of 8e-3 (bf16 noise of the update times the step size)."""
    gen = torch.Generator().manual_seed(9)
    ps = [torch.randn(s, generator=gen) * 0.02 for s in SHAPES]
    gs = [torch.randn(s, generator=gen) for s in SHAPES]
    mine = [nn.Parameter(p.clone().to(gpu)) for p in ps]
    for p, g in zip(mine, gs):
        p.grad = g.to(gpu)
    opt = HipMuon(mine, lr=2e-2, weight_decay=0.1, coeffs=COEFFS, nesterov=True, beta=0.95, ns_steps=5, eps=1e-7,
                  adjust_lr_fn="spectral_unclamped")
    opt.step()
    torch.cuda.synchronize()
    keep = np.float32(1 - 2e-2 * 0.1)
    for p, p0, g in zip(mine, ps, gs):
        exp_p, exp_m, exp_u = oracle.muon.muon_update(p0.numpy(), g.numpy(), np.zeros(p0.shape, np.float32),
                                                      lr=2e-2, weight_decay=0.1, beta=0.95, nesterov=True,
                                                      coeffs=COEFFS, ns_steps=5, eps=1e-7,
                                                      adjust_lr_fn="spectral_unclamped")
        assert np.array_equal(opt.momentum[p].cpu().numpy(), exp_m)
        adj = oracle.muon.adjust_lr(2e-2, "spectral_unclamped", p0.shape)
        got_u = (p0.numpy().astype(np.float64) * keep - p.detach().cpu().numpy()) / adj
        assert rel_fro(got_u, exp_u) <= 1e-2, p0.shape
        # parameter differences are adj * (bf16 noise of the update), as in the oracle's own pin
        np.testing.assert_allclose(p.detach().cpu().numpy(), exp_p, atol=adj * 8e-3, rtol=0)


# ---- GradScaler and LR schedules against the torch optimizers -----------------

def _small_named(dev, seed):
    gen = torch.Generator(device=dev).manual_seed(seed)
    lay = [(n, sh, b) for n, sh, b in gpt2_layout(n_layer=2, vocab=512) if not n.startswith("wpe")]
    return [(n, nn.Parameter(torch.empty(sh, device=dev).normal_(0.0, 0.02, generator=gen)), b) for n, sh, b in lay]


def _muon_updates_close(mine, theirs, before_m, before_t, mc, tag):
    keep = 1 - mc.lr * mc.weight_decay
    for (n, p, b), (_, q, _), p0, q0 in zip(mine, theirs, before_m, before_t):
        if b != "muon":
            continue
        adj = mc.lr * math.sqrt(max(1.0, p.shape[0] / p.shape[1]))
        u_m = (p0.double() * keep - p.detach().double()) / adj
        u_t = (q0.double() * keep - q.detach().double()) / adj
        err = ((u_m - u_t).norm() / u_t.norm()).item()
        assert err <= 1e-2, f"{tag} {n}: update rel err {err}"


def _adam_close(mine, theirs, tag):
    for (n, p, b), (_, q, _) in zip(mine, theirs):
        if b == "adam":
            torch.testing.assert_close(p.detach(), q.detach(), atol=1e-6, rtol=0, msg=f"{tag} {n}")


def test_grad_scaler_against_torch_optimizers(gpu):
    mc = _mc()
    mine, theirs = _small_named(gpu, 21), _small_named(gpu, 21)
    opt = MuonAdamW(_split(mine), muon_config=mc, adam_config=AC, parameter_split="explicit")
    ref = PyTorchMuonAdamW(_split(theirs), muon_config=mc, adam_config=AC, parameter_split="explicit")
    s_m = torch.amp.GradScaler("cuda", init_scale=2048.0, growth_interval=1000)
    s_t = torch.amp.GradScaler("cuda", init_scale=2048.0, growth_interval=1000)
    for sc in (s_m, s_t):
        sc.scale(torch.ones((), device=gpu))  # initialise the scale on the device
    gen = torch.Generator(device=gpu).manual_seed(22)
    for it in range(4):
        grads = [torch.empty(p.shape, device=gpu).normal_(0.0, 1e-3, generator=gen) for _, p, _ in mine]
        if it == 2:  # one non-finite gradient in each branch: every optimizer skips the step
            grads[[k for k, (_, _, b) in enumerate(mine) if b == "adam"][0]].view(-1)[0] = float("inf")
            grads[[k for k, (_, _, b) in enumerate(mine) if b == "muon"][0]].view(-1)[0] = float("nan")
        scale = s_m.get_scale()
        assert scale == s_t.get_scale()
        for (_, p, _), (_, q, _), g in zip(mine, theirs, grads):
            p.grad = g * scale
            q.grad = g * scale
        before_m = [p.detach().clone() for _, p, _ in mine]
        before_t = [q.detach().clone() for _, q, _ in theirs]
        s_m.step(opt)
        s_m.update()
        s_t.step(ref.adamw)
        s_t.step(ref.muon)
        s_t.update()
        torch.cuda.synchronize()
        if it == 2:
            assert all(torch.equal(p.detach(), p0) for (_, p, _), p0 in zip(mine, before_m))
            assert all(torch.equal(q.detach(), q0) for (_, q, _), q0 in zip(theirs, before_t))
            continue
        _adam_close(mine, theirs, f"step {it}")
        _muon_updates_close(mine, theirs, before_m, before_t, mc, f"step {it}")
    assert opt.adamw.step_num == 3
    assert all(int(st["step"]) == 3 for st in ref.adamw.state.values())
    assert s_m.get_scale() == s_t.get_scale() == 1024.0


@pytest.mark.filterwarnings("ignore:Detected call of")
def test_lr_schedule_against_torch_optimizers(gpu):
    mc = _mc()
    mine, theirs = _small_named(gpu, 31), _small_named(gpu, 31)
    opt = MuonAdamW(_split(mine), muon_config=mc, adam_config=AC, parameter_split="explicit")
    ref = PyTorchMuonAdamW(_split(theirs), muon_config=mc, adam_config=AC, parameter_split="explicit")
    rate = lambda k: 0.6 ** k  # noqa: E731
    sched = torch.optim.lr_scheduler.LambdaLR(opt, rate)
    sched_a = torch.optim.lr_scheduler.LambdaLR(ref.adamw, rate)
    sched_u = torch.optim.lr_scheduler.LambdaLR(ref.muon, rate)
    gen = torch.Generator(device=gpu).manual_seed(32)
    for k in range(4):
        for (_, p, _), (_, q, _) in zip(mine, theirs):
            g = torch.empty(p.shape, device=gpu).normal_(0.0, 1e-3, generator=gen)
            p.grad, q.grad = g, g.clone()
        before_m = [p.detach().clone() for _, p, _ in mine]
        before_t = [q.detach().clone() for _, q, _ in theirs]
        opt.step()
        ref.step()
        torch.cuda.synchronize()
        _adam_close(mine, theirs, f"step {k}")
        lr_k = mc.lr * rate(k)
        _muon_updates_close(mine, theirs, before_m, before_t, MuonConfig(**{**mc.__dict__, "lr": lr_k}),
                            f"step {k}")
        sched.step()
        sched_a.step()
        sched_u.step()
    assert math.isclose(opt.param_groups[1]["lr"], mc.lr * rate(4))
    assert math.isclose(ref.muon.param_groups[0]["lr"], mc.lr * rate(4))
