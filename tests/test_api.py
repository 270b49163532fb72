"""Drop-in API: configs, routing, errors and step semantics that need no GPU.

Mirrors the behaviour of the reference's optimizer.py (configs :14-67,
routing :105-130, errors :107-111, attributes :132-154, state_dict :166-175)
and its branch classes (triton_adam.py:106-161, triton_muon.py:375-456).
"""

import dataclasses
import math
import importlib

import numpy as np
import pytest
import torch
import torch.nn as nn

import oracle
from triton_muon_adamw import AdamConfig, MuonAdamW, MuonConfig, PyTorchMuonAdamW, split_parameters
from triton_muon_adamw.muon.hip_muon import scaled_lr


class TinyLM(nn.Module):
    """Embedding + position embedding + 2 Linear + LayerNorm + head (optionally tied)."""

    def __init__(self, tied=False, vocab=50, d=16):
        super().__init__()
        self.wte = nn.Embedding(vocab, d)
        self.wpe = nn.Embedding(8, d)
        self.fc = nn.Linear(d, 4 * d)
        self.proj = nn.Linear(4 * d, d, bias=False)
        self.ln = nn.LayerNorm(d)
        self.head = nn.Linear(d, vocab, bias=False)
        if tied:
            self.head.weight = self.wte.weight

    def get_input_embeddings(self):
        return self.wte

    def get_output_embeddings(self):
        return self.head


def test_config_defaults_match_reference():
    a = AdamConfig()
    assert (a.lr, a.betas, a.eps, a.weight_decay) == (1e-3, (0.9, 0.999), 1e-7, 0.01)
    m = MuonConfig()
    assert (m.lr, m.beta, m.eps, m.weight_decay) == (1e-3, 0.95, 1e-7, 0.1)
    assert m.coeffs == (3.445, -4.775, 2.0315)
    assert (m.nesterov, m.ns_steps, m.adjust_lr_fn) == (True, 5, "original")
    assert [f.name for f in dataclasses.fields(AdamConfig)] == ["lr", "betas", "eps", "weight_decay"]
    assert [f.name for f in dataclasses.fields(MuonConfig)] == [
        "lr", "beta", "eps", "weight_decay", "coeffs", "nesterov", "ns_steps", "adjust_lr_fn"]


def test_auto_routing():
    model = TinyLM()
    adam, muon = split_parameters(model, "auto")
    ids = lambda ps: {id(p) for p in ps}  # noqa: E731
    # 2-D parameters go to Muon except the input embedding and the head;
    # the position embedding (2-D, not the input embedding) goes to Muon.
    assert ids(muon) == ids([model.wpe.weight, model.fc.weight, model.proj.weight])
    assert ids(adam) == ids([model.wte.weight, model.fc.bias, model.ln.weight, model.ln.bias, model.head.weight])
    # order follows model.parameters()
    assert [id(p) for p in muon] == [id(model.wpe.weight), id(model.fc.weight), id(model.proj.weight)]


def test_auto_routing_tied_frozen_and_no_head():
    model = TinyLM(tied=True)
    model.fc.bias.requires_grad_(False)
    adam, muon = split_parameters(model, "auto")
    assert sum(p is model.wte.weight for p in adam) == 1  # tied head deduplicated by data_ptr
    assert all(p is not model.fc.bias for p in adam + muon)
    model.get_output_embeddings = lambda: None
    adam, muon = split_parameters(model, "auto")
    assert any(p is model.head.weight for p in adam)  # tied: same tensor as the embedding


def test_explicit_routing_and_errors():
    p1, p2 = nn.Parameter(torch.zeros(3, 4)), nn.Parameter(torch.zeros(4))
    assert split_parameters({"muon": [p1]}, "explicit") == ([], [p1])
    assert split_parameters({"adam": [p2]}, "explicit") == ([p2], [])
    with pytest.raises(ValueError, match="explicit"):
        split_parameters(TinyLM(), "explicit")
    with pytest.raises(ValueError, match="auto"):
        split_parameters({"adam": [], "muon": []}, "auto")
    with pytest.raises(AttributeError):
        split_parameters(nn.Linear(3, 3), "auto")


def test_muonadamw_attributes_and_state_dict():
    model = TinyLM()
    opt = MuonAdamW(model, MuonConfig(lr=0.02), AdamConfig(lr=3e-4), "auto")
    assert opt.param_group["adam"] is opt.adamw.model_params
    assert opt.param_group["muon"] is opt.muon.model_params
    assert opt.muon.lr == 0.02 and opt.adamw.lr == 3e-4
    sd = opt.state_dict()  # optimizer state, not the parameter lists (those stay in param_group)
    assert set(sd) == {"adam", "muon"} and "state" in sd["adam"] and "state" in sd["muon"]
    # the reference's format (parameter lists, optimizer.py:170-175) still reassigns the lists
    new = [nn.Parameter(torch.zeros(2, 2))]
    opt.load_state_dict({"muon": new})
    assert opt.muon.model_params is new and opt.param_group["muon"] is new
    assert opt.param_groups[1]["params"] is new
    # a parameter that joined a branch that way gets zero state on first use
    mom = opt.state_dict()["muon"]["state"][0]["momentum_buffer"]
    assert mom.shape == (2, 2) and mom.dtype == torch.float32 and not mom.any()
    new_a = [nn.Parameter(torch.zeros(3))]
    opt.load_state_dict({"adam": new_a})
    opt.adamw.step_num = 1  # state_dict lists the moments only after a step, as torch does
    st = opt.state_dict()["adam"]["state"][0]
    assert st["exp_avg"].shape == (3,) and not st["exp_avg"].any() and not st["exp_avg_sq"].any()
    # state shapes: fp32 moments for AdamW, parameter-shaped momentum for Muon
    for p in opt.adamw.model_params:
        assert opt.adamw.m[p].shape == p.shape and opt.adamw.m[p].dtype == torch.float32
    for p in model.fc.weight, model.proj.weight:
        assert opt.muon.momentum[p].shape == p.shape


def test_parameters_join_a_branch_through_its_list():
    """add_param_group is refused after construction (the two groups are the two
    branches); a parameter appended to a branch's list joins that branch, with
    zero state from its first use, and the torch.optim groups see it."""
    opt = MuonAdamW(TinyLM())
    with pytest.raises(ValueError, match="two fixed parameter groups"):
        opt.add_param_group({"params": [nn.Parameter(torch.zeros(3))]})
    extra = nn.Parameter(torch.zeros(4, 6))
    opt.param_group["muon"].append(extra)
    assert opt.param_groups[1]["params"][-1] is extra
    mom = opt.state_dict()["muon"]["state"][len(opt.muon.model_params) - 1]["momentum_buffer"]
    assert mom.shape == (4, 6) and not mom.any()


def test_invalid_adjust_lr_fn_raises_assertion():
    with pytest.raises(AssertionError, match="Invalid adjust_lr_fn"):
        MuonAdamW(TinyLM(), MuonConfig(adjust_lr_fn="bogus"))
    # also when set through param_groups (checked before anything runs), where
    # torch's None stands for "original"
    opt = MuonAdamW(TinyLM())
    opt.param_groups[1]["adjust_lr_fn"] = None
    opt._pull_groups()
    assert opt.muon.adjust_lr_fn == "original"
    opt.param_groups[1]["adjust_lr_fn"] = "bogus"
    with pytest.raises(AssertionError, match="Invalid adjust_lr_fn"):
        opt.step()


def test_zero_grad_zero_fills():
    model = TinyLM()
    opt = MuonAdamW(model)
    for p in model.parameters():
        p.grad = torch.ones_like(p)
    opt.zero_grad()
    for p in model.parameters():
        assert p.grad is not None and not p.grad.any()


def test_step_on_cpu_tensors_fails_loudly():
    model = TinyLM()
    opt = MuonAdamW(model)
    for p in model.parameters():
        p.grad = torch.ones_like(p)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        opt.step()
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        opt.muon.step()


def test_non_2d_muon_parameter_raises_assertion():
    p = nn.Parameter(torch.zeros(2, 3, 4))
    p.grad = torch.zeros_like(p)
    opt = MuonAdamW({"muon": [p]}, parameter_split="explicit")
    with pytest.raises(AssertionError, match="2D"):
        opt.step()


def test_scaled_lr_closed_forms():
    assert scaled_lr(0.01, "original", 2048, 512) == 0.01 * 2.0
    assert scaled_lr(0.01, "original", 512, 2048) == 0.01
    assert scaled_lr(0.01, "match_rms_adamw", 512, 2048) == oracle.muon.adjust_lr(0.01, "match_rms_adamw",
                                                                                    (512, 2048))
    assert scaled_lr(0.01, "spectral_unclamped", 512, 2048) == 0.005


def test_exports_and_shim():
    pkg = importlib.import_module("triton_muon_adamw")
    for name in ("AdamConfig", "MuonAdamW", "MuonConfig", "PyTorchMuonAdamW"):
        assert name in pkg.__all__
    from triton_muon_adamw.adamw import TritonAdamW
    from triton_muon_adamw.muon import TritonMuon

    assert issubclass(MuonAdamW, TritonMuon) and issubclass(MuonAdamW, TritonAdamW)
    shim = importlib.import_module("MuonAdamW")
    assert shim.MuonAdamW is MuonAdamW and shim.PyTorchMuonAdamW is PyTorchMuonAdamW


def test_pytorch_wrapper_matches_oracle_on_cpu():
    torch.manual_seed(0)
    model = nn.Sequential(nn.Linear(32, 64), nn.LayerNorm(64), nn.Linear(64, 32))
    for p in model.parameters():
        p.grad = torch.randn_like(p) * 1e-3
    p0 = [p.detach().numpy().copy() for p in model.parameters()]
    g0 = [p.grad.numpy().copy() for p in model.parameters()]
    mc = MuonConfig(lr=0.02, coeffs=(3.4445, -4.775, 2.0315))
    ac = AdamConfig(lr=3e-4, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1)
    split = {"adam": [p for p in model.parameters() if p.ndim == 1],
             "muon": [p for p in model.parameters() if p.ndim == 2]}
    ref = PyTorchMuonAdamW(split, mc, ac, "explicit")
    ref.step()
    for p, a, g in zip(model.parameters(), p0, g0):
        if p.ndim == 1:
            b1, b2 = oracle.adamw.bias_corrections(0.9, 0.95, 1)
            e, _, _ = oracle.adamw.adamw_update(a, g, np.zeros_like(a), np.zeros_like(a), lr=3e-4, bias1=b1,
                                                bias2=b2, beta1=0.9, beta2=0.95, weight_decay=0.1, eps=1e-8)
            np.testing.assert_allclose(p.detach().numpy(), e, rtol=0, atol=1e-7)
        else:
            e, _, _ = oracle.muon.muon_update(a, g, np.zeros_like(a), lr=0.02, weight_decay=0.1, beta=0.95,
                                              coeffs=mc.coeffs)
            np.testing.assert_allclose(p.detach().numpy(), e, rtol=0, atol=0.02 * 8e-3)
    sd = ref.state_dict()
    assert set(sd) == {"adam", "muon"}
    ref.load_state_dict(sd)


def test_adamw_step_counter_host_and_device_views():
    """step_num is a host int until a gradient-scaler (or capturable) step moves
    the counter to the device; reading it then reads the device counter back,
    and assigning it (e.g. load_state_dict) fills that same counter tensor in
    place, so a step captured in a graph keeps advancing the live counter."""
    from triton_muon_adamw.adamw import HipAdamW

    opt = HipAdamW([nn.Parameter(torch.zeros(4))])
    assert opt.step_num == 0 and opt._dev_steps == {}
    opt.step_num = 7
    assert opt.step_num == 7
    counter = torch.tensor(9.0)
    opt._dev_steps = {torch.device("cpu"): counter}  # as _step_amp leaves it
    assert opt.step_num == 9
    opt.step_num = 3
    assert opt.step_num == 3 and opt._dev_steps[torch.device("cpu")] is counter and counter.item() == 3.0
    assert MuonAdamW._step_supports_amp_scaling


def test_capturable_flag():
    """``capturable`` is keyword-only, off by default, passed to the AdamW
    branch and reported in its state dict as torch.optim.AdamW does; a step
    with no gradients keeps a device-side counter on the device."""
    from triton_muon_adamw.adamw import HipAdamW

    lin = nn.Linear(8, 8)
    groups = {"adam": [lin.bias], "muon": [lin.weight]}
    assert MuonAdamW(groups, parameter_split="explicit").adamw.capturable is False
    opt = MuonAdamW(groups, parameter_split="explicit", capturable=True)
    assert opt.adamw.capturable is True
    assert opt.adamw.state_dict()["param_groups"][0]["capturable"] is True
    with pytest.raises(TypeError):
        MuonAdamW(groups, MuonConfig(), AdamConfig(), "explicit", True)
    a = HipAdamW([nn.Parameter(torch.zeros(4))], capturable=True)
    a._dev_steps = {torch.device("cpu"): torch.tensor(2.0)}  # as the first capturable step leaves it
    a.step()  # no gradient: the counter alone advances, where it lives
    assert a._dev_steps and a.step_num == 3


def _brute_cost(sizes, m, n, cus):
    """Modelled time of a split, counted tile by tile: each product's rounds of
    CU slots times its reduction length times the relative k-step time of its
    tile (the group's tile: 256 from m = 2048, or from m = 1024 for groups of 8
    or more when the padding allows; on the 128 tile, 256-wide updates from
    m = 1024 when the padded edges allow), plus a quarter round of each
    product per group."""
    w = {128: 1.0, 256: 1.4}
    slots = {128: 2 * cus, 256: cus}
    rup = lambda x, t: -(-x // t) * t  # noqa: E731
    total = 0.0
    for k in sizes:
        tile = 256 if m >= 2048 or (m >= 1024 and k >= 8 and rup(m, 256) * rup(n, 256) * 16
                                    <= rup(m, 128) * rup(n, 128) * 17) else 128
        mp, np_ = rup(m, tile), rup(n, tile)
        utile = 256 if (tile == 128 and m >= 1024 and mp % 256 == 0 and np_ % 256 == 0) else tile
        tm = mp // tile
        sym = sum(1 for i in range(tm) for j in range(tm) if j >= i) * k
        full = sum(1 for i in range(mp // utile) for j in range(np_ // utile)) * k
        total += math.ceil(sym / slots[tile]) * w[tile] * (n + m) + math.ceil(full / slots[utile]) * w[utile] * m
        total += 0.25 * (w[tile] * (n + m) + w[utile] * m)
    return total


def _compositions(count, cap):
    if count == 0:
        yield []
        return
    for k in range(1, min(cap, count) + 1):
        for rest in _compositions(count - k, cap):
            yield [k] + rest


@pytest.mark.parametrize("count,cap,m,n", [
    (96, 32, 4096, 14336), (96, 20, 4096, 14336), (64, 32, 4096, 4096), (64, 32, 1024, 4096),
    (33, 32, 4096, 4096), (24, 32, 768, 3072), (1, 32, 768, 768), (7, 2, 2048, 2048), (40, 9, 1024, 1024)])
def test_launch_group_sizes(count, cap, m, n):
    """Group sizing: covers every matrix, respects the cap, and never costs
    more than the even split under the cap (same model, counted tile by tile)."""
    from triton_muon_adamw.muon.hip_muon import group_sizes
    sizes = group_sizes(count, cap, m, n, 256)
    assert sum(sizes) == count and max(sizes) <= cap and min(sizes) >= 1
    g = -(-count // cap)
    even = [count // g + (1 if i < count % g else 0) for i in range(g)]
    assert _brute_cost(sizes, m, n, 256) <= _brute_cost(even, m, n, 256) + 1e-6


@pytest.mark.parametrize("count,cap,m,n", [(12, 5, 1024, 4096), (10, 4, 4096, 4096), (9, 9, 768, 3072),
                                           (11, 6, 2048, 8192)])
def test_launch_group_sizes_optimal(count, cap, m, n):
    """The dynamic programme finds the cheapest split: every composition of a
    small count into groups of at most cap, by brute force."""
    from triton_muon_adamw.muon.hip_muon import group_sizes
    sizes = group_sizes(count, cap, m, n, 256)
    best = min(_brute_cost(c, m, n, 256) for c in _compositions(count, cap))
    assert abs(_brute_cost(sizes, m, n, 256) - best) < 1e-6


def test_launch_group_sizes_llama():
    """The Llama-3-8B classes: groups of 32 where the 136 symmetric tiles of a
    4096-row Gram fill whole rounds of 256 CUs (17 rounds for 32 matrices,
    where 20 matrices take 11 rounds for 62.5% of the work); the 64 k/v
    (1024 x 4096) matrices as 24 + 24 + 16 on 256-wide tiles (10 symmetric
    tiles per matrix: one round per group; updates 6 + 6 + 4 whole rounds;
    measured 5.76 ms for the class's step against 6.17 ms as 28 + 28 + 8 on
    the 128 tile)."""
    from triton_muon_adamw.muon.hip_muon import group_sizes
    assert group_sizes(96, 32, 4096, 14336, 256) == [32, 32, 32]
    assert group_sizes(64, 32, 4096, 4096, 256) == [32, 32]
    assert group_sizes(64, 32, 1024, 4096, 256) == [24, 24, 16]
    assert group_sizes(0, 32, 4096, 4096, 256) == []


@pytest.mark.parametrize("classes,n_side,caller,groups", [
    # config 3: the 4096 x 14336 class on the caller's stream, the rest on one side stream
    ([(1, 768, 3072), (2, 1024, 4096), (1, 4096, 4096), (1, 4096, 14336)], 1, 3, [[2, 1, 0]]),
    # GPT-2: 24 x 768 x 3072 on the caller's stream
    ([(12, 768, 2304), (12, 768, 768), (24, 768, 3072)], 1, 2, [[0, 1]]),
    # the reference's hybrid MLP: batch-1 classes of small grids need a third lane
    ([(1, 1024, 2048), (1, 2048, 4096), (1, 4096, 4096), (1, 1024, 4096)], 2, 2, [[1], [3, 0]]),
    # five small classes of similar estimated time (the GPU test's "five_classes"): three side
    # streams, the most there are, although the third ends after the caller's class
    ([(2, 256, 512), (2, 384, 384), (2, 128, 640), (2, 320, 448), (2, 192, 576)], 3, 3, [[1], [4], [0, 2]]),
])
def test_concurrent_class_lanes(monkeypatch, classes, n_side, caller, groups):
    """Concurrent shape classes: the class with the longest estimated time
    (launch rounds, not flops) runs on the caller's stream (lane None); the
    others, longest first, share the fewest side streams (up to 3) that all
    finish within it.  ``groups`` lists each side stream's classes in order."""
    from triton_muon_adamw import _lib
    from triton_muon_adamw.muon import hip_muon
    made = []

    def fake_side_streams(dev, count):
        made.append((dev, count))
        return [f"{dev}/s{i}" for i in range(count)]

    monkeypatch.setattr(_lib, "side_streams", fake_side_streams)
    calls = [hip_muon._Call("d0", None, b, 0, m, n, g) for g, (b, m, n) in enumerate(classes)]
    lanes, times = hip_muon._lanes(calls, 5, {"d0": 256})
    assert lanes[("d0", caller)] is None
    assert made == [("d0", n_side)]
    by_stream = {}
    for g in sorted(range(len(classes)), key=lambda g: -times[("d0", g)]):
        if lanes[("d0", g)] is not None:
            by_stream.setdefault(lanes[("d0", g)], []).append(g)
    assert [by_stream[f"d0/s{i}"] for i in range(n_side)] == groups
    side_time = [sum(times[("d0", g)] for g in grp) for grp in groups]
    if n_side < 3:
        assert max(side_time) <= times[("d0", caller)]


def test_lane_split():
    """The fewest side streams (1 to 3) whose loads fit within the longest
    class, least loaded first; three when even three do not fit."""
    from triton_muon_adamw.muon.hip_muon import _lane_split
    assert _lane_split([10.0, 4.0, 3.0, 2.0]) == (1, [0, 0, 0])
    assert _lane_split([10.0, 6.0, 5.0]) == (2, [0, 1])
    assert _lane_split([10.0, 9.0, 8.0, 7.0]) == (3, [0, 1, 2])
    assert _lane_split([5.0, 5.0, 5.0, 5.0, 5.0]) == (3, [0, 1, 2, 0])
    assert _lane_split([3.0, 1.0]) == (1, [0])


def test_concurrent_class_lanes_one_class_per_device(monkeypatch):
    from triton_muon_adamw import _lib
    from triton_muon_adamw.muon import hip_muon
    monkeypatch.setattr(_lib, "side_streams", lambda dev, count: [f"{dev}/s{i}" for i in range(count)])
    calls = [hip_muon._Call("d0", None, 2, 0, 512, 512, 0), hip_muon._Call("d1", None, 1, 0, 256, 256, 1),
             hip_muon._Call("d1", None, 1, 0, 2048, 4096, 2)]
    lanes, _ = hip_muon._lanes(calls, 5, {"d0": 256, "d1": 256})
    assert lanes[("d0", 0)] is None and lanes[("d1", 2)] is None and lanes[("d1", 1)] == "d1/s0"


def test_side_streams_of_ended_threads_are_reused():
    """A thread's side streams go back to a free list when it ends and the
    next thread takes them from there (stand-in objects for the streams, a
    device index no GPU has: nothing here calls HIP)."""
    import gc
    import threading

    from triton_muon_adamw import _lib

    dev = torch.device("cuda", 97)

    def first():
        _lib._thread_side_streams.streams = _lib._ThreadStreams()
        _lib._thread_side_streams.streams.by_device[97] = ["s0", "s1"]

    t = threading.Thread(target=first)
    t.start()
    t.join()
    gc.collect()
    try:
        assert sorted(_lib._free_side_streams.get(97, [])) == ["s0", "s1"]
        got = []
        t = threading.Thread(target=lambda: got.extend(_lib.side_streams(dev, 2)))
        t.start()
        t.join()
        gc.collect()
        assert sorted(got) == ["s0", "s1"]
        assert sorted(_lib._free_side_streams.get(97, [])) == ["s0", "s1"]  # returned again
    finally:
        _lib._free_side_streams.pop(97, None)
