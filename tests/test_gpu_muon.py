"""GPU parity of the Muon kernels (gfx950) through the C ABI.

Building blocks (Gram, polynomial, update GEMMs) against float64 products of
the same bf16 inputs: every output within one bf16 rounding of the exact
value.  The full Muon step against the CPU oracle (oracle/muon.py): momentum
bit-exact, the orthogonalised update within bf16 noise (relative Frobenius
error <= 1e-2; two correct bf16 implementations differ by 0.3-0.6%), and the
parameters within the reference tolerance (atol = rtol = 1e-2,
muon_benchmark.py:105) and far tighter.  Batched launches must equal
single-matrix launches bit for bit.
"""

import numpy as np
import pytest
import torch

import oracle
from helpers import muon_inputs, rel_fro
from triton_muon_adamw.muon import HipMuon, muon_step, newton_shultz_step
from triton_muon_adamw.muon import solve_ns_kernel_1, solve_ns_kernel_2, solve_ns_kernel_3
from triton_muon_adamw.muon.hip_muon import scaled_lr

pytestmark = pytest.mark.gpu

COEFFS = (3.4445, -4.7750, 2.0315)


def _bf16_close(got: torch.Tensor, exact: np.ndarray, rel_floor: float = 1e-5):
    """|got - exact| <= one bf16 ulp of exact (+ a floor for cancellation)."""
    g = got.float().cpu().numpy().astype(np.float64)
    e = np.asarray(exact, dtype=np.float64)
    ulp = np.exp2(np.floor(np.log2(np.maximum(np.abs(e), 1e-30))) - 7)
    bad = np.abs(g - e) > ulp + rel_floor * np.abs(e).max()
    assert not bad.any(), f"{bad.sum()} elements off by more than 1 bf16 ulp (max err {np.abs(g - e).max()})"


def _rand_bf16(shape, seed, std=1.0):
    gen = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=gen) * std).bfloat16()


@pytest.mark.parametrize("m,k", [(128, 64), (256, 640), (200, 333), (2048, 1024)])
def test_gram_exact_symmetric(gpu, m, k):
    X = _rand_bf16((m, k), 11, std=k**-0.5)
    A = torch.empty((m, m), dtype=torch.bfloat16, device=gpu)
    solve_ns_kernel_1(X.to(gpu), A)
    torch.cuda.synchronize()
    assert torch.equal(A, A.T), "Gram output must be exactly symmetric"
    Xd = X.double().numpy()
    _bf16_close(A, Xd @ Xd.T)


@pytest.mark.parametrize("m", [128, 384, 2048])
def test_poly_exact_symmetric(gpu, m):
    X = _rand_bf16((m, 2 * m), 12, std=(2 * m) ** -0.5)
    A = torch.empty((m, m), dtype=torch.bfloat16, device=gpu)
    solve_ns_kernel_1(X.to(gpu), A)
    B = torch.empty_like(A)
    b, c = COEFFS[1], COEFFS[2]
    solve_ns_kernel_2(A, b, c, B)
    torch.cuda.synchronize()
    assert torch.equal(B, B.T), "polynomial output must be exactly symmetric"
    Ad = A.double().cpu().numpy()
    _bf16_close(B, b * Ad + c * (Ad @ Ad))


@pytest.mark.parametrize("m,n", [(128, 128), (256, 768), (100, 300), (2048, 4096)])
def test_update_exact(gpu, m, n):
    X = _rand_bf16((m, n), 13, std=n**-0.5).to(gpu)
    A = torch.empty((m, m), dtype=torch.bfloat16, device=gpu)
    solve_ns_kernel_1(X, A)
    B = torch.empty_like(A)
    solve_ns_kernel_2(A, COEFFS[1], COEFFS[2], B)
    out = torch.empty_like(X)
    solve_ns_kernel_3(X, B, COEFFS[0], out)
    torch.cuda.synchronize()
    Xd = X.double().cpu().numpy()
    Bd = B.double().cpu().numpy()
    _bf16_close(out, COEFFS[0] * Xd + Bd @ Xd)


def test_newton_shultz_step_matches_blocks(gpu):
    X = _rand_bf16((256, 512), 14, std=512**-0.5).to(gpu)
    out = torch.empty_like(X)
    newton_shultz_step(X, *COEFFS, out)
    A = torch.empty((256, 256), dtype=torch.bfloat16, device=gpu)
    B = torch.empty_like(A)
    ref = torch.empty_like(X)
    solve_ns_kernel_1(X, A)
    solve_ns_kernel_2(A, COEFFS[1], COEFFS[2], B)
    solve_ns_kernel_3(X, B, COEFFS[0], ref)
    torch.cuda.synchronize()
    assert torch.equal(out, ref)


def _run_muon(shapes, gpu, seed=1, lr=2e-2, **kw):
    ps, gs, ms = muon_inputs(shapes, seed=seed)
    params = [torch.nn.Parameter(p.to(gpu)) for p in ps]
    opt = HipMuon(params, lr=lr, coeffs=COEFFS, **kw)
    for p, g, m in zip(params, gs, ms):
        p.grad = g.to(gpu)
        opt.momentum[p].copy_(m)
    return ps, gs, ms, params, opt


SMALL_SHAPES = [(128, 256), (256, 128), (100, 37), (37, 100), (512, 512), (640, 1280), (1, 5), (300, 1)]


# Ragged shapes over several prep tiles (64 x 128 parameter elements) and
# scale tiles (128 x 64 of X) in both orientations, tall and wide in one class.
RAGGED_SHAPES = [(300, 1000), (1000, 300), (1000, 300), (200, 520), (520, 200)]


@pytest.mark.parametrize("nesterov,ns_steps", [(True, 5), (False, 5), (True, 1), (True, 0), (True, 2)])
def test_muon_step_vs_oracle(gpu, nesterov, ns_steps):
    _check_vs_oracle(gpu, SMALL_SHAPES, nesterov, ns_steps)


def test_ragged_multi_tile_vs_oracle(gpu):
    _check_vs_oracle(gpu, RAGGED_SHAPES, True, 5)


def _check_vs_oracle(gpu, shapes, nesterov, ns_steps):
    ps, gs, ms, params, opt = _run_muon(shapes, gpu, nesterov=nesterov, ns_steps=ns_steps)
    outs = []
    for p in params:  # update outputs through muon_step's `out` on a copy of each matrix
        outs.append(torch.empty_like(p))
    w2 = [p.detach().clone() for p in params]
    mom2 = [m.to(gpu) for m in ms]
    g2 = [g.to(gpu) for g in gs]
    for w, g, m, o, shp in zip(w2, g2, mom2, outs, shapes):
        muon_step(w, g, m, opt.beta, *COEFFS, opt.lr, scaled_lr(opt.lr, "original", *shp), opt.weight_decay,
                  ns_steps, opt.eps, nesterov, out=o)
    opt.step()
    torch.cuda.synchronize()
    for i, shp in enumerate(shapes):
        ep, em, eo = oracle.muon.muon_update(ps[i].numpy(), gs[i].numpy(), ms[i].numpy(), lr=opt.lr,
                                             weight_decay=opt.weight_decay, beta=opt.beta, nesterov=nesterov,
                                             coeffs=COEFFS, ns_steps=ns_steps, eps=opt.eps)
        assert np.array_equal(opt.momentum[params[i]].cpu().numpy(), em), f"momentum {shp}"
        assert torch.equal(params[i].detach(), w2[i]), f"batched step != single muon_step {shp}"
        upd = outs[i].cpu().numpy()
        err = rel_fro(upd, eo)
        assert err <= 1e-2, f"{shp}: update rel err {err}"
        exact = oracle.muon.zeropower_ns(
            oracle.muon.lerp(gs[i].numpy(), em, opt.beta) if nesterov else em, COEFFS, ns_steps, opt.eps,
            exact=True)
        assert rel_fro(upd, exact) <= 3e-2, f"{shp}: far from exact NS"
        got = params[i].detach().cpu().numpy()
        np.testing.assert_allclose(got, ep, atol=1e-2, rtol=1e-2)
        # the apply epilogue itself: p*(1 - lr*wd) - slr*update, one fma in fp32
        keep = np.float32(1 - opt.lr * opt.weight_decay)
        slr = np.float32(scaled_lr(opt.lr, "original", *shp))
        np.testing.assert_allclose(got, oracle.muon.fma32(-slr, upd, ps[i].numpy() * keep), rtol=0, atol=1e-7)


def test_batched_equals_single(gpu):
    shapes = [(256, 512)] * 3 + [(512, 256)] * 2
    ps, gs, ms, params, opt = _run_muon(shapes, gpu, seed=4)
    singles = []
    for p, g, m in zip(ps, gs, ms):
        q = torch.nn.Parameter(p.to(gpu))
        q.grad = g.to(gpu)
        o = HipMuon([q], lr=opt.lr, coeffs=COEFFS)
        o.momentum[q].copy_(m)
        o.step()
        singles.append(q)
    opt.step()
    torch.cuda.synchronize()
    for a, b in zip(params, singles):
        assert torch.equal(a.detach(), b.detach())


def test_parameter_listed_twice_steps_twice(gpu):
    """A matrix listed twice gets two Muon updates in sequence (momentum and
    parameter), as the reference's per-parameter loop gives it
    (triton_muon.py:415-448, state keyed by the parameter): its second
    occurrence goes to a later launch.  Equal bit for bit to the same matrix
    stepped twice alone; the other member once."""
    ps, gs, ms = muon_inputs([(256, 512), (512, 256)], seed=6)
    w, u = (torch.nn.Parameter(p.to(gpu)) for p in ps)
    opt = HipMuon([w, u, w], lr=2e-2, coeffs=COEFFS)
    for p, g, m in zip((w, u), gs, ms):
        p.grad = g.to(gpu)
        opt.momentum[p].copy_(m)
    opt.step()
    assert [c.n for c in opt._calls] == [2, 1]
    for p, p0, g, m, times in ((w, ps[0], gs[0], ms[0], 2), (u, ps[1], gs[1], ms[1], 1)):
        q = torch.nn.Parameter(p0.to(gpu))
        q.grad = g.to(gpu)
        o = HipMuon([q], lr=2e-2, coeffs=COEFFS)
        o.momentum[q].copy_(m)
        for _ in range(times):
            o.step()
        torch.cuda.synchronize()
        assert torch.equal(p.detach(), q.detach())
        assert torch.equal(opt.momentum[p], o.momentum[q])


def test_rect_tile_does_not_change_the_bits(gpu):
    """Twelve 768 x 3072 matrices (the tall and the wide orientation) in one
    launch group run their updates on 128 x 192 tiles (1152 tiles, at least
    two rounds); each alone runs them on 128 x 128 tiles.  Every output
    element sums the same products in the same order under either tile, so
    parameters and momenta agree bit for bit (two steps)."""
    from triton_muon_adamw import _lib
    shapes = [(768, 3072)] * 6 + [(3072, 768)] * 6
    ps, gs, ms, params, opt = _run_muon(shapes, gpu, seed=12)
    singles = []
    for p, g, m in zip(ps, gs, ms):
        q = torch.nn.Parameter(p.to(gpu))
        q.grad = g.to(gpu)
        o = HipMuon([q], lr=opt.lr, coeffs=COEFFS)
        o.momentum[q].copy_(m)
        singles.append((q, o))

    def tiles_of(step_fn):
        _lib.prof_start()
        step_fn()
        _lib.prof_stop()
        return {(r["kernel"].split(":")[1], r["variant"] // 8) for r in _lib.prof_collect()
                if r["kernel"].startswith("ns_gemm")}

    assert tiles_of(opt.step) == {("gram", 128), ("poly", 128), ("update", 192), ("apply", 192)}
    assert tiles_of(lambda: [o.step() for _, o in singles]) == {("gram", 128), ("poly", 128), ("update", 128),
                                                                ("apply", 128)}
    opt.step()
    for q, o in singles:
        o.step()
    torch.cuda.synchronize()
    for a, (b, o) in zip(params, singles):
        assert torch.equal(a.detach(), b.detach())
        assert torch.equal(opt.momentum[a], o.momentum[b])


def test_tile_edge_does_not_change_the_bits(gpu):
    """Eight 1024 x 2048 matrices in one launch group run on 256-wide tiles
    (m >= 1024 and 8 matrices) with lower-triangle A and B; each alone runs
    its Gram and polynomial on 128-wide tiles with mirrored A and B (the
    updates take 256-wide tiles from m = 1024 either way).  Every output
    element sums the same products in the same order under either tile and
    layout, so parameters and momenta agree bit for bit (two steps)."""
    from triton_muon_adamw import _lib
    shapes = [(1024, 2048)] * 8
    ps, gs, ms, params, opt = _run_muon(shapes, gpu, seed=9)
    singles = []
    for p, g, m in zip(ps, gs, ms):
        q = torch.nn.Parameter(p.to(gpu))
        q.grad = g.to(gpu)
        o = HipMuon([q], lr=opt.lr, coeffs=COEFFS)
        o.momentum[q].copy_(m)
        singles.append((q, o))

    def tiles_of(step_fn):
        _lib.prof_start()
        step_fn()
        _lib.prof_stop()
        return {(r["kernel"].split(":")[1], r["variant"] // 8) for r in _lib.prof_collect()
                if r["kernel"].startswith("ns_gemm")}

    assert tiles_of(opt.step) == {("gram", 256), ("poly", 256), ("update", 256), ("apply", 256)}
    assert [c.n for c in opt._calls] == [8]
    # alone: 128-wide Gram and polynomial, 256-wide updates (m = 1024)
    assert tiles_of(lambda: [o.step() for _, o in singles]) == {("gram", 128), ("poly", 128), ("update", 256),
                                                                 ("apply", 256)}
    opt.step()
    for q, o in singles:
        o.step()
    torch.cuda.synchronize()
    for a, (b, o) in zip(params, singles):
        assert torch.equal(a.detach(), b.detach())
        assert torch.equal(opt.momentum[a], o.momentum[b])


# Shape classes of a small step: three (two side streams beside the caller's),
# and five whose estimated times make _lanes use three side streams
# (tests/test_api.py checks that split on the CPU).
CONCURRENT_SETS = {
    "three_classes": [(256, 512)] * 3 + [(512, 256)] * 2 + [(384, 384)] * 2 + [(128, 640)],
    "five_classes": [(256, 512), (512, 256), (384, 384)] * 1 + [(384, 384), (128, 640), (640, 128), (320, 448),
                                                                (448, 320), (192, 576), (576, 192)],
}


@pytest.mark.parametrize("classes", sorted(CONCURRENT_SETS))
@pytest.mark.parametrize("on_side_stream", [False, True])
def test_concurrent_classes_equal_in_order(gpu, on_side_stream, classes):
    """Shape classes on their own streams (small steps) give the same bits as one after another,
    also when the caller steps on a non-default stream and reads the result there."""
    shapes = CONCURRENT_SETS[classes]
    ps, gs, ms = muon_inputs(shapes, seed=7)
    runs = []
    for limit in (0.0, HipMuon.concurrent_flops_limit):
        params = []
        for p, g in zip(ps, gs):
            q = torch.nn.Parameter(p.to(gpu))
            q.grad = g.to(gpu)
            params.append(q)
        opt = HipMuon(params, lr=1e-3, coeffs=COEFFS)
        opt.concurrent_flops_limit = limit
        for q, m in zip(params, ms):
            opt.momentum[q].copy_(m)
        stream = torch.cuda.Stream(device=gpu) if on_side_stream else torch.cuda.current_stream(gpu)
        stream.wait_stream(torch.cuda.current_stream(gpu))
        with torch.cuda.stream(stream):
            for _ in range(3):
                opt.step()
            assert opt._concurrent == (limit > 0)
            if limit > 0:
                side = {id(st) for st in opt._lanes.values() if st is not None}
                assert len(side) == (3 if classes == "five_classes" else 2)
            out = [q.detach().clone() for q in params] + [opt.momentum[q].clone() for q in params]
        torch.cuda.current_stream(gpu).wait_stream(stream)
        runs.append(out)
    torch.cuda.synchronize()
    for a, b in zip(*runs):
        assert torch.equal(a, b)


# Launch groups that exercise the tile and storage choices: two block rows
# (m just above 128, lower-triangle A and B), ragged n, tall matrices, the
# 256-wide tile from m = 1024 in groups of 8 or more (and the padding rule
# that keeps the 128 tile), m >= 2048, and the 128 x 192 update tile on
# ragged matrices.
SWEEP = [(3, (200, 520)), (5, (700, 260)), (1, (129, 4000)), (8, (1024, 1300)), (9, (1100, 2100)),
         (8, (1024, 2100)), (8, (1280, 2560)), (8, (4096, 1024)), (2, (2100, 2300)),
         # 128 x 192 update tiles over ragged edges (padded 768 x 768, 32 x 6 x 4 = 768 tiles), both orientations
         (32, (700, 760)), (32, (760, 700))]


@pytest.mark.parametrize("count,shape", SWEEP)
def test_group_sweep_vs_torch(gpu, count, shape):
    """A launch group of ``count`` matrices of ``shape``: every matrix's update
    (recovered from the parameter change, in float64) against torch's
    Newton-Schulz (``torch.optim._muon._zeropower_via_newtonschulz``) of the
    same Nesterov blend, relative Frobenius error <= 1e-2."""
    from torch.optim._muon import _zeropower_via_newtonschulz
    from triton_muon_adamw.muon.hip_muon import gemm_tile
    lr, wd = 2e-2, 0.1
    ps, gs, ms, params, opt = _run_muon([shape] * count, gpu, seed=11, lr=lr, weight_decay=wd)
    mom0 = [opt.momentum[p].clone() for p in params]
    opt.step()
    torch.cuda.synchronize()
    assert [c.n for c in opt._calls] == [count]
    m_, n_ = min(shape), max(shape)
    assert gemm_tile(m_, n_, count) == (256 if m_ >= 2048 or shape in ((1024, 2100), (1280, 2560), (4096, 1024))
                                        else 128)
    keep = 1 - lr * wd
    slr = scaled_lr(lr, "original", *shape)
    for p0, p, g, m0 in zip(ps, params, gs, mom0):
        g = g.to(gpu)
        mom = m0.lerp(g, 1 - 0.95)
        ref = _zeropower_via_newtonschulz(g.lerp(mom, 0.95), COEFFS, 5, 1e-7).double()
        u = (p0.to(gpu).double() * keep - p.detach().double()) / slr
        err = ((u - ref).norm() / ref.norm()).item()
        assert err <= 1e-2, f"{count} x {shape}: update rel err {err} against torch's Newton-Schulz"


@pytest.mark.parametrize("shape", [(200, 520), (520, 200)])
def test_zero_gradient_members_only_decay(gpu, shape):
    """A launch group whose members 1 and 3 have zero gradient and zero
    momentum: X = 0, so ||X|| = 0 and X / max(||X||, eps) = 0 (torch's
    clamp), the Newton-Schulz iterate stays 0 and the parameter only decays,
    p * (1 - lr * wd) bit for bit as torch computes it; the momentum stays 0.
    The other members, in the same launches, match torch's Newton-Schulz."""
    from torch.optim._muon import _zeropower_via_newtonschulz
    lr, wd, zero = 2e-2, 0.1, (1, 3)
    ps, gs, ms, params, opt = _run_muon([shape] * 5, gpu, seed=13, lr=lr, weight_decay=wd)
    for i in zero:
        params[i].grad.zero_()
        opt.momentum[params[i]].zero_()
    mom0 = [opt.momentum[p].clone() for p in params]
    opt.step()
    torch.cuda.synchronize()
    assert [c.n for c in opt._calls] == [5]
    keep = 1 - lr * wd
    slr = scaled_lr(lr, "original", *shape)
    for i, (p0, p, g, m0) in enumerate(zip(ps, params, gs, mom0)):
        p0 = p0.to(gpu)
        if i in zero:
            assert torch.equal(p.detach(), p0 * keep), f"member {i}: not a pure decay"
            assert not opt.momentum[p].any()
            continue
        g = g.to(gpu)
        mom = m0.lerp(g, 1 - 0.95)
        ref = _zeropower_via_newtonschulz(g.lerp(mom, 0.95), COEFFS, 5, 1e-7).double()
        u = (p0.double() * keep - p.detach().double()) / slr
        err = ((u - ref).norm() / ref.norm()).item()
        assert err <= 1e-2, f"member {i}: update rel err {err} against torch's Newton-Schulz"


@pytest.mark.parametrize("shape", [(768, 3072), (1024, 4096), (4096, 4096), (14336, 4096)])
def test_config3_ns_vs_torch(gpu, shape):
    """Config 3 shapes: blend momentum (beta 0.95, Nesterov), NS in bf16 vs torch's routine on the GPU."""
    from torch.optim._muon import _zeropower_via_newtonschulz

    ps, gs, ms = muon_inputs([shape], seed=1)
    p = torch.nn.Parameter(ps[0].to(gpu))
    g = gs[0].to(gpu)
    m = ms[0].to(gpu)
    out = torch.empty_like(p)
    w = p.detach().clone()
    m_ref = m.clone()
    muon_step(w, g, m, 0.95, *COEFFS, 1e-3, scaled_lr(1e-3, "original", *shape), 0.1, 5, 1e-7, True, out=out)
    m_ref.lerp_(g, 1 - 0.95)
    u = g.lerp(m_ref, 0.95)
    ref = _zeropower_via_newtonschulz(u, COEFFS, 5, 1e-7).float()
    torch.cuda.synchronize()
    torch.testing.assert_close(m, m_ref, atol=0, rtol=2.4e-7)  # lerp with one fma: <= 2 ulp of torch's
    err = (out - ref).norm().item() / ref.norm().item()
    assert err <= 1e-2, f"{shape}: NS rel err vs torch {err}"



def test_config3_concurrent_step_vs_torch(gpu):
    """Config 3 as bench.py times it: the five matrices in one HipMuon.step(),
    whose four shape classes run concurrently (the longest on the caller's
    stream, the others on side streams), with the seeded values of
    bench_ns_c3 (params N(0, 0.02), gradients N(0, 1), momentum N(0, 1e-3)).
    Every matrix: momentum within 2 ulp of torch's lerp_, and the update
    against torch's Newton-Schulz of the same Nesterov blend, relative
    Frobenius error <= 1e-2 (muon_benchmark.py:105)."""
    from helpers import C3_SHAPES
    from torch.optim._muon import _zeropower_via_newtonschulz

    gen = torch.Generator(device=gpu).manual_seed(1)
    params = []
    for s in C3_SHAPES:
        p = torch.nn.Parameter(torch.empty(s, device=gpu).normal_(0.0, 0.02, generator=gen))
        p.grad = torch.empty(s, device=gpu).normal_(0.0, 1.0, generator=gen)
        params.append(p)
    opt = HipMuon(params, lr=1e-3, weight_decay=0.1, coeffs=COEFFS, nesterov=True, beta=0.95, ns_steps=5, eps=1e-7)
    for p in params:
        opt.momentum[p].normal_(0.0, 1e-3, generator=gen)
    p0 = [p.detach().clone() for p in params]
    m0 = [opt.momentum[p].clone() for p in params]
    opt.step()
    torch.cuda.synchronize()
    assert opt._concurrent and len({c.group for c in opt._calls}) == 4
    assert any(st is not None for st in opt._lanes.values())
    keep = 1 - 1e-3 * 0.1
    for q0, p, mom0 in zip(p0, params, m0):
        g = p.grad
        mom = mom0.lerp(g, 1 - 0.95)
        torch.testing.assert_close(opt.momentum[p], mom, atol=0, rtol=2.4e-7)
        ref = _zeropower_via_newtonschulz(g.lerp(mom, 0.95), COEFFS, 5, 1e-7).double()
        u = (q0.double() * keep - p.detach().double()) / scaled_lr(1e-3, "original", *p.shape)
        err = ((u - ref).norm() / ref.norm()).item()
        assert err <= 1e-2, f"{tuple(p.shape)}: update rel err {err} against torch's Newton-Schulz"


def _orthogonal_signs(rows, cols, rng, order=4096):
    """rows x cols, rows mutually orthogonal: distinct rows of the Sylvester
    Hadamard matrix of order `order` (entry (-1)^popcount(i & j)), with random
    column signs, placed on `order` random columns (zero elsewhere)."""
    r = rng.choice(order, size=rows, replace=False)
    x = np.bitwise_and.outer(r, np.arange(order))
    pop = np.zeros_like(x)
    while x.any():
        pop += x & 1
        x >>= 1
    h = np.where(pop & 1, -1.0, 1.0).astype(np.float32) * rng.choice([-1.0, 1.0], size=order).astype(np.float32)
    out = np.zeros((rows, cols), np.float32)
    out[:, rng.permutation(cols)[:order]] = h
    return out



@pytest.mark.parametrize("count,shape,order", [(16, (1024, 4096), 4096), (1, (14336, 4096), 4096),
                                               (16, (512, 2304), 2048)])
def test_ns_exact_on_orthogonal_rows(gpu, count, shape, order):
    """The whole Newton-Schulz pipeline on inputs where every product is exact
    in any summation order, so the result is known bit for bit.

    The gradients' rows (in the m x n orientation) are orthogonal +-1 vectors
    with `order` nonzeros (4096 or 2048); with zero momentum, beta = 0 and no
    Nesterov blend, X0 = G / ||G||_F = +-2^-e exactly (||G||_F^2 = m * order
    = 2^2e), every Gram partial sum is an integer multiple of 2^-2e below 2^24
    of them, and A = X0 X0^T = lam I with lam = order * 2^-2e.  Coefficients (0, 1/lam, 0) make B = I and
    every iterate X0 again, so with zero parameters the step writes
    -slr * X0 = -s G for one scalar s = slr * 2^-e.  A k block lost, doubled
    or summed into another tile, a block of A or B above the diagonal read
    from the wrong place, or an iterate tile written to the wrong place moves
    A off lam I or the iterates off X0 (a lost 64-column block moves 80-90% of
    an off-diagonal tile of A).  The 16 matrices of 1024 x 4096 run on
    256-wide tiles with lower-triangle A and B; each stepped alone (128-wide
    Gram and polynomial, mirrored A and B) gives the same bits.  The
    14336 x 4096 matrix runs transposed.  The 16 matrices of 512 x 2304 run
    their updates on 128 x 192 tiles (768 of them); each alone on 128 x 128."""
    from triton_muon_adamw import _lib
    rng = np.random.default_rng(17)
    m_, n_ = min(shape), max(shape)
    grads = []
    for _ in range(count):
        x = _orthogonal_signs(m_, n_, rng, order)
        grads.append(torch.from_numpy(x if shape[0] <= shape[1] else np.ascontiguousarray(x.T)))
    e2 = int(np.log2(m_)) + int(np.log2(order))  # ||G||_F^2 = m * order = 2^e2
    assert m_ * order == 2 ** e2 and e2 % 2 == 0
    e = e2 // 2
    lam = order * 2.0 ** (-2 * e)
    coeffs = (0.0, 1.0 / lam, 0.0)
    lr = 2e-2

    def make(gs):
        params = [torch.nn.Parameter(torch.zeros(shape, device=gpu)) for _ in gs]
        for q, g in zip(params, gs):
            q.grad = g.to(gpu)
        return params, HipMuon(params, lr=lr, coeffs=coeffs, beta=0.0, nesterov=False, weight_decay=0.1)

    params, opt = make(grads)
    _lib.prof_start()
    opt.step()
    _lib.prof_stop()
    assert [c.n for c in opt._calls] == [count]
    update_tiles = {r["variant"] // 8 for r in _lib.prof_collect() if r["kernel"] in ("ns_gemm_kernel:update",
                                                                                     "ns_gemm_kernel:apply")}
    assert update_tiles == ({192} if shape == (512, 2304) else {256})
    slr = scaled_lr(lr, "original", *shape)
    for i, (q, g) in enumerate(zip(params, grads)):
        got = q.detach().cpu()
        s = got.abs().max().item()
        assert torch.equal(got, -s * g), f"matrix {i}: not -s * G ({(got != -s * g).sum().item()} elements off)"
        assert abs(s - slr * 2.0 ** -e) <= 1e-6 * slr * 2.0 ** -e, f"matrix {i}: {s}"
    if count > 1:
        singles = [make([g]) for g in grads]
        for _, o in singles:
            o.step()
        for q, (qs, _) in zip(params, singles):
            assert torch.equal(q.detach(), qs[0].detach())


def test_side_streams_are_per_thread(gpu):
    """The library's side streams are made once per calling thread and device:
    the same thread gets the same streams again, another thread its own (a
    graph capture on one thread forks its streams into the capture, so they
    must not be shared with a thread stepping eagerly meanwhile); a thread
    that ends hands its streams on to the next thread."""
    import gc
    import threading

    from triton_muon_adamw import _lib
    mine = [s.cuda_stream for s in _lib.side_streams(gpu, 2)]
    assert [s.cuda_stream for s in _lib.side_streams(gpu, 2)] == mine
    assert [s.cuda_stream for s in _lib.side_streams(gpu, 1)] == mine[:1]
    other = []
    t = threading.Thread(target=lambda: other.extend(s.cuda_stream for s in _lib.side_streams(gpu, 2)))
    t.start()
    t.join()
    assert len(other) == 2 and not set(other) & set(mine)
    # the ended thread's streams go to the next thread instead of new ones
    gc.collect()
    later = []
    t = threading.Thread(target=lambda: later.extend(s.cuda_stream for s in _lib.side_streams(gpu, 2)))
    t.start()
    t.join()
    assert set(later) == set(other)
