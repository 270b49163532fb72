"""bf16 parameters and gradients with fp32 optimizer state, on the GPU.

No counterpart in the reference (its kernels compute in the parameter's dtype,
triton_adam.py:79-85, triton_muon.py:407-412).  Semantics (oracle/adamw.py,
oracle/muon.py; pinned there against torch.optim in fp32 with the parameter
rounded to bf16 after every step): bf16 values are widened exactly, the update
runs in fp32 with fp32 moments / momentum, and a bf16 parameter is rounded
back to nearest-even.

* AdamW, every combination of bf16 / fp32 parameter and gradient, ragged sizes
  (vector and scalar paths, an unaligned view): bit-exact against the oracle.
* Muon, bf16 parameter and gradient, wide and tall: momentum bit-exact, the
  parameter within one bf16 ulp plus the bf16 noise of the orthogonalised
  update (the fp32 Muon tests' tolerance), and always a bf16 value.
"""

import numpy as np
import pytest
import torch

import oracle
from triton_muon_adamw.adamw import HipAdamW
from triton_muon_adamw.muon import HipMuon

pytestmark = pytest.mark.gpu

HP = dict(lr=3e-4, betas=(0.9, 0.95), weight_decay=0.1, eps=1e-8)
SIZES = [1, 3, 5, 1000, 1023, 1024, 1025, 4099, 12288]


@pytest.mark.parametrize("pdt,gdt", [(torch.bfloat16, torch.bfloat16), (torch.float32, torch.bfloat16),
                                     (torch.bfloat16, torch.float32)])
def test_adamw_bf16_bitexact_vs_oracle(gpu, pdt, gdt):
    gen = torch.Generator().manual_seed(11)
    host = [(torch.randn(n, generator=gen) * 0.02).to(pdt) for n in SIZES]
    params = [torch.nn.Parameter(h.to(gpu)) for h in host]
    base = (torch.randn(3001, generator=gen) * 0.02).to(pdt).to(gpu)
    params.append(torch.nn.Parameter(base[1:]))  # 2-byte / 4-byte offset view: scalar path
    if pdt != gdt:
        for p in params:
            p.grad_dtype = None  # torch otherwise insists that grad.dtype == param.dtype
    opt = HipAdamW(params, **HP)
    ref = oracle.adamw.AdamWOracle([p.detach().float().cpu().numpy().copy() for p in params], **HP,
                                   param_bf16=pdt == torch.bfloat16)
    for _ in range(3):
        grads = [(torch.randn(p.shape, generator=gen) * 1e-3).to(gdt) for p in params]
        for p, g in zip(params, grads):
            p.grad = g.to(gpu)
        opt.step()
        ref.step([g.float().numpy() for g in grads])
    torch.cuda.synchronize()
    for i, p in enumerate(params):
        assert p.dtype == pdt
        assert np.array_equal(p.detach().float().cpu().numpy(), ref.params[i]), f"tensor {i} ({p.numel()})"
        assert np.array_equal(opt.m[p].cpu().numpy(), ref.m[i])
        assert np.array_equal(opt.v[p].cpu().numpy(), ref.v[i])


@pytest.mark.parametrize("shape", [(256, 512), (512, 256), (100, 37), (640, 1280)])
def test_muon_bf16_vs_oracle(gpu, shape):
    gen = torch.Generator().manual_seed(12)
    p0 = (torch.randn(shape, generator=gen) * 0.02).bfloat16()
    g0 = torch.randn(shape, generator=gen).bfloat16()
    m0 = torch.randn(shape, generator=gen) * 1e-3
    p = torch.nn.Parameter(p0.to(gpu))
    opt = HipMuon([p], lr=2e-2, weight_decay=0.1, coeffs=(3.4445, -4.7750, 2.0315), nesterov=True, beta=0.95,
                  ns_steps=5, eps=1e-7)
    assert opt.momentum[p].dtype == torch.float32
    opt.momentum[p].copy_(m0.to(gpu))
    p.grad = g0.to(gpu)
    opt.step()
    torch.cuda.synchronize()
    op, om_, _ = oracle.muon.muon_update(p0.float().numpy(), g0.float().numpy(), m0.numpy(), lr=2e-2,
                                         weight_decay=0.1, beta=0.95, nesterov=True,
                                         coeffs=(3.4445, -4.7750, 2.0315), ns_steps=5, eps=1e-7,
                                         param_bf16=True)
    assert p.dtype == torch.bfloat16
    assert np.array_equal(opt.momentum[p].cpu().numpy(), om_)
    got = p.detach().float().cpu().numpy()
    adj = oracle.muon.adjust_lr(2e-2, "original", shape)
    ulp = np.exp2(np.floor(np.log2(np.maximum(np.abs(op), 1e-30))) - 7)
    assert (np.abs(got - op) <= ulp + adj * 8e-3).all()
    keep = np.float32(1 - 2e-2 * 0.1)
    u_got = (p0.float().numpy() * keep - got) / adj
    u_ref = (p0.float().numpy() * keep - op) / adj
    # A bf16 parameter quantises the step: one ulp of p (~1.2e-4 at |p| ~ 0.02) is a quarter of a typical
    # update (adj * |u| ~ 5e-4), so elements whose update sits near a rounding boundary flip by one ulp.
    assert np.linalg.norm(u_got - u_ref) / np.linalg.norm(u_ref) < 5e-2


@pytest.mark.parametrize("shapes,tile", [([(1024, 2048)] * 4 + [(2048, 1024)] * 4, 256),
                                         ([(768, 3072)] * 6 + [(3072, 768)] * 6, 192)])
def test_muon_bf16_params_batched_equal_single(gpu, shapes, tile):
    """bf16 parameters through the batched APPLY epilogues of the 256 x 256
    tile and of the 128 x 192 update tile (the group of 8 or 12) against each
    matrix stepped alone (128 x 128 tiles): the same products in the same
    order, so parameters and momenta agree bit for bit, both orientations."""
    from triton_muon_adamw import _lib
    gen = torch.Generator().manual_seed(13)
    vals = [((torch.randn(s, generator=gen) * 0.02).bfloat16(), torch.randn(s, generator=gen).bfloat16(),
             torch.randn(s, generator=gen) * 1e-3) for s in shapes]
    kw = dict(lr=2e-2, weight_decay=0.1, coeffs=(3.4445, -4.7750, 2.0315), nesterov=True, beta=0.95, ns_steps=5,
              eps=1e-7)

    def make(p0, g0, m0):
        p = torch.nn.Parameter(p0.to(gpu))
        p.grad = g0.to(gpu)
        return p

    group = [make(*v) for v in vals]
    opt = HipMuon(group, **kw)
    for p, v in zip(group, vals):
        opt.momentum[p].copy_(v[2].to(gpu))
    _lib.prof_start()
    opt.step()
    _lib.prof_stop()
    assert {r["variant"] // 8 for r in _lib.prof_collect() if r["kernel"] == "ns_gemm_kernel:apply"} == {tile}
    for v, p in zip(vals, group):
        q = make(*v)
        o = HipMuon([q], **kw)
        o.momentum[q].copy_(v[2].to(gpu))
        o.step()
        torch.cuda.synchronize()
        assert q.dtype == torch.bfloat16
        assert torch.equal(p.detach(), q.detach())
        assert torch.equal(opt.momentum[p], o.momentum[q])
