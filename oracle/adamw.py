"""AdamW oracle (test infrastructure only).

Restates the reference's AdamW kernel, ``adamw_step``
(``MuonAdamW package/triton_muon_adamw/adamw/triton_adam.py:53-59``), in IEEE
float32 with one rounding per operation (numpy never fuses a multiply-add):

    m_t = beta1 * m + (1 - beta1) * g                       (:53)
    v_t = beta2 * v + (1 - beta2) * (g * g)                 (:54)
    m_c = m_t / bias1                                       (:55)
    v_c = v_t / bias2                                       (:56)
    p   = (1 - lr * weight_decay) * p                       (:58)
    p   = p - lr * (m_c / (sqrt(v_c) + eps))                (:59)

and the step-loop semantics of ``TritonAdamW.step`` (:132-153): one global
step counter incremented on every call, bias corrections computed on the
host in float64 and passed to the kernel as float32, parameters whose grad is
``None`` skipped.

bf16 parameters and gradients (no counterpart in the reference, whose kernel
computes in the parameter's dtype, triton_adam.py:79-85): the values are
widened exactly, the update above runs in fp32 with fp32 moments, and a bf16
parameter is rounded back to nearest-even (``param_bf16=True``).  Pinned
against torch.optim.AdamW in fp32 with the parameter rounded to bf16 after
every step.
"""

from __future__ import annotations

import numpy as np

from .bf16 import round_bf16

F32 = np.float32


def bias_corrections(beta1: float, beta2: float, step: int) -> tuple[np.float32, np.float32]:
    """(1 - beta1**t, 1 - beta2**t) in float64, then float32 (triton_adam.py:147-148)."""
    return F32(1 - beta1**step), F32(1 - beta2**step)


def adamw_update(p, g, m, v, *, lr, bias1, bias2, beta1, beta2, weight_decay, eps, param_bf16=False):
    """One AdamW update of float32 arrays; returns new (p, m, v) (triton_adam.py:53-59).

    ``param_bf16``: the parameter is bf16 (its bf16 values arrive as float32);
    the new value is rounded to bf16 (returned as float32).
    """
    p = np.asarray(p, dtype=F32)
    g = np.asarray(g, dtype=F32)
    m = np.asarray(m, dtype=F32)
    v = np.asarray(v, dtype=F32)
    lr, bias1, bias2 = F32(lr), F32(bias1), F32(bias2)
    beta1, beta2, wd, eps = F32(beta1), F32(beta2), F32(weight_decay), F32(eps)
    one = F32(1)
    m_t = beta1 * m + (one - beta1) * g
    v_t = beta2 * v + (one - beta2) * (g * g)
    m_c = m_t / bias1
    v_c = v_t / bias2
    p_decay = (one - lr * wd) * p
    p_new = p_decay - lr * (m_c / (np.sqrt(v_c) + eps))
    if param_bf16:
        p_new = round_bf16(p_new.astype(F32))
    return p_new.astype(F32), m_t.astype(F32), v_t.astype(F32)


class AdamWOracle:
    """CPU model of ``TritonAdamW`` (triton_adam.py:106-161) on numpy arrays.

    ``params`` is a list of float32 arrays updated in place; ``grads`` given
    to :meth:`step` is a parallel list whose entries may be ``None``.
    """

    def __init__(self, params, lr=1e-3, betas=(0.9, 0.999), weight_decay=1e-2, eps=1e-7, param_bf16=False):
        self.params = params
        self.param_bf16 = param_bf16
        self.lr, self.beta1, self.beta2 = lr, betas[0], betas[1]
        self.weight_decay, self.eps = weight_decay, eps
        self.step_num = 0
        self.m = [np.zeros_like(p, dtype=F32) for p in params]
        self.v = [np.zeros_like(p, dtype=F32) for p in params]

    def step(self, grads):
        self.step_num += 1
        bias1, bias2 = bias_corrections(self.beta1, self.beta2, self.step_num)
        for i, (p, g) in enumerate(zip(self.params, grads)):
            if g is None:
                continue
            p_new, self.m[i], self.v[i] = adamw_update(
                p, g, self.m[i], self.v[i], lr=self.lr, bias1=bias1, bias2=bias2,
                beta1=self.beta1, beta2=self.beta2, weight_decay=self.weight_decay, eps=self.eps,
                param_bf16=self.param_bf16)
            p[...] = p_new
