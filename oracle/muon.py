"""Muon oracle (test infrastructure only).

Restates one Muon update of a 2-D fp32 parameter as the reference defines it:
``muon_step`` (``MuonAdamW package/triton_muon_adamw/muon/triton_muon.py:327-372``)
and, for the rounding points, the torch routine the reference's wrapper
``PyTorchMuonAdamW`` delegates to (``optimizer.py:228-241`` ->
``torch/optim/_muon.py:31-84,304-318``, torch 2.10):

    momentum = lerp(momentum, grad, 1 - beta)            _muon.py:310  (triton_muon.py:346)
    u        = lerp(grad, momentum, beta) if nesterov     _muon.py:311  (triton_muon.py:348-349)
    X        = bf16(u), transposed if rows > cols         _muon.py:55-57 (triton_muon.py:351-354)
    X        = bf16(X / bf16(max(bf16(||X||_F), eps)))    _muon.py:59    (triton_muon.py:356)
    repeat ns_steps:                                      _muon.py:61-66 (triton_muon.py:358-363)
        A = bf16(X X^T)                                   fp32 accumulate
        B = bf16(c * (A A) + b * A)                       addmm epilogue in fp32
        X = bf16(a * X + B X)
    param    = param * (1 - lr * weight_decay)            _muon.py:317   (triton_muon.py:370)
    param    = param - adjusted_lr * X (transposed back)  _muon.py:318   (triton_muon.py:365-372)

``lerp`` is torch's (ATen Lerp.h): weights below 0.5 interpolate from the
start, others from the end, each with one fused multiply-add in fp32.
numpy has no fma; ``fma32`` evaluates it in float64 and rounds once to
float32 (exact except for double-rounding ties, about 1 in 2**29 inputs).
"""

from __future__ import annotations

import math

import numpy as np

from .bf16 import round_bf16

F32 = np.float32


def fma32(a, b, c) -> np.ndarray:
    """float32 fused multiply-add a*b + c (float64 evaluation, one final rounding)."""
    return (np.float64(a) * np.asarray(b, dtype=np.float64) + np.asarray(c, dtype=np.float64)).astype(F32)


def lerp(start, end, weight) -> np.ndarray:
    """torch.lerp(start, end, weight) for float32 arrays and a scalar weight."""
    start = np.asarray(start, dtype=F32)
    end = np.asarray(end, dtype=F32)
    w = F32(weight)
    diff = end - start
    if abs(w) < F32(0.5):
        return fma32(w, diff, start)
    return fma32(w - F32(1), diff, end)


def adjust_lr(lr: float, adjust_lr_fn: str | None, shape) -> float:
    """Shape-dependent learning rate.

    "original"            lr * sqrt(max(1, R/C))   torch/optim/_muon.py:77-79, triton_muon.py:424-425
    "match_rms_adamw"     lr * 0.2 * sqrt(max(R,C)) torch/optim/_muon.py:80-81 (the reference's
                          triton_muon.py:428 calls max() on an int and raises TypeError)
    "spectral_unclamped"  lr * sqrt(R/C)           triton_muon.py:430-431 (reference only)
    """
    A, B = shape[0], shape[1]
    if adjust_lr_fn is None or adjust_lr_fn == "original":
        return lr * math.sqrt(max(1, A / B))
    if adjust_lr_fn == "match_rms_adamw":
        return lr * (0.2 * math.sqrt(max(A, B)))
    if adjust_lr_fn == "spectral_unclamped":
        return lr * math.sqrt(A / B)
    raise AssertionError(f"Invalid adjust_lr_fn: {adjust_lr_fn}")


def frobenius_norm_bf16(X: np.ndarray) -> np.float32:
    """bf16(||X||_F) for bf16-valued X: sum of squares, sqrt, round to bf16."""
    s = np.sum(np.square(X, dtype=np.float64))
    return round_bf16(np.float32(math.sqrt(s)))[()]


def zeropower_ns(G, coeffs=(3.4445, -4.7750, 2.0315), ns_steps=5, eps=1e-7, exact=False) -> np.ndarray:
    """Newton-Schulz orthogonalisation of a 2-D array (torch/optim/_muon.py:31-70).

    ``exact=False``: bf16 iterates with fp32 products, rounded where torch rounds.
    ``exact=True``:  the same recurrence in float64 with no rounding (the
    closed form on singular values applies to it exactly).
    """
    a, b, c = coeffs
    G = np.asarray(G)
    tall = G.shape[0] > G.shape[1]
    if exact:
        X = G.astype(np.float64)
        if tall:
            X = X.T
        X = X / max(np.linalg.norm(X), eps)
        for _ in range(ns_steps):
            A = X @ X.T
            B = b * A + c * (A @ A)
            X = a * X + B @ X
        return X.T if tall else X
    X = round_bf16(G.astype(F32))
    if tall:
        X = np.ascontiguousarray(X.T)
    nrm = frobenius_norm_bf16(X)
    nrm = round_bf16(np.maximum(nrm, F32(eps)))[()]
    X = round_bf16(X / nrm)
    a32, b32, c32 = F32(a), F32(b), F32(c)
    for _ in range(ns_steps):
        A = round_bf16(X @ X.T)
        B = round_bf16(c32 * (A @ A) + b32 * A)
        X = round_bf16(a32 * X + B @ X)
    return np.ascontiguousarray(X.T) if tall else X


def muon_update(param, grad, momentum, *, lr, weight_decay, beta, nesterov=True,
                coeffs=(3.4445, -4.7750, 2.0315), ns_steps=5, eps=1e-7, adjust_lr_fn="original",
                param_bf16=False):
    """One Muon update; returns (new_param, new_momentum, orthogonalised update).

    ``param_bf16``: the parameter is bf16 (values arrive as float32); the
    update runs in fp32 with an fp32 momentum and the new parameter is rounded
    to bf16.  A bf16 gradient needs nothing: its values are exact in fp32.
    """
    param = np.asarray(param, dtype=F32)
    grad = np.asarray(grad, dtype=F32)
    mom = lerp(momentum, grad, 1 - beta)
    u = lerp(grad, mom, beta) if nesterov else mom
    O = zeropower_ns(u, coeffs, ns_steps, eps)
    adj = adjust_lr(lr, adjust_lr_fn, param.shape)
    p = param * F32(1 - lr * weight_decay)
    p = fma32(F32(-adj), O, p)
    if param_bf16:
        p = round_bf16(np.asarray(p, dtype=F32))
    return p, mom, O


class MuonOracle:
    """CPU model of one Muon branch (triton_muon.py:375-448) on numpy arrays."""

    def __init__(self, params, lr=1e-3, weight_decay=0.1, coeffs=(3.445, -4.775, 2.0315),
                 nesterov=True, beta=0.95, ns_steps=5, eps=1e-7, adjust_lr_fn="original", param_bf16=False):
        self.params = params
        self.kw = dict(lr=lr, weight_decay=weight_decay, beta=beta, nesterov=nesterov,
                       coeffs=coeffs, ns_steps=ns_steps, eps=eps, adjust_lr_fn=adjust_lr_fn,
                       param_bf16=param_bf16)
        self.momentum = [np.zeros_like(p, dtype=F32) for p in params]

    def step(self, grads):
        for i, (p, g) in enumerate(zip(self.params, grads)):
            if g is None:
                continue
            p_new, self.momentum[i], _ = muon_update(p, g, self.momentum[i], **self.kw)
            p[...] = p_new
