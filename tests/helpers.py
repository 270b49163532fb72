"""Seeded synthetic inputs shared by the tests and bench.py.

Every value is drawn on the CPU from a seeded ``torch.Generator`` so CPU and
GPU runs see identical bits.
"""

from __future__ import annotations

import numpy as np
import torch

GPT2_MUON_SHAPES = [(768, 2304), (768, 768), (768, 3072), (3072, 768)]  # per layer: qkv, proj, fc, mlp-proj


def c2_sizes(n: int = 256, total: int = 1 << 26, seed: int = 0) -> list[int]:
    """Config 2 tensor sizes: log-uniform in [1e3, 4e6], scaled to sum to ``total``."""
    rng = np.random.default_rng(seed)
    raw = np.exp(rng.uniform(np.log(1e3), np.log(4e6), n))
    sizes = np.clip(np.round(raw * total / raw.sum()), 1000, 4_000_000).astype(np.int64)
    order = np.argsort(-sizes)
    diff = int(total - sizes.sum())
    i = 0
    while diff != 0:  # nudge the largest tensors until the sum is exact
        j = order[i % n]
        step = max(diff, -(int(sizes[j]) - 1000)) if diff < 0 else min(diff, 4_000_000 - int(sizes[j]))
        sizes[j] += step
        diff -= step
        i += 1
    return [int(s) for s in sizes]


def randn(shape, std: float, gen: torch.Generator) -> torch.Tensor:
    return torch.randn(shape, generator=gen, dtype=torch.float32) * std


def adamw_state(sizes, seed: int = 0):
    """(params, grads, exp_avg, exp_avg_sq) lists of CPU fp32 tensors, config 2 distributions."""
    gen = torch.Generator().manual_seed(seed)
    ps = [randn(s, 0.02, gen) for s in sizes]
    gs = [randn(s, 1e-3, gen) for s in sizes]
    ms = [randn(s, 1e-4, gen) for s in sizes]
    vs = [randn(s, 1e-6, gen).abs() for s in sizes]
    return ps, gs, ms, vs


def muon_inputs(shapes, seed: int = 1, grad_std: float = 1.0, mom_std: float = 1e-3, param_std: float = 0.02):
    """(params, grads, momentum) lists of CPU fp32 tensors for the given shapes."""
    gen = torch.Generator().manual_seed(seed)
    ps = [randn(s, param_std, gen) for s in shapes]
    gs = [randn(s, grad_std, gen) for s in shapes]
    ms = [randn(s, mom_std, gen) for s in shapes]
    return ps, gs, ms


def rel_fro(a, b) -> float:
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


# ---------------------------------------------------------------------------
# Parameter layouts of the benchmark configurations: (name, shape, branch).

def gpt2_layout(n_layer: int = 12, d: int = 768, vocab: int = 50257, n_ctx: int = 1024):
    """GPT-2-small (config 4), HF Conv1D weight layout (in, out); tied LM head.

    Explicit routing as config 4: the four per-layer matrices to Muon,
    embeddings, LayerNorms and biases to AdamW (48 Muon + 100 AdamW tensors).
    """
    out = [("wte", (vocab, d), "adam"), ("wpe", (n_ctx, d), "adam")]
    for i in range(n_layer):
        out += [
            (f"h{i}.ln_1.w", (d,), "adam"), (f"h{i}.ln_1.b", (d,), "adam"),
            (f"h{i}.attn.c_attn.w", (d, 3 * d), "muon"), (f"h{i}.attn.c_attn.b", (3 * d,), "adam"),
            (f"h{i}.attn.c_proj.w", (d, d), "muon"), (f"h{i}.attn.c_proj.b", (d,), "adam"),
            (f"h{i}.ln_2.w", (d,), "adam"), (f"h{i}.ln_2.b", (d,), "adam"),
            (f"h{i}.mlp.c_fc.w", (d, 4 * d), "muon"), (f"h{i}.mlp.c_fc.b", (4 * d,), "adam"),
            (f"h{i}.mlp.c_proj.w", (4 * d, d), "muon"), (f"h{i}.mlp.c_proj.b", (d,), "adam"),
        ]
    out += [("ln_f.w", (d,), "adam"), ("ln_f.b", (d,), "adam")]
    return out


def llama8b_layout(n_layer: int = 32, d: int = 4096, kv: int = 1024, ffn: int = 14336, vocab: int = 128256):
    """Llama-3-8B (config 5), torch Linear layout (out, in); untied LM head.

    Muon: q, k, v, o, gate, up, down of every layer (224 matrices); AdamW:
    embedding, LM head and the 65 RMSNorm weights (67 tensors).
    """
    out = [("embed", (vocab, d), "adam")]
    for i in range(n_layer):
        out += [
            (f"l{i}.attn_norm", (d,), "adam"),
            (f"l{i}.q", (d, d), "muon"), (f"l{i}.k", (kv, d), "muon"), (f"l{i}.v", (kv, d), "muon"),
            (f"l{i}.o", (d, d), "muon"),
            (f"l{i}.mlp_norm", (d,), "adam"),
            (f"l{i}.gate", (ffn, d), "muon"), (f"l{i}.up", (ffn, d), "muon"), (f"l{i}.down", (d, ffn), "muon"),
        ]
    out += [("norm", (d,), "adam"), ("lm_head", (vocab, d), "adam")]
    return out


C3_SHAPES = [(768, 3072), (1024, 4096), (4096, 4096), (1024, 4096), (14336, 4096)]


def ns_flops(shape, ns_steps: int = 5) -> float:
    """Symmetric-minimal Newton-Schulz work: ns_steps * (3 m^2 n + m^3), m = min, n = max."""
    m, n = min(shape), max(shape)
    return float(ns_steps) * (3.0 * m * m * n + float(m) ** 3)
