"""Seeded synthetic workloads for the MoE FFN configurations.

The five configurations are the ones the drop-in is measured and checked on:

* C1 toy fp32: T=32, H=64, F=128, E=8, k=2, renormalised weights.
* C2 Mixtral-8x7B bf16: H=4096, F=14336, E=8, k=2, T in {16, 512, 4096}.
* C3 Qwen3-30B-A3B bf16: H=2048, F=768, E=128, k=8, T in {64, 2048, 8192},
  router logits biased per expert by Zipf(1.1).
* C4 DeepSeek-V2-Lite bf16: H=2048, F=1408, E=64, k=6, T in {1, 4, 16, 64}.
* C5 Mixtral fp8-e4m3 weights (per-output-channel scales), bf16 activations,
  T in {16, 4096}.

Distributions: activations N(0, 1); router and expert weights N(0, 0.02^2).
Token rows whose router probabilities have an adjacent gap below ``margin``
among the top-(k+1) are redrawn, so that top-k selection and slot order do
not depend on floating-point summation order (exact-tie order is the one
thing the reference leaves implementation-defined).  The Zipf skew of C3 is
expressed through the reference signature, which has no bias input: hidden
channel 0 of every token is 1.0 and router column 0 holds
``-1.1 * ln(rank_e)`` for a seeded permutation ``rank`` of 1..E.

Expert weights are drawn on the GPU with a seeded torch generator (one
Mixtral projection is 470M values) in the reference layout
``[n_out, n_in, E]``; tests copy them to the host for the oracle.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import Tuple

import numpy as np
import torch


@dataclass(frozen=True)
class Config:
    name: str
    n_embd: int
    n_ff: int
    n_expert: int
    n_expert_used: int
    tokens: Tuple[int, ...]
    act: str  # "f32" | "bf16"
    weights: str  # "f32" | "bf16" | "fp8"
    normalize: bool
    margin: float
    zipf: float = 0.0
    rtol: float = 1e-4
    seed: int = 0
    extra: dict = field(default_factory=dict)


CONFIGS = {
    "C1": Config("C1", 64, 128, 8, 2, (32,), "f32", "f32", True, 1e-6, rtol=1e-4, seed=1),
    "C2": Config("C2", 4096, 14336, 8, 2, (16, 512, 4096), "bf16", "bf16", False, 1e-3, rtol=2e-2, seed=2),
    "C3": Config("C3", 2048, 768, 128, 8, (64, 2048, 8192), "bf16", "bf16", True, 1e-4, zipf=1.1,
                 rtol=2e-2, seed=3),
    "C4": Config("C4", 2048, 1408, 64, 6, (1, 4, 16, 64), "bf16", "bf16", False, 1e-4, rtol=2e-2, seed=4),
    "C5": Config("C5", 4096, 14336, 8, 2, (16, 4096), "bf16", "fp8", False, 1e-3, rtol=5e-2, seed=5),
}


def scaled(cfg: Config, n_embd: int, n_ff: int, **kw) -> Config:
    """The same configuration at a smaller hidden/ffn size (for fast tests)."""
    d = dict(cfg.__dict__)
    d.update(n_embd=n_embd, n_ff=n_ff, name=cfg.name + f"-h{n_embd}f{n_ff}")
    d.update(kw)
    return Config(**d)


def bf16_round_np(a: np.ndarray) -> np.ndarray:
    """fp32 -> nearest bf16 (ties to even) -> fp32, through torch's cast."""
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(torch.bfloat16).float().numpy()


def _probs(x: np.ndarray, wr: np.ndarray) -> np.ndarray:
    logits = x.astype(np.float64) @ wr.astype(np.float64).T  # [T, E]
    e = np.exp(logits - logits.max(axis=1, keepdims=True))
    return e / e.sum(axis=1, keepdims=True)


def min_adjacent_gap(x: np.ndarray, wr: np.ndarray, k: int) -> np.ndarray:
    """Per token, the smallest gap between adjacent sorted probabilities among
    the top-(k+1) (top-k when k == E)."""
    p = -np.sort(-_probs(x, wr), axis=1)
    m = min(k + 1, p.shape[1])
    if m < 2:
        return np.full(p.shape[0], np.inf)
    return (p[:, : m - 1] - p[:, 1:m]).min(axis=1)


def router_inputs(cfg: Config, n_tokens: int, seed: int | None = None, max_rounds: int = 200):
    """-> (x [T, H] float32, wr [E, H] float32, stats), both already rounded
    to the activation dtype, with every token meeting the router margin."""
    rng = np.random.default_rng(cfg.seed * 1000003 + n_tokens if seed is None else seed)
    H, E, k = cfg.n_embd, cfg.n_expert, cfg.n_expert_used
    rnd = bf16_round_np if cfg.act == "bf16" else (lambda a: np.asarray(a, np.float32))
    wr = (rng.standard_normal((E, H), dtype=np.float32) * np.float32(0.02)).astype(np.float32)
    if cfg.zipf:
        rank = rng.permutation(E) + 1
        wr[:, 0] = (-cfg.zipf * np.log(rank)).astype(np.float32)
    wr = rnd(wr)

    def draw(n):
        x = rng.standard_normal((n, H), dtype=np.float32)
        if cfg.zipf:
            x[:, 0] = 1.0
        return rnd(x)

    x = draw(n_tokens)
    redrawn = 0
    for _ in range(max_rounds):
        bad = np.nonzero(min_adjacent_gap(x, wr, k) < cfg.margin)[0]
        if bad.size == 0:
            break
        redrawn += bad.size
        x[bad] = draw(bad.size)
    else:
        raise RuntimeError(f"{cfg.name}: could not meet router margin {cfg.margin}")
    return x, wr, {"redrawn_rows": int(redrawn)}


def expert_weights(cfg: Config, device, seed: int | None = None, dtype=torch.float32, std: float = 0.02):
    """(up [F,H,E], gate [F,H,E], down [H,F,E]) ~ N(0, std^2) (0.02 by
    default), drawn with a seeded torch generator on `device`, returned in
    `dtype`."""
    H, F, E = cfg.n_embd, cfg.n_ff, cfg.n_expert
    g = torch.Generator(device=device)
    g.manual_seed(cfg.seed * 7919 + 17 if seed is None else seed)
    out = []
    for shape in ((F, H, E), (F, H, E), (H, F, E)):
        w = torch.empty(shape, dtype=torch.float32, device=device)
        w.normal_(0.0, std, generator=g)
        out.append(w.to(dtype))
    return tuple(out)


def _rms_norm64(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    x = x.astype(np.float64)
    return x / np.sqrt(np.mean(x * x, axis=1, keepdims=True) + eps) * w.astype(np.float64)


def sublayer_inputs(cfg: Config, n_tokens: int, seed: int | None = None, eps: float = 1e-5,
                    scale_range=(0.25, 4.0), max_rounds: int = 200):
    """Inputs of the MoE FFN sub-layer (ffn_norm -> block -> residual add):
    -> (residual [T, H], ffn_norm_w [H], wr [E, H], eps, stats), rounded to the
    activation dtype.

    Residual rows are N(0, 1) times a per-row scale, log-uniform in
    ``scale_range`` (so the norm has work to do; the block's output does not
    depend on it); the norm weight is 1 + N(0, 0.1^2).  The router margin is
    enforced on the NORMALISED rows -- what the router sees -- both exact and
    rounded to the activation dtype.  For the Zipf configuration channel 0 of
    the residual equals the row's RMS scale and its norm weight is 1, so the
    normalised channel 0 stays near 1 and router column 0 keeps its bias."""
    rng = np.random.default_rng(cfg.seed * 1000033 + n_tokens + 7 if seed is None else seed)
    H, E, k = cfg.n_embd, cfg.n_expert, cfg.n_expert_used
    rnd = bf16_round_np if cfg.act == "bf16" else (lambda a: np.asarray(a, np.float32))
    wr = (rng.standard_normal((E, H), dtype=np.float32) * np.float32(0.02)).astype(np.float32)
    if cfg.zipf:
        rank = rng.permutation(E) + 1
        wr[:, 0] = (-cfg.zipf * np.log(rank)).astype(np.float32)
    wr = rnd(wr)
    nw = (1.0 + 0.1 * rng.standard_normal(H)).astype(np.float32)
    if cfg.zipf:
        nw[0] = 1.0
    nw = rnd(nw)

    def draw(n):
        lo, hi = scale_range
        scale = np.exp(rng.uniform(np.log(lo), np.log(hi), (n, 1))).astype(np.float32)
        x = rng.standard_normal((n, H), dtype=np.float32) * scale
        if cfg.zipf:
            x[:, 0] = scale[:, 0]
        return rnd(x)

    def gap(rows):
        xn = _rms_norm64(rows, nw, eps)
        return np.minimum(min_adjacent_gap(xn, wr, k), min_adjacent_gap(rnd(xn.astype(np.float32)), wr, k))

    res = draw(n_tokens)
    redrawn = 0
    for _ in range(max_rounds):
        bad = np.nonzero(gap(res) < cfg.margin)[0]
        if bad.size == 0:
            break
        redrawn += bad.size
        res[bad] = draw(bad.size)
    else:
        raise RuntimeError(f"{cfg.name}: could not meet router margin {cfg.margin}")
    return res, nw, wr, eps, {"redrawn_rows": int(redrawn)}
