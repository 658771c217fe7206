"""Input recipes of the golden fixtures whose inputs are regenerated rather
than stored (test infrastructure: imported by make_golden.py, which writes
the fixtures, and by the tests, which check a fixture's input digest first)."""
from __future__ import annotations

import hashlib

import numpy as np
import torch


def bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().contiguous().view(torch.int16).numpy().view(np.uint16)


def real_shape_inputs(T: int, H: int, E: int, seed: int, zipf_s: float | None):
    """Inputs of the Qwen3-30B-A3B-shaped router fixtures, regenerated from
    numpy's PCG64 by the test that reads the fixture: hidden N(0, 1), router
    N(0, 0.02), both rounded to bf16 by torch (round to nearest even).  With
    ``zipf_s``, the Zipf popularity bias b_e = log p_{pi(e)} (p_r ~ r^-s,
    pi a seeded permutation) is folded in: hidden feature 0 := 1, router
    column 0 := b.  Returns bf16 tensors (hidden [T,H], router [E,H])."""
    rng = np.random.default_rng(seed)
    router = rng.standard_normal((E, H), dtype=np.float32) * np.float32(0.02)
    hidden = rng.standard_normal((T, H), dtype=np.float32)
    if zipf_s is not None:
        perm = rng.permutation(E)
        p = np.arange(1, E + 1, dtype=np.float64) ** -zipf_s
        p /= p.sum()
        bias = np.empty(E, np.float64)
        bias[perm] = np.log(p)
        hidden[:, 0] = 1.0
        router[:, 0] = bias.astype(np.float32)
    return (torch.from_numpy(hidden).to(torch.bfloat16),
            torch.from_numpy(router).to(torch.bfloat16))


def input_digest(hidden: torch.Tensor, router: torch.Tensor) -> str:
    return hashlib.sha256(bits(hidden).tobytes() + bits(router).tobytes()).hexdigest()


