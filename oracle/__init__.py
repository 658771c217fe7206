"""CPU oracle of the offloaded Qwen3-MoE verification path.

TEST INFRASTRUCTURE ONLY.  Only ``tests/``, ``__graft_entry__.smoke()`` and
the ``cpu_baseline`` leg of ``bench.py`` may import this package, and only to
check results (or as the timed CPU baseline).  The product path
(``specfit_amd``) never imports it and fails loudly when its HIP library is
missing.

What it restates (paths relative to the SpecFit tree; ``tf:`` is
transformers/models/qwen3_moe/modeling_qwen3_moe.py):

* ``router``        tf:258-267 -- bit-exact with the GPU kernel: the fp32
  summation order of the logit dot products and of the softmax sum and the
  ``exp`` are fixed by contract and evaluated in C (``oracle.c``).
* ``dispatch``      qwen3_offloaded_experts.py:173-178 (stable sort of routes
  by expert id, counts, offsets) -- C counting sort.
* ``combine``       qwen3_offloaded_experts.py:144-164, 200-202 (index_add_
  in canonical or arrival order, bf16 or fp32 accumulation) -- C.
* ``expert_forward_bf16`` qwen3_offloaded_experts.py:38-62 with the bf16
  rounding points of the eager reference (numpy fp32 GEMMs, bf16 rounding
  after each op), ``expert_forward_fp32`` the same without rounding.
* ``moe_forward_bf16`` / ``moe_forward_fp32``: whole MoE layer (router output
  given) -- the per-expert loop of qwen3_offloaded_experts.py:98-164.
* ``lru`` module: the cache's LRU victim rule and access sequence,
  src/specfit/replay.py:217-279 / gpu_expert_cache.py:224-266,495-518.

How each part is pinned (tests/test_oracle_*.py): router against
transformers' Qwen3MoeTopKRouter on torch CPU (golden fixtures) and the exact
fp64 dot products; dispatch against numpy's stable argsort; combine against
the reference test's known answer (1 + 2^-8 - 1) and torch CPU index_add_;
expert math against transformers' eager Qwen3MoeExperts (golden fixtures) and
the fp32 closed form; LRU against the reference's known answers.
"""
from __future__ import annotations

import ctypes
import os
from typing import Sequence

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "liboracle.so")
_lib = None


def build() -> str:
    """Compile oracle.c into _build/liboracle.so (gcc, -ffp-contract=off)."""
    import subprocess

    subprocess.run(["make", "-s", "-B", "-C", _HERE], check=True)
    return _LIB_PATH


def _load():
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(_LIB_PATH):
        build()
    lib = ctypes.CDLL(_LIB_PATH)
    p = ctypes.c_void_p
    i = ctypes.c_int
    lib.oracle_router.argtypes = [p, p, i, i, i, i, i, p, p, p, p]
    lib.oracle_router.restype = None
    lib.oracle_dispatch.argtypes = [p, i, i, i, p, p, p, p]
    lib.oracle_dispatch.restype = None
    lib.oracle_combine.argtypes = [p, p, p, p, i, i, i, i, i, p]
    lib.oracle_combine.restype = None
    lib.oracle_exp_nonpos.argtypes = [ctypes.c_float]
    lib.oracle_exp_nonpos.restype = ctypes.c_float
    _lib = lib
    return lib


def _ptr(a: np.ndarray | None):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


# ------------------------------------------------------------------ bf16 --
def bf16_bits(x: np.ndarray) -> np.ndarray:
    """fp32 values -> bf16 bit patterns (uint16), round to nearest even."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    if nan.any():
        r = np.where(nan, ((u >> 16) | 0x40).astype(np.uint16), r)
    return r


def bf16_float(bits: np.ndarray) -> np.ndarray:
    """bf16 bit patterns -> fp32 values (exact)."""
    return (np.ascontiguousarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def round_bf16(x: np.ndarray) -> np.ndarray:
    return bf16_float(bf16_bits(x))


def exp_nonpos(x: float) -> float:
    return float(_load().oracle_exp_nonpos(float(x)))


# ---------------------------------------------------------------- router --
def router(hidden_bits: np.ndarray, weight_bits: np.ndarray, top_k: int,
           norm_topk_prob: bool = True):
    """Returns (logits bf16 bits [T,E], weights bf16 bits [T,K], index int64
    [T,K], probs fp32 [T,E])."""
    h = np.ascontiguousarray(hidden_bits, dtype=np.uint16)
    w = np.ascontiguousarray(weight_bits, dtype=np.uint16)
    T, H = h.shape
    E = w.shape[0]
    if w.shape[1] != H or not 1 <= top_k <= min(E, 32) or E > 256:
        raise ValueError("unsupported router shape")
    logits = np.zeros((T, E), np.uint16)
    topw = np.zeros((T, top_k), np.uint16)
    topi = np.zeros((T, top_k), np.int64)
    probs = np.zeros((T, E), np.float32)
    if T:
        _load().oracle_router(_ptr(h), _ptr(w), T, H, E, top_k, int(bool(norm_topk_prob)),
                              _ptr(logits), _ptr(topw), _ptr(topi), _ptr(probs))
    return logits, topw, topi, probs


# -------------------------------------------------------------- dispatch --
def dispatch(index: np.ndarray, num_experts: int):
    """Returns (counts [E+1] (last = invalid entries), offsets [E+1],
    perm_pos [N], inv_perm [N])."""
    idx = np.ascontiguousarray(index, dtype=np.int64)
    T, K = idx.shape
    n = T * K
    counts = np.zeros(num_experts + 1, np.int32)
    offsets = np.zeros(num_experts + 1, np.int32)
    perm = np.full(n, -1, np.int32)
    inv = np.full(n, -1, np.int32)
    _load().oracle_dispatch(_ptr(idx), T, K, num_experts, _ptr(counts), _ptr(offsets),
                            _ptr(perm), _ptr(inv))
    return counts, offsets, perm, inv


# --------------------------------------------------------------- combine --
def combine(rows_bits: np.ndarray, index: np.ndarray, inv_perm: np.ndarray,
            num_experts: int, expert_rank: Sequence[int] | None = None,
            accumulate_fp32: bool = False) -> np.ndarray:
    rows = np.ascontiguousarray(rows_bits, dtype=np.uint16)
    idx = np.ascontiguousarray(index, dtype=np.int64)
    inv = np.ascontiguousarray(inv_perm, dtype=np.int32)
    T, K = idx.shape
    H = rows.shape[1] if rows.ndim == 2 else 0
    out = np.zeros((T, H), np.uint16)
    rank = None if expert_rank is None else np.ascontiguousarray(expert_rank, dtype=np.int32)
    if T and H:
        _load().oracle_combine(_ptr(rows), _ptr(idx), _ptr(inv), _ptr(rank), T, K,
                               num_experts, H, int(bool(accumulate_fp32)), _ptr(out))
    return out


# ----------------------------------------------------------- expert math --
def _split(packed: np.ndarray, H: int, I: int):
    p = np.asarray(packed, dtype=np.float32).reshape(-1)
    if p.size != 3 * H * I:
        raise ValueError("packed expert has the wrong size")
    gu = p[: 2 * H * I].reshape(2 * I, H)
    down = p[2 * H * I:].reshape(H, I)
    return gu, down


def _silu(x: np.ndarray) -> np.ndarray:
    return (x / (1.0 + np.exp(-x.astype(np.float64)))).astype(np.float32)


def expert_forward_bf16(x: np.ndarray, packed: np.ndarray, H: int, I: int) -> np.ndarray:
    """bf16 eager semantics of _expert_forward: fp32 GEMMs, bf16 rounding after
    the gate/up GEMM, after silu, after the product and after the down GEMM.
    x and packed hold fp32 values of bf16 numbers; returns fp32 values of bf16
    numbers."""
    gu, down = _split(packed, H, I)
    g_u = round_bf16(np.asarray(x, np.float32) @ gu.T)
    g, u = g_u[:, :I], g_u[:, I:]
    act = round_bf16(round_bf16(_silu(g)) * u)
    return round_bf16(act @ down.T)


def expert_forward_fp32(x: np.ndarray, packed: np.ndarray, H: int, I: int) -> np.ndarray:
    """Same closed form with no intermediate rounding (fp64 accumulate)."""
    gu, down = _split(packed, H, I)
    g_u = np.asarray(x, np.float64) @ gu.T.astype(np.float64)
    g, u = g_u[:, :I], g_u[:, I:]
    act = g / (1.0 + np.exp(-g)) * u
    return (act @ down.T.astype(np.float64)).astype(np.float32)


def moe_rows_bf16(hidden: np.ndarray, index: np.ndarray, weights: np.ndarray,
                  experts: dict, H: int, I: int, num_experts: int):
    """Scaled expert output rows in dispatch order (what the GPU's grouped
    SwiGLU writes): row r = bf16(bf16(expert(x_t)) * w_route)."""
    counts, offsets, perm, inv = dispatch(index, num_experts)
    K = index.shape[1]
    rows = np.zeros((perm.size, H), np.float32)
    wflat = np.asarray(weights, np.float32).reshape(-1)
    for e in range(num_experts):
        a, b = int(offsets[e]), int(offsets[e + 1])
        if a == b:
            continue
        pos = perm[a:b]
        y = expert_forward_bf16(hidden[pos // K], experts[e], H, I)
        rows[a:b] = round_bf16(y * wflat[pos][:, None])
    return rows, counts, offsets, perm, inv


def moe_forward_bf16(hidden: np.ndarray, index: np.ndarray, weights: np.ndarray,
                     experts: dict, H: int, I: int, num_experts: int,
                     expert_rank: Sequence[int] | None = None,
                     accumulate_fp32: bool = False) -> np.ndarray:
    """HF-eager bf16 semantics of one MoE layer (router output given):
    per-expert SwiGLU, bf16 weight scale, sequential bf16 index_add_ in
    canonical (or the given) expert order.  Returns fp32 values of bf16."""
    rows, counts, offsets, perm, inv = moe_rows_bf16(hidden, index, weights, experts, H, I,
                                                     num_experts)
    if counts[num_experts]:
        raise KeyError("routing index outside the expert range")
    out = combine(bf16_bits(rows), index, inv, num_experts, expert_rank, accumulate_fp32)
    return bf16_float(out)


def moe_forward_fp32(hidden: np.ndarray, index: np.ndarray, weights: np.ndarray,
                     experts: dict, H: int, I: int) -> np.ndarray:
    """fp32 reference of one MoE layer: out[t] = sum_j w[t,j] * expert_j(x_t),
    no intermediate rounding (weights upcast)."""
    T, K = index.shape
    out = np.zeros((T, H), np.float64)
    w = np.asarray(weights, np.float64)
    for e in np.unique(index):
        tok, j = np.nonzero(index == e)
        y = expert_forward_fp32(hidden[tok], experts[int(e)], H, I).astype(np.float64)
        np.add.at(out, tok, y * w[tok, j][:, None])
    return out.astype(np.float32)
