"""Pins the oracle's router (oracle.router / oracle.c) on the CPU.

Checks: its exp() against math.exp; its logits against the exact (fp64) dot
products rounded to bf16; its softmax against fp64; its top-k against
numpy's stable argsort of the probabilities (ties -> lower expert id); its
renormalised weights against fp64; and everything against transformers'
Qwen3MoeTopKRouter on torch CPU (golden fixtures, tests/golden/).
"""
import math
import os

import numpy as np
import pytest

import oracle

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def _rand_bits(shape, seed, std=1.0):
    rng = np.random.default_rng(seed)
    return oracle.bf16_bits((rng.standard_normal(shape) * std).astype(np.float32))


def test_exp_against_math_exp():
    xs = np.concatenate([-np.geomspace(1e-8, 86.9, 4000), np.linspace(-86.9, 0, 4001)])
    worst = 0.0
    for x in xs.astype(np.float32):
        got = oracle.exp_nonpos(float(x))
        ref = math.exp(float(x))
        worst = max(worst, abs(got - ref) / ref)
    assert worst <= 4.0e-7  # about 3 fp32 ulp
    assert oracle.exp_nonpos(0.0) == 1.0
    assert oracle.exp_nonpos(-88.0) == 0.0
    assert oracle.exp_nonpos(-1e9) == 0.0


def _exact_logits(h_bits, w_bits):
    h = oracle.bf16_float(h_bits).astype(np.float64)
    w = oracle.bf16_float(w_bits).astype(np.float64)
    return h @ w.T


def test_logits_are_the_rounded_dot_products():
    h, w = _rand_bits((32, 2048), 1), _rand_bits((128, 2048), 2, 0.02)
    logits, _, _, _ = oracle.router(h, w, 8, True)
    exact = _exact_logits(h, w)
    got = oracle.bf16_float(logits).astype(np.float64)
    want = oracle.bf16_float(oracle.bf16_bits(exact.astype(np.float32))).astype(np.float64)
    # fp32 accumulation may flip a rounding only when the exact value sits
    # next to a bf16 rounding boundary: at most 1 ulp and rarely.
    ulp = np.abs(want) * 2.0 ** -7 + 1e-30
    assert np.all(np.abs(got - want) <= ulp)
    assert np.mean(got == want) >= 0.999


def test_softmax_topk_and_weights_against_fp64_and_stable_sort():
    h, w = _rand_bits((64, 2048), 3), _rand_bits((128, 2048), 4, 0.02)
    for K, norm in ((8, True), (8, False), (1, True), (32, True)):
        logits, tw, ti, probs = oracle.router(h, w, K, norm)
        lg = oracle.bf16_float(logits).astype(np.float64)
        p64 = np.exp(lg - lg.max(axis=1, keepdims=True))
        p64 /= p64.sum(axis=1, keepdims=True)
        assert np.max(np.abs(probs - p64) / p64) <= 2e-6
        order = np.argsort(-probs, axis=1, kind="stable")[:, :K]
        np.testing.assert_array_equal(ti, order)
        v = np.take_along_axis(probs, ti, axis=1).astype(np.float64)
        want = v / v.sum(axis=1, keepdims=True) if norm else v
        got = oracle.bf16_float(tw).astype(np.float64)
        assert np.all(np.abs(got - want) <= np.abs(want) * 2.0 ** -8 + 1e-12)


def test_ties_resolve_to_the_lower_expert_id():
    h = np.zeros((2, 64), np.uint16)  # all logits 0
    w = _rand_bits((16, 64), 5, 0.02)
    _, tw, ti, _ = oracle.router(h, w, 4, True)
    assert ti.tolist() == [[0, 1, 2, 3]] * 2
    assert np.all(oracle.bf16_float(tw) == 0.25)
    w2 = _rand_bits((16, 64), 6, 0.02)
    w2[11] = w2[2]
    _, _, ti2, p2 = oracle.router(_rand_bits((6, 64), 7), w2, 16, True)
    for row, prob in zip(ti2, p2):
        assert list(row).index(2) < list(row).index(11)
        assert prob[2] == prob[11]


@pytest.mark.parametrize("name", ["router_hf_t16_h256_e64_k8.npz", "router_hf_t8_h32_e4_k2_nonorm.npz"])
def test_router_against_transformers_golden(name):
    f = np.load(os.path.join(GOLDEN, name))
    K, norm = int(f["top_k"]), bool(int(f["norm"]))
    logits, tw, ti, probs = oracle.router(f["hidden"], f["router"], K, norm)
    hf_lg = oracle.bf16_float(f["logits"])
    lg = oracle.bf16_float(logits)
    assert np.all(np.abs(lg - hf_lg) <= np.abs(hf_lg) * 2.0 ** -7 + 1e-30)
    exact_rows = np.all(logits == f["logits"], axis=1)
    assert exact_rows.mean() >= 0.5
    boundary_ties = 0
    for t in np.nonzero(exact_rows)[0]:
        # Same logits: same experts, except that torch.topk leaves the order
        # of equal probabilities unspecified -- inside the top-k and across
        # the k-th/(k+1)-th boundary, where the lower-id rule may keep a
        # different expert.  Every difference must be such a tie.
        kth = probs[t, ti[t][-1]]
        for e in set(ti[t]) ^ set(f["index"][t]):
            assert probs[t, e] == kth
            boundary_ties += 1
        for a, b in zip(ti[t], f["index"][t]):
            if a != b:
                assert probs[t, a] == probs[t, b]
        got_w = oracle.bf16_float(tw[t])
        hf_w = oracle.bf16_float(f["weights"][t])
        assert np.all(np.abs(np.sort(got_w) - np.sort(hf_w)) <= np.abs(hf_w).max() * 2.0 ** -7)
    print(f"{name}: {exact_rows.sum()} rows with bitwise-equal logits, "
          f"{boundary_ties // 2} top-k boundary ties resolved differently by torch.topk")


REAL_SHAPE = [("router_hf_t256_h2048_e128_k8_uniform.npz", None),
              ("router_hf_t256_h2048_e128_k8_zipf.npz", 1.1)]


def real_shape_case(name):
    """(fixture, hidden bits, router bits) of a Qwen3-30B-A3B-shaped router
    fixture; its inputs are regenerated and checked against the stored
    digest first."""
    import sys

    sys.path.insert(0, GOLDEN)
    import inputs

    f = np.load(os.path.join(GOLDEN, name))
    zipf = float(f["zipf_s"])
    hidden, weight = inputs.real_shape_inputs(int(f["tokens"]), 2048, 128, int(f["seed"]),
                                              None if zipf < 0 else zipf)
    assert inputs.input_digest(hidden, weight) == str(f["input_sha256"]), \
        "regenerated router inputs differ from the ones the fixture was made from"
    return f, inputs.bits(hidden), inputs.bits(weight)


@pytest.mark.parametrize("name,zipf", REAL_SHAPE)
def test_router_agreement_with_transformers_at_the_qwen3_shape(name, zipf):
    """H 2048, E 128, top-8 renormalised, 256 tokens: logits within one
    bf16 ulp of transformers', and every expert-set difference is a tie at
    the 8th logit (rows with equal logits) or a one-ulp flip at the
    boundary."""
    from _router_agreement import classify

    f, h, w = real_shape_case(name)
    logits, tw, ti, _ = oracle.router(h, w, 8, True)
    a = classify(logits, ti, f["logits"], f["index"], 8)
    print(f"{name}: {a.rows} rows, {a.exact_logit_rows} with bitwise-equal logits, "
          f"{a.same_set_rows} same expert set ({a.agreement:.2%}); differences: "
          f"{a.tie_rows} ties at the 8th logit, {a.flip_set_rows} one-ulp flips "
          f"({a.flip_rows} rows with a flipped logit)")
    assert a.exact_logit_rows >= 0.95 * a.rows
    assert a.agreement >= 0.95
    # weights of rows with the same expert set agree within one bf16 ulp
    for t in range(a.rows):
        if set(ti[t]) == set(f["index"][t]):
            ours = dict(zip(ti[t].tolist(), oracle.bf16_float(tw[t]).tolist()))
            hf = dict(zip(f["index"][t].tolist(), oracle.bf16_float(f["weights"][t]).tolist()))
            for e, v in ours.items():
                assert abs(v - hf[e]) <= abs(hf[e]) * 2.0 ** -7
