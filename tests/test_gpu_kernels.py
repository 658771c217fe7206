"""Parity of the HIP kernels (through the C-ABI) with the CPU oracle.

Bar: router logits / weights / indices and the dispatch permutation
bit-exact; combine bit-exact given the same rows; expert SwiGLU within the
MoE tolerance (max |y - y32| / max |y32| <= 1e-2 against the fp32 oracle,
rtol = atol = 1.6e-2 against the bf16 eager oracle).
"""
import numpy as np
import pytest
import torch

import oracle
from specfit_amd import ops
from specfit_amd.workloads import make_hidden, make_layer, zipf_bias

pytestmark = pytest.mark.gpu


def _bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def _from_bits(a: np.ndarray, device) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(torch.bfloat16).to(device)


def _randn_bf16(shape, seed, std=1.0):
    g = torch.Generator("cpu").manual_seed(seed)
    return (torch.randn(*shape, generator=g) * std).to(torch.bfloat16)


def _router_case(device, T, H, E, K, renorm, seed, hidden=None, weight=None):
    h = hidden if hidden is not None else _randn_bf16((T, H), seed)
    w = weight if weight is not None else _randn_bf16((E, H), seed + 1, 0.02)
    logits, tw, ti = ops.router_topk(h.to(device), w.to(device), K, renorm)
    torch.cuda.synchronize()
    o_logits, o_w, o_i, _ = oracle.router(_bits(h), _bits(w), K, renorm)
    print(f"router case T={T} H={H} E={E} K={K} renorm={renorm} seed={seed}", flush=True)
    np.testing.assert_array_equal(_bits(logits), o_logits)
    np.testing.assert_array_equal(ti.cpu().numpy(), o_i)
    np.testing.assert_array_equal(_bits(tw), o_w)


@pytest.mark.parametrize("T,seed", [(16, 0), (64, 1), (1, 2), (128, 3), (300, 5)])
def test_router_bitexact_qwen3_shape(device, T, seed):
    _router_case(device, T, 2048, 128, 8, True, seed)


def test_router_bitexact_zipf_biased(device):
    layer_bias = zipf_bias(128, 1.1, 1.0, 5)
    w = _randn_bf16((128, 2048), 9, 0.02)
    w[:, 0] = layer_bias.to(torch.bfloat16)
    h = make_hidden(64, 2048, seed=11, zipf_fold=True)
    _router_case(device, 64, 2048, 128, 8, True, 0, hidden=h, weight=w)


@pytest.mark.parametrize("T,H,E,K,renorm", [
    (4, 32, 4, 2, False),     # tiny test config (norm_topk_prob default False)
    (5, 100, 60, 4, True),    # H not a multiple of 8: scalar path
    (3, 8192, 256, 32, True), # largest expert count / top-k
    (7, 2048, 128, 8, False),
    (20, 4096, 128, 8, True), # Qwen3-235B-A22B router (8 chunks per lane)
    (6, 512, 64, 32, True),   # 1 expert per lane, top-32
    (5, 256, 65, 8, True),    # 2 per lane with one expert in the second slice
    (4, 256, 129, 1, False),  # 4 per lane, top-1
    (9, 1024, 200, 32, False),
])
def test_router_bitexact_other_shapes(device, T, H, E, K, renorm):
    _router_case(device, T, H, E, K, renorm, 21)


def test_router_ties_resolve_to_lower_id(device):
    h = torch.zeros(3, 256, dtype=torch.bfloat16)
    w = _randn_bf16((16, 256), 4, 0.02)
    logits, tw, ti = ops.router_topk(h.to(device), w.to(device), 4, True)
    assert ti.cpu().tolist() == [[0, 1, 2, 3]] * 3
    assert torch.all(tw.cpu().float() == 0.25)
    # duplicated router rows -> exactly equal logits -> lower id first
    w2 = _randn_bf16((16, 256), 5, 0.02)
    w2[9] = w2[3]
    h2 = _randn_bf16((8, 256), 6)
    _router_case(device, 8, 256, 16, 16, True, 0, hidden=h2, weight=w2)


def _dispatch_case(device, idx: np.ndarray, E: int):
    t = torch.from_numpy(idx).to(device)
    plan = ops.dispatch(t, E)
    torch.cuda.synchronize()
    counts, offsets, perm, inv = oracle.dispatch(idx, E)
    np.testing.assert_array_equal(plan.counts.cpu().numpy(), counts)
    np.testing.assert_array_equal(plan.offsets.cpu().numpy(), offsets)
    valid = int(offsets[E])
    np.testing.assert_array_equal(plan.perm_pos.cpu().numpy()[:valid], perm[:valid])
    np.testing.assert_array_equal(plan.inv_perm.cpu().numpy(), inv)
    # The kernel's own write of [counts; offsets] into pinned host memory
    # (read after waiting for the kernel only) and the copied read agree.
    host = torch.full((2, E + 1), -7, dtype=torch.int32, pin_memory=True)
    plan2 = ops.dispatch(t, E, host_meta=host)
    got = plan2.fetch_counts().numpy()
    np.testing.assert_array_equal(got[0], counts)
    np.testing.assert_array_equal(got[1], offsets)
    assert plan2.count_list == counts.tolist()
    np.testing.assert_array_equal(plan.fetch_counts().numpy(), got)


@pytest.mark.parametrize("T,K,E,seed", [(64, 8, 128, 0), (1, 8, 128, 1), (16, 8, 128, 2),
                                        (200, 8, 128, 3), (513, 7, 256, 4), (4, 2, 4, 5),
                                        # chunk and kernel-width boundaries: 256 routes
                                        # (last 256-thread case), 264, 1024 (one full
                                        # 1024 chunk), 1032 (a second chunk of 8)
                                        (32, 8, 128, 6), (33, 8, 128, 7), (128, 8, 256, 8),
                                        (129, 8, 64, 9)])
def test_dispatch_bitexact(device, T, K, E, seed):
    rng = np.random.default_rng(seed)
    idx = rng.integers(0, E, size=(T, K)).astype(np.int64)
    _dispatch_case(device, idx, E)


def test_dispatch_duplicates_skew_and_invalid(device):
    rng = np.random.default_rng(7)
    idx = rng.integers(0, 3, size=(300, 8)).astype(np.int64)   # heavy collisions, 3 chunks
    idx[0, 2] = idx[0, 0]
    _dispatch_case(device, idx, 128)
    bad = np.array([[0, 5], [130, 2], [-1, 1]], dtype=np.int64)
    _dispatch_case(device, bad, 128)
    plan = ops.dispatch(torch.from_numpy(bad).to(device), 128)
    assert int(plan.fetch_counts()[0][128]) == 2


def test_dispatch_empty(device):
    plan = ops.dispatch(torch.zeros((0, 8), dtype=torch.int64, device=device), 128)
    assert plan.fetch_counts()[0].sum().item() == 0
    host = torch.full((2, 129), 5, dtype=torch.int32, pin_memory=True)
    plan = ops.dispatch(torch.zeros((0, 8), dtype=torch.int64, device=device), 128, host_meta=host)
    assert plan.fetch_counts().sum().item() == 0 and plan.count_list == [0] * 129


def test_dispatch_rejects_unmapped_host_meta(device):
    idx = torch.zeros((4, 8), dtype=torch.int64, device=device)
    with pytest.raises(ValueError, match="pinned"):
        ops.dispatch(idx, 128, host_meta=torch.zeros((2, 129), dtype=torch.int32))
    with pytest.raises(ValueError, match="pinned"):
        ops.dispatch(idx, 128, host_meta=torch.zeros((2, 128), dtype=torch.int32,
                                                     pin_memory=True))


def test_combine_bitexact_both_modes(device):
    rng = np.random.default_rng(3)
    T, K, E, H = 33, 8, 128, 2048
    idx = np.stack([rng.choice(E, K, replace=False) for _ in range(T)]).astype(np.int64)
    idx[5, 3] = idx[5, 1]  # duplicated expert in a row
    rows = oracle.bf16_bits(rng.standard_normal((T * K, H)).astype(np.float32))
    plan = ops.dispatch(torch.from_numpy(idx).to(device), E)
    inv = plan.inv_perm.cpu().numpy()
    rank = list(rng.permutation(E))
    for acc32 in (False, True):
        for r in (None, rank):
            out = ops.combine(_from_bits(rows, device), torch.from_numpy(idx).to(device), plan, H,
                              expert_rank=r, accumulate_fp32=acc32)
            ref = oracle.combine(rows, idx, inv, E, r, acc32)
            np.testing.assert_array_equal(_bits(out), ref)


def test_combine_known_answer_order(device):
    # 1 + 2^-8 - 1 in bf16: ascending order loses 2^-8, order (0,2,1) keeps it
    # (reference test_qwen3_offloaded_experts.py:379-458).
    idx = torch.tensor([[0, 1, 2]], dtype=torch.int64, device=device)
    plan = ops.dispatch(idx, 3)
    rows = torch.tensor([[1.0], [2.0 ** -8], [-1.0]], dtype=torch.bfloat16, device=device)
    assert ops.combine(rows, idx, plan, 1).item() == 0.0
    assert ops.combine(rows, idx, plan, 1, expert_rank=[0, 2, 1]).item() == 2.0 ** -8
    assert ops.combine(rows, idx, plan, 1, accumulate_fp32=True).item() == 2.0 ** -8


def _moe_rows(device, layer, hidden, K, experts_list):
    """K3 rows for the given experts, plus the oracle's."""
    H, I, E = layer.hidden_size, layer.intermediate_size, layer.num_experts
    h_dev = hidden.to(device)
    logits, w, idx = ops.router_topk(h_dev, layer.router.to(device), K, True)
    plan = ops.dispatch(idx, E)
    T = hidden.shape[0]
    act = torch.empty((T * K, I), dtype=torch.bfloat16, device=device)
    rows = torch.zeros((T * K, H), dtype=torch.bfloat16, device=device)
    slots = layer.experts.to(device)
    ops.grouped_swiglu(h_dev, plan, w.reshape(-1).contiguous(), experts_list,
                       [slots[e] for e in experts_list], H, I, act, rows)
    torch.cuda.synchronize()
    return h_dev, idx, w, plan, rows, slots


def test_grouped_swiglu_matches_oracle_qwen3_shape(device):
    layer = make_layer(seed=0, num_experts=16)
    hidden = make_hidden(40, seed=1)
    h_dev, idx, w, plan, rows, _ = _moe_rows(device, layer, hidden, 8, list(range(16)))
    x = oracle.bf16_float(_bits(hidden))
    experts = {e: oracle.bf16_float(_bits(layer.experts[e])) for e in range(16)}
    ref_rows, *_ = oracle.moe_rows_bf16(x, idx.cpu().numpy(), oracle.bf16_float(_bits(w)), experts,
                                        2048, 768, 16)
    got = oracle.bf16_float(_bits(rows))
    np.testing.assert_allclose(got, ref_rows, rtol=1.6e-2, atol=1.6e-2)
    # fp32 closed form of the whole layer
    out = ops.combine(rows, idx, plan, 2048)
    y32 = oracle.moe_forward_fp32(x, idx.cpu().numpy(), oracle.bf16_float(_bits(w)), experts, 2048, 768)
    err = np.abs(oracle.bf16_float(_bits(out)) - y32).max() / np.abs(y32).max()
    print(f"grouped swiglu max normalised error vs fp32 oracle: {err:.3e}", flush=True)
    assert err <= 1e-2


def test_grouped_swiglu_is_independent_of_grouping(device):
    layer = make_layer(seed=3, num_experts=12)
    hidden = make_hidden(24, seed=4)
    _, idx, w, plan, rows_all, slots = _moe_rows(device, layer, hidden, 8, list(range(12)))
    H, I = 2048, 768
    h_dev = hidden.to(device)
    act = torch.empty((24 * 8, I), dtype=torch.bfloat16, device=device)
    rows_one = torch.zeros_like(rows_all)
    for e in reversed(range(12)):
        ops.grouped_swiglu(h_dev, plan, w.reshape(-1).contiguous(), [e], [slots[e]], H, I, act,
                           rows_one)
    rows_tab = torch.zeros_like(rows_all)
    table = torch.arange(12, dtype=torch.int32, device=device)
    ops.grouped_swiglu_table(h_dev, plan, w.reshape(-1).contiguous(), table, slots, H, I, act,
                             rows_tab)
    torch.cuda.synchronize()
    assert torch.equal(rows_one, rows_all)
    assert torch.equal(rows_tab, rows_all)
    # dense single-expert seam equals the unscaled grouped rows of expert 5
    counts = plan.fetch_counts()
    a, b = int(counts[1][5]), int(counts[1][6])
    pos = plan.perm_pos[a:b].long()
    tokens = (pos // 8)
    y = ops.expert_swiglu(h_dev[tokens], slots[5], H, I)
    scaled = (y.float() * w.reshape(-1)[pos].float()[:, None]).to(torch.bfloat16)
    assert torch.equal(scaled, rows_all[a:b])


def test_grouped_swiglu_row_classes_streams_and_table(device):
    """Calls whose largest expert falls in each row class (<= 16 / 32 / 64 /
    more rows), thirty calls in a row, calls running concurrently on two
    streams and the slot-table form all give the rows of one-expert calls,
    bit for bit.  One-expert calls of <= 16 rows run narrow tiles (8 gate/up,
    16 down columns per workgroup); the all-expert calls (more than 24
    experts) run wide ones (16 / 32), so this also pins that the two widths
    agree bit for bit."""
    E, T, K, H, I = 32, 128, 8, 2048, 768
    layer = make_layer(seed=11, num_experts=E, zipf_s=1.1)
    hidden = make_hidden(T, seed=12, zipf_fold=True)
    h_dev, idx, w, plan, rows_all, slots = _moe_rows(device, layer, hidden, K, list(range(E)))
    ms = [int(c) for c in plan.fetch_counts()[0]]
    print(f"row-class case E={E} T={T} rows per expert {ms}", flush=True)
    assert max(ms) > 64 and 0 < min(m for m in ms if m) <= 16  # every row class occurs
    wflat = w.reshape(-1).contiguous()
    act = torch.empty((T * K, I), dtype=torch.bfloat16, device=device)
    ref = torch.zeros_like(rows_all)
    active = [e for e in range(E) if ms[e]]
    assert len(active) > 24  # the all-expert calls take the wide tiles
    assert sum(0 < m <= 16 for m in ms) >= 2  # some one-expert calls take the narrow ones
    for e in active:
        ops.grouped_swiglu(h_dev, plan, wflat, [e], [slots[e]], H, I, act, ref)
    torch.cuda.synchronize()
    assert torch.equal(ref, rows_all)
    offs = plan.fetch_counts()[1]

    def rows_of(experts):
        return torch.cat([torch.arange(int(offs[e]), int(offs[e + 1]), device=device)
                          for e in experts])

    for lo, hi in ((1, 16), (17, 32), (33, 64), (65, T * K)):
        sel = [e for e in active if lo <= ms[e] <= hi]
        if not sel:
            continue
        out = torch.zeros_like(rows_all)
        ops.grouped_swiglu(h_dev, plan, wflat, sel, [slots[e] for e in sel], H, I, act, out)
        torch.cuda.synchronize()
        r = rows_of(sel)
        assert torch.equal(out[r], ref[r]), (lo, hi)
    side = torch.cuda.Stream(device)
    main = torch.cuda.current_stream(device)
    outs = [torch.zeros_like(rows_all) for _ in range(30)]
    acts = [torch.empty_like(act) for _ in range(30)]
    torch.cuda.synchronize()
    for i in range(30):
        with torch.cuda.stream(side if i % 3 == 2 else main):
            ops.grouped_swiglu(h_dev, plan, wflat, active, [slots[e] for e in active], H, I,
                               acts[i], outs[i])
    torch.cuda.synchronize()
    for i, out in enumerate(outs):
        assert torch.equal(out, ref), i
    table = torch.arange(E, dtype=torch.int32, device=device)
    table[::4] = -1
    out = torch.zeros_like(rows_all)
    ops.grouped_swiglu_table(h_dev, plan, wflat, table, slots, H, I, act, out)
    torch.cuda.synchronize()
    with_slot = [e for e in active if e % 4]
    r = rows_of(with_slot)
    assert torch.equal(out[r], ref[r])
    r0 = rows_of([e for e in active if e % 4 == 0])
    assert not out[r0].any()


def test_grouped_swiglu_qwen3_235b_shape(device):
    """The MFMA path's second compiled expert shape (Qwen3-235B-A22B: hidden
    4096, intermediate 1536), with Zipf-skewed experts spanning the row
    classes: one grouped launch gives the rows of one-expert launches bit
    for bit, and the bf16-eager oracle's rows within tolerance."""
    E, T, K = 8, 96, 4
    layer = make_layer(seed=3, hidden_size=4096, intermediate_size=1536, num_experts=E,
                       top_k=K, zipf_s=1.1)
    H, I = 4096, 1536
    hidden = make_hidden(T, H, seed=4, zipf_fold=True)
    h_dev, idx, w, plan, rows, slots = _moe_rows(device, layer, hidden, K, list(range(E)))
    ms = [int(c) for c in plan.fetch_counts()[0][:E]]
    print(f"235b-shape case rows per expert {ms}", flush=True)
    assert min(ms) <= 32 and max(ms) > 64
    wflat = w.reshape(-1).contiguous()
    act = torch.empty((T * K, I), dtype=torch.bfloat16, device=device)
    one = torch.zeros_like(rows)
    for e in range(E):
        if ms[e]:
            ops.grouped_swiglu(h_dev, plan, wflat, [e], [slots[e]], H, I, act, one)
    torch.cuda.synchronize()
    assert torch.equal(one, rows)
    x = oracle.bf16_float(_bits(hidden))
    experts = {e: oracle.bf16_float(_bits(layer.experts[e])) for e in range(E)}
    ref_rows, *_ = oracle.moe_rows_bf16(x, idx.cpu().numpy(), oracle.bf16_float(_bits(w)), experts,
                                        H, I, E)
    np.testing.assert_allclose(oracle.bf16_float(_bits(rows)), ref_rows, rtol=1.6e-2, atol=1.6e-2)


@pytest.mark.parametrize("H,I,m", [(4, 3, 2), (32, 16, 5), (96, 64, 70), (2048, 768, 48),
                                   (2048, 768, 130), (4096, 1536, 20), (4096, 1536, 70)])
def test_expert_swiglu_generic_and_mfma_paths(device, H, I, m):
    g = torch.Generator("cpu").manual_seed(H + I + m)
    x = torch.randn(m, H, generator=g).to(torch.bfloat16)
    packed = (torch.randn(3 * H * I, generator=g) * 0.05).to(torch.bfloat16)
    y = ops.expert_swiglu(x.to(device), packed.to(device), H, I)
    torch.cuda.synchronize()
    ref = oracle.expert_forward_bf16(oracle.bf16_float(_bits(x)), oracle.bf16_float(_bits(packed)), H, I)
    np.testing.assert_allclose(oracle.bf16_float(_bits(y)), ref, rtol=1.6e-2, atol=1.6e-2)
    if H >= 32:
        # With H=4 the reference's own bf16 rounding points are ~3% from fp32,
        # so the 1e-2 bound against the fp32 closed form applies from H=32 on.
        y32 = oracle.expert_forward_fp32(oracle.bf16_float(_bits(x)), oracle.bf16_float(_bits(packed)), H, I)
        err = np.abs(oracle.bf16_float(_bits(y)) - y32).max() / max(np.abs(y32).max(), 1e-30)
        assert err <= 1e-2


def test_h2d_copy_roundtrip(device):
    src = torch.arange(1 << 20, dtype=torch.int32).view(torch.bfloat16).pin_memory()
    dst = torch.empty(src.shape, dtype=torch.bfloat16, device=device)
    s = torch.cuda.Stream(device=device)
    ops.copy_h2d(dst, src, s)
    s.synchronize()
    assert torch.equal(dst.cpu().view(torch.int32), src.view(torch.int32))
