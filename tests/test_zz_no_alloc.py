"""The allocation-free slot-table K3 entry point against the allocating one.

Both are called through the C ABI on the same dispatched routes and slot
table; the rows they write must be identical bits.  Two calls in a row, the
second with fewer tokens (the scratch array keeps the first call's
contents); calls at the size limit (341 tokens at the Qwen3-30B-A3B expert
shape, the most that fit, and a shape whose activations fill the 4 MiB
array exactly); then the over-limit call, which must be refused on the host
before anything is launched.
"""
from __future__ import annotations

import pytest
import torch

from specfit_amd import _native, ops
from specfit_amd.workloads import make_hidden, make_layer

pytestmark = pytest.mark.gpu

H, I, K, E = 2048, 768, 8, 16
SCRATCH_BYTES = 4 << 20


def _routes(device, tokens: int, seed: int, h_: int, i_: int):
    layer = make_layer(seed=seed, num_experts=E, hidden_size=h_, intermediate_size=i_)
    hidden = make_hidden(tokens, h_, seed=seed + 1).to(device)
    _, w, idx = ops.router_topk(hidden, layer.router.to(device), K, True)
    plan = ops.dispatch(idx, E)
    return layer, hidden, w.reshape(-1).contiguous(), plan


def _call_both(device, tokens: int, seed: int, h_: int = H, i_: int = I):
    layer, hidden, w, plan, = _routes(device, tokens, seed, h_, i_)
    storage = layer.experts.to(device)  # [E, 3*H*I]: expert e in slot e ...
    # ... but the table maps experts to shuffled slots and leaves two out.
    table_host = [(5 * e) % E for e in range(E)]
    table_host[3] = table_host[11] = -1
    order = torch.tensor([table_host.index(s) if s in table_host else 0 for s in range(E)])
    slots = storage[order].contiguous()  # slot s holds the expert the table maps to it
    table = torch.tensor(table_host, dtype=torch.int32, device=device)
    N = tokens * K
    sentinel = torch.full((N, h_), 0x7FC1, dtype=torch.int16, device=device).view(torch.bfloat16)
    out_ref = sentinel.clone()
    out_new = sentinel.clone()
    act = torch.empty((N, i_), dtype=torch.bfloat16, device=device)
    lib = _native.lib()
    stream = torch.cuda.current_stream(device).cuda_stream
    common = (hidden.data_ptr(), plan.perm_pos.data_ptr(), plan.offsets.data_ptr(), w.data_ptr(),
              tokens, K, h_, i_, E, N, table.data_ptr(), slots.data_ptr(), slots.stride(0))
    print(f"no-alloc case: tokens={tokens} seed={seed} H={h_} I={i_} allocating entry point",
          flush=True)
    _native.check(lib.sf_grouped_swiglu_table(*common, act.data_ptr(), out_ref.data_ptr(), stream),
                  "sf_grouped_swiglu_table")
    print(f"no-alloc case: tokens={tokens} seed={seed} H={h_} I={i_} allocation-free entry point",
          flush=True)
    _native.check(lib.sf_grouped_swiglu_table_noalloc(*common, out_new.data_ptr(), stream),
                  "sf_grouped_swiglu_table_noalloc")
    torch.cuda.synchronize()
    return out_ref, out_new, plan, table_host


def test_noalloc_matches_allocating_entry_point_twice(device):
    ref1, new1, plan1, table = _call_both(device, 64, 3)
    assert torch.equal(ref1.view(torch.int16), new1.view(torch.int16))
    # every routed row of a table expert was written (the sentinel is gone)
    counts = plan1.fetch_counts()[1].tolist()
    written = [r for e in range(E) if table[e] >= 0 for r in range(counts[e], counts[e + 1])]
    assert written and not (new1[written].view(torch.int16) == 0x7FC1).all(dim=1).any()
    # second call, fewer tokens: the array still holds the first call's rows
    ref2, new2, _, _ = _call_both(device, 16, 9)
    assert torch.equal(ref2.view(torch.int16), new2.view(torch.int16))


@pytest.mark.parametrize("tokens,h_,i_", [
    (SCRATCH_BYTES // (K * I * 2), H, I),  # 341 tokens: the most that fit at this shape
    (256, 64, 1024),                       # activations of exactly 4 MiB (loop kernels)
])
def test_noalloc_at_the_scratch_limit(device, tokens, h_, i_):
    need = tokens * K * i_ * 2
    assert need <= SCRATCH_BYTES and (tokens + 1) * K * i_ * 2 > SCRATCH_BYTES
    ref, new, plan, table = _call_both(device, tokens, 21, h_, i_)
    assert torch.equal(ref.view(torch.int16), new.view(torch.int16))
    counts = plan.fetch_counts()[1].tolist()
    written = [r for e in range(E) if table[e] >= 0 for r in range(counts[e], counts[e + 1])]
    assert written and not (new[written].view(torch.int16) == 0x7FC1).all(dim=1).any()


def test_noalloc_refuses_inputs_beyond_its_scratch(device):
    lib = _native.lib()
    buf = torch.zeros(64, dtype=torch.int32, device=device)
    p = buf.data_ptr()
    tokens = SCRATCH_BYTES // (K * I * 2) + 1  # one token past the 4 MiB scratch
    rc = lib.sf_grouped_swiglu_table_noalloc(p, p, p, p, tokens, K, H, I, E, tokens * K, p, p,
                                             3 * H * I, p,
                                             torch.cuda.current_stream(device).cuda_stream)
    assert rc == 5  # SF_ERR_SCRATCH_LIMIT
    assert "scratch" in _native.error_string(rc)
