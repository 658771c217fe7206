"""Host checks of the exponent-coded expert records (specfit_amd.codec):
record sizes against the C library, a hand-built known answer, round trips
through the host definition of the decode, the table rule and the raw
fallback.  The device decode is checked against the same bytes in
tests/test_gpu_codec.py."""
import numpy as np
import pytest
import torch

from specfit_amd import _native
from specfit_amd.codec import (CompressedExperts, decode_record_reference, encode_record,
                               record_bytes, section_offsets)


def _bits(t: torch.Tensor) -> np.ndarray:
    return t.view(torch.int16).numpy().view(np.uint16)


def _chunk_table_ok(rec: np.ndarray, n: int, n_esc: int) -> bool:
    """EC[k] = number of escapes below value 4096 k, for k = 0 .. ceil(n/4096)."""
    _, _, off_ei, _, off_ec = section_offsets(n, n_esc)
    idx = rec[off_ei:off_ei + 4 * n_esc].view("<u4")
    chunks = -(-n // 4096)
    ec = rec[off_ec:off_ec + 4 * (chunks + 1)].view("<u4")
    want = [int(np.count_nonzero(idx < 4096 * k)) for k in range(chunks + 1)]
    return ec.tolist() == want


def _roundtrip(values: torch.Tensor, force: bool = False):
    rec, n_esc, table = encode_record(values, force=force)
    assert rec is not None
    out = decode_record_reference(rec.numpy(), values.numel(), n_esc, table)
    assert np.array_equal(out, _bits(values))
    assert _chunk_table_ok(rec.numpy(), values.numel(), n_esc)
    return rec, n_esc, table


@pytest.mark.parametrize("n,e", [(0, 0), (1, 0), (5, 0), (4096, 3), (4_718_592, 700),
                                 (4_718_593, 4_718_593)])
def test_record_size_matches_the_library(n, e):
    assert record_bytes(n, e) == _native.lib().sf_expert_record_bytes(n, e)
    off = section_offsets(n, e)
    assert len(off) == 5 and all(o % 256 == 0 for o in off) and off == tuple(sorted(off))
    assert _native.lib().sf_expert_record_bytes(5, 6) == -1
    with pytest.raises(ValueError):
        record_bytes(5, 6)


def test_known_answer_record():
    # 1.0, -2.0, 0.5, 1.5, 1.0: exponents 127, 128, 126, 127, 127
    values = torch.tensor([1.0, -2.0, 0.5, 1.5, 1.0], dtype=torch.bfloat16)
    rec, n_esc, table = encode_record(values, force=True)
    assert n_esc == 0
    assert table == bytes([127, 126, 128]) + bytes(13)  # by count, ties to the lower exponent
    r = rec.numpy()
    # S at 0, X at 256, no escapes, the chunk table [0, 0] at 512
    assert r.size == 768 and r[:5].tolist() == [0x00, 0x80, 0x00, 0x40, 0x00]
    assert r[256:259].tolist() == [0x20, 0x01, 0x00]  # codes 0,2 | 1,0 | 0
    assert not r[5:256].any() and not r[259:].any()
    # too small to gain anything: the expert stays raw
    assert encode_record(values)[0] is None


def test_gaussian_expert_roundtrip_and_size():
    g = torch.Generator().manual_seed(3)
    values = (torch.randn(100_003, generator=g) * 0.02).to(torch.bfloat16)
    rec, n_esc, table = _roundtrip(values)
    assert n_esc < 100  # |x| < 2^-18 is rare at this scale
    assert rec.numel() < 0.77 * 2 * values.numel()
    # the table is the 15 most frequent exponents
    exps = (_bits(values) >> 7) & 0xFF
    counts = np.bincount(exps, minlength=256)
    top = sorted(range(256), key=lambda x: (-counts[x], x))[:15]
    assert list(table[:15]) == top


def test_every_bit_pattern_roundtrips():
    values = torch.arange(65536, dtype=torch.int32).to(torch.int16).view(torch.bfloat16)
    rec, n_esc, table = _roundtrip(values, force=True)
    assert n_esc == 65536 - 15 * 256  # 15 exponents in the table, 256 values each
    # without force the record would be larger than the raw bytes
    assert encode_record(values)[0] is None


@pytest.mark.parametrize("n", [1, 2, 3, 17, 4095, 4097])
def test_short_and_odd_lengths(n):
    g = torch.Generator().manual_seed(n)
    values = (torch.randn(n, generator=g) * 0.02).to(torch.bfloat16)
    _roundtrip(values, force=True)


def test_image_layout_and_raw_fallback():
    g = torch.Generator().manual_seed(0)
    n = 3 * 4096 + 10
    sources = {("l", e): (torch.randn(n, generator=g) * 0.02).to(torch.bfloat16) for e in range(3)}
    # an expert of arbitrary bit patterns: its record would be larger
    noise = torch.randint(-32768, 32768, (n,), generator=g, dtype=torch.int32)
    sources[("l", 3)] = noise.to(torch.int16).view(torch.bfloat16)
    image = CompressedExperts.encode(sources)
    assert image.numel == n and image.raw_bytes == 4 * 2 * n
    raw = image.records[("l", 3)]
    assert raw.raw and raw.nbytes == 2 * n
    coded = [image.records[("l", e)] for e in range(3)]
    assert all(not r.raw and r.offset % 256 == 0 for r in coded)
    spans = sorted((r.offset, r.offset + r.nbytes) for r in coded)
    assert all(a[1] <= b[0] for a, b in zip(spans, spans[1:]))
    assert image.transfer_bytes == sum(r.nbytes for r in coded) + 2 * n
    assert image.staging_bytes() == max(r.nbytes for r in coded)
    for e in range(3):
        r = image.records[("l", e)]
        out = decode_record_reference(image.record_view(("l", e)).numpy(), n, r.n_escapes, r.table)
        assert np.array_equal(out, _bits(sources[("l", e)]))
    with pytest.raises(ValueError, match="stored raw"):
        image.record_view(("l", 3))
    with pytest.raises(ValueError, match="same number"):
        CompressedExperts.encode({0: torch.zeros(4, dtype=torch.bfloat16),
                                  1: torch.zeros(5, dtype=torch.bfloat16)})
