"""Host checks of the exponent-coded expert records (specfit_amd.codec):
record sizes against the C library, hand-built known answers for every
section (planes, level-2 and level-3 codes, raw bytes, chunk tables), round
trips through the host definition of the decode, the table rule and the raw
fallback.  The device decode is checked against the same
bytes in tests/test_gpu_codec.py."""
import numpy as np
import pytest
import torch

from specfit_amd import _native
from specfit_amd.codec import CompressedExperts, encode_record, record_bytes, section_offsets

from codec_reference import decode_record_reference


def _bits(t: torch.Tensor) -> np.ndarray:
    return t.view(torch.int16).numpy().view(np.uint16)


def _from_bits(bits) -> torch.Tensor:
    return torch.tensor(np.asarray(bits, dtype=np.uint16).view(np.int16)).view(torch.bfloat16)


def _levels(values: torch.Tensor, table: bytes):
    """Positions of the values that reach level 2, level 3 and a raw byte,
    from the exponents and the record's table alone."""
    exps = (_bits(values) >> 7) & 0xFF
    n_used = len(set(exps.tolist()))
    used = lambda lo, k: list(table[lo:lo + min(k, n_used)])
    at2 = np.nonzero(~np.isin(exps, used(0, 3)))[0]
    at3 = at2[~np.isin(exps[at2], used(8, 3))]
    at_raw = at3[~np.isin(exps[at3], used(16, 15))]
    return at2, at3, at_raw


def _chunk_tables_ok(rec: np.ndarray, values: torch.Tensor, counts, table: bytes) -> bool:
    """C2[k] / C3[k] / CR[k] = level-2 / level-3 / raw entries of the values
    below 4096 k, and the counts match."""
    n = values.numel()
    off = section_offsets(n, counts)
    levels = _levels(values, table)
    if tuple(len(p) for p in levels) != tuple(counts):
        return False
    chunks = -(-n // 4096)
    for key, pos in zip(("C2", "C3", "CR"), levels):
        got = rec[off[key]:off[key] + 4 * (chunks + 1)].view("<u4").tolist()
        if got != [int(np.count_nonzero(pos < 4096 * k)) for k in range(chunks + 1)]:
            return False
    return True


def _roundtrip(values: torch.Tensor, force: bool = False):
    rec, counts, table = encode_record(values, force=force)
    assert rec is not None
    out = decode_record_reference(rec.numpy(), values.numel(), counts, table)
    assert np.array_equal(out, _bits(values))
    return rec, counts, table


@pytest.mark.parametrize("n,counts", [(0, (0, 0, 0)), (1, (0, 0, 0)), (5, (0, 0, 0)),
                                      (4096, (3, 2, 1)), (4_718_592, (1_300_000, 190_000, 7)),
                                      (4_718_593, (4_718_593,) * 3)])
def test_record_size_matches_the_library(n, counts):
    lib = _native.lib()
    assert record_bytes(n, counts) == lib.sf_expert_record_bytes(n, *counts)
    off = section_offsets(n, counts)
    order = [off[k] for k in ("S", "P", "L2", "L3", "R", "C2", "C3", "CR", "size")]
    assert all(o % 256 == 0 for o in order) and order == sorted(order)
    for bad in ((6, 0, 0), (2, 3, 0), (3, 2, 3), (-1, 0, 0)):
        assert lib.sf_expert_record_bytes(5, *bad) == -1
        with pytest.raises(ValueError):
            record_bytes(5, bad)


def test_known_answer_record():
    # 1.0, -2.0, 0.5, 1.5, 1.0: exponents 127, 128, 126, 127, 127
    values = torch.tensor([1.0, -2.0, 0.5, 1.5, 1.0], dtype=torch.bfloat16)
    rec, counts, table = encode_record(values, force=True)
    assert counts == (0, 0, 0)
    # level 1 by count, ties to the lower exponent; nothing reaches level 2
    assert table == bytes([127, 126, 128]) + bytes(29)
    b = rec.numpy()
    # S at 0; planes at 256 and 512 (codes 0, 2, 1, 0, 0); L2, L3, R empty;
    # C2, C3, CR at 768, 1024, 1280
    assert b.size == 1536 and b[:5].tolist() == [0x00, 0x80, 0x00, 0x40, 0x00]
    assert b[256:258].tolist() == [0b100, 0] and b[512:514].tolist() == [0b10, 0]
    assert not b[5:256].any() and not b[258:512].any() and not b[514:].any()
    # too small to gain anything: the expert stays raw
    assert encode_record(values)[0] is None


def _cascade_exponents():
    """Exponents 100..102 four times each (level 1), 103..105 three times
    (level 2), 106..120 twice (level 3), 121 and 122 once (raw): 53 values."""
    return ([e for e in range(100, 103) for _ in range(4)]
            + [e for e in range(103, 106) for _ in range(3)]
            + [e for e in range(106, 121) for _ in range(2)] + [121, 122])


def test_known_answer_cascade():
    exps = _cascade_exponents()
    bits = [(e << 7) | (j % 128) | (0x8000 if j % 3 == 0 else 0) for j, e in enumerate(exps)]
    values = _from_bits(bits)
    rec, counts, table = _roundtrip(values, force=True)
    assert table == (bytes([100, 101, 102]) + bytes(5) + bytes([103, 104, 105]) + bytes(5)
                     + bytes(range(106, 121)) + bytes(1))
    assert counts == (41, 32, 2)
    b = rec.numpy()
    off = section_offsets(53, counts)
    # level 2 in value order: 103 x3 -> 0, 104 x3 -> 1, 105 x3 -> 2, then 32 x 3
    l2 = b[off["L2"]:off["L2"] + 11].tolist()
    assert l2[:3] == [0x40, 0xA5, 0xFE] and l2[3:10] == [0xFF] * 7 and l2[10] == 0x03
    # level 3: 106..120 twice each -> codes 0..14, then 121, 122 -> 15
    l3 = b[off["L3"]:off["L3"] + 16].tolist()
    assert l3 == [0x11 * c for c in range(15)] + [0xFF]
    assert b[off["R"]:off["R"] + 2].tolist() == [121, 122]
    assert _chunk_tables_ok(b, values, counts, table)


def test_known_answer_cascade_interleaved():
    # the same exponents in a fixed shuffled order, repeated across three chunks
    exps = np.array(_cascade_exponents() * 240)  # 12,720 values
    np.random.default_rng(5).shuffle(exps)
    j = np.arange(exps.size)
    bits = ((exps.astype(np.uint16) << 7) | (j % 128).astype(np.uint16)
            | ((j % 3 == 0) << 15).astype(np.uint16))
    values = _from_bits(bits)
    rec, counts, table = _roundtrip(values, force=True)
    assert counts == (41 * 240, 32 * 240, 2 * 240)
    assert _chunk_tables_ok(rec.numpy(), values, counts, table)


def test_gaussian_expert_roundtrip_and_size():
    g = torch.Generator().manual_seed(3)
    values = (torch.randn(100_003, generator=g) * 0.02).to(torch.bfloat16)
    rec, counts, table = _roundtrip(values)
    n = values.numel()
    assert 0.25 < counts.n_second / n < 0.30 and 0.03 < counts.n_third / n < 0.05
    assert counts.n_raw < 100
    assert rec.numel() < 0.68 * 2 * n
    assert _chunk_tables_ok(rec.numpy(), values, counts, table)
    exps = (_bits(values) >> 7) & 0xFF
    hist = np.bincount(exps, minlength=256)
    ranked = [e for e in sorted(range(256), key=lambda x: (-hist[x], x)) if hist[e]]
    assert list(table[:3]) == ranked[:3] and list(table[8:11]) == ranked[3:6]
    third = ranked[6:21]
    assert list(table[16:16 + len(third)]) == third
    assert not any(table[3:8]) and not any(table[11:16])  # unused entries are 0
    assert not any(table[16 + len(third):])


def test_every_bit_pattern_roundtrips():
    values = torch.arange(65536, dtype=torch.int32).to(torch.int16).view(torch.bfloat16)
    rec, counts, table = _roundtrip(values, force=True)
    assert counts == (65536 - 3 * 256, 65536 - 6 * 256, 65536 - 21 * 256)
    assert _chunk_tables_ok(rec.numpy(), values, counts, table)
    # without force the record would be larger than the raw bytes
    assert encode_record(values)[0] is None


@pytest.mark.parametrize("n", [1, 2, 3, 17, 4095, 4097])
def test_short_and_odd_lengths(n):
    g = torch.Generator().manual_seed(n)
    values = (torch.randn(n, generator=g) * 0.02).to(torch.bfloat16)
    rec, counts, table = _roundtrip(values, force=True)
    assert _chunk_tables_ok(rec.numpy(), values, counts, table)


def test_reference_decode_catches_a_wrong_level():
    """A record whose level-2 code of one value is changed decodes to a
    different exponent there and nowhere else (the definition reads each
    list at the value's rank)."""
    exps = _cascade_exponents()
    values = _from_bits([(e << 7) | 5 for e in exps])
    rec, counts, table = encode_record(values, force=True)
    off = section_offsets(values.numel(), counts)
    bad = rec.numpy().copy()
    bad[off["L2"]] ^= 0b01  # entry 0: code 0 (103) -> 1 (104)
    out = decode_record_reference(bad, values.numel(), counts, table)
    diff = np.nonzero(out != _bits(values))[0]
    assert diff.tolist() == [12] and (out[12] >> 7) & 0xFF == 104


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
        out = decode_record_reference(image.record_view(("l", e)).numpy(), n, r.counts, r.table)
        assert np.array_equal(out, _bits(sources[("l", e)]))
    with pytest.raises(ValueError, match="stored raw"):
        image.record_view(("l", 3))
    with pytest.raises(ValueError, match="same number"):
        CompressedExperts.encode({0: torch.zeros(4, dtype=torch.bfloat16),
                                  1: torch.zeros(5, dtype=torch.bfloat16)})
