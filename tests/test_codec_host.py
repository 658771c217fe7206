"""Host checks of the exponent-coded expert records (specfit_amd.codec):
record sizes against the C library, hand-built known answers, round trips
through the host definition of the decode, the chunk tables, the table
rules and the raw fallback.  The device decode is checked against the same
bytes in tests/test_gpu_codec.py."""
import numpy as np
import pytest
import torch

from specfit_amd import _native
from specfit_amd.codec import (CompressedExperts, decode_record_reference, encode_record,
                               record_bytes, section_offsets)


def _bits(t: torch.Tensor) -> np.ndarray:
    return t.view(torch.int16).numpy().view(np.uint16)


def _from_bits(bits) -> torch.Tensor:
    return torch.tensor(np.asarray(bits, dtype=np.uint16).view(np.int16)).view(torch.bfloat16)


def _chunk_tables_ok(rec: np.ndarray, values: torch.Tensor, q: int, r: int, table: bytes) -> bool:
    """QC[k] / RC[k] = secondary / raw entries of the values below 4096 k."""
    n = values.numel()
    off = section_offsets(n, q, r)
    exps = (_bits(values) >> 7) & 0xFF
    distinct = len(set(exps.tolist()))
    primary = list(table[:min(7, distinct)])  # the entries in use (the rest are padding)
    secondary = list(table[16:16 + min(15, max(0, distinct - 7))])
    in_primary = np.isin(exps, primary)
    sec_pos = np.nonzero(~in_primary)[0]
    raw_pos = sec_pos[~np.isin(exps[sec_pos], secondary)]
    chunks = -(-n // 4096)
    qc = rec[off["QC"]:off["QC"] + 4 * (chunks + 1)].view("<u4")
    rc = rec[off["RC"]:off["RC"] + 4 * (chunks + 1)].view("<u4")
    want_q = [int(np.count_nonzero(sec_pos < 4096 * k)) for k in range(chunks + 1)]
    want_r = [int(np.count_nonzero(raw_pos < 4096 * k)) for k in range(chunks + 1)]
    return (len(sec_pos), len(raw_pos)) == (q, r) and qc.tolist() == want_q and rc.tolist() == want_r


def _roundtrip(values: torch.Tensor, force: bool = False):
    rec, q, r, table = encode_record(values, force=force)
    assert rec is not None
    out = decode_record_reference(rec.numpy(), values.numel(), q, r, table)
    assert np.array_equal(out, _bits(values))
    return rec, q, r, table


@pytest.mark.parametrize("n,q,r", [(0, 0, 0), (1, 0, 0), (5, 0, 0), (4096, 3, 1),
                                   (4_718_592, 96_000, 700), (4_718_593, 4_718_593, 4_718_593)])
def test_record_size_matches_the_library(n, q, r):
    lib = _native.lib()
    assert record_bytes(n, q, r) == lib.sf_expert_record_bytes(n, q, r)
    off = section_offsets(n, q, r)
    order = [off[k] for k in ("S", "P", "Q", "R", "QC", "RC", "size")]
    assert all(o % 256 == 0 for o in order) and order == sorted(order)
    assert lib.sf_expert_record_bytes(5, 6, 0) == -1 and lib.sf_expert_record_bytes(5, 2, 3) == -1
    with pytest.raises(ValueError):
        record_bytes(5, 2, 3)


def test_known_answer_record():
    # 1.0, -2.0, 0.5, 1.5, 1.0: exponents 127, 128, 126, 127, 127
    values = torch.tensor([1.0, -2.0, 0.5, 1.5, 1.0], dtype=torch.bfloat16)
    rec, q, r, table = encode_record(values, force=True)
    assert (q, r) == (0, 0)
    # primary by count, ties to the lower exponent; no secondary exponents
    assert table == bytes([127, 126, 128]) + bytes(13) + bytes(16)
    b = rec.numpy()
    # S at 0; planes at 256, 512, 768 (codes 0, 2, 1, 0, 0); QC at 1024, RC at 1280
    assert b.size == 1536 and b[:5].tolist() == [0x00, 0x80, 0x00, 0x40, 0x00]
    assert b[256:258].tolist() == [0b100, 0] and b[512:514].tolist() == [0b10, 0]
    assert not b[768:].any() and not b[5:256].any() and not b[258:512].any()
    assert not b[514:768].any()
    # too small to gain anything: the expert stays raw
    assert encode_record(values)[0] is None


def test_known_answer_secondary_and_raw_codes():
    # 23 exponents 100 .. 122: the first 7 twice, the others once (30 values)
    exps = [100 + j for j in range(7)] * 2 + [107 + j for j in range(16)]
    bits = [(e << 7) | (j % 128) | (0x8000 if j % 3 == 0 else 0) for j, e in enumerate(exps)]
    values = _from_bits(bits)
    rec, q, r, table = _roundtrip(values, force=True)
    assert table[:7] == bytes(range(100, 107)) and table[7] == 0
    assert table[16:31] == bytes(range(107, 122)) and table[31] == 0
    assert (q, r) == (16, 1)  # exponents 107..122 go secondary, 122 raw
    assert _chunk_tables_ok(rec.numpy(), values, q, r, table)


def test_gaussian_expert_roundtrip_and_size():
    g = torch.Generator().manual_seed(3)
    values = (torch.randn(100_003, generator=g) * 0.02).to(torch.bfloat16)
    rec, q, r, table = _roundtrip(values)
    assert 0.01 < q / values.numel() < 0.03 and r < 100
    assert rec.numel() < 0.70 * 2 * values.numel()
    assert _chunk_tables_ok(rec.numpy(), values, q, r, table)
    exps = (_bits(values) >> 7) & 0xFF
    counts = np.bincount(exps, minlength=256)
    ranked = [e for e in sorted(range(256), key=lambda x: (-counts[x], x)) if counts[e]]
    sec = ranked[7:22]
    assert list(table[:7]) == ranked[:7] and list(table[16:16 + len(sec)]) == sec
    assert not any(table[16 + len(sec):])  # unused secondary entries are 0


def test_every_bit_pattern_roundtrips():
    values = torch.arange(65536, dtype=torch.int32).to(torch.int16).view(torch.bfloat16)
    rec, q, r, table = _roundtrip(values, force=True)
    assert (q, r) == (65536 - 7 * 256, 65536 - 22 * 256)
    assert _chunk_tables_ok(rec.numpy(), values, q, r, table)
    # without force the record would be larger than the raw bytes
    assert encode_record(values)[0] is None


@pytest.mark.parametrize("n", [1, 2, 3, 17, 4095, 4097])
def test_short_and_odd_lengths(n):
    g = torch.Generator().manual_seed(n)
    values = (torch.randn(n, generator=g) * 0.02).to(torch.bfloat16)
    rec, q, r, table = _roundtrip(values, force=True)
    assert _chunk_tables_ok(rec.numpy(), values, q, r, table)


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
        out = decode_record_reference(image.record_view(("l", e)).numpy(), n, r.n_secondary,
                                      r.n_raw, r.table)
        assert np.array_equal(out, _bits(sources[("l", e)]))
    with pytest.raises(ValueError, match="stored raw"):
        image.record_view(("l", 3))
    with pytest.raises(ValueError, match="same number"):
        CompressedExperts.encode({0: torch.zeros(4, dtype=torch.bfloat16),
                                  1: torch.zeros(5, dtype=torch.bfloat16)})
