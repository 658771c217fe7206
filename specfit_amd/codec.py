"""Exponent-coded expert records: fewer bytes over the host link, same slot.

The offloaded path is bound by the host-to-device link: every miss moves a
whole packed expert (9,437,184 B at the Qwen3-30B-A3B shape) from pinned
host memory into an HBM slot (gpu_expert_cache.py:556-561 of the reference
copies the raw bf16 bytes).  A bf16 weight is sign | 8-bit exponent | 7-bit
mantissa, and the weights of an expert use few exponents: N(0, 0.02) values
put 98% of their mass in 7 binades, and trained checkpoints look alike.  A
record keeps, per value, one byte of sign and mantissa and a 3-bit code into
a 7-entry primary exponent table; code 7 defers to a 4-bit secondary code
(15 more exponents) kept only for those values, and its code 15 to a raw
exponent byte.  For N(0, 0.02) weights that is ~11.1 bits per value, 69% of
the raw bytes.  The cache copies the record into a device staging buffer
and the HIP decoder (``sf_expert_decode``) writes the expert's exact bf16
bytes into the slot, so everything downstream sees what a raw copy
delivers.  An expert whose record would not be smaller stays raw.

Record layout (``sf_expert_record_bytes`` / include/specfit_amd.h), every
section 256-byte aligned: S [n] uint8 (sign << 7 | mantissa); P, three bit
planes of ceil(n/16) uint16 words (plane p, word g: bit p of the primary
codes of values 16g .. 16g+15); Q [ceil(q/2)] uint8 (secondary codes of the
values with primary code 7, in value order, entry 2j in the low nibble of
byte j); R [r] uint8 (raw exponents of the values with secondary code 15,
in value order); QC and RC [ceil(n/4096) + 1] uint32 (Q and R entries of
the values before each 4096-value chunk).
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Hashable, Mapping

import torch

PRIMARY = 7           # exponents of the primary table; code 7 defers to the secondary
SECONDARY = 15        # exponents of the secondary table; code 15 defers to a raw byte
CHUNK = 4096          # values per entry of the chunk tables (SF_DECODE_CHUNK)
_ALIGN = 256


def _align(x: int) -> int:
    return (x + _ALIGN - 1) // _ALIGN * _ALIGN


def section_offsets(n_values: int, n_secondary: int, n_raw: int) -> dict:
    """Byte offsets of the sections of a record (and its ``size``)."""
    if n_values < 0 or not 0 <= n_raw <= n_secondary <= n_values:
        raise ValueError("invalid record counts")
    chunks = -(-n_values // CHUNK)
    plane = _align(2 * -(-n_values // 16))
    off = {"S": 0, "P": _align(n_values)}
    off["Q"] = off["P"] + 3 * plane
    off["R"] = off["Q"] + _align((n_secondary + 1) // 2)
    off["QC"] = off["R"] + _align(n_raw)
    off["RC"] = off["QC"] + _align(4 * (chunks + 1))
    off["size"] = off["RC"] + _align(4 * (chunks + 1))
    off["plane_bytes"] = plane
    return off


def record_bytes(n_values: int, n_secondary: int, n_raw: int) -> int:
    """Size of a record (the formula of sf_expert_record_bytes)."""
    return section_offsets(n_values, n_secondary, n_raw)["size"]


@dataclass(frozen=True)
class ExpertRecord:
    """Where one expert's record sits in a ``CompressedExperts`` blob."""

    offset: int        # byte offset in the blob (256-byte aligned)
    nbytes: int        # bytes the transfer moves
    n_secondary: int   # values with primary code 7
    n_raw: int         # values with secondary code 15
    table: bytes       # 32 bytes: primary exponents at 0..6, secondary at 16..30
    raw: bool          # True: no record, the transfer moves the raw bytes


def _top(hist: torch.Tensor, k: int) -> torch.Tensor:
    """The k most frequent exponents with a nonzero count, ties to the lower."""
    order = torch.sort(hist, descending=True, stable=True).indices[:k]
    return order[hist[order] > 0]


def encode_record(values: torch.Tensor, *, force: bool = False
                  ) -> tuple[torch.Tensor | None, int, int, bytes]:
    """(record uint8 tensor on values' device, secondary count, raw count,
    32-byte table) of a 1-D bf16 tensor; the record is None when it would
    not be smaller than the raw bytes (unless ``force``).  The primary table
    holds the 7 most frequent exponents, the secondary the next 15."""
    if values.dtype != torch.bfloat16 or values.dim() != 1:
        raise ValueError("encode_record expects a 1-D bf16 tensor")
    n = values.numel()
    dev = values.device
    u = values.view(torch.int16).to(torch.int32) & 0xFFFF
    exponent = (u >> 7) & 0xFF
    hist = torch.bincount(exponent, minlength=256)
    primary = _top(hist, PRIMARY)
    rest = hist.clone()
    rest[primary] = 0
    secondary = _top(rest, SECONDARY)
    lut1 = torch.full((256,), PRIMARY, dtype=torch.int32, device=dev)
    lut1[primary] = torch.arange(primary.numel(), dtype=torch.int32, device=dev)
    lut2 = torch.full((256,), SECONDARY, dtype=torch.int32, device=dev)
    lut2[secondary] = torch.arange(secondary.numel(), dtype=torch.int32, device=dev)
    code1 = lut1[exponent]
    esc1 = torch.nonzero(code1 == PRIMARY).flatten()      # values with a secondary code
    code2 = lut2[exponent[esc1]]
    raw_at = esc1[code2 == SECONDARY]                      # values with a raw exponent
    q, r = int(esc1.numel()), int(raw_at.numel())
    off = section_offsets(n, q, r)
    table = (bytes(primary.tolist()) + bytes(16 - primary.numel())
             + bytes(secondary.tolist()) + bytes(16 - secondary.numel()))
    if off["size"] >= 2 * n and not force:
        return None, q, r, table
    rec = torch.zeros(off["size"], dtype=torch.uint8, device=dev)
    rec[:n] = (((u >> 8) & 0x80) | (u & 0x7F)).to(torch.uint8)
    groups = -(-n // 16)
    padded = torch.zeros(groups * 16, dtype=torch.int32, device=dev)
    padded[:n] = code1
    weights = torch.tensor([1 << k for k in range(16)], dtype=torch.int32, device=dev)
    for p in range(3):
        words = (((padded >> p) & 1).view(groups, 16) * weights).sum(1)
        base = off["P"] + p * off["plane_bytes"]
        rec[base:base + 2 * groups] = words.to(torch.int32).to(torch.int16).view(torch.uint8)
    if q:
        c2 = code2 if q % 2 == 0 else torch.cat([code2, code2.new_zeros(1)])
        rec[off["Q"]:off["Q"] + c2.numel() // 2] = (c2[0::2] | (c2[1::2] << 4)).to(torch.uint8)
    if r:
        rec[off["R"]:off["R"] + r] = exponent[raw_at].to(torch.uint8)
    starts = torch.arange(0, n + CHUNK, CHUNK, device=dev)[:-(-n // CHUNK) + 1]
    for key, positions in (("QC", esc1), ("RC", raw_at)):
        first = torch.searchsorted(positions, starts).to(torch.int32)
        rec[off[key]:off[key] + 4 * first.numel()] = first.view(torch.uint8)
    return rec, q, r, table


class CompressedExperts:
    """One cache's experts as exponent-coded records in ONE page-locked
    blob (``blob``, uint8), with each expert's ``ExpertRecord``."""

    def __init__(self, blob: torch.Tensor, records: dict, numel: int) -> None:
        self.blob = blob
        self.records = records
        self.numel = numel

    @classmethod
    def encode(cls, sources: Mapping[Hashable, torch.Tensor], *,
               device: torch.device | str = "cpu") -> "CompressedExperts":
        """Encode every source (bf16, any shape, all the same numel) on
        ``device`` (a GPU encodes a 1.1 GiB layer in well under a second)."""
        if not sources:
            raise ValueError("no experts to encode")
        device = torch.device(device)
        numel = None
        encoded = {}
        for key, src in sources.items():
            if src.dtype != torch.bfloat16:
                raise ValueError(f"expert {key!r} is not bf16")
            if numel is None:
                numel = src.numel()
            elif src.numel() != numel:
                raise ValueError("all experts must have the same number of values")
            encoded[key] = encode_record(src.reshape(-1).to(device, non_blocking=False))
        offset = 0
        layout = {}
        for key, (rec, q, r, table) in encoded.items():
            if rec is None:
                layout[key] = ExpertRecord(0, 2 * numel, q, r, table, True)
            else:
                layout[key] = ExpertRecord(offset, rec.numel(), q, r, table, False)
                offset += rec.numel()
        blob = torch.empty(max(offset, 1), dtype=torch.uint8, pin_memory=torch.cuda.is_available())
        for key, (rec, _, _, _) in encoded.items():
            if rec is not None:
                r = layout[key]
                blob[r.offset:r.offset + r.nbytes].copy_(rec)
        return cls(blob, layout, numel)

    @property
    def raw_bytes(self) -> int:
        """Bytes the same experts move as raw bf16."""
        return 2 * self.numel * len(self.records)

    @property
    def transfer_bytes(self) -> int:
        """Bytes the records move (raw experts at their raw size)."""
        return sum(r.nbytes for r in self.records.values())

    def staging_bytes(self) -> int:
        """Largest record: the size of a device staging buffer."""
        return max((r.nbytes for r in self.records.values() if not r.raw), default=0)

    def record_view(self, key: Hashable) -> torch.Tensor:
        r = self.records[key]
        if r.raw:
            raise ValueError(f"expert {key!r} is stored raw")
        return self.blob[r.offset:r.offset + r.nbytes]


def decode_record_reference(record, n_values: int, n_secondary: int, n_raw: int,
                            table: bytes):
    """The values a record stands for, on the host (numpy uint16 bit
    patterns): the definition ``sf_expert_decode`` implements."""
    import numpy as np

    rec = np.asarray(record, dtype=np.uint8)
    off = section_offsets(n_values, n_secondary, n_raw)
    sm = rec[:n_values].astype(np.uint16)
    groups = -(-n_values // 16)
    code1 = np.zeros(groups * 16, dtype=np.uint8)
    for p in range(3):
        base = off["P"] + p * off["plane_bytes"]
        words = rec[base:base + 2 * groups].view("<u2")
        bits = (words[:, None] >> np.arange(16, dtype=np.uint16)) & 1
        code1 |= (bits.reshape(-1) << p).astype(np.uint8)
    code1 = code1[:n_values]
    tbl = np.frombuffer(bytes(table), dtype=np.uint8).astype(np.uint16)
    exponent = tbl[code1]
    esc1 = np.nonzero(code1 == PRIMARY)[0]
    if n_secondary:
        packed = rec[off["Q"]:off["Q"] + (n_secondary + 1) // 2]
        code2 = np.empty(2 * packed.size, dtype=np.uint8)
        code2[0::2] = packed & 15
        code2[1::2] = packed >> 4
        code2 = code2[:n_secondary]
        exponent[esc1] = tbl[16 + code2]
        raw_at = esc1[code2 == SECONDARY]
        exponent[raw_at] = rec[off["R"]:off["R"] + n_raw]
    return ((sm & 0x80) << 8) | (exponent << 7) | (sm & 0x7F)
