"""Exponent-coded expert records: fewer bytes over the host link, same slot.

The offloaded path is bound by the host-to-device link: every miss moves a
whole packed expert (9,437,184 B at the Qwen3-30B-A3B shape) from pinned
host memory into an HBM slot (gpu_expert_cache.py:556-561 of the reference
copies the raw bf16 bytes).  A bf16 weight is sign | 8-bit exponent | 7-bit
mantissa, and the weights of an expert use few exponents: N(0, 0.02) values
put 96% of their mass in 7 binades, and trained checkpoints look alike.  An
``ExpertRecord`` keeps, per value, one byte of sign and mantissa and a 4-bit
code into a 15-entry exponent table chosen per expert, plus an escape list
(index, exponent byte) for values outside the table: 12 bits per value, 75%
of the raw bytes.  The cache copies the record into a device staging buffer
and the HIP decoder (``sf_expert_decode``) writes the expert's exact bf16
bytes into the slot, so everything downstream sees what a raw copy delivers.
An expert whose record would not be smaller stays raw.

Record layout (``sf_expert_record_bytes`` / include/specfit_amd.h): S
[n] uint8, X [ceil(n/2)] uint8 (value i's code in byte i/2, low nibble for
even i), EI [e] uint32 ascending, EE [e] uint8, EC [ceil(n/4096) + 1]
uint32 (EC[k] = escapes below value 4096 k); each section 256-byte aligned.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Hashable, Mapping

import torch

ESCAPE = 15           # the code of a value whose exponent is not in the table
TABLE_SIZE = 15       # exponents a table holds
CHUNK = 4096          # values per entry of the chunk table (SF_DECODE_CHUNK)
_ALIGN = 256


def _align(x: int) -> int:
    return (x + _ALIGN - 1) // _ALIGN * _ALIGN


def record_bytes(n_values: int, n_escapes: int) -> int:
    """Size of the record of ``n_values`` values with ``n_escapes`` escapes
    (the formula of sf_expert_record_bytes)."""
    if n_values < 0 or not 0 <= n_escapes <= n_values:
        raise ValueError("invalid record counts")
    ec = section_offsets(n_values, n_escapes)[4]
    return ec + _align(4 * (-(-n_values // CHUNK) + 1))


def section_offsets(n_values: int, n_escapes: int) -> tuple[int, int, int, int, int]:
    """Byte offsets of S, X, EI, EE and EC in a record."""
    x = _align(n_values)
    ei = x + _align((n_values + 1) // 2)
    ee = ei + _align(4 * n_escapes)
    ec = ee + _align(n_escapes)
    return 0, x, ei, ee, ec


@dataclass(frozen=True)
class ExpertRecord:
    """Where one expert's record sits in a ``CompressedExperts`` blob."""

    offset: int      # byte offset in the blob (256-byte aligned)
    nbytes: int      # bytes the transfer moves
    n_escapes: int
    table: bytes     # 16 exponent bytes; entry c is the exponent of code c
    raw: bool        # True: no record, the transfer moves the raw bytes


def encode_record(values: torch.Tensor, *, force: bool = False
                  ) -> tuple[torch.Tensor | None, int, bytes]:
    """(record uint8 tensor on values' device, escapes, 16-byte table) of a
    1-D bf16 tensor; the record is None when it would not be smaller than
    the raw bytes (unless ``force``).  The table holds the 15 most frequent
    exponents, ties to the lower exponent."""
    if values.dtype != torch.bfloat16 or values.dim() != 1:
        raise ValueError("encode_record expects a 1-D bf16 tensor")
    n = values.numel()
    dev = values.device
    u = values.view(torch.int16).to(torch.int32) & 0xFFFF
    exponent = (u >> 7) & 0xFF
    hist = torch.bincount(exponent, minlength=256)
    order = torch.sort(hist, descending=True, stable=True).indices[:TABLE_SIZE]
    used = order[hist[order] > 0]
    lut = torch.full((256,), ESCAPE, dtype=torch.int32, device=dev)
    lut[used] = torch.arange(used.numel(), dtype=torch.int32, device=dev)
    code = lut[exponent]
    escapes = torch.nonzero(code == ESCAPE).flatten()
    n_esc = int(escapes.numel())
    size = record_bytes(n, n_esc)
    table = bytes(used.tolist()) + bytes(16 - used.numel())
    if size >= 2 * n and not force:
        return None, n_esc, table
    _, off_x, off_ei, off_ee, off_ec = section_offsets(n, n_esc)
    rec = torch.zeros(size, dtype=torch.uint8, device=dev)
    rec[:n] = (((u >> 8) & 0x80) | (u & 0x7F)).to(torch.uint8)
    if n % 2:
        code = torch.cat([code, code.new_zeros(1)])
    rec[off_x:off_x + code.numel() // 2] = (code[0::2] | (code[1::2] << 4)).to(torch.uint8)
    if n_esc:
        rec[off_ei:off_ei + 4 * n_esc] = escapes.to(torch.int32).view(torch.uint8)
        rec[off_ee:off_ee + n_esc] = exponent[escapes].to(torch.uint8)
    starts = torch.arange(0, n + CHUNK, CHUNK, device=dev)[:-(-n // CHUNK) + 1]
    first = torch.searchsorted(escapes, starts).to(torch.int32)
    rec[off_ec:off_ec + 4 * first.numel()] = first.view(torch.uint8)
    return rec, n_esc, table


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
            rec, n_esc, table = encode_record(src.reshape(-1).to(device, non_blocking=False))
            encoded[key] = (rec, n_esc, table)
        offset = 0
        layout = {}
        for key, (rec, n_esc, table) in encoded.items():
            if rec is None:
                layout[key] = ExpertRecord(0, 2 * numel, n_esc, table, True)
            else:
                layout[key] = ExpertRecord(offset, rec.numel(), n_esc, table, False)
                offset += rec.numel()
        blob = torch.empty(max(offset, 1), dtype=torch.uint8, pin_memory=torch.cuda.is_available())
        for key, (rec, _, _) in encoded.items():
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


def decode_record_reference(record, n_values: int, n_escapes: int, table: bytes):
    """The values a record stands for, on the host (numpy uint16 bit
    patterns): the definition ``sf_expert_decode`` implements."""
    import numpy as np

    rec = np.asarray(record, dtype=np.uint8)
    _, off_x, off_ei, off_ee, _ = section_offsets(n_values, n_escapes)
    sm = rec[:n_values].astype(np.uint16)
    packed = rec[off_x:off_x + (n_values + 1) // 2]
    codes = np.empty(2 * packed.size, dtype=np.uint8)
    codes[0::2] = packed & 15
    codes[1::2] = packed >> 4
    codes = codes[:n_values]
    tbl = np.frombuffer(bytes(table), dtype=np.uint8).astype(np.uint16)
    exponent = tbl[codes]
    if n_escapes:
        idx = rec[off_ei:off_ei + 4 * n_escapes].view("<u4").astype(np.int64)
        exponent[idx] = rec[off_ee:off_ee + n_escapes]
    return ((sm & 0x80) << 8) | (exponent << 7) | (sm & 0x7F)
