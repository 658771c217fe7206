"""Host definition of the exponent-coded record format (test helper).

The values a record stands for, computed on the host from the layout that
``specfit_amd.codec`` writes and ``sf_expert_decode`` reads.  Tests check
round trips through it against the raw bf16 bits, and the device decode
against the same bits; the library never calls it.
"""
import numpy as np

from specfit_amd.codec import section_offsets


def decode_record_reference(record, n_values: int, counts, table: bytes):
    """The values a record stands for, on the host (numpy uint16 bit
    patterns): the definition ``sf_expert_decode`` implements."""
    rec = np.asarray(record, dtype=np.uint8)
    off = section_offsets(n_values, counts)
    n2, n3, nr = counts
    sm = rec[:n_values].astype(np.uint16)
    groups = -(-n_values // 16)
    code1 = np.zeros(groups * 16, dtype=np.uint8)
    for p in range(2):
        base = off["P"] + p * off["plane_bytes"]
        words = rec[base:base + 2 * groups].view("<u2")
        bits = (words[:, None] >> np.arange(16, dtype=np.uint16)) & 1
        code1 |= (bits.reshape(-1) << p).astype(np.uint8)
    code1 = code1[:n_values]
    tbl = np.frombuffer(bytes(table), dtype=np.uint8).astype(np.uint16)
    exponent = tbl[code1]

    def unpack(key, count, bits):
        per = 8 // bits
        packed = rec[off[key]:off[key] + -(-count // per)]
        shifts = (np.arange(per) * bits).astype(np.uint8)
        return ((packed[:, None] >> shifts) & ((1 << bits) - 1)).reshape(-1)[:count]

    at2 = np.nonzero(code1 == 3)[0]
    code2 = unpack("L2", n2, 2)
    exponent[at2] = tbl[8 + code2]
    at3 = at2[code2 == 3]
    code3 = unpack("L3", n3, 4)
    exponent[at3] = tbl[16 + code3]
    at_raw = at3[code3 == 15]
    exponent[at_raw] = rec[off["R"]:off["R"] + nr]
    return ((sm & 0x80) << 8) | (exponent << 7) | (sm & 0x7F)
