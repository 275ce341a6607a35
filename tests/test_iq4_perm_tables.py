"""CPU: the two-table IQ4_NL lookup of the GEMV's block dot (iq4_dot8 in
qwen35_amd/csrc/qhip_device.hpp) gives every codebook value.

The kernel looks each 4-bit index n up twice with v_perm_b32 -- selector n in
the low table, n ^ 8 in the high table -- and multiplies both bytes into the
dot.  This restates v_perm_b32's byte selection as the gfx9 ISA defines it
(selector 0..7: that byte of {src0:src1}; 8..11: the sign of byte 1, 3, 5, 7
replicated; 12: 0x00; 13 and above: 0xFF) and checks, for all 16 indices,
that the two int8 bytes add up to the codebook value the oracle decodes
(an IQ4_NL block with d = 1 dequantizes to the codebook entries)."""
import re
from pathlib import Path

import numpy as np

import pyoracle as po

HDR = Path(__file__).resolve().parents[1] / "qwen35_amd" / "csrc" / "qhip_device.hpp"


def const(name):
    m = re.search(rf"constexpr uint32_t {name} = (0x[0-9A-Fa-f]+)u;", HDR.read_text())
    assert m, name
    return int(m.group(1), 16)


def perm_byte(src0, src1, sel):
    data = (src0 << 32) | src1
    if sel >= 13:
        return 0xFF
    if sel == 12:
        return 0x00
    if sel >= 8:
        bit = [15, 31, 47, 63][sel - 8]
        return 0xFF if (data >> bit) & 1 else 0x00
    return (data >> (8 * sel)) & 0xFF


def s8(b):
    return b - 256 if b >= 128 else b


def test_two_lookups_add_up_to_the_codebook(oracle):
    # the codebook as the oracle decodes it: block bytes d = 1.0, index byte j
    # = j (values 0..15 in the low nibbles), so value j = codebook[j]
    blk = np.zeros(18, np.uint8)
    blk[0:2] = [0x00, 0x3C]
    blk[2:18] = np.arange(16, dtype=np.uint8)
    book = oracle.dequant_row(po.TT_IQ4_NL, blk, 32)[:16]
    assert np.array_equal(book, np.round(book))
    L0, L1, H0, H1 = const("IQ4_L0"), const("IQ4_L1"), const("IQ4_H0"), const("IQ4_H1")
    for n in range(16):
        lo = s8(perm_byte(L1, L0, n))
        hi = s8(perm_byte(H1, H0, n ^ 8))
        assert lo + hi == int(book[n]), (n, lo, hi, book[n])


def test_select_lookup_matches_the_codebook(oracle):
    """The byte-decoding lookup (iq4_lookup, used where a decoded byte is
    reused: MMQ staging and the multi-token GEMV) on the same restatement."""
    blk = np.zeros(18, np.uint8)
    blk[0:2] = [0x00, 0x3C]
    blk[2:18] = np.arange(16, dtype=np.uint8)
    book = oracle.dequant_row(po.TT_IQ4_NL, blk, 32)[:16]
    T0, T1, T2, T3 = const("IQ4_T0"), const("IQ4_T1"), const("IQ4_T2"), const("IQ4_T3")
    for n in range(16):
        s7, pick = n & 7, ((n >> 1) & 4)
        lo, hi = perm_byte(T1, T0, s7), perm_byte(T3, T2, s7)
        got = perm_byte(hi, lo, pick)  # result byte 0 of perm(hi, lo, pick | 0x03020100)
        assert s8(got) == int(book[n]), n
