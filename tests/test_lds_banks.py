"""LDS bank conflicts of the direct GEMM's fragment reads, under gfx950's measured bank rules.

The rules were measured on an MI355X with eight waves per CU issuing one read
pattern back to back and counting shader clocks per instruction:

* ``ds_read_b128``: 4.4 clocks when conflict-free. A wave's 64 lanes go in
  four passes of 16; lane ``l`` is in pass ``(b2^b3^b4, b5)`` of its index
  bits. Within a pass, lanes whose addresses differ but fall in the same
  16-byte slot of a 256-byte bank row (``(addr >> 4) & 15``) serialise:
  two-way costs 8.0 clocks, sixteen-way 64.
* ``ds_read_b64`` and ``ds_read_b64_tr_b16``: 2.5 clocks when conflict-free.
  Two passes, lanes 0-31 then 32-63, over 32 eight-byte slots
  (``(addr >> 3) & 31``); a two-way conflict costs 4.0.

Both rules reproduce every measured pattern (32 for the 16-byte reads, 15 for
the 8-byte reads) to within 30% of the predicted multiple. The patterns below
are the fragment reads of ``csrc/gemm_direct.h`` for both MFMA shapes the
library uses (16x16x32: 16 rows x 4 lane groups; 32x32x16: 32 rows x 2 lane
groups), at every k step of a 64-wide slice and both tile widths of B.
"""

from __future__ import annotations

import re
from pathlib import Path

import pytest

GEMM_DIRECT = Path(__file__).resolve().parent.parent / "kernelforge" / "csrc" / "gemm_direct.h"
LANES = range(64)


def _parity(x: int) -> int:
    return bin(x).count("1") & 1


def b128_multiplicity(addrs: list[int]) -> int:
    worst = 0
    for p in range(4):
        slots: dict[int, set[int]] = {}
        for lane in LANES:
            if (_parity(lane & 0b011100) | ((lane >> 5) << 1)) == p:
                slots.setdefault((addrs[lane] >> 4) & 15, set()).add(addrs[lane])
        worst = max(worst, max(len(v) for v in slots.values()))
    return worst


def b64_multiplicity(addrs: list[int]) -> int:
    worst = 0
    for half in (range(32), range(32, 64)):
        slots: dict[int, set[int]] = {}
        for lane in half:
            slots.setdefault((addrs[lane] >> 3) & 31, set()).add(addrs[lane] & ~7)
        worst = max(worst, max(len(v) for v in slots.values()))
    return worst


# The kernel's swizzles (gemm_direct.h swz_k / swz_n); test_the_swizzles_are_the_kernels
# keeps these in step with the header.
def swz_k(chunk: int, row: int) -> int:
    return chunk ^ ((row >> 1) & 7)


def swz_n(chunk: int, row: int, row_chunks: int) -> int:
    if row_chunks >= 16:
        return chunk ^ (((row & 3) << 2) ^ (((row >> 3) & 1) << 1))
    return chunk ^ ((row & 3) << 1)


def a_reads_16(c: int) -> list[int]:
    """16x16x32: lane (g, li) reads row li, k chunk 4c + g (c = 0, 1)."""
    return [(l & 15) * 128 + swz_k(c * 4 + (l >> 4), l & 15) * 16 for l in LANES]


def a_reads_32(c: int) -> list[int]:
    """32x32x16: lane (h, l32) reads row l32, k chunk 2c + h (c = 0..3)."""
    return [(l & 31) * 128 + swz_k(c * 2 + (l >> 5), l & 31) * 16 for l in LANES]


def b_reads_16(c: int, j: int, bn: int, second: bool) -> list[int]:
    out = []
    for l in LANES:
        g, li = l >> 4, l & 15
        col = j * 16 + (li & 3) * 4
        r0 = c * 32 + 8 * g + (li >> 2) + (4 if second else 0)
        out.append(r0 * bn * 2 + swz_n(col >> 3, r0, bn // 8) * 16 + (col & 7) * 2)
    return out


def b_reads_32(c: int, j: int, bn: int, second: bool) -> list[int]:
    out = []
    for l in LANES:
        grp, i16 = l >> 4, l & 15
        col = j * 32 + 16 * (grp & 1) + (i16 & 3) * 4
        r0 = c * 16 + 8 * (grp >> 1) + (i16 >> 2) + (4 if second else 0)
        out.append(r0 * bn * 2 + swz_n(col >> 3, r0, bn // 8) * 16 + (col & 7) * 2)
    return out


def test_the_rules_reproduce_the_measured_anchor_patterns():
    # Measured: linear 16-byte reads 4.4 clocks, the earlier A swizzle
    # (row & 7) ^ ((row >> 3) & 1) on 16x16x32 fragments 8.0, all 64 lanes in
    # one slot 64.0; linear 8-byte reads 2.5, slots repeating every 16 lanes 4.0.
    assert b128_multiplicity([l * 16 for l in LANES]) == 1
    old = [(l & 15) * 128 + (((l >> 4) ^ (l & 7) ^ ((l >> 3) & 1)) * 16) for l in LANES]
    assert b128_multiplicity(old) == 2
    assert b128_multiplicity([l * 256 for l in LANES]) == 16
    assert b64_multiplicity([l * 8 for l in LANES]) == 1
    assert b64_multiplicity([l * 256 + (l & 15) * 8 for l in LANES]) == 2


@pytest.mark.parametrize("c", range(2))
def test_a_fragments_16x16x32_are_conflict_free(c):
    assert b128_multiplicity(a_reads_16(c)) == 1


@pytest.mark.parametrize("c", range(4))
def test_a_fragments_32x32x16_are_conflict_free(c):
    assert b128_multiplicity(a_reads_32(c)) == 1


@pytest.mark.parametrize("bn", (128, 256))
def test_b_transposing_reads_are_conflict_free(bn):
    for c in range(2):
        for j in range(bn // 64):
            for second in (False, True):
                assert b64_multiplicity(b_reads_16(c, j, bn, second)) == 1
    for c in range(4):
        for j in range(bn // 64):
            for second in (False, True):
                assert b64_multiplicity(b_reads_32(c, j, bn, second)) == 1


def test_swizzles_keep_the_immediate_row_steps():
    # Fragment rows 16 and 32 apart (A) share the k swizzle; B rows r and r + 4
    # (a fragment's second transposing read; the first read's row has bit 2
    # clear) and rows 16 apart share the n one.
    for r in range(64):
        for ch in range(8):
            assert swz_k(ch, r) == swz_k(ch, r + 16) == swz_k(ch, r + 32)
        for ch in range(32):
            assert swz_n(ch, r, 32) == swz_n(ch, r + 16, 32)
            if not r & 4:
                assert swz_n(ch, r, 32) == swz_n(ch, r + 4, 32)
            assert 0 <= swz_n(ch, r, 32) < 32
        for ch in range(16):
            assert 0 <= swz_n(ch, r, 16) < 16


def test_the_swizzles_are_the_kernels():
    src = GEMM_DIRECT.read_text()
    k = re.search(r"int swz_k\(int chunk, int row\) \{\s*return (.+?);", src)
    n = re.search(r"if constexpr \(ROW_CHUNKS >= 16\) return (.+?);", src)
    assert k and k.group(1) == "chunk ^ ((row >> 1) & 7)"
    assert n and n.group(1) == "chunk ^ (((row & 3) << 2) ^ (((row >> 3) & 1) << 1))"
