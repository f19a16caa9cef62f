"""LDS layout invariants of the attention kernels (CPU): the XOR swizzle
tables in pdum_dsl_amd/csrc/attn_common.h must keep the operand reads the
kernels issue bank-conflict free, for 32 and for 64 four-byte banks.

The read patterns (one 16-byte slot per lane for row reads, two 8-byte halves
of a 16-byte slot pair per 16-lane group for ds_read_b64_tr_b16) are the ones
the kernels issue; a table that breaks any of them costs LDS cycles, never
correctness, so this pins a performance property the GPU tests cannot see."""

import re
from pathlib import Path

import pytest

HDR = Path(__file__).resolve().parents[1] / "pdum_dsl_amd" / "csrc" / "attn_common.h"


def _table(D):
    src = HDR.read_text()
    m = re.search(r"kTable = D == 128 \? (0x[0-9a-fA-F]+)ull : (0x[0-9a-fA-F]+)ull", src)
    assert m, "swizzle table constants not found"
    v = int(m.group(1 if D == 128 else 2), 16)
    return [(v >> (4 * i)) & 15 for i in range(16)]


def swap23(r):
    return (r & ~12) | ((r & 4) << 1) | ((r & 8) >> 1)


def _slot(row, chunk, f, cpr):
    """16-byte slot index (in LDS order) holding chunk `chunk` of `row`."""
    return row * cpr + (chunk ^ f[row % 16])


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("banks", [32, 64])
def test_row_operand_reads_are_conflict_free(D, banks):
    f, cpr = _table(D), D // 8
    per = banks * 4 // 16  # 16-byte slots served per cycle
    lanes = per  # b128 reads: one slot per lane
    for kb in range(2):
        for c in range(cpr):
            rows = [kb * 32 + swap23(r) for r in range(lanes)]
            slots = {_slot(r, c, f, cpr) % per for r in rows}
            assert len(slots) == lanes, (D, banks, c)


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("banks", [32, 64])
def test_transposed_reads_are_conflict_free(D, banks):
    f, cpr = _table(D), D // 8
    groups = banks * 4 // 128  # 16-lane groups (8 bytes each) served per cycle
    for s in range(2):
        for h in range(2):
            for db in range(D // 32):
                for g0 in range(0, 4, groups):
                    halves = set()
                    for G in range(g0, g0 + groups):
                        for kk in range(4):
                            row = 16 * s + 8 * (G >> 1) + 4 * h + kk
                            for c4 in range(4):
                                chunk = 4 * db + 2 * (G & 1) + (c4 >> 1)
                                halves.add((_slot(row, chunk, f, cpr) * 2 + (c4 & 1)) % (banks * 4 // 8))
                    assert len(halves) == 16 * groups, (D, banks, s, h, db, g0)


@pytest.mark.parametrize("D", [64, 128])
def test_the_table_is_a_permutation_per_row(D):
    f, cpr = _table(D), D // 8
    for r in range(16):
        assert f[r] < cpr
        assert sorted(c ^ f[r] for c in range(cpr)) == list(range(cpr))


# ---- the forward's 16x16x32 layout (flash_fwd.hip swz16_k / swz16_v)

FWD = Path(__file__).resolve().parents[1] / "pdum_dsl_amd" / "csrc" / "flash_fwd.hip"


def _fwd_swizzle(name):
    """The swizzle function `name` of flash_fwd.hip as a Python callable
    (its one return statement, a C conditional over `row` and `D`)."""
    src = FWD.read_text()
    m = re.search(r"int %s\(int row\) \{\s*return (.*?);\s*\}" % name, src, re.S)
    assert m, f"{name} not found"
    cond, a, b = re.match(r"(D == 128) \? (.*) : (.*)$", m.group(1).strip()).groups()
    return lambda row, D: eval(a if D == 128 else b, {"row": row})


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("banks", [32, 64])
def test_forward_k_reads_are_conflict_free(D, banks):
    """Lanes 16 G + c read K row c (of a 16-row half) at chunk 4 ks + G, 16
    bytes each: every group of lanes served in one cycle hits distinct banks."""
    swz, cpr = _fwd_swizzle("swz16_k"), D // 8
    per = banks * 4 // 16
    for half in range(2):
        for ks in range(D // 32):
            for l0 in range(0, 64, per):
                slots = set()
                for lane in range(l0, l0 + per):
                    G, c = lane >> 4, lane & 15
                    row, chunk = 16 * half + c, 4 * ks + G
                    slots.add((row * cpr + (chunk ^ swz(row, D))) % per)
                assert len(slots) == per, (D, banks, half, ks, l0)


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("banks", [32, 64])
def test_forward_v_transposed_reads_are_conflict_free(D, banks):
    """ds_read_b64_tr_b16: lane 16 G + 4 k + c addresses 8 bytes of V row
    4 G + k (+ 16), features 16 fb + 4 c; the lanes served in one cycle
    (banks * 4 / 8 of them) must hit distinct 8-byte bank pairs."""
    swz, cpr = _fwd_swizzle("swz16_v"), D // 8
    per = banks * 4 // 8
    for half in range(2):
        for fb in range(D // 16):
            for l0 in range(0, 64, per):
                halves = set()
                for lane in range(l0, l0 + per):
                    G, k, c = lane >> 4, (lane >> 2) & 3, lane & 3
                    row, chunk = 16 * half + 4 * G + k, 2 * fb + (c >> 1)
                    halves.add(((row * cpr + (chunk ^ swz(row, D))) * 2 + (c & 1)) % per)
                assert len(halves) == per, (D, banks, half, fb, l0)


@pytest.mark.parametrize("name", ["swz16_k", "swz16_v"])
@pytest.mark.parametrize("D", [64, 128])
def test_forward_swizzles_permute_each_row(name, D):
    swz, cpr = _fwd_swizzle(name), D // 8
    for r in range(32):
        assert sorted(c ^ swz(r, D) for c in range(cpr)) == list(range(cpr))
