"""LDS layout invariants of the attention kernels (CPU): the XOR swizzles of
pdum_dsl_amd/csrc/flash_fwd.hip and flash_bwd.hip must keep the operand reads
the kernels issue bank-conflict free, for 32 and for 64 four-byte banks.

The read patterns (one 16-byte slot per lane for row reads, 8-byte halves of
16-byte slot pairs for ds_read_b64_tr_b16) are the ones the kernels issue; a
swizzle that breaks any of them costs LDS cycles, never correctness, so this
pins a performance property the GPU tests cannot see."""

import re
from pathlib import Path

import pytest

BWD = Path(__file__).resolve().parents[1] / "pdum_dsl_amd" / "csrc" / "flash_bwd.hip"


def _table(D):
    """The backward's per-row XOR table (swz16_rt): entry i masks row i % 16."""
    src = BWD.read_text()
    m = re.search(r"kTable = D == 128 \? (0x[0-9a-fA-F]+)ull : (0x[0-9a-fA-F]+)ull", src)
    assert m, "swizzle table constants not found"
    v = int(m.group(1 if D == 128 else 2), 16)
    return [(v >> (4 * i)) & 15 for i in range(16)]


def _row_reads_conflict_free(swz, D, banks):
    """Lanes 16 G + c read row c (+ 16 half) at chunk 4 ks + G, 16 bytes each."""
    cpr, per = D // 8, banks * 4 // 16
    for half in range(2):
        for ks in range(D // 32):
            for l0 in range(0, 64, per):
                slots = set()
                for lane in range(l0, l0 + per):
                    G, c = lane >> 4, lane & 15
                    row, chunk = 16 * half + c, 4 * ks + G
                    slots.add((row * cpr + (chunk ^ swz(row))) % per)
                if len(slots) != per:
                    return False
    return True


def _transposed_reads_conflict_free(swz, D, banks):
    """ds_read_b64_tr_b16: lane 16 G + 4 k + c addresses 8 bytes of row 4 G + k
    (+ 16 half), features 16 fb + 4 c; the lanes served in one cycle
    (banks * 4 / 8 of them) must hit distinct 8-byte bank pairs."""
    cpr, per = D // 8, banks * 4 // 8
    for half in range(2):
        for fb in range(D // 16):
            for l0 in range(0, 64, per):
                halves = set()
                for lane in range(l0, l0 + per):
                    G, k, c = lane >> 4, (lane >> 2) & 3, lane & 3
                    row, chunk = 16 * half + 4 * G + k, 2 * fb + (c >> 1)
                    halves.add(((row * cpr + (chunk ^ swz(row))) * 2 + (c & 1)) % per)
                if len(halves) != per:
                    return False
    return True


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("banks", [32, 64])
def test_backward_tiles_serve_both_read_patterns_conflict_free(D, banks):
    """Q, dO and K tiles are read as rows AND transposed from one layout."""
    f = _table(D)
    swz = lambda row: f[row % 16]  # noqa: E731
    assert _row_reads_conflict_free(swz, D, banks)
    assert _transposed_reads_conflict_free(swz, D, banks)


@pytest.mark.parametrize("D", [64, 128])
def test_the_table_is_a_permutation_per_row(D):
    f, cpr = _table(D), D // 8
    for r in range(16):
        assert f[r] < cpr
        assert sorted(c ^ f[r] for c in range(cpr)) == list(range(cpr))


def test_a_planted_table_error_is_caught():
    """The checkers are not vacuous: a table whose rows 0 and 1 share a mask
    breaks a read pattern."""
    f = _table(128)
    f[1] = f[0]
    swz = lambda row: f[row % 16]  # noqa: E731
    assert not (_row_reads_conflict_free(swz, 128, 32) and _transposed_reads_conflict_free(swz, 128, 64)
                and _row_reads_conflict_free(swz, 128, 64) and _transposed_reads_conflict_free(swz, 128, 32))


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
    """K rows are read as rows (the A operand of S^T = K Q^T)."""
    swz = _fwd_swizzle("swz16_k")
    assert _row_reads_conflict_free(lambda row: swz(row, D), D, banks)


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("banks", [32, 64])
def test_forward_v_transposed_reads_are_conflict_free(D, banks):
    """V rows are read transposed (the A operand of O^T += V^T P^T)."""
    swz = _fwd_swizzle("swz16_v")
    assert _transposed_reads_conflict_free(lambda row: swz(row, D), D, banks)


@pytest.mark.parametrize("name", ["swz16_k", "swz16_v"])
@pytest.mark.parametrize("D", [64, 128])
def test_forward_swizzles_permute_each_row(name, D):
    swz, cpr = _fwd_swizzle(name), D // 8
    for r in range(32):
        assert sorted(c ^ swz(r, D) for c in range(cpr)) == list(range(cpr))
