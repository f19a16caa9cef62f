"""The C ABI boundary on the CPU: the built library loads and exports every
symbol include/pdhip.h declares; no compute is launched."""

import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]


def _declared():
    text = (ROOT / "include" / "pdhip.h").read_text()
    return sorted(set(re.findall(r"\b(pdh_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_binding_table():
    from pdum_dsl_amd._lib import EXPORTS

    assert _declared() == sorted(EXPORTS)


def test_library_exports_every_declared_symbol():
    from pdum_dsl_amd import _lib

    if not _lib.LIB_PATH.exists():
        pytest.fail("libpdhip.so is not built: run __graft_entry__.build() first")
    lib = _lib.lib()
    for name in _declared():
        assert hasattr(lib, name), name
    assert lib.pdh_version() == 100


def test_validation_errors_need_no_device():
    """Shape checks fire before any HIP call, so they run here without a GPU."""
    import ctypes as C

    from pdum_dsl_amd import _lib

    lib = _lib.lib()
    rc = lib.pdh_row_softmax(None, None, 4, 0, 0, 0, None)
    assert rc == _lib.PDH_EINVAL and "cols >= 1" in _lib.last_error()
    g = _lib.AttnGeom()
    g.batch, g.heads_q, g.heads_kv, g.t, g.s, g.e, g.od = 1, 3, 2, 8, 8, 64, 64
    rc = lib.pdh_flash_fwd(None, None, None, None, None, None, None, C.byref(g), 1, 1.0, -1e9, 0, 0, 0, 1, None)
    assert rc == _lib.PDH_EINVAL and "multiple of heads_kv" in _lib.last_error()
    assert lib.pdh_attn_decode_workspace(C.byref(g), 4) == 1 * 3 * 8 * 4 * (2 + 64) * 4
    # the key-split forward: its workspace, and an nsplit out of range refused before anything runs
    assert lib.pdh_flash_fwd_workspace(C.byref(g), 5) == 5 * (1 * 3 * 8) * (64 + 3) * 4
    assert lib.pdh_flash_fwd_workspace(C.byref(g), 1) == 0
    rc = lib.pdh_flash_fwd_split(None, None, None, None, None, None, None, C.byref(g), 1, 1.0, -1e9, 0, 0, 0, 1, 65,
                                 None, 0, None)
    assert rc == _lib.PDH_EINVAL and "nsplit 65" in _lib.last_error()
    # the row reduction's reducer code
    p = _lib.EwProgram()
    rc = lib.pdh_reduce_rows_ex(C.byref(p), 1, C.byref(p), None, 0, None, 0, 3, None)
    assert rc == _lib.PDH_EINVAL and "reducer 3" in _lib.last_error()
    # in-place contraction views: fp32 only, one unit stride per operand, no empty k slice
    fake = C.c_void_p(256)  # never dereferenced: every call below is refused first

    def views(sa, sb, k=1000, ksplit=1, dt=_lib.PDH_F32):
        return lib.pdh_contract_views(fake, *sa, fake, *sb, 1, 100, 100, k, ksplit, C.byref(p), None, fake, dt, None)

    assert views((0, 1000, 1), (0, 1000, 1), dt=_lib.PDH_BF16) == _lib.PDH_EUNSUPPORTED
    assert views((0, 1000, 2), (0, 1000, 1)) == _lib.PDH_EINVAL and "contiguous" in _lib.last_error()
    assert views((0, 1, 100), (0, 1000, 1), ksplit=5) == _lib.PDH_EINVAL and "slice empty" in _lib.last_error()
    assert views((0, 1, 100), (0, -1, 1)) == _lib.PDH_EINVAL and "negative" in _lib.last_error()


def test_the_forward_split_picker():
    """Key splits only for grids that cannot fill the chip: gpt2's 12 heads x
    1024 rows take 4 runs of 8 key tiles; the C3 headline (8192 query blocks)
    and short rows take none."""
    pytest.importorskip("torch")
    from pdum_dsl_amd.kernels import pick_fwd_splits

    assert pick_fwd_splits(12, 1024, 1024, cus=256) == 4
    assert pick_fwd_splits(8 * 32, 4096, 4096, cus=256) == 1
    assert pick_fwd_splits(1, 4096, 4096, cus=256) == 16
    assert pick_fwd_splits(4, 256, 256, cus=256) == 1  # 8 key tiles a row
    assert pick_fwd_splits(0, 0, 1, cus=256) == 1
