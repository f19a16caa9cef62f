"""ctypes binding of libpdhip.so (the C ABI declared in include/pdhip.h).

The library is loaded once per process. There is no fallback: a missing or
stale library raises, so nothing on the execution path can silently run
anywhere but the HIP kernels."""

from __future__ import annotations

import ctypes as C
import threading
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libpdhip.so"

PDH_OK, PDH_EINVAL, PDH_EUNSUPPORTED, PDH_ELAUNCH = 0, 1, 2, 3
PDH_F32, PDH_BF16, PDH_F16 = 0, 1, 2
DECODE_SCRATCH_BYTES = 16 << 20  # PDH_DECODE_SCRATCH_BYTES: pdh_attn_decode_noalloc's per-GPU array
PDH_MASK_NONE, PDH_MASK_BAND = 0, 1

I64_MIN = -(2**63)
I64_MAX = 2**63 - 1

# every symbol include/pdhip.h declares (checked by the CPU test suite)
EXPORTS = (
    "pdh_version",
    "pdh_last_error",
    "pdh_device_cus",
    "pdh_row_softmax",
    "pdh_layernorm",
    "pdh_row_softmax_dt",
    "pdh_layernorm_dt",
    "pdh_take_rows",
    "pdh_scatter_add_rows",
    "pdh_flash_fwd",
    "pdh_flash_fwd_workspace",
    "pdh_flash_fwd_split",
    "pdh_flash_bwd",
    "pdh_attn_decode_workspace",
    "pdh_attn_decode",
    "pdh_attn_decode_noalloc",
    "pdh_map_chain",
    "pdh_contract",
    "pdh_contract_strided",
    "pdh_contract_strided_ksplit",
    "pdh_contract_views",
    "pdh_contract_views_pro",
    "pdh_contract_views_rowred",
    "pdh_reduce_rows",
    "pdh_reduce_rows_ex",
    "pdh_scan",
    "pdh_ew_set_jit",
    "pdh_contract_set_f32_mode",
    "pdh_ew_jit_stats",
    "pdh_ew_jit_source",
    "pdh_ew_jit_compile",
    "pdh_probe_mfma",
)


class PdhError(RuntimeError):
    """A nonzero status from libpdhip, with the library's own message."""

    def __init__(self, fn: str, code: int, msg: str):
        self.fn, self.code = fn, code
        super().__init__(f"{fn} failed (status {code}): {msg}")


class AttnGeom(C.Structure):
    """pdh_attn_geom: instance / shape / element-stride description."""

    _fields_ = [
        (n, C.c_int64)
        for n in (
            "batch heads_q heads_kv t s e od "
            "q_sb q_sh q_st k_sb k_sh k_st v_sb v_sh v_st o_sb o_sh o_st"
        ).split()
    ]


# elementwise programs (pdh_ew_program): limits and opcodes, as include/pdhip.h
EW_MAX_INSNS, EW_MAX_REGS, EW_MAX_OPERANDS, EW_MAX_DIMS = 64, 16, 8, 4
EW_OPS = (
    "LOAD ACC CONST IOTA NEG EXP LOG SQRT TANH SIN COS ABS FLOOR ADD SUB MUL DIV MAX MIN "
    "EQ NE LT LE GT GE WHERE RBF16 RF16"
).split()
EW = {name: i for i, name in enumerate(EW_OPS)}


class EwInsn(C.Structure):
    _fields_ = [("op", C.c_uint8), ("dst", C.c_uint8), ("a", C.c_uint8), ("b", C.c_uint8), ("c", C.c_uint8),
                ("pad0", C.c_uint8), ("pad1", C.c_uint8), ("pad2", C.c_uint8), ("imm", C.c_float)]


class EwProgram(C.Structure):
    """pdh_ew_program: a register program over one output lattice."""

    _fields_ = [
        ("n_insns", C.c_int32), ("n_operands", C.c_int32), ("ndim", C.c_int32), ("out_reg", C.c_int32),
        ("shape", C.c_int64 * EW_MAX_DIMS), ("start", C.c_int64 * EW_MAX_DIMS),
        ("out_stride", C.c_int64 * EW_MAX_DIMS), ("in_stride", (C.c_int64 * EW_MAX_DIMS) * EW_MAX_OPERANDS),
        ("insns", EwInsn * EW_MAX_INSNS),
    ]


_lock = threading.Lock()
_lib = None


def _declare(lib) -> None:
    vp, i64, i32, f32 = C.c_void_p, C.c_int64, C.c_int, C.c_float
    fp = C.POINTER(C.c_float)
    gp = C.POINTER(AttnGeom)
    sigs = {
        "pdh_version": (i32, []),
        "pdh_last_error": (C.c_size_t, [C.c_char_p, C.c_size_t]),
        "pdh_device_cus": (i32, []),
        "pdh_row_softmax": (i32, [vp, vp, i64, i64, i64, i64, vp]),
        "pdh_layernorm": (i32, [vp, vp, vp, vp, i64, i64, i64, i64, f32, vp]),
        "pdh_row_softmax_dt": (i32, [vp, vp, i64, i64, i64, i64, i32, vp]),
        "pdh_layernorm_dt": (i32, [vp, vp, vp, vp, i64, i64, i64, i64, f32, i32, vp]),
        "pdh_take_rows": (i32, [vp, vp, vp, i64, i64, i64, i64, i64, i32, vp, vp]),
        "pdh_scatter_add_rows": (i32, [vp, vp, vp, i64, i64, i64, i64, i64, i32, vp, vp]),
        "pdh_flash_fwd": (i32, [vp, vp, vp, vp, vp, vp, vp, gp, i32, f32, f32, i32, i64, i64, i32, vp]),
        "pdh_flash_fwd_workspace": (C.c_size_t, [gp, i32]),
        "pdh_flash_fwd_split": (i32, [vp, vp, vp, vp, vp, vp, vp, gp, i32, f32, f32, i32, i64, i64, i32, i32, vp,
                                      C.c_size_t, vp]),
        "pdh_flash_bwd": (i32, [vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, gp, i32, f32, f32, i32, i64, i64, vp]),
        "pdh_attn_decode_workspace": (C.c_size_t, [gp, i32]),
        "pdh_attn_decode": (i32, [vp, vp, vp, vp, vp, gp, i32, f32, i32, vp, C.c_size_t, vp]),
        "pdh_attn_decode_noalloc": (i32, [vp, vp, vp, vp, vp, gp, i32, f32, i32, vp]),
        "pdh_map_chain": (i32, [C.POINTER(EwProgram), C.POINTER(vp), vp, i32, vp]),
        "pdh_contract": (i32, [vp, vp, i64, i64, i64, i64, i64, C.POINTER(EwProgram), C.POINTER(vp), vp, i32, vp]),
        "pdh_contract_strided": (
            i32, [vp, i64, i64, vp, i64, i64, i64, i64, i64, i64, C.POINTER(EwProgram), C.POINTER(vp), vp, i32, vp]),
        "pdh_contract_strided_ksplit": (
            i32, [vp, i64, i64, vp, i64, i64, i64, i64, i64, i64, i64, C.POINTER(EwProgram), C.POINTER(vp), vp, i32,
                  vp]),
        "pdh_contract_views": (
            i32, [vp, i64, i64, i64, vp, i64, i64, i64, i64, i64, i64, i64, i64, C.POINTER(EwProgram), C.POINTER(vp),
                  vp, i32, vp]),
        "pdh_contract_views_pro": (
            i32, [vp, i64, i64, i64, C.POINTER(EwProgram), C.POINTER(vp), vp, i64, i64, i64, C.POINTER(EwProgram),
                  C.POINTER(vp), i64, i64, i64, i64, i64, C.POINTER(EwProgram), C.POINTER(vp), vp, i32, vp]),
        "pdh_contract_views_rowred": (
            i32, [vp, i64, i64, i64, vp, i64, i64, i64, i64, i64, i64, i64, C.POINTER(EwProgram), C.POINTER(vp), i32,
                  vp, i32, vp]),
        "pdh_reduce_rows": (i32, [C.POINTER(EwProgram), i32, C.POINTER(EwProgram), C.POINTER(vp), i32, vp, i32, vp]),
        "pdh_reduce_rows_ex": (i32, [C.POINTER(EwProgram), i32, C.POINTER(EwProgram), C.POINTER(vp), i32, vp, i32, i32,
                                     vp]),
        "pdh_scan": (i32, [vp, vp, i64, i64, i64, i32, i32, i32, vp]),
        "pdh_ew_set_jit": (i32, [i32]),
        "pdh_contract_set_f32_mode": (i32, [i32]),
        "pdh_ew_jit_stats": (None, [C.POINTER(i64)]),
        "pdh_ew_jit_source": (C.c_size_t, [C.POINTER(EwProgram), i32, i32, C.c_char_p, C.c_size_t]),
        "pdh_ew_jit_compile": (i32, [C.POINTER(EwProgram), i32, i32]),
        "pdh_probe_mfma": (i32, [vp, vp, vp, vp, vp, vp, vp]),
    }
    del fp
    for name, (res, args) in sigs.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args


def lib():
    """The loaded library; raises if libpdhip.so has not been built."""
    global _lib
    if _lib is None:
        with _lock:
            if _lib is None:
                if not LIB_PATH.exists():
                    raise RuntimeError(
                        f"{LIB_PATH} is missing: build the HIP backend first "
                        "(python -m pdum_dsl_amd.build or __graft_entry__.build())"
                    )
                handle = C.CDLL(str(LIB_PATH))
                _declare(handle)
                _lib = handle
    return _lib


def last_error() -> str:
    buf = C.create_string_buffer(1024)
    lib().pdh_last_error(buf, len(buf))
    return buf.value.decode(errors="replace")


def check(fn: str, code: int) -> None:
    if code != PDH_OK:
        raise PdhError(fn, code, last_error())


def call(fn: str, *args) -> None:
    """Call a status-returning entry point; raise PdhError on failure."""
    check(fn, getattr(lib(), fn)(*args))
