"""Device-resident entry points: torch tensors in, torch tensors out, every
call a launch of the HIP kernels behind libpdhip's C ABI on the current
stream (no host copies, no synchronization).

Torch is plumbing here — device memory and streams. Shapes follow the
reference's dims: attention tensors are [batch, heads, rows, features]
(the reference template's 2-D q:(t,e), k:(s,e), v:(s,o) per instance,
fusion.py:517-523, with batch and head as independent instances)."""

from __future__ import annotations

import ctypes as C
import math
from dataclasses import dataclass

import torch

from . import _lib
from ._lib import (
    I64_MAX,
    I64_MIN,
    PDH_BF16,
    PDH_F16,
    PDH_F32,
    PDH_MASK_BAND,
    PDH_MASK_NONE,
    AttnGeom,
)

_DT = {torch.float32: PDH_F32, torch.bfloat16: PDH_BF16, torch.float16: PDH_F16}


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def _ptr(t: torch.Tensor | None):
    return None if t is None else C.c_void_p(t.data_ptr())


def _require_cuda(*ts: torch.Tensor) -> None:
    for t in ts:
        if t is not None and not t.is_cuda:
            raise ValueError("HIP kernels take device tensors (got a CPU tensor)")


@dataclass(frozen=True)
class Band:
    """Score mask: key s is live for query row t iff lo <= s - t <= hi.
    ``None`` ends are unbounded. Causal le(iota_s, iota_t) is Band(None, 0)."""

    lo: int | None = None
    hi: int | None = None

    def c_args(self):
        return (
            I64_MIN if self.lo is None else int(self.lo),
            I64_MAX if self.hi is None else int(self.hi),
        )


CAUSAL = Band(None, 0)


# ---------------------------------------------------------------------- rows


def row_softmax(x: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """softmax over the last axis (rows = all leading dims); fp32, bf16 or
    f16 storage, fp32 arithmetic."""
    _require_cuda(x)
    if x.dtype not in _DT:
        raise ValueError(f"row_softmax stores f32, bf16 or f16 (got {x.dtype})")
    x2 = x.reshape(-1, x.shape[-1])
    if x2.stride(-1) != 1:
        x2 = x2.contiguous()
    y = torch.empty_like(x2) if out is None else out.reshape(-1, x.shape[-1])
    if y.dtype != x.dtype or y.stride(-1) != 1:
        raise ValueError("out must share x's element type and have contiguous rows")
    if x.dtype == torch.float32:
        _lib.call(
            "pdh_row_softmax",
            _ptr(x2), _ptr(y), x2.shape[0], x2.shape[1], x2.stride(0), y.stride(0), C.c_void_p(_stream()),
        )
    else:
        _lib.call(
            "pdh_row_softmax_dt",
            _ptr(x2), _ptr(y), x2.shape[0], x2.shape[1], x2.stride(0), y.stride(0), _DT[x.dtype],
            C.c_void_p(_stream()),
        )
    return y.reshape(x.shape)


def layernorm(
    x: torch.Tensor,
    gamma: torch.Tensor | None = None,
    beta: torch.Tensor | None = None,
    eps: float = 1e-5,
    out: torch.Tensor | None = None,
) -> torch.Tensor:
    """Two-pass layernorm over the last axis, optional affine epilogue; fp32,
    bf16 or f16 storage (x, gamma, beta alike), fp32 arithmetic."""
    _require_cuda(x, gamma, beta)
    if x.dtype not in _DT:
        raise ValueError(f"layernorm stores f32, bf16 or f16 (got {x.dtype})")
    for t in (gamma, beta):
        if t is not None and t.dtype != x.dtype:
            raise ValueError("gamma / beta must share x's element type")
    n = x.shape[-1]
    for nm, t in (("gamma", gamma), ("beta", beta)):
        if t is not None and (t.numel() != n or not t.is_contiguous()):
            raise ValueError(f"{nm} must be a contiguous vector of {n} elements")
    x2 = x.reshape(-1, n)
    if x2.stride(-1) != 1:
        x2 = x2.contiguous()
    y = torch.empty_like(x2) if out is None else out.reshape(-1, n)
    if y.dtype != x.dtype or y.stride(-1) != 1:
        raise ValueError("out must share x's element type and have contiguous rows")
    if x.dtype == torch.float32:
        _lib.call(
            "pdh_layernorm",
            _ptr(x2), _ptr(gamma), _ptr(beta), _ptr(y), x2.shape[0], n, x2.stride(0), y.stride(0),
            C.c_float(eps), C.c_void_p(_stream()),
        )
    else:
        _lib.call(
            "pdh_layernorm_dt",
            _ptr(x2), _ptr(gamma), _ptr(beta), _ptr(y), x2.shape[0], n, x2.stride(0), y.stride(0),
            C.c_float(eps), _DT[x.dtype], C.c_void_p(_stream()),
        )
    return y.reshape(x.shape)


def take_rows(table: torch.Tensor, idx: torch.Tensor, out: torch.Tensor | None = None,
              bad: torch.Tensor | None = None) -> torch.Tensor:
    """out[i, ...] = table[idx[i], ...]: a gather along the table's leading
    dim (idx int64, any shape; the rest of the table's dims ride). An index
    out of range gives a zero row and counts in ``bad`` (an int32 device
    scalar) when given."""
    _require_cuda(table, idx)
    if table.dtype not in _DT or idx.dtype != torch.int64:
        raise ValueError("take_rows: table f32/bf16/f16, idx int64")
    rows = table.reshape(table.shape[0], -1)
    if rows.stride(-1) != 1:
        raise ValueError("take_rows: the table's trailing dims must be contiguous")
    flat = idx.reshape(-1).contiguous()
    y = torch.empty((flat.numel(), rows.shape[1]), dtype=table.dtype, device=table.device) if out is None else \
        out.reshape(flat.numel(), rows.shape[1])
    if y.dtype != table.dtype or y.stride(-1) != 1:
        raise ValueError("take_rows: out must share the table's element type with contiguous rows")
    if bad is not None and (bad.dtype != torch.int32 or bad.numel() < 1):
        raise ValueError("take_rows: bad is an int32 device scalar")
    _lib.call(
        "pdh_take_rows",
        _ptr(rows), _ptr(flat), _ptr(y), flat.numel(), rows.shape[1], rows.shape[0], rows.stride(0), y.stride(0),
        _DT[table.dtype], _ptr(bad), C.c_void_p(_stream()),
    )
    return y.reshape(tuple(idx.shape) + tuple(table.shape[1:]))


SCATTER_MAX_IDX = 1 << 16  # positions pdh_scatter_add_rows takes per launch


def scatter_add_rows(values: torch.Tensor, idx: torch.Tensor, n_rows: int, out: torch.Tensor | None = None,
                     bad: torch.Tensor | None = None) -> torch.Tensor:
    """out[v, ...] = sum of values[i, ...] over the positions i with
    idx[i] == v: the gather's adjoint along out's leading dim (values has
    idx's shape followed by the row dims; rows nothing lands in are zero).
    Deterministic (increasing i, fp32 sums, one rounding). An index out of
    range is dropped and counts in ``bad`` (an int32 device scalar) when
    given. At most ``SCATTER_MAX_IDX`` positions (the kernel's owner scan is
    quadratic in them); more raise ``PdhError``."""
    _require_cuda(values, idx)
    if values.dtype not in _DT or idx.dtype != torch.int64:
        raise ValueError("scatter_add_rows: values f32/bf16/f16, idx int64")
    if tuple(values.shape[:idx.dim()]) != tuple(idx.shape):
        raise ValueError(f"scatter_add_rows: values {tuple(values.shape)} do not lead with idx's shape {tuple(idx.shape)}")
    rest = tuple(values.shape[idx.dim():])
    n = idx.numel()
    rows = values.reshape(n, -1) if n else values.new_empty((0, math.prod(rest)))
    if rows.shape[1] < 1:
        raise ValueError("scatter_add_rows: empty rows")
    if n and rows.stride(-1) != 1:
        raise ValueError("scatter_add_rows: the values' row dims must be contiguous")
    y = torch.empty((n_rows, rows.shape[1]), dtype=values.dtype, device=values.device) if out is None else \
        out.reshape(n_rows, rows.shape[1])
    if y.dtype != values.dtype or y.stride(-1) != 1:
        raise ValueError("scatter_add_rows: out must share the values' element type with contiguous rows")
    if bad is not None and (bad.dtype != torch.int32 or bad.numel() < 1):
        raise ValueError("scatter_add_rows: bad is an int32 device scalar")
    flat = idx.reshape(-1).contiguous()
    _lib.call(
        "pdh_scatter_add_rows",
        _ptr(rows), _ptr(flat), _ptr(y), n, rows.shape[1], n_rows, max(rows.stride(0), rows.shape[1]), y.stride(0),
        _DT[values.dtype], _ptr(bad), C.c_void_p(_stream()),
    )
    return y.reshape((n_rows,) + rest)


# ----------------------------------------------------------------- attention


def _geom(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, o: torch.Tensor) -> AttnGeom:
    for nm, t in (("q", q), ("k", k), ("v", v), ("o", o)):
        if t.dim() != 4:
            raise ValueError(f"{nm} must be [batch, heads, rows, features] (got shape {tuple(t.shape)})")
        if t.stride(-1) != 1:
            raise ValueError(f"{nm}'s feature axis must be contiguous")
    B, Hq, T, E = q.shape
    Bk, Hkv, S, Ek = k.shape
    if (Bk, Ek) != (B, E) or v.shape[:3] != k.shape[:3] or o.shape[:3] != q.shape[:3] or o.shape[3] != v.shape[3]:
        raise ValueError(
            f"shape mismatch: q {tuple(q.shape)} k {tuple(k.shape)} v {tuple(v.shape)} o {tuple(o.shape)}"
        )
    if Hq % Hkv:
        raise ValueError(f"query heads ({Hq}) must be a multiple of key/value heads ({Hkv})")
    g = AttnGeom()
    g.batch, g.heads_q, g.heads_kv, g.t, g.s, g.e, g.od = B, Hq, Hkv, T, S, E, v.shape[3]
    g.q_sb, g.q_sh, g.q_st = q.stride(0), q.stride(1), q.stride(2)
    g.k_sb, g.k_sh, g.k_st = k.stride(0), k.stride(1), k.stride(2)
    g.v_sb, g.v_sh, g.v_st = v.stride(0), v.stride(1), v.stride(2)
    g.o_sb, g.o_sh, g.o_st = o.stride(0), o.stride(1), o.stride(2)
    return g


@dataclass
class FlashOut:
    o: torch.Tensor
    lse: torch.Tensor | None
    m: torch.Tensor | None
    den: torch.Tensor | None


def flash_fwd(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    *,
    scale: float | None = None,
    band: Band | None = None,
    fill: float = -1e9,
    prune: bool = True,
    want_lse: bool = True,
    want_artifacts: bool = False,
    out: torch.Tensor | None = None,
    nsplit: int | None = None,
) -> FlashOut:
    """Flash-attention forward over [B, H, T, E] q and [B, Hkv, S, E] k / v.

    ``band`` None means every key is live; masked scores take ``fill``.
    Returns the output plus lse and, with ``want_artifacts``, the reference's
    (m, den) artifacts ([B, H, T] fp32). ``nsplit`` > 1 splits each query
    block's keys over that many workgroups (pdh_flash_fwd_split); None picks
    it (``pick_fwd_splits``): 1 unless the grid is too small to fill the chip."""
    _require_cuda(q, k, v)
    if not (q.dtype == k.dtype == v.dtype) or q.dtype not in _DT:
        raise ValueError(f"q/k/v must share one dtype of f32/bf16/f16 (got {q.dtype}, {k.dtype}, {v.dtype})")
    B, H, T, _ = q.shape
    o = torch.empty(q.shape[:3] + (v.shape[3],), dtype=q.dtype, device=q.device) if out is None else out
    g = _geom(q, k, v, o)
    st = dict(dtype=torch.float32, device=q.device)
    lse = torch.empty((B, H, T), **st) if want_lse else None
    m = torch.empty((B, H, T), **st) if want_artifacts else None
    den = torch.empty((B, H, T), **st) if want_artifacts else None
    sc = 1.0 / math.sqrt(q.shape[3]) if scale is None else float(scale)
    kind, (lo, hi) = (PDH_MASK_NONE, (0, 0)) if band is None else (PDH_MASK_BAND, band.c_args())
    if nsplit is None:
        nsplit = pick_fwd_splits(B * H, T, k.shape[2]) if q.dtype != torch.float32 else 1
    if nsplit > 1 and q.dtype != torch.float32:
        need = _lib.lib().pdh_flash_fwd_workspace(C.byref(g), int(nsplit))
        ws = torch.empty((need + 3) // 4, dtype=torch.float32, device=q.device)
        _lib.call(
            "pdh_flash_fwd_split",
            _ptr(q), _ptr(k), _ptr(v), _ptr(o), _ptr(m), _ptr(den), _ptr(lse), C.byref(g), _DT[q.dtype],
            C.c_float(sc), C.c_float(fill), kind, lo, hi, int(bool(prune)), int(nsplit), _ptr(ws),
            C.c_size_t(ws.numel() * 4), C.c_void_p(_stream()),
        )
        return FlashOut(o, lse, m, den)
    _lib.call(
        "pdh_flash_fwd",
        _ptr(q), _ptr(k), _ptr(v), _ptr(o), _ptr(m), _ptr(den), _ptr(lse), C.byref(g), _DT[q.dtype],
        C.c_float(sc), C.c_float(fill), kind, lo, hi, int(bool(prune)), C.c_void_p(_stream()),
    )
    return FlashOut(o, lse, m, den)


def flash_fwd_prepared(q, k, v, *, scale: float | None = None, band: Band | None = None, fill: float = -1e9,
                       prune: bool = True, out: torch.Tensor | None = None, lse: torch.Tensor | None = None):
    """``flash_fwd`` (one workgroup sweep per query block, no key split, no
    artifacts) with its geometry, pointers and stream bound once: returns a
    function of no arguments that launches the kernel into ``out`` (and
    ``lse``) on the stream current now. For loops that call the same shapes
    many times (serving, small heads), where the per-call wrapper's host work
    outweighs the launch. The tensors must stay alive and in place."""
    _require_cuda(q, k, v)
    if not (q.dtype == k.dtype == v.dtype) or q.dtype not in _DT:
        raise ValueError(f"q/k/v must share one dtype of f32/bf16/f16 (got {q.dtype}, {k.dtype}, {v.dtype})")
    B, H, T, _ = q.shape
    o = torch.empty(q.shape[:3] + (v.shape[3],), dtype=q.dtype, device=q.device) if out is None else out
    g = _geom(q, k, v, o)
    if lse is None:
        lse = torch.empty((B, H, T), dtype=torch.float32, device=q.device)
    elif lse.shape != (B, H, T) or lse.dtype != torch.float32 or not lse.is_contiguous():
        raise ValueError("lse must be a contiguous fp32 [batch, heads, rows] tensor")
    sc = 1.0 / math.sqrt(q.shape[3]) if scale is None else float(scale)
    kind, (lo, hi) = (PDH_MASK_NONE, (0, 0)) if band is None else (PDH_MASK_BAND, band.c_args())
    _lib.lib()  # loaded and declared (raises if the library is missing)
    # the same symbol through a handle without argtypes: the arguments are built
    # once as their exact C types, so a call does no per-argument conversion
    fn = getattr(C.CDLL(str(_lib.LIB_PATH)), "pdh_flash_fwd")
    fn.restype = C.c_int
    i64, i32 = C.c_int64, C.c_int
    args = (_ptr(q), _ptr(k), _ptr(v), _ptr(o), C.c_void_p(None), C.c_void_p(None), _ptr(lse), C.byref(g),
            i32(_DT[q.dtype]), C.c_float(sc), C.c_float(fill), i32(kind), i64(lo), i64(hi), i32(int(bool(prune))),
            C.c_void_p(_stream()))
    keep = (q, k, v, o, lse, g)  # the bound pointers' owners live as long as the call

    def call():
        rc = fn(*args)
        if rc:
            _lib.check("pdh_flash_fwd", rc)
        return keep[3]

    call.o, call.lse = o, lse
    return call


def pick_fwd_splits(ninst: int, t: int, s: int, cus: int | None = None) -> int:
    """Key splits for the 16-bit forward: 1 when the instances x 128-row query
    blocks give every CU two workgroups, or a row has under 16 key tiles
    (512 keys); otherwise runs of at least 8 key tiles (256 keys), up to
    three workgroups per CU in all."""
    if cus is None:
        cus = _lib.lib().pdh_device_cus() or 256
    blocks = ninst * ((t + 127) // 128)
    ntiles = (s + 31) // 32
    if blocks == 0 or blocks >= 2 * cus or ntiles < 16:
        return 1
    return int(max(1, min(ntiles // 8, (3 * cus) // blocks, 64)))


def flash_bwd(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    o: torch.Tensor,
    do: torch.Tensor,
    lse: torch.Tensor,
    *,
    m: torch.Tensor | None = None,
    den: torch.Tensor | None = None,
    scale: float | None = None,
    band: Band | None = None,
    fill: float = -1e9,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Gradients (dq, dk, dv) of flash attention given the forward's lse
    (and optionally its (m, den) artifacts, exact for fully-masked rows)."""
    _require_cuda(q, k, v, o, do, lse, m, den)
    if do.shape != o.shape or do.stride() != o.stride():
        raise ValueError("dO must match O's shape and strides")
    g = _geom(q, k, v, o)
    dq = torch.empty_like(q)
    dk = torch.empty_like(k)
    dv = torch.empty_like(v)
    if dq.stride() != q.stride() or dk.stride() != k.stride() or dv.stride() != v.stride():
        raise ValueError("q/k/v must be dense (their gradients share their strides)")
    for nm, t in (("lse", lse), ("m", m), ("den", den)):
        if t is not None and (t.dtype != torch.float32 or not t.is_contiguous() or t.shape != q.shape[:3]):
            raise ValueError(f"{nm} must be contiguous fp32 [batch, heads, rows]")
    if (m is None) != (den is None):
        raise ValueError("pass both m and den, or neither")
    ws = torch.empty((3,) + tuple(q.shape[:3]), dtype=torch.float32, device=q.device)
    sc = 1.0 / math.sqrt(q.shape[3]) if scale is None else float(scale)
    kind, (lo, hi) = (PDH_MASK_NONE, (0, 0)) if band is None else (PDH_MASK_BAND, band.c_args())
    _lib.call(
        "pdh_flash_bwd",
        _ptr(q), _ptr(k), _ptr(v), _ptr(o), _ptr(do), _ptr(lse), _ptr(m), _ptr(den), _ptr(dq), _ptr(dk), _ptr(dv),
        _ptr(ws), C.byref(g), _DT[q.dtype], C.c_float(sc), C.c_float(fill), kind, lo, hi, C.c_void_p(_stream()),
    )
    return dq, dk, dv


def attn_decode(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    *,
    scale: float | None = None,
    nsplit: int | None = None,
    want_lse: bool = True,
    workspace: torch.Tensor | None = None,
) -> tuple[torch.Tensor, torch.Tensor | None]:
    """Split-K decode attention: q [B, Hq, t, D] (small t) against the cache
    k / v [B, Hkv, S, D]; every cache row is live."""
    _require_cuda(q, k, v)
    B, Hq, T, D = q.shape
    o = torch.empty((B, Hq, T, v.shape[3]), dtype=q.dtype, device=q.device)
    g = _geom(q, k, v, o)
    if nsplit is None:
        nsplit = pick_decode_splits(B * k.shape[1], k.shape[2])
    need = _lib.lib().pdh_attn_decode_workspace(C.byref(g), int(nsplit))
    if workspace is None or workspace.numel() * workspace.element_size() < need:
        workspace = torch.empty((max(need, 16) + 3) // 4, dtype=torch.float32, device=q.device)
    lse = torch.empty((B, Hq, T), dtype=torch.float32, device=q.device) if want_lse else None
    sc = 1.0 / math.sqrt(D) if scale is None else float(scale)
    _lib.call(
        "pdh_attn_decode",
        _ptr(q), _ptr(k), _ptr(v), _ptr(o), _ptr(lse), C.byref(g), _DT[q.dtype], C.c_float(sc), int(nsplit),
        _ptr(workspace), C.c_size_t(workspace.numel() * workspace.element_size()), C.c_void_p(_stream()),
    )
    return o, lse


def attn_decode_static(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    o: torch.Tensor,
    lse: torch.Tensor | None,
    *,
    nsplit: int,
    scale: float | None = None,
) -> None:
    """attn_decode into caller-provided o / lse with the split partials in the
    library's per-GPU scratch array (pdh_attn_decode_noalloc): nothing is
    allocated, so the call can be captured in a HIP graph. Calls that overlap
    on one GPU share that array and race."""
    _require_cuda(q, k, v, o, lse)
    g = _geom(q, k, v, o)
    if lse is not None and (lse.dtype != torch.float32 or not lse.is_contiguous() or lse.shape != q.shape[:3]):
        raise ValueError("lse must be contiguous fp32 [batch, heads_q, t]")
    sc = 1.0 / math.sqrt(q.shape[3]) if scale is None else float(scale)
    _lib.call(
        "pdh_attn_decode_noalloc",
        _ptr(q), _ptr(k), _ptr(v), _ptr(o), _ptr(lse), C.byref(g), _DT[q.dtype], C.c_float(sc), int(nsplit),
        C.c_void_p(_stream()),
    )


# ------------------------------------------------- elementwise programs


def _max_offset(prog, strides, ndim) -> int:
    return sum((int(prog.shape[d]) - 1) * int(strides[d]) for d in range(ndim))


def _check_views(prog, operands, out, ndim):
    """Every view the program reads or writes stays inside its tensor."""
    if len(operands) != prog.n_operands:
        raise ValueError(f"program reads {prog.n_operands} operands, {len(operands)} given")
    dt = out.dtype
    for i, t in enumerate(operands):
        if t.dtype != dt:
            raise ValueError(f"operand {i} is {t.dtype}, the output {dt}: one element type per call")
        if _max_offset(prog, prog.in_stride[i], ndim) >= t.numel() or t.storage_offset() < 0:
            raise ValueError(f"operand {i}: the program's view reaches past the tensor")
    if _max_offset(prog, prog.out_stride, ndim) >= out.numel():
        raise ValueError("the program's output view reaches past the output tensor")


def map_chain(prog: _lib.EwProgram, operands: list, out: torch.Tensor) -> torch.Tensor:
    """Run an elementwise program (ewprog.lower) over its output lattice:
    operands and ``out`` share one element type; strides come from the program."""
    _require_cuda(out, *operands)
    if out.dtype not in _DT:
        raise ValueError(f"element type {out.dtype} (f32, bf16, f16)")
    _check_views(prog, operands, out, prog.ndim)
    table = (C.c_void_p * max(1, len(operands)))(*[t.data_ptr() for t in operands])
    _lib.call("pdh_map_chain", C.byref(prog), table, _ptr(out), _DT[out.dtype], C.c_void_p(_stream()))
    return out


# How fp32 contractions run (pdh_contract_set_f32_mode): bf16 matrix-core
# products of split operands (6: fp32 grade, 3, or 1: bf16-rounded operands
# with fp32 accumulation, an autocast's numerics), or fp32 VALU fma.
F32_CONTRACT = {"bf16x6": 6, "bf16x3": 3, "bf16": 1, "fma": 0}


def set_f32_contract(mode: str) -> str:
    """Set how fp32 contractions run, process-wide; returns the previous mode."""
    if mode not in F32_CONTRACT:
        raise ValueError(f"f32 contraction mode {mode!r}: one of {sorted(F32_CONTRACT)}")
    prev = _lib.lib().pdh_contract_set_f32_mode(F32_CONTRACT[mode])
    return next(k for k, v in F32_CONTRACT.items() if v == prev)


def _with_f32_mode(mode, dtype, launch):
    if mode is None or dtype != torch.float32:
        return launch()
    prev = set_f32_contract(mode)
    try:
        return launch()
    finally:
        set_f32_contract(prev)


def contract(a: torch.Tensor, bt: torch.Tensor, k: int, epi: _lib.EwProgram, operands: list,
             out: torch.Tensor, f32_mode: str | None = None) -> torch.Tensor:
    """acc[b, m, n] = sum_k a[b, m, k] bt[b, n, k]; out = epi(acc, operands).
    a: [batch, m, kp], bt: [batch, n, kp] contiguous, kp % 64 == 0, columns
    k..kp-1 zero. The epilogue program's lattice is (batch, m, n).
    ``f32_mode`` (fp32 operands only) picks F32_CONTRACT's mode for this call."""
    _require_cuda(a, bt, out, *operands)
    if a.dim() != 3 or bt.dim() != 3 or not a.is_contiguous() or not bt.is_contiguous():
        raise ValueError("a and bt must be contiguous [batch, rows, kp]")
    B, M, KP = a.shape
    if bt.shape[0] != B or bt.shape[2] != KP or a.dtype != bt.dtype or out.dtype != a.dtype:
        raise ValueError("a / bt / out shapes or dtypes disagree")
    N = bt.shape[1]
    if tuple(epi.shape[d] for d in range(3)) != (B, M, N) or epi.ndim != 3:
        raise ValueError("the epilogue's lattice must be (batch, m, n)")
    _check_views(epi, operands, out, 3)
    table = (C.c_void_p * max(1, len(operands)))(*[t.data_ptr() for t in operands])
    _with_f32_mode(f32_mode, a.dtype, lambda: _lib.call(
        "pdh_contract", _ptr(a), _ptr(bt), B, M, N, int(k), KP, C.byref(epi), table, _ptr(out), _DT[a.dtype],
        C.c_void_p(_stream()),
    ))
    return out


def contract_strided(a: torch.Tensor, a_strides, bt: torch.Tensor, bt_strides, shape, epi: _lib.EwProgram,
                     operands: list, out: torch.Tensor, f32_mode: str | None = None, ksplit: int = 1) -> torch.Tensor:
    """acc[b, m, n] = sum_k a[b, m, k] bt[b, n, k] with a and bt read through
    (batch, row) element strides from their tensors' first elements; k is
    contiguous and a multiple of 64. ``shape`` = (batch, m, n, k). With
    ``ksplit`` > 1 each batch entry's k runs in that many slices and the
    epilogue's lattice is (batch * ksplit, m, n): index e * ksplit + s holds
    entry e's products over the s-th slice (pdh_contract_strided_ksplit)."""
    _require_cuda(a, bt, out, *operands)
    B, M, N, Kd = (int(x) for x in shape)
    if a.dtype != bt.dtype or a.dtype not in _DT or out.dtype != a.dtype:
        raise ValueError("a / bt / out element types disagree")
    for t, (sb, sr), rows in ((a, a_strides, M), (bt, bt_strides, N)):
        reach = t.storage_offset() + (B - 1) * sb + (rows - 1) * sr + Kd
        if reach > t.untyped_storage().nbytes() // t.element_size():
            raise ValueError("a strided operand's view reaches past its storage")
    if tuple(epi.shape[d] for d in range(3)) != (B * ksplit, M, N) or epi.ndim != 3:
        raise ValueError("the epilogue's lattice must be (batch * ksplit, m, n)")
    _check_views(epi, operands, out, 3)
    table = (C.c_void_p * max(1, len(operands)))(*[t.data_ptr() for t in operands])
    if ksplit == 1:
        call = lambda: _lib.call(  # noqa: E731
            "pdh_contract_strided", _ptr(a), int(a_strides[0]), int(a_strides[1]), _ptr(bt), int(bt_strides[0]),
            int(bt_strides[1]), B, M, N, Kd, C.byref(epi), table, _ptr(out), _DT[a.dtype], C.c_void_p(_stream()))
    else:
        call = lambda: _lib.call(  # noqa: E731
            "pdh_contract_strided_ksplit", _ptr(a), int(a_strides[0]), int(a_strides[1]), _ptr(bt),
            int(bt_strides[0]), int(bt_strides[1]), B, M, N, Kd, int(ksplit), C.byref(epi), table, _ptr(out),
            _DT[a.dtype], C.c_void_p(_stream()))
    _with_f32_mode(f32_mode, a.dtype, call)
    return out


def contract_views(a: torch.Tensor, a_strides, bt: torch.Tensor, bt_strides, shape, epi: _lib.EwProgram,
                   operands: list, out: torch.Tensor, f32_mode: str | None = None, ksplit: int = 1) -> torch.Tensor:
    """The fp32 contraction over operands read in place (pdh_contract_views):
    acc[b, m, n] = sum_k a[b, m, k] bt[b, n, k], a[b, m, k] at element
    b sa_b + m sa_r + k sa_k of ``a`` (``a_strides`` = (sa_b, sa_r, sa_k)),
    each operand with k or its rows contiguous; k (``shape`` = (batch, m, n,
    k)) is any size. With ``ksplit`` > 1 the epilogue's lattice is
    (batch * ksplit, m, n), as for :func:`contract_strided`."""
    _require_cuda(a, bt, out, *operands)
    B, M, N, Kd = (int(x) for x in shape)
    if a.dtype != torch.float32 or bt.dtype != torch.float32 or out.dtype != torch.float32:
        raise ValueError("contract_views takes fp32 a / bt / out")
    for t, (sb, sr, sk), rows in ((a, a_strides, M), (bt, bt_strides, N)):
        if min(sb, sr, sk) < 0 or (sk != 1 and sr != 1):
            raise ValueError("each operand needs k or its rows contiguous, with non-negative strides")
        reach = t.storage_offset() + (B - 1) * sb + (rows - 1) * sr + (Kd - 1) * sk + 1
        if reach > t.untyped_storage().nbytes() // t.element_size():
            raise ValueError("a strided operand's view reaches past its storage")
    if tuple(epi.shape[d] for d in range(3)) != (B * ksplit, M, N) or epi.ndim != 3:
        raise ValueError("the epilogue's lattice must be (batch * ksplit, m, n)")
    _check_views(epi, operands, out, 3)
    table = (C.c_void_p * max(1, len(operands)))(*[t.data_ptr() for t in operands])
    sa, sb_ = [int(x) for x in a_strides], [int(x) for x in bt_strides]
    _with_f32_mode(f32_mode, a.dtype, lambda: _lib.call(
        "pdh_contract_views", _ptr(a), *sa, _ptr(bt), *sb_, B, M, N, Kd, int(ksplit), C.byref(epi), table,
        _ptr(out), _DT[a.dtype], C.c_void_p(_stream())))
    return out


def contract_views_pro(a, a_strides, bt, bt_strides, shape, epi: _lib.EwProgram, operands: list,
                       out: torch.Tensor, pro_a=None, pro_b=None, f32_mode: str | None = None,
                       ksplit: int = 1) -> torch.Tensor:
    """:func:`contract_views` with either operand computed in the k loop
    (pdh_contract_views_pro): ``pro_a`` = (program, operands), the program over
    the lattice (batch, m, k) whose value at (b, r, kk) is a[b, r, kk] (``a`` /
    ``a_strides`` are then unused and may be None); ``pro_b`` likewise over
    (batch, n, k) for bt. fp32, or bf16 with both operands computed (a stored
    one as :func:`view_program`)."""
    B, M, N, Kd = (int(x) for x in shape)
    if pro_a is None and pro_b is None:
        raise ValueError("contract_views_pro needs a prologue (contract_views reads both operands)")
    _require_cuda(out, *operands, *[t for t in (a, bt) if t is not None],
                  *[t for pr in (pro_a, pro_b) if pr is not None for t in pr[1]])
    dt = out.dtype
    if dt not in (torch.float32, torch.bfloat16):
        raise ValueError("contract_views_pro takes fp32 or bf16")
    if dt != torch.float32 and (pro_a is None or pro_b is None):
        raise ValueError("bf16 contract_views_pro computes both operands (a stored one as view_program)")
    tables, progs, reads = [], [], []
    for t, st, pr, rows, nm in ((a, a_strides, pro_a, M, "a"), (bt, bt_strides, pro_b, N, "bt")):
        if pr is None:
            if t is None or t.dtype != torch.float32:
                raise ValueError(f"{nm} must be an fp32 tensor when it has no prologue")
            sb, sr, sk = (int(x) for x in st)
            if min(sb, sr, sk) < 0 or (sk != 1 and sr != 1):
                raise ValueError("each operand needs k or its rows contiguous, with non-negative strides")
            reach = t.storage_offset() + (B - 1) * sb + (rows - 1) * sr + (Kd - 1) * sk + 1
            if reach > t.untyped_storage().nbytes() // t.element_size():
                raise ValueError("a strided operand's view reaches past its storage")
            tables.append(None)
            progs.append(None)
            reads.append((_ptr(t), sb, sr, sk))
            continue
        prog, ops = pr
        if prog.ndim != 3 or tuple(int(prog.shape[d]) for d in range(3)) != (B, rows, Kd):
            raise ValueError(f"the {nm} prologue's lattice must be (batch, {'m' if nm == 'a' else 'n'}, k)")
        if len(ops) != prog.n_operands:
            raise ValueError(f"the {nm} prologue reads {prog.n_operands} operands, {len(ops)} given")
        for i, o in enumerate(ops):
            if o.dtype != dt:
                raise ValueError(f"{nm} prologue operand {i} is {o.dtype}, the output {dt}: one element type")
            if _max_offset(prog, prog.in_stride[i], 3) >= o.numel() or o.storage_offset() < 0:
                raise ValueError(f"{nm} prologue operand {i}: the program's view reaches past the tensor")
        tables.append((C.c_void_p * max(1, len(ops)))(*[o.data_ptr() for o in ops]))
        progs.append(C.byref(prog))
        reads.append((C.c_void_p(0), 0, 0, 1))
    if tuple(epi.shape[d] for d in range(3)) != (B * ksplit, M, N) or epi.ndim != 3:
        raise ValueError("the epilogue's lattice must be (batch * ksplit, m, n)")
    _check_views(epi, operands, out, 3)
    table = (C.c_void_p * max(1, len(operands)))(*[t.data_ptr() for t in operands])
    null_prog = C.POINTER(_lib.EwProgram)()
    (pa, sab, sar, sak), (pb, sbb, sbr, sbk) = reads
    _with_f32_mode(f32_mode, dt, lambda: _lib.call(
        "pdh_contract_views_pro", pa, sab, sar, sak, progs[0] if progs[0] is not None else null_prog,
        tables[0], pb, sbb, sbr, sbk, progs[1] if progs[1] is not None else null_prog, tables[1],
        B, M, N, Kd, int(ksplit), C.byref(epi), table, _ptr(out), _DT[dt], C.c_void_p(_stream())))
    return out


def view_program(shape3, strides) -> _lib.EwProgram:
    """A one-LOAD prologue: operand 0 read through ``strides`` over the
    lattice ``shape3`` = (batch, rows, k) (a stored operand of
    :func:`contract_views_pro`)."""
    p = _lib.EwProgram()
    p.n_insns, p.n_operands, p.ndim, p.out_reg = 1, 1, 3, 0
    acc = 1
    for d in (2, 1, 0):
        p.shape[d] = int(shape3[d])
        p.out_stride[d] = acc
        p.in_stride[0][d] = int(strides[d])
        acc *= int(shape3[d])
    p.insns[0].op = _lib.EW["LOAD"]
    return p


_REDUCERS = {"sum": 0, "max": 1, "min": 2}


def contract_views_rowred(a: torch.Tensor, a_strides, bt: torch.Tensor, bt_strides, shape, epi: _lib.EwProgram,
                          operands: list, reducer: str, partials: torch.Tensor,
                          f32_mode: str | None = None) -> torch.Tensor:
    """Row partials of an fp32 contraction's epilogue values
    (pdh_contract_views_rowred): partials[b, r, j] = the ``reducer`` ("sum",
    "max", "min") of epi(acc)[b, r, 32 j .. 32 j + 31] (columns under n),
    fp32 [batch, m, ceil(n / 32)]. Operands as for :func:`contract_views`."""
    _require_cuda(a, bt, partials, *operands)
    B, M, N, Kd = (int(x) for x in shape)
    if a.dtype != torch.float32 or bt.dtype != torch.float32:
        raise ValueError("contract_views_rowred takes fp32 a / bt")
    if reducer not in _REDUCERS:
        raise ValueError(f"reducer {reducer!r} (sum, max, min)")
    nblk = -(-N // 32)
    if partials.dtype != torch.float32 or tuple(partials.shape) != (B, M, nblk) or not partials.is_contiguous():
        raise ValueError(f"partials must be contiguous fp32 of shape {(B, M, nblk)}")
    for t, (sb, sr, sk), rows in ((a, a_strides, M), (bt, bt_strides, N)):
        if min(sb, sr, sk) < 0 or (sk != 1 and sr != 1):
            raise ValueError("each operand needs k or its rows contiguous, with non-negative strides")
        reach = t.storage_offset() + (B - 1) * sb + (rows - 1) * sr + (Kd - 1) * sk + 1
        if reach > t.untyped_storage().nbytes() // t.element_size():
            raise ValueError("a strided operand's view reaches past its storage")
    if tuple(epi.shape[d] for d in range(3)) != (B, M, N) or epi.ndim != 3:
        raise ValueError("the epilogue's lattice must be (batch, m, n)")
    if len(operands) != epi.n_operands:
        raise ValueError(f"program reads {epi.n_operands} operands, {len(operands)} given")
    for i in range(epi.n_operands):
        if _max_offset(epi, epi.in_stride[i], 3) >= operands[i].numel():
            raise ValueError(f"epilogue operand {i}: its view reaches past the tensor")
    table = (C.c_void_p * max(1, len(operands)))(*[t.data_ptr() for t in operands])
    sa, sb_ = [int(x) for x in a_strides], [int(x) for x in bt_strides]
    _with_f32_mode(f32_mode, a.dtype, lambda: _lib.call(
        "pdh_contract_views_rowred", _ptr(a), *sa, _ptr(bt), *sb_, B, M, N, Kd, C.byref(epi), table,
        _REDUCERS[reducer], _ptr(partials), _DT[a.dtype], C.c_void_p(_stream())))
    return partials


def reduce_rows(summand: _lib.EwProgram, nk: int, epi: _lib.EwProgram, operands: list,
                out: torch.Tensor, reducer: str = "sum") -> torch.Tensor:
    """out[r] = epi(sum over the last nk summand dims of summand(r, k)): the
    rowsum / plain contraction shapes. Both programs read ``operands``."""
    _require_cuda(out, *operands)
    if out.dtype not in _DT:
        raise ValueError(f"element type {out.dtype} (f32, bf16, f16)")
    if summand.ndim != epi.ndim + nk or nk < 1:
        raise ValueError("the summand's lattice is the epilogue's plus nk reduced dims")
    for prog, nd in ((summand, summand.ndim), (epi, epi.ndim)):
        for i in range(prog.n_operands):
            t = operands[i]
            if t.dtype != out.dtype:
                raise ValueError(f"operand {i} is {t.dtype}, the output {out.dtype}")
            if _max_offset(prog, prog.in_stride[i], nd) >= t.numel():
                raise ValueError(f"operand {i}: a program's view reaches past the tensor")
    if _max_offset(epi, epi.out_stride, epi.ndim) >= out.numel():
        raise ValueError("the epilogue's output view reaches past the output tensor")
    table = (C.c_void_p * max(1, len(operands)))(*[t.data_ptr() for t in operands])
    _lib.call("pdh_reduce_rows_ex", C.byref(summand), int(nk), C.byref(epi), table, len(operands), _ptr(out),
              _DT[out.dtype], _REDUCERS[reducer], C.c_void_p(_stream()))
    return out


_SCAN = {"sum": 0, "max": 1, "min": 2, "prod": 3, "mean": 4}


def scan(x: torch.Tensor, dim: int, f: str = "sum", *, reverse: bool = False,
         out: torch.Tensor | None = None) -> torch.Tensor:
    """Inclusive prefix reduce of contiguous ``x`` along ``dim`` (tl.scan):
    sum, max, min, prod or mean (running count); ``reverse`` folds suffixes."""
    _require_cuda(x)
    if x.dtype not in _DT:
        raise ValueError(f"scan stores f32, bf16 or f16 (got {x.dtype})")
    if f not in _SCAN:
        raise ValueError(f"scan reducer {f!r} (sum, max, min, prod, mean)")
    if not x.is_contiguous():
        raise ValueError("scan takes a contiguous tensor")
    dim = dim % x.dim()
    y = torch.empty_like(x) if out is None else out
    if y.shape != x.shape or y.dtype != x.dtype or not y.is_contiguous():
        raise ValueError("out must match x's shape and element type, contiguous")
    if x.numel() == 0:
        return y
    outer = math.prod(x.shape[:dim])
    inner = math.prod(x.shape[dim + 1:])
    _lib.call("pdh_scan", _ptr(x), _ptr(y), outer, x.shape[dim], inner, _DT[x.dtype], _SCAN[f],
              1 if reverse else 0, C.c_void_p(_stream()))
    return y


def pick_decode_splits(groups: int, s: int, cus: int | None = None) -> int:
    """Splits so the (batch x kv-head x split) grid covers the chip ~8 deep,
    with at least 256 keys per split."""
    if cus is None:
        cus = _lib.lib().pdh_device_cus() or 256
    want = max(1, (8 * cus + groups - 1) // groups)
    return int(max(1, min(want, s // 256 if s >= 256 else 1)))


def probe_mfma(a32, b32, a16, b16):
    """Run the MFMA lane-layout probe; inputs are bf16 device tensors."""
    c32 = torch.empty((32, 32), dtype=torch.float32, device=a32.device)
    c16 = torch.empty((16, 16), dtype=torch.float32, device=a32.device)
    _lib.call(
        "pdh_probe_mfma", _ptr(a32), _ptr(b32), _ptr(c32), _ptr(a16), _ptr(b16), _ptr(c16), C.c_void_p(_stream())
    )
    return c32, c16
