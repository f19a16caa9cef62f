"""compile_tile_hip — the HIP seat of the reference's tile runner.

Same contract as compile_tile (conformance/triton_tile.py:662-698):

    run = compile_tile_hip(region, launch=(), prune=())
    out = run(values)   # numpy arrays positional per param, each in its
                        # param's type-dim order; returns one array in the
                        # yield's dim order, or (out, m, den) for artifacts
    run.source          # readable kernel-selection descriptor
    run.grid            # program count of the plan's launch (prod of cdivs)
    run.checked

Instead of emitting code node by node, the seat RECOGNIZES the tile region
a fusion template generated and binds it to a hand-written gfx950 kernel:

  flash tile (fusion.py:542-615)          -> pdh_flash_fwd (mask forest -> band)
  flash joint (autodiff.grad of a flash,  -> pdh_flash_fwd with (m, den) artifacts, then
    claimed whole by partition.plan_model)   pdh_flash_bwd: yields (out, *grads)
  staged row softmax (fusion.py:339-350)  -> pdh_row_softmax
  staged row statistics (layernorm core + gamma/beta epilogue) -> pdh_layernorm
  map-chain (fusion.py:844-854)           -> pdh_map_chain: the chain lowered to
                                             an elementwise register program
  contraction-epilogue, GEMM shape        -> pdh_contract: the k-tiled fold's
    (fusion.py:268-324)                      operands (prologue chains run first
                                             through pdh_map_chain), the epilogue
                                             program fused onto the accumulator

Anything else raises Untranslatable naming what it could not bind — the
refusal law of triton_tile.py:216-226 and :617-621. The runner uploads,
launches, synchronizes and downloads like the reference's; nothing in it
computes on the host.
"""

from __future__ import annotations

import contextlib
import math

import numpy as np

from .tl.fusion import FOLD_KW, contract_core, flash_step, forest_is_closed, match_rowstat, match_softmax
from .tl.ir import Node, Region, walk, walk_deep

HIP_FP = ("tile_hip", "gfx950")


class Untranslatable(Exception):
    """The region (or launch) has no binding to a HIP kernel."""


# --------------------------------------------------------------- helpers


def _carried_dims(region: Region, root=None) -> set:
    """Dims a fold scans or a reduce contracts, among the nodes ``root``
    depends on (the whole region when ``root`` is None), fold steps included."""
    if root is None:
        nodes = walk_deep(region)
    else:
        nodes = walk_deep(Region(params=region.params, body=(Node("core.yield", root.type, (root,)),)))
    out = set()
    for n in nodes:
        if n.op == "tl.fold":
            out.add(n.attr("dim"))
        if n.op == "tl.reduce":
            d = n.attr("dims")
            out.update((d,) if isinstance(d, str) else d)
    return out


def _grid(region: Region, launch: tuple) -> int:
    """Launch legality and the derived program count (triton_tile.py:598-632)."""
    y = region.body[-1].args[0]
    if y.op == "core.tuple":
        y = y.args[0]
    out_dims = {d.name: d for d in y.type.dims}
    carried = _carried_dims(region, y)  # what the first output depends on (a joint's grads reduce over t)
    grid = 1
    for name, tile in launch:
        if name not in out_dims:
            raise Untranslatable(f"launch dim {name!r} is not an output dim")
        if name in carried:
            raise Untranslatable(f"launch dim {name!r} is carried/reduced — not griddable")
        grid *= -(-out_dims[name].size // int(tile))
    return grid


def _unstage(n):
    while n.op == "tl.stage":
        n = n.args[0]
    return n


_CLOSED_PW = {
    "add": np.add, "sub": np.subtract, "mul": np.multiply, "neg": np.negative, "maximum": np.maximum,
    "minimum": np.minimum, "le": np.less_equal, "lt": np.less, "ge": np.greater_equal, "gt": np.greater,
    "eq": np.equal, "ne": np.not_equal, "where": np.where, "abs": np.abs,
}


def _eval_closed(n, t: str, s: str, ti: np.ndarray, si: np.ndarray):
    """Evaluate a closed mask forest at coordinates (ti[:, None], si[None, :])."""
    if n.op == "tl.iota":
        nm = n.attr("name")
        if nm == t:
            return ti[:, None]
        if nm == s:
            return si[None, :]
        raise Untranslatable(f"mask iota over dim {nm!r} (only {t!r}, {s!r} index the score lattice)")
    if n.op in ("core.const", "tl.const"):
        return float(n.attr("value"))
    if n.op in ("tl.repeat_like", "tl.repeat"):
        return _eval_closed(n.args[0], t, s, ti, si)
    if n.op == "tl.pointwise" and n.attr("f") in _CLOSED_PW:
        return _CLOSED_PW[n.attr("f")](*(_eval_closed(a, t, s, ti, si) for a in n.args))
    raise Untranslatable(f"mask op {n.op} ({n.attr('f')}) has no closed-form binding")


def mask_to_band(mask, t: str, s: str, T: int, S: int, block: int = 1024):
    """The closed mask forest as a band lo <= s - t <= hi (None = unbounded),
    or ("none",) when every score is live. Exact: the band is re-evaluated
    against the forest on the whole lattice; a forest that is not a band
    refuses."""
    s_idx = np.arange(S)
    lo_c, hi_c = set(), set()
    all_live = True
    firsts, lasts, empty = np.empty(T, np.int64), np.empty(T, np.int64), np.zeros(T, bool)
    for r0 in range(0, T, block):
        r1 = min(T, r0 + block)
        live = np.broadcast_to(np.asarray(_eval_closed(mask, t, s, np.arange(r0, r1), s_idx), dtype=bool),
                               (r1 - r0, S))
        if not live.all():
            all_live = False
        any_ = live.any(axis=1)
        first = np.argmax(live, axis=1)
        last = S - 1 - np.argmax(live[:, ::-1], axis=1)
        if np.any(any_ & (live.sum(axis=1) != last - first + 1)):
            raise Untranslatable("mask forest is not a band (a row's live keys are not contiguous)")
        firsts[r0:r1], lasts[r0:r1], empty[r0:r1] = first, last, ~any_
    if all_live:
        return ("none",)
    rows = np.arange(T)
    ok = ~empty
    lo_c = set((firsts - rows)[ok & (firsts > 0)].tolist())
    hi_c = set((lasts - rows)[ok & (lasts < S - 1)].tolist())
    if len(lo_c) > 1 or len(hi_c) > 1:
        raise Untranslatable("mask forest is not a band (the live window's offsets vary by row)")
    lo = lo_c.pop() if lo_c else None
    hi = hi_c.pop() if hi_c else None
    if empty.any() and hi is None and lo is None:
        raise Untranslatable("mask forest masks whole rows without a band shape")
    if empty.all():  # every row masked: a band no key satisfies
        return ("band", 1, 0)
    # verify exactly, block by block
    for r0 in range(0, T, block):
        r1 = min(T, r0 + block)
        d = s_idx[None, :] - np.arange(r0, r1)[:, None]
        want = np.ones_like(d, dtype=bool)
        if lo is not None:
            want &= d >= lo
        if hi is not None:
            want &= d <= hi
        got = np.broadcast_to(np.asarray(_eval_closed(mask, t, s, np.arange(r0, r1), s_idx), dtype=bool), want.shape)
        if not np.array_equal(got, want):
            raise Untranslatable("mask forest is not a band")
    return ("band", lo, hi)


# --------------------------------------------------------- recognizers


def recognize_flash(region: Region):
    """Bind a flash tile region: (out | (out, m, den)) over two/three fold
    nodes sharing the online-softmax step. Returns a binding dict or None."""
    y = region.body[-1].args[0]
    f_m = None
    if y.op == "core.tuple":
        if len(y.args) != 3:
            return None
        y, f_m, f_den_a = y.args
    if y.op != "tl.pointwise" or y.attr("f") != "div" or len(y.args) != 2:
        return None
    f_o, rl = y.args
    if f_o.op != "tl.fold" or rl.op != "tl.repeat_like" or rl.args[1] is not f_o:
        return None
    f_den = rl.args[0]
    folds = [f_o, f_den] + ([f_m] if f_m is not None else [])
    outs = (("final", 2), ("final", 1), ("final", 0))
    for fnode, want in zip(folds, outs):
        if fnode.op != "tl.fold" or tuple(fnode.attr("out")) != want:
            return None
        if fnode.args != f_o.args or fnode.regions != f_o.regions:
            return None
        for k, v in FOLD_KW.items():
            if fnode.attr(k) != v:
                return None
    if f_m is not None and f_den_a is not f_den:
        return None
    m0, den0, o0, qr, kt, vt, mt = f_o.args
    for c, val in ((m0, -1e30), (den0, 0.0), (o0, 0.0)):
        if c.op != "tl.const" or float(c.attr("value")) != val:
            return None
    if qr.op != "tl.repeat" or qr.attr("name") != "so" or qr.args[0].op != "core.param":
        return None
    if not (kt.op == vt.op == mt.op == "tl.split"):
        return None
    s = kt.attr("name")
    parts = kt.attr("parts")
    if vt.attr("name") != s or mt.attr("name") != s or vt.attr("parts") != parts or mt.attr("parts") != parts:
        return None
    if tuple(p for p, _ in parts) != ("so", "si"):
        return None
    q, k, v = qr.args[0], kt.args[0], vt.args[0]
    if k.op != "core.param" or v.op != "core.param":
        return None
    if len(region.params) != 3 or {id(q), id(k), id(v)} != {id(p) for p in region.params}:
        return None
    step = f_o.regions[0]
    # the step's contracted dim and fill, then the step must BE the template's step
    red_e = [n for n in walk(step) if n.op == "tl.reduce" and n.attr("f") == "sum" and contract_core(n) is not None
             and n.attr("dims") != ("si",)]
    wh = [n for n in walk(step) if n.op == "tl.pointwise" and n.attr("f") == "where"]
    if len(red_e) != 1 or len(wh) != 1 or wh[0].args[2].op != "core.const":
        return None
    e = red_e[0].attr("dims")[0]
    fill = float(wh[0].args[2].attr("value"))
    types = tuple(p.type for p in step.params)
    if step.key != flash_step(types, e, fill).key:
        return None
    t = next(nm for nm in q.type.names if nm != e)
    o = next(nm for nm in v.type.names if nm != s)
    mask = mt.args[0]
    if not forest_is_closed(mask):
        raise Untranslatable("flash mask forest reads data (the template needs a closed form)")
    if q.type.names != (t, e) and q.type.names != (e, t):
        return None
    return {
        "q": q, "k": k, "v": v, "mask": mask, "fill": fill, "t": t, "s": s, "e": e, "o": o,
        "T": q.type.dim(t).size, "S": k.type.dim(s).size, "E": q.type.dim(e).size, "OD": v.type.dim(o).size,
        "si": int(dict(parts)["si"]), "artifacts": f_m is not None,
    }


def recognize_softmax(region: Region):
    sm = match_softmax(region.body[-1].args[0])
    if sm is None or len(region.params) != 1:
        return None
    x = _unstage(sm["sm"])
    if x is not region.params[0]:
        return None
    return {"x": x, "s": sm["s"]}


def recognize_layernorm(region: Region):
    y = region.body[-1].args[0]
    gamma = beta = None
    node = y
    if node.op == "tl.pointwise" and node.attr("f") == "add" and len(node.args) == 2 and node.args[1].op == "tl.repeat_like":
        beta = _unstage(node.args[1].args[0])
        node = node.args[0]
    if node.op == "tl.pointwise" and node.attr("f") == "mul" and len(node.args) == 2 and node.args[1].op == "tl.repeat_like":
        gamma = _unstage(node.args[1].args[0])
        node = node.args[0]
    rs = match_rowstat(node)
    if rs is None:
        return None
    x = _unstage(rs["x"])
    feat = rs["feat"]
    want = [p for p in (x, gamma, beta) if p is not None]
    if any(p.op != "core.param" for p in want) or {id(p) for p in want} != {id(p) for p in region.params}:
        return None
    for p in (gamma, beta):
        if p is not None and p.type.names != (feat,):
            return None
    return {"x": x, "feat": feat, "eps": rs["eps"], "gamma": gamma, "beta": beta}


# ------------------------------------------------------------- runners


def _torch():
    import torch

    if not torch.cuda.is_available():
        raise RuntimeError("compile_tile_hip runners launch HIP kernels: no GPU is visible")
    return torch


def _index(region, node):
    return next(i for i, p in enumerate(region.params) if p is node)


def compile_tile_hip(region: Region, launch: tuple = (), prune: tuple = (), *, dtype: str = "f32"):
    """Bind a template tile region to a gfx950 kernel; see the module doc."""
    grid = _grid(region, tuple(launch))
    if dtype not in ("f32", "bf16", "f16"):
        raise Untranslatable(f"element type {dtype!r} (f32, bf16, f16)")

    fb = recognize_flash(region)
    if fb is not None:
        return _flash_runner(region, fb, grid, bool(prune), dtype)
    from .tl.partition import match_flash_joint

    fj = match_flash_joint(region)
    if fj is not None:
        return _flash_joint_runner(region, fj, grid, dtype)
    sb = recognize_softmax(region)
    if sb is not None:
        return _softmax_runner(region, sb, grid, dtype)
    lb = recognize_layernorm(region)
    if lb is not None:
        return _layernorm_runner(region, lb, grid, dtype)
    cb = recognize_contraction(region)
    if cb is not None and cb["shape"] != "gemm":
        return _reduce_runner(region, cb, grid, dtype)
    if cb is not None:
        return _contraction_runner(region, cb, grid, dtype)
    if recognize_map_chain(region):
        return _map_chain_runner(region, grid, dtype)
    ops = sorted({n.op for n in walk(region)} - {"core.param", "core.yield"})
    raise Untranslatable(
        f"no HIP binding for this tile region (ops: {', '.join(ops)}); bound templates: flash, "
        "row-normalization, row-statistics, flash-joint, map-chain, contraction-epilogue (GEMM shape)"
    )


def _finish(dev, source: str, grid: int, template: str, region: Region, dtype: str):
    """The seat's ``run(values)`` over the device form ``run.run_dev``.

    ``run_dev(tensors, stream=None)`` takes device tensors positional per
    param, each laid out in its param's type-dim order (any float dtype;
    converted to the column's), launches on ``stream`` (a torch stream; the
    current one when None) and returns device tensors in
    the yield's type-dim order, without synchronizing: the per-call host
    copies stay out of a benchmark's timed region. ``run(values)`` is the
    reference runner's contract (triton_tile.py:662-698): numpy in, upload,
    launch, synchronize, numpy out."""
    shapes = [tuple(d.size for d in p.type.dims) for p in region.params]

    def run_dev(tensors, stream=None):
        torch = _torch()
        tdt = getattr(torch, _TORCH_DT[dtype])
        if len(tensors) != len(shapes):
            raise ValueError(f"{len(tensors)} param tensors given, the region has {len(shapes)} params")
        for t, shp in zip(tensors, shapes):
            if tuple(t.shape) != shp:
                raise ValueError(f"a param tensor has shape {tuple(t.shape)}, the region wants {shp}")
        with torch.cuda.stream(stream) if stream is not None else contextlib.nullcontext():
            return dev([t.to(device="cuda", dtype=tdt).contiguous() for t in tensors])

    def run(values):
        torch = _torch()
        got = run_dev([torch.as_tensor(np.asarray(v, dtype=np.float32)) for v in values])
        torch.cuda.synchronize()
        if isinstance(got, tuple):
            return tuple(g.float().cpu().numpy() for g in got)
        return got.float().cpu().numpy()

    run.run_dev = run_dev
    run.source = source
    run.grid = grid
    run.checked = True  # precision is by construction: the MFMA / VALU instruction is chosen, not inferred
    run.template = template
    return run


def _flash_runner(region, fb, grid, prune, dtype):
    from . import kernels as K

    T, S, E, OD = fb["T"], fb["S"], fb["E"], fb["OD"]
    band = mask_to_band(fb["mask"], fb["t"], fb["s"], T, S)
    kband = None if band[0] == "none" else K.Band(band[1], band[2])
    if dtype != "f32" and not (E == OD and E in (64, 128)):
        raise Untranslatable(f"{dtype} flash needs e == od in {{64, 128}} (got {E}, {OD})")
    iq, ik, iv = (_index(region, fb[x]) for x in ("q", "k", "v"))
    tq = fb["q"].type.names

    def dev(ts):
        def mat(t, names, want, rows, cols):
            return (t if names == want else t.t()).contiguous().view(1, 1, rows, cols)

        res = K.flash_fwd(mat(ts[iq], tq, (fb["t"], fb["e"]), T, E), mat(ts[ik], fb["k"].type.names, (fb["s"], fb["e"]), S, E),
                          mat(ts[iv], fb["v"].type.names, (fb["s"], fb["o"]), S, OD), scale=1.0, band=kband,
                          fill=fb["fill"], prune=prune, want_lse=False, want_artifacts=fb["artifacts"])
        out = res.o.view(T, OD)
        if fb["artifacts"]:
            return out, res.m.view(T), res.den.view(T)
        return out

    kern = "flash_fwd_generic_f32" if dtype == "f32" else f"flash_fwd_m16<{dtype},{E}>"
    bdesc = "all" if kband is None else f"band({band[1]},{band[2]})"
    src = (
        f"hip:{kern} t={T} s={S} e={E} od={OD} si={fb['si']} mask={bdesc} fill={fb['fill']:g} "
        f"prune={'on' if prune else 'off'} sweeps=1 stores={3 if fb['artifacts'] else 1}"
    )
    return _finish(dev, src, grid, "flash", region, dtype)


def _softmax_runner(region, sb, grid, dtype="f32"):
    from . import kernels as K

    names = sb["x"].type.names
    s = sb["s"]
    out_names = region.body[-1].args[0].type.names

    def dev(ts):
        order = tuple(n for n in names if n != s) + (s,)
        x = ts[0].permute([names.index(n) for n in order]).contiguous()
        y = K.row_softmax(x)
        return y.permute([order.index(n) for n in out_names])

    n_rows = math.prod(d.size for d in sb["x"].type.dims if d.name != s)
    src = f"hip:row_softmax rows={n_rows} cols={sb['x'].type.dim(s).size} reduce={s} dtype={dtype} sweeps=1 stores=1"
    return _finish(dev, src, grid, "row-normalization", region, dtype)


def _layernorm_runner(region, lb, grid, dtype="f32"):
    from . import kernels as K

    names = lb["x"].type.names
    feat = lb["feat"]
    out_names = region.body[-1].args[0].type.names
    ix = _index(region, lb["x"])
    ig = _index(region, lb["gamma"]) if lb["gamma"] is not None else None
    ib = _index(region, lb["beta"]) if lb["beta"] is not None else None

    def dev(ts):
        order = tuple(n for n in names if n != feat) + (feat,)
        x = ts[ix].permute([names.index(n) for n in order]).contiguous()
        y = K.layernorm(x, None if ig is None else ts[ig], None if ib is None else ts[ib], eps=lb["eps"])
        return y.permute([order.index(n) for n in out_names])

    n_rows = math.prod(d.size for d in lb["x"].type.dims if d.name != feat)
    src = (
        f"hip:layernorm rows={n_rows} cols={lb['x'].type.dim(feat).size} mean/N=/ {lb['x'].type.dim(feat).size} "
        f"eps={lb['eps']:g} affine={'gamma' if ig is not None else ''}{'+beta' if ib is not None else ''} dtype={dtype} "
        "sweeps=1 stores=1"
    )
    return _finish(dev, src, grid, "row-statistics", region, dtype)


def _flash_joint_runner(region, fj, grid, dtype):
    """(out, *grads) of a flash joint: the forward with its (m, den)
    artifacts, then the fused backward seeded by the joint's last param."""
    from . import kernels as K

    q_, k_, v_ = fj["q"], fj["k"], fj["v"]
    t, s, e, o = fj["t"], fj["s"], fj["e"], fj["o"]
    T, S, E, OD = q_.type.dim(t).size, k_.type.dim(s).size, q_.type.dim(e).size, v_.type.dim(o).size
    band = mask_to_band(fj["mask"], t, s, T, S)
    kband = None if band[0] == "none" else K.Band(band[1], band[2])
    if dtype != "f32" and not (E == OD and E in (64, 128)):
        raise Untranslatable(f"{dtype} flash joint needs e == od in {{64, 128}} (got {E}, {OD})")
    iq, ik, iv = (_index(region, x) for x in (q_, k_, v_))
    iseed = len(region.params) - 1
    y = region.body[-1].args[0]
    grad_types = [g.type for g in y.args[1:]]
    wrt = fj["wrt"]
    out_names = y.args[0].type.names

    def dev(ts):
        def mat(t, node, order, rows, cols):
            return t.permute([node.type.names.index(n) for n in order]).contiguous().view(1, 1, rows, cols)

        q = mat(ts[iq], q_, (t, e), T, E)
        k = mat(ts[ik], k_, (s, e), S, E)
        v = mat(ts[iv], v_, (s, o), S, OD)
        do = mat(ts[iseed], region.params[iseed], (t, o), T, OD)
        res = K.flash_fwd(q, k, v, scale=1.0, band=kband, fill=fj["fill"], want_artifacts=True)
        dq, dk, dv = K.flash_bwd(q, k, v, res.o, do, res.lse, m=res.m, den=res.den, scale=1.0, band=kband,
                                 fill=fj["fill"])
        outs = {"q": (dq.view(T, E), (t, e)), "k": (dk.view(S, E), (s, e)), "v": (dv.view(S, OD), (s, o))}
        ys = [res.o.view(T, OD).permute([(t, o).index(n) for n in out_names])]
        for nm, gt in zip(wrt, grad_types):
            x, order = outs[nm]
            ys.append(x.permute([order.index(n) for n in gt.names]))
        return tuple(ys)

    kern = "flash_fwd_generic_f32 + bwd_rows_f32" if dtype == "f32" else f"flash_fwd_m16<{dtype},{E}> + bwd_main<{dtype},{E}>"
    bdesc = "all" if kband is None else f"band({band[1]},{band[2]})"
    src = (
        f"hip:{kern} t={T} s={S} e={E} od={OD} mask={bdesc} fill={fj['fill']:g} wrt={','.join(wrt)} "
        "artifacts=m,den launches=fwd+bwd"
    )
    return _finish(dev, src, grid, "flash-joint", region, dtype)


# ------------------------------------------- map-chain and contraction-epilogue

_CHAIN_OPS = {"core.param", "core.yield", "core.const", "tl.const", "tl.iota", "tl.pointwise", "tl.repeat_like",
              "tl.repeat", "tl.stage", "tl.rename", "tl.shift", "tl.slice", "tl.window", "tl.decimate", "tl.diagonal"}
_TORCH_DT = {"f32": "float32", "bf16": "bfloat16", "f16": "float16"}


def recognize_map_chain(region: Region) -> bool:
    y = region.body[-1].args[0]
    if y.op == "core.tuple" or not hasattr(y.type, "dims") or not y.type.dims:
        return False
    return all(n.op in _CHAIN_OPS for n in walk(region))


def _arrange(torch, t, names, order, pad_last=None):
    """A device tensor with dims ``names`` as a contiguous tensor with dims
    ``order`` (absent dims as size 1), optionally zero-padded in the last dim
    to ``pad_last``."""
    x = t.permute([names.index(n) for n in order if n in names]).contiguous()
    shape = [t.shape[names.index(n)] if n in names else 1 for n in order]
    x = x.reshape(shape)
    if pad_last is not None and pad_last != shape[-1]:
        full = torch.zeros(shape[:-1] + [pad_last], device="cuda", dtype=t.dtype)
        full[..., : shape[-1]] = x
        x = full
    return x


def _map_chain_runner(region, grid, dtype):
    from . import ewprog
    from . import kernels as K

    y = region.body[-1].args[0]
    dims = y.type.dims
    leaves = {id(p): p for p in region.params}
    try:
        low = ewprog.lower(y, dims, leaves, allow_views=True)
    except ewprog.Unlowerable as exc:
        raise Untranslatable(f"map-chain: {exc}") from None
    idx = [_index(region, p) for p in low.bases]
    out_names = y.type.names
    shifted = low.offset_reads()

    def dev(ts):
        torch = _torch()
        ops, strides = [], []
        for j, (i, base) in enumerate(zip(idx, low.bases)):
            t = ts[i]  # each param once; shifted reads are offset views of it
            st, off = low.operand_view(j, dict(zip(base.type.names, t.stride())))
            if off < 0:
                raise Untranslatable("a shifted read starts before its tensor")
            ops.append(t.reshape(-1)[off:])
            strides.append(st)
        out = torch.empty(tuple(d.size for d in dims), device="cuda", dtype=getattr(torch, _TORCH_DT[dtype]))
        K.map_chain(low.program(out.stride(), strides), ops, out)
        return out

    tmpl = "stencil" if shifted else "map-chain"
    src = (f"hip:map_chain lattice=({','.join(out_names)}) insns={len(low.insns)} operands={len(low.operands)} "
           f"shifted_reads={shifted} sweeps=1 stores=1")
    return _finish(dev, src, grid, tmpl, region, dtype)


def recognize_contraction(region: Region):
    """Bind a contraction-epilogue tile (fusion.py:268-324): the k-tiled
    accumulation fold over split operand chains, an epilogue over its result.
    Returns the binding or None; shapes other than GEMM raise Untranslatable."""
    folds = [n for n in walk(region) if n.op == "tl.fold"]
    if len(folds) != 1:
        return None
    f = folds[0]
    if tuple(f.attr("state")) != ("acc",) or f.attr("dim") != "ko" or tuple(f.attr("out")) != ("final", 0):
        return None
    init, *srcs = f.args
    if init.op != "tl.const" or float(init.attr("value")) != 0.0:
        return None
    if not srcs or any(x.op != "tl.split" for x in srcs):
        return None
    k = srcs[0].attr("name")
    parts = tuple(srcs[0].attr("parts"))
    if tuple(p for p, _ in parts) != ("ko", "ki") or any(x.attr("name") != k or tuple(x.attr("parts")) != parts
                                                        for x in srcs):
        return None
    step = f.regions[0]
    y = step.body[-1].args[0]
    if y.op != "tl.pointwise" or y.attr("f") != "add" or y.args[0] is not step.params[0]:
        return None
    part = y.args[1]
    if part.op != "tl.reduce" or part.attr("f") != "sum":
        return None
    rdims = (part.attr("dims"),) if isinstance(part.attr("dims"), str) else tuple(part.attr("dims"))
    contracted = (k,) + tuple(d for d in rdims if d != "ki")
    prod = part.args[0]
    if len(srcs) == 1:  # PLAIN: the one operand chain summed
        if prod.op != "tl.stage" or prod.args[0] is not step.params[1]:
            return None
        return {"fold": f, "k": k, "shape": "plain", "a": srcs[0].args[0], "b": None, "contracted": contracted}
    if len(srcs) != 2:
        return None
    if prod.op == "tl.pointwise" and prod.attr("f") == "mul" and all(x.op == "tl.stage" for x in prod.args) and \
            prod.args[0].args[0] is step.params[1] and prod.args[1].args[0] is step.params[2]:
        return {"fold": f, "k": k, "shape": "rowsum", "a": srcs[0].args[0], "b": srcs[1].args[0],
                "contracted": contracted}
    a_s = b_s = None
    if prod.op == "tl.pointwise" and prod.attr("f") == "mul" and all(x.op == "tl.repeat_like" for x in prod.args):
        a_s, b_s = prod.args[0].args[0], prod.args[1].args[0]
    if a_s is None or a_s.op != "tl.stage" or b_s.op != "tl.stage" or a_s.args[0] is not step.params[1] \
            or b_s.args[0] is not step.params[2]:
        return None
    if rdims != ("ki",):
        raise Untranslatable(f"contraction-epilogue: one contracted dim on HIP (the step reduces {rdims})")
    ca, cb = srcs[0].args[0], srcs[1].args[0]
    keep_a = [nm for nm in ca.type.names if nm != k]
    keep_b = [nm for nm in cb.type.names if nm != k]
    riders = [nm for nm in keep_a if nm in keep_b]
    mdims = [nm for nm in keep_a if nm not in riders]
    ndims = [nm for nm in keep_b if nm not in riders]
    if len(riders) > 1 or len(mdims) > 1 or len(ndims) > 1:
        raise Untranslatable("contraction-epilogue: at most one batch, one m and one n dim on HIP")
    return {"fold": f, "k": k, "a": ca, "b": cb, "rider": riders[0] if riders else None,
            "m": mdims[0] if mdims else None, "n": ndims[0] if ndims else None,
            "K": ca.type.dim(k).size, "shape": "gemm"}


def _reduce_runner(region, cb, grid, dtype):
    """The ROWSUM / PLAIN shapes: the summand (the same-space product, or the
    one operand chain) over (output dims..., contracted dims...) summed by
    pdh_reduce_rows, the epilogue on the sum."""
    from . import ewprog
    from . import kernels as K
    from .tl.dialect import OPS
    from .tl.ir import Builder, Dim

    y = region.body[-1].args[0]
    if y.op == "core.tuple":
        raise Untranslatable("contraction-epilogue with several yields")
    fold, ca, cbn = cb["fold"], cb["a"], cb["b"]
    summand = ca if cb["shape"] == "plain" else Builder(OPS).emit("tl.pointwise", ca, cbn, f="mul")
    rows = tuple(fold.type.dims) or (Dim("_unit_r", 0, 1),)
    kdims = tuple(d for d in ca.type.dims if d.name in cb["contracted"])
    lat = rows + kdims
    if len(lat) > 4:
        raise Untranslatable(f"a reduction over {len(lat)} lattice dims (max 4)")
    leaves = {id(p): p for p in region.params}
    try:
        ls = ewprog.lower(summand, lat, leaves)
        le = ewprog.lower(y, rows, leaves, acc=fold)
    except ewprog.Unlowerable as exc:
        raise Untranslatable(f"row reduction: {exc}") from None
    idx = [_index(region, b) for b in ls.bases + le.bases]
    nodes = ls.operands + le.operands
    n_s = len(ls.operands)

    def dev(ts):
        torch = _torch()
        ops = [ts[i] for i in idx]
        st = [ewprog.strides_over(t.stride(), nd.type.names, lat) for t, nd in zip(ops[:n_s], nodes[:n_s])]
        se = [ewprog.strides_over(t.stride(), nd.type.names, rows) for t, nd in zip(ops[n_s:], nodes[n_s:])]
        out = torch.empty(tuple(d.size for d in rows), device="cuda", dtype=getattr(torch, _TORCH_DT[dtype]))
        ps = ewprog.with_slots(ls.program([0] * len(lat), st), 0, len(ops))
        pe = ewprog.with_slots(le.program(out.stride(), se), n_s, len(ops))
        K.reduce_rows(ps, len(kdims), pe, ops, out)
        if not y.type.dims:
            return out.reshape(())
        names = [d.name for d in rows]
        return out.permute([names.index(nm) for nm in y.type.names])

    src = (f"hip:reduce_rows shape={cb['shape']} rows={math.prod(d.size for d in rows)} "
           f"k={math.prod(d.size for d in kdims)} summand_insns={len(ls.insns)} epilogue_insns={len(le.insns)} stores=1")
    return _finish(dev, src, grid, "contraction-epilogue", region, dtype)


def _contraction_runner(region, cb, grid, dtype):
    from . import ewprog
    from .tl.ir import Dim
    from . import kernels as K

    y = region.body[-1].args[0]
    if y.op == "core.tuple":
        raise Untranslatable("contraction-epilogue with several yields")
    fold = cb["fold"]
    out_t = fold.type
    size = {d.name: d for d in out_t.dims}
    lattice = tuple(size[nm] if nm is not None else Dim(f"_unit{i}", 0, 1)
                    for i, nm in enumerate((cb["rider"], cb["m"], cb["n"])))
    lnames = tuple(d.name for d in lattice)
    leaves = {id(p): p for p in region.params}
    try:
        epi = ewprog.lower(y, lattice, leaves, acc=fold)
    except ewprog.Unlowerable as exc:
        raise Untranslatable(f"contraction epilogue: {exc}") from None
    Kdim = cb["K"]
    KP = -(-Kdim // 64) * 64
    k = cb["k"]
    B_, M_, N_ = (d.size for d in lattice)
    a_order = (lnames[0], lnames[1], k)
    b_order = (lnames[0], lnames[2], k)

    def operand(node, order):
        """A param uploads as is. A prologue chain is computed in the k loop
        (pdh_contract_views_pro) at fp32 and bf16 (where the other operand,
        a param, is then read by a one-LOAD program), and runs first through
        pdh_map_chain at f16."""
        if node.op == "core.param":
            return ("param", _index(region, node))
        adims = tuple(size.get(nm) or (node.type.dim(nm) if node.type.has(nm) else Dim(nm, 0, 1)) for nm in order)
        try:
            low = ewprog.lower(node, adims, leaves)
        except ewprog.Unlowerable as exc:
            raise Untranslatable(f"contraction prologue: {exc}") from None
        return ("chain", low)

    pa, pb = operand(cb["a"], a_order), operand(cb["b"], b_order)
    epi_idx = [_index(region, p) for p in epi.bases]

    fused = dtype in ("f32", "bf16") and "chain" in (pa[0], pb[0])

    def dev(ts):
        torch = _torch()
        tdt = getattr(torch, _TORCH_DT[dtype])

        def prologue(spec, rows):
            """(program over (batch, rows, k), its operands) of a chain operand."""
            low = spec[1]
            ins = [ts[_index(region, b)] for b in low.bases]
            st = [ewprog.strides_over(t.stride(), p.type.names, low.dims) for t, p in zip(ins, low.operands)]
            return low.program((rows * Kdim, Kdim, 1), st), ins

        def build(spec, node, order, rows):
            if spec[0] == "param":
                return _arrange(torch, ts[spec[1]], node.type.names, order, pad_last=KP)
            low = spec[1]
            ins = [ts[_index(region, b)] for b in low.bases]
            st = [ewprog.strides_over(t.stride(), p.type.names, low.dims) for t, p in zip(ins, low.operands)]
            buf = torch.zeros((low.dims[0].size, rows, KP), device="cuda", dtype=tdt)
            K.map_chain(low.program(buf.stride(), st), ins, buf)
            return buf

        ops = [ts[i] for i in epi_idx]
        st = [ewprog.strides_over(t.stride(), p.type.names, lattice) for t, p in zip(ops, epi.operands)]
        out = torch.empty((B_, M_, N_), device="cuda", dtype=tdt)
        if fused:  # chain operands evaluated in the k loop, params read as packed
            sides = []
            for spec, node, order, rows in ((pa, cb["a"], a_order, M_), (pb, cb["b"], b_order, N_)):
                if spec[0] == "chain":
                    sides.append((None, None, prologue(spec, rows)))
                elif dtype == "bf16":  # both computed at 16 bits: the param through a one-LOAD program
                    t = _arrange(torch, ts[spec[1]], node.type.names, order)
                    sides.append((None, None, (K.view_program(tuple(t.shape), t.stride()), [t])))
                else:
                    t = build(spec, node, order, rows)
                    sides.append((t, t.stride(), None))
            (a, sta, pra), (bt, stb, prb) = sides
            K.contract_views_pro(a, sta, bt, stb, (B_, M_, N_, Kdim), epi.program(out.stride(), st), ops, out,
                                 pro_a=pra, pro_b=prb)
        else:
            a = build(pa, cb["a"], a_order, M_)
            bt = build(pb, cb["b"], b_order, N_)
            K.contract(a, bt, Kdim, epi.program(out.stride(), st), ops, out)
        present = [nm for nm in lnames if nm in y.type.names]  # the unit stand-ins drop out
        full = out.reshape(tuple(size[nm].size for nm in present))
        return full.permute([present.index(nm) for nm in y.type.names])

    kern = "contract_views_pro" if fused else ("contract_f32" if dtype == "f32" else f"contract_mfma<{dtype}>")
    src = (f"hip:{kern} batch={B_} m={M_} n={N_} k={Kdim} kp={KP} prologue={pa[0]},{pb[0]} "
           f"epilogue_insns={len(epi.insns)} operands={len(epi.operands)} stores=1")
    return _finish(dev, src, grid, "contraction-epilogue", region, dtype)
